"""CPU test of the decode matvec's kernel-form rule (qmm_decode_form, the rule the launchers apply): every row's units
fit the kernel it takes, and the unguarded form is taken only where the row fills every lane's units exactly.  A row
of 192 units once took the unguarded four-unit form and read a fourth unit past its end."""
import ctypes

import pytest

import qmm

TYPES = [(qmm.Q4K, 0), (qmm.Q6K, 0), (qmm.Q5K, 0), (qmm.IQ4XS, 0), (qmm.Q8_0, 0), (qmm.Q4_0, 0), (qmm.Q5_0, 0),
         (qmm.Q8_0, 1), (qmm.Q4_0, 1), (qmm.Q5_0, 1)]


def form(t, k, nc, q8_0):
    out = (ctypes.c_int * 4)()
    assert qmm.lib().qmm_decode_form(t, k, nc, q8_0, out) == 0, qmm.last_error()
    return tuple(out)


@pytest.mark.parametrize("t,q8_0", TYPES)
def test_units_fit_the_form(t, q8_0):
    bs = qmm.BLOCK_SIZE[t]
    seen = set()
    for k in range(bs if bs == 256 else 64, 24577, bs if bs == 256 else 64):
        for nc in range(1, 9):
            kernel, s, full, units = form(t, k, nc, q8_0)
            seen.add(units)
            if kernel == 2:  # k_mmvq takes any row in passes
                assert units > 64 * 4 and not full
                continue
            cap = 256 if kernel == 1 else 64 * s
            assert s in (1, 2, 4)
            assert units <= cap, (k, nc, units, cap)
            assert full == (units == cap), (k, nc, units, cap, full)
            if kernel == 1:
                assert 128 < units <= 256 and nc <= 2
    for u in (192, 224, 256):  # three, three-and-a-half and four units per lane
        assert u in seen, u


@pytest.mark.parametrize("t,q8_0,k", [(qmm.Q6K, 0, 12288), (qmm.Q4K, 0, 12288), (qmm.Q8_0, 1, 12288)])
def test_192_unit_rows_are_guarded(t, q8_0, k):
    for nc in range(1, 9):
        kernel, s, full, units = form(t, k, nc, q8_0)
        assert not full, (nc, kernel, s, units)


def test_bad_arguments():
    out = (ctypes.c_int * 4)()
    L = qmm.lib()
    assert L.qmm_decode_form(qmm.Q4K, 100, 1, 0, out) == -1
    assert "decode_form" in qmm.last_error()
    L.qmm_clear_error()
    assert L.qmm_decode_form(qmm.Q4K, 256, 9, 0, out) == -1
    L.qmm_clear_error()
    assert L.qmm_decode_form(qmm.Q4K, 256, 1, 1, out) == -1
    L.qmm_clear_error()
