"""The committed golden fixtures (tests/golden/, written by tests/golden/make_goldens.py from the C oracle):
the oracle and the host quantizer must still reproduce them exactly.  A change in either shows up here as a
byte or bit difference against data that was produced before the change."""
import ctypes
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = {O.Q8_0: "q8_0", O.Q4K: "q4_k", O.Q6K: "q6_k"}
SEED = 20260601  # tests/golden/make_goldens.py


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


@pytest.mark.parametrize("gtype", list(TYPES))
def test_oracle_reproduces_the_qmatmul_fixture(gtype):
    g = load(f"qmatmul_{TYPES[gtype]}.npz")
    n, k = int(g["n"]), int(g["k"])
    assert np.array_equal(O.quantize(O.ACT_TYPE[gtype], g["x"]).reshape(-1), g["xq_bytes"].reshape(-1))
    y = O.matmul(gtype, g["x"], g["w_bytes"].reshape(-1), n)
    assert np.array_equal(y.astype(np.float32), g["y"])
    # the weight bytes come from the seeded generator through the restated reference quantizer
    rng = np.random.default_rng(SEED + gtype)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    assert np.array_equal(O.quantize(gtype, w).reshape(-1), g["w_bytes"].reshape(-1))


def test_oracle_reproduces_the_indexed_moe_fixture():
    g = load("indexed_moe_q4_k.npz")
    e, n, k = int(g["experts"]), int(g["n"]), int(g["k"])
    y = O.indexed_moe(O.Q4K, g["w_bytes"].reshape(-1), e, n, k, g["x"], g["ids"])
    assert np.array_equal(y, g["y"])


@pytest.mark.parametrize("gtype", list(TYPES))
def test_host_quantizer_reproduces_the_fixture(gtype):
    """The C++ host layer's CPU quantizers (QTensor::quantize) write the fixture's activation blocks."""
    import qmm
    host = ctypes.CDLL(qmm.HOST_LIB_PATH)
    host.qmm_quantize_cpu.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    g = load(f"qmatmul_{TYPES[gtype]}.npz")
    x = np.ascontiguousarray(g["x"])
    out = np.zeros(g["xq_bytes"].size, dtype=np.uint8)
    assert host.qmm_quantize_cpu(O.ACT_TYPE[gtype], x.ctypes.data, x.size, out.ctypes.data) == 0
    assert np.array_equal(out, g["xq_bytes"].reshape(-1))
