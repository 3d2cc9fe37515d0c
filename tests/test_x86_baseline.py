"""CPU tests of the x86 restatement of the reference's CPU QMatMul (oracle/x86.c), the timed CPU baseline.

The reference on x86-64 runs repacked 16-row tiles with vpdpbusd (AVX-512 VNNI, AVX-VNNI or AVX2) and AMX for
Q4_K at m >= 32 (crates/inference-tensor/src/quantized/repack_x86.rs, repack.rs:232-262), or avx.rs's AVX2
vec_dot where select() declines the tiles.  Its sums are the same integer block dots with the f32 scaling
regrouped (d*sc pre-multiplied per row, the min term through the bsums), so each path is held to the scalar
oracle and to a float64 brute force over the dequantized operands within f32 reordering error, at every
instruction level this host can run, on the route select() picks.
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import assert_parity, terms

LEVELS = {3: {}, 2: {"MISTRALRS_FORCE_AVXVNNI": "1"}, 1: {"MISTRALRS_FORCE_AVX2": "1"}}


def cpu_flags():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def runnable_levels():
    flags = cpu_flags()
    out = []
    if "avx512_vnni" in flags and "avx512f" in flags:
        out.append(3)
    if "avx_vnni" in flags and "avx2" in flags:
        out.append(2)  # forcing AVX-VNNI on a CPU without it would run instructions it lacks
    if "avx2" in flags and "fma" in flags:
        out.append(1)
    return out


@pytest.fixture(params=runnable_levels() or [None])
def level(request, monkeypatch):
    if request.param is None:
        pytest.skip("host has no AVX2")
    for k, v in LEVELS[request.param].items():
        monkeypatch.setenv(k, v)
    assert O.x86_level() == request.param
    return request.param


def brute(gtype, x, wq, n):
    import test_oracle as T
    m, k = x.shape
    a = T.NP_DEQUANT[O.ACT_TYPE[gtype]](O.quantize(O.ACT_TYPE[gtype], x)).reshape(m, k).astype(np.float64)
    w = T.NP_DEQUANT[gtype](wq).reshape(n, k).astype(np.float64)
    return a @ w.T


@pytest.mark.parametrize("gtype,n,k", [(O.Q4K, 48, 768), (O.Q6K, 32, 512), (O.Q8_0, 32, 512), (O.Q8_0, 16, 352)])
@pytest.mark.parametrize("m", [1, 2, 4, 7, 33])
def test_x86_path_matches_oracle_and_brute_force(level, gtype, n, k, m):
    rng = np.random.default_rng(1000 * gtype + 10 * m + level)
    wq = O.quantize(gtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    got, path = O.X86Weight(gtype, wq, n, k).matmul(x, threads=3)
    want_path = "tiles"
    if gtype == O.Q6K and m == 1 or gtype == O.Q8_0 and m == 1 and level == 1:
        want_path = "compact_avx2"  # select() keeps these on the compact blocks (repack_x86.rs:112-117)
    elif gtype == O.Q4K and m >= 32 and O.x86_amx():
        want_path = "amx"
    assert path == want_path
    t = terms(gtype, x, wq, n)
    assert_parity(got, O.matmul(gtype, x, wq, n), t, what=f"vs oracle {path}")
    assert_parity(got, brute(gtype, x, wq, n), t, what=f"vs float64 {path}")


def test_x86_shapes_the_tiles_do_not_take_fall_back():
    """n not a multiple of 16 (select() declines, repack_x86.rs:106-108): the scalar vec_dot route."""
    rng = np.random.default_rng(5)
    n, k = 24 + 3, 512
    wq = O.quantize(O.Q4K, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((3, k)).astype(np.float32)
    got, path = O.X86Weight(O.Q4K, wq, n, k).matmul(x)
    assert path == "scalar"
    assert np.array_equal(got, O.matmul(O.Q4K, x, wq, n))


def test_x86_select_matches_the_reference_rules():
    lv = O.x86_level()
    sel = O.lib().oracle_x86_select
    assert sel(O.Q4K, 1, 4096, 4096) == 1
    assert sel(O.Q6K, 1, 4096, 4096) == 0 and sel(O.Q6K, 2, 4096, 4096) == 1
    assert sel(O.Q8_0, 1, 4096, 4096) == (1 if lv != 1 else 0)
    assert sel(O.Q4K, 4, 4100, 4096) == 0  # n % 16
    assert sel(O.Q4K, 4, 4096, 4000) == 0  # k % 256
    assert sel(O.Q8_0, 4, 4096, 4000) == 1  # Q8_0 rows of whole 32-value blocks, padded to superblocks
    assert sel(O.Q5K, 4, 4096, 4096) == 0


def test_x86_threads_do_not_change_the_result():
    """Each output is computed by one unit whatever the thread count, so the bits cannot depend on it."""
    rng = np.random.default_rng(9)
    n, k = 64, 1024
    wq = O.quantize(O.Q4K, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w = O.X86Weight(O.Q4K, wq, n, k)
    x = rng.standard_normal((40, k)).astype(np.float32)
    a, _ = w.matmul(x, threads=1)
    b, _ = w.matmul(x, threads=5)
    assert np.array_equal(a, b)


def test_x86_q8_0_zero_and_tied_blocks():
    """Zero activation blocks (d = 0, sums = 0) and a weight row of zeros through the +128 offset tiles."""
    rng = np.random.default_rng(11)
    n, k = 16, 256
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[3] = 0.0
    wq = O.quantize(O.Q8_0, w)
    x = rng.standard_normal((2, k)).astype(np.float32)
    x[0, 64:160] = 0.0
    x[1, :] = 0.0
    got, _ = O.X86Weight(O.Q8_0, wq, n, k).matmul(x)
    want = O.matmul(O.Q8_0, x, wq, n)
    assert np.all(got[1] == 0.0) and np.all(got[:, 3] == 0.0)
    assert_parity(got, want, terms(O.Q8_0, x, wq, n))


def test_x86_describe_names_the_level():
    s = O.x86_describe()
    assert any(name in s for name in ("AVX-512 VNNI", "AVX-VNNI", "AVX2", "no AVX2"))
    assert O.x86_physical_cores() >= 1
    assert "MISTRALRS_FORCE_AVX2" not in os.environ
