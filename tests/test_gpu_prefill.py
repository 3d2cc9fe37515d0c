"""GPU parity of the prefill path through the C ABI: the tile-layout Q8_K / Q8_0 quantizers (bit-exact) and the
int8-MFMA matmul for Q4_K / Q6_K / Q8_0 and, on the Q8_0 kernel, Q4_0 / Q5_0 (max rel. error <= 1e-3 against the
oracle's CPU QMatMul)."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, terms, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def tiles_to_blocks(buf, rows, kp, at):
    """Prefill tile layout -> the oracle's block array [rows, nsb] (bytes)."""
    nsb = kp // 256
    b = buf[: rows * nsb * (292 if at == O.Q8K else 272)]
    qs = b[: nsb * rows * 256].reshape(nsb, rows, 256)
    if at == O.Q8K:
        d = b[nsb * rows * 256: nsb * rows * 260].view(np.float32).reshape(nsb, rows)
        # bsums are stored as f16 (exact for |bsum| <= 2048)
        bs = b[nsb * rows * 260:].view(np.float16).reshape(nsb, rows, 16).astype(np.int16)
        out = np.zeros((rows, nsb), dtype=O.BLOCK_DTYPES[O.Q8K])
        out["d"] = d.T
        out["qs"] = qs.transpose(1, 0, 2)
        out["bsums"] = bs.transpose(1, 0, 2)
        return out.view(np.uint8).reshape(-1)
    d8 = b[nsb * rows * 256:].view(np.uint16).reshape(nsb, rows, 8)
    out = np.zeros((rows, nsb * 8), dtype=O.BLOCK_DTYPES[O.Q8_0])
    out["d"] = d8.transpose(1, 0, 2).reshape(rows, nsb * 8)
    out["qs"] = qs.transpose(1, 0, 2).reshape(rows, nsb * 8, 32)
    return out.view(np.uint8).reshape(-1)


@pytest.mark.parametrize("wtype", [O.Q4K, O.Q8_0])
@pytest.mark.parametrize("m,k", [(5, 256), (130, 1024), (3, 300), (64, 4096)])
def test_prefill_quantizer_is_bit_exact(wtype, m, k):
    rng = np.random.default_rng(m * 7 + k)
    x = acts(rng, m, k)
    if k >= 512:
        x[0, :256] = 0.0
        x[-1, 10], x[-1, 100] = -9.0, 9.0
    y, kp = qmm.quantize_prefill(wtype, to_dev(x))
    at = O.ACT_TYPE[wtype]
    xp = np.zeros((m, kp), np.float32)
    xp[:, :k] = x
    want = O.quantize(at, xp).reshape(-1)
    got = tiles_to_blocks(y.cpu().numpy(), m, kp, at)
    assert np.array_equal(got, want)


def test_prefill_quantizer_row_gather():
    rng = np.random.default_rng(3)
    x = acts(rng, 10, 512)
    ids = np.array([7, 7, 0, 9, 3], dtype=np.int32)
    y, kp = qmm.quantize_prefill(O.Q4K, to_dev(x), ids=to_dev(ids))
    want = O.quantize(O.Q8K, x[ids]).reshape(-1)
    assert np.array_equal(tiles_to_blocks(y.cpu().numpy(), 5, kp, O.Q8K), want)


CASES = [
    # (gtype, m, n, k)
    (O.Q4K, 40, 64, 512), (O.Q4K, 128, 128, 256), (O.Q4K, 130, 200, 1024), (O.Q4K, 1, 128, 4096),
    (O.Q4K, 512, 256, 4096), (O.Q4K, 17, 33, 2048),
    (O.Q6K, 40, 64, 512), (O.Q6K, 130, 200, 1024), (O.Q6K, 64, 96, 14336), (O.Q6K, 255, 129, 256),
    (O.Q8_0, 40, 64, 512), (O.Q8_0, 33, 48, 1056), (O.Q8_0, 130, 200, 1024), (O.Q8_0, 9, 32, 2688),
    (O.Q4_0, 40, 64, 512), (O.Q4_0, 33, 48, 1056), (O.Q4_0, 130, 200, 4096), (O.Q4_0, 9, 32, 2720),
    (O.Q5_0, 40, 64, 512), (O.Q5_0, 33, 48, 1056), (O.Q5_0, 130, 200, 4096), (O.Q5_0, 9, 32, 2720),
    # 32-value types with K a multiple of 256: the run-loading kernel, 32-row tiles with K split across
    # workgroups (f32 atomics), 64-row tiles, a ragged last weight tile
    (O.Q8_0, 17, 300, 4096), (O.Q4_0, 20, 130, 2048), (O.Q5_0, 64, 257, 1280), (O.Q8_0, 300, 129, 768),
    # Q5_K: the K-quant kernel with the fifth-bit plane (32-row tiles with split K, 64-row tiles, ragged edges)
    (O.Q5K, 40, 64, 512), (O.Q5K, 130, 200, 1024), (O.Q5K, 17, 300, 4096), (O.Q5K, 255, 129, 256),
]


@pytest.mark.parametrize("gtype,m,n,k", CASES)
def test_mmq_matches_the_cpu_qmatmul(gtype, m, n, k):
    rng = np.random.default_rng(gtype * 1000 + m + n + k)
    w = weights(rng, n, k)
    x = acts(rng, m, k)
    x[:, ::64] *= 60.0
    wq = O.quantize(gtype, w)
    want = O.matmul(gtype, x, wq, n)
    got = qmm.qmatmul_prefill(gtype, to_dev(wq), to_dev(x), n).cpu().numpy()
    assert_parity(got, want, terms(gtype, x, wq, n), what=f"t{gtype} m{m} n{n} k{k}")


@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_mmq_half_outputs(out):
    rng = np.random.default_rng(11)
    m, n, k = 64, 128, 1024
    wq = O.quantize(O.Q4K, weights(rng, n, k))
    x = acts(rng, m, k)
    want = O.matmul(O.Q4K, x, wq, n)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[out]
    got = qmm.qmatmul_prefill(O.Q4K, to_dev(wq), to_dev(x), n, out_dtype=tdt).float().cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max())


@pytest.mark.parametrize("gtype,n,k", [(O.Q4K, 14336, 4096), (O.Q6K, 4096, 14336), (O.Q8_0, 14336, 4096),
                                       (O.Q5K, 14336, 4096)])
def test_mmq_config_shapes(gtype, n, k):
    """[512, K] activations; checked against the oracle on 24 sampled activation rows."""
    rng = np.random.default_rng(20261203 + gtype)
    m = 512
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, m, k)
    got = qmm.qmatmul_prefill(gtype, to_dev(wq), to_dev(x), n).cpu().numpy()
    rows = np.sort(rng.choice(m, 24, replace=False))
    want = O.matmul(gtype, x[rows], wq, n)
    r = assert_parity(got[rows], want, what=f"t{gtype}")
    print(f"type {gtype} [{m},{k}]x[{n},{k}]: max rel err {r:.2e}")
