"""GPU parity of the adjacent GGUF types (Q4_0, Q5_0, Q5_K, IQ4_XS) through the C ABI: the decode matvec
launch_mmvq_gguf_<t>_<dtype>_plain against the oracle's CPU QMatMul on the same bytes and the same (bit-exact)
activation blocks, max rel. error <= 1e-3 and per element <= 1e-5 * sum|terms|; the dequantizers bit-exact with the
oracle's to_float (f16 / bf16 outputs: the f32 values rounded to nearest even)."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, decode_act_blocks, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
TYPES = [O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS]


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def weight_bytes(gtype, n, k, rng, random_bytes=False):
    if gtype == O.IQ4XS or random_bytes:
        return O.random_blocks(gtype, n * k, rng, 0.002).reshape(n, -1)
    return O.quantize(gtype, weights(rng, n, k))


def terms(gtype, aq, wq, m, n, k):
    import test_oracle as T
    a = T.NP_DEQUANT[O.ACT_TYPE[gtype]](aq).reshape(m, -1)[:, :k]
    w = T.NP_DEQUANT[gtype](wq).reshape(n, k)
    return np.abs(a) @ np.abs(w).T


def run_matvec(gtype, wq, x, n, out_dtype=torch.float32):
    m, k = x.shape
    w = to_dev(wq.reshape(-1))
    vy, kp = qmm.quantize_decode(gtype, to_dev(x))
    got = qmm.mmvq(gtype, w, vy, k, n, m, kp, out_dtype=out_dtype)
    torch.cuda.synchronize()
    # the activation blocks the GPU made, as the oracle's blocks of the first k values (bit-exact with the oracle's own
    # quantizer, checked below); the oracle's matmul on them
    aq = decode_act_blocks(gtype, vy.cpu().numpy(), m, kp, k)
    want = O.matmul_preq(gtype, aq, m, k, wq, n)
    return got.float().cpu().numpy(), want, aq


def _k_cases(gtype):
    # 32-value types: even and odd block counts (the block-pair and the one-block unit); super-block types: one to
    # many super-blocks, including counts that leave a wave's lanes partly idle
    return [32, 96, 512, 1056, 4096, 14336] if O.BLOCK_SIZE[gtype] == 32 else [256, 768, 4096, 5120, 14336]


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("kidx", range(5))
@pytest.mark.parametrize("b", [1, 2, 5, 8, 16])
def test_adjacent_matvec_matches_the_oracle(gtype, kidx, b):
    k = _k_cases(gtype)[kidx]
    rng = np.random.default_rng(1000 * gtype + 10 * kidx + b)
    n = 37 if k > 4096 else 300
    wq = weight_bytes(gtype, n, k, rng)
    x = acts(rng, b, k)
    x[:, ::64] *= 30.0
    got, want, aq = run_matvec(gtype, wq, x, n)
    assert np.array_equal(aq, O.quantize(O.ACT_TYPE[gtype], x).reshape(-1))
    assert_parity(got, want, terms(gtype, aq, wq, b, n, k), what=f"type {gtype} k={k} b={b}")


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_adjacent_matvec_half_outputs(gtype, out):
    rng = np.random.default_rng(77 + gtype)
    k = 4096
    n = 513
    wq = weight_bytes(gtype, n, k, rng, random_bytes=True)
    x = acts(rng, 3, k)
    odt = {"f16": torch.float16, "bf16": torch.bfloat16}[out]
    got, want, _ = run_matvec(gtype, wq, x, n, out_dtype=odt)
    # the f32 result rounded once to the output type: the north-star bound plus half an ulp of each value
    ulp = 2.0 ** -8 if out == "bf16" else 2.0 ** -11
    want = np.asarray(want, np.float64)
    err = np.abs(np.asarray(got, np.float64) - want)
    assert np.all(err <= 1e-3 * np.abs(want).max() + ulp * np.abs(want)), f"type {gtype} {out}"


@pytest.mark.parametrize("gtype", [O.Q4_0, O.Q5_0])
def test_odd_block_rows_and_unaligned_weights(gtype):
    """Rows of an odd number of 32-value blocks and a weight pointer that is only 2-byte aligned take the one-block
    unit; the result is the same arithmetic."""
    rng = np.random.default_rng(5 + gtype)
    k, n = 160, 77
    wq = weight_bytes(gtype, n, k, rng)
    x = acts(rng, 4, k)
    buf = torch.zeros(wq.size + 2, dtype=torch.uint8, device=DEV)
    buf[2:] = to_dev(wq.reshape(-1))
    vy, kp = qmm.quantize_decode(gtype, to_dev(x))
    got = qmm.mmvq(gtype, buf[2:], vy, k, n, 4, kp).cpu().numpy()
    want = O.matmul(gtype, x, wq, n)
    assert_parity(got, want, what="odd/unaligned")
    # a 64-multiple K through the same 2-byte-aligned pointer
    k = 256
    wq = weight_bytes(gtype, n, k, rng)
    x = acts(rng, 2, k)
    buf = torch.zeros(wq.size + 2, dtype=torch.uint8, device=DEV)
    buf[2:] = to_dev(wq.reshape(-1))
    vy, kp = qmm.quantize_decode(gtype, to_dev(x))
    got = qmm.mmvq(gtype, buf[2:], vy, k, n, 2, kp).cpu().numpy()
    assert_parity(got, O.matmul(gtype, x, wq, n), what="aligned-K, unaligned pointer")


def test_q5k_and_iq4xs_reject_misaligned_weights():
    w = torch.zeros(176 * 4 + 16, dtype=torch.uint8, device=DEV)
    vy, kp = qmm.quantize_decode(qmm.Q5K, torch.zeros((1, 256), device=DEV))
    with pytest.raises(qmm.QmmError, match="aligned"):
        qmm.mmvq(qmm.Q5K, w[4:], vy, 256, 4, 1, kp)
    with pytest.raises(qmm.QmmError, match="aligned"):
        qmm.mmvq(qmm.IQ4XS, w[2:], vy, 256, 4, 1, kp)


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("out", ["f32", "f16", "bf16"])
def test_adjacent_dequantize_is_bit_exact(gtype, out):
    rng = np.random.default_rng(31 + gtype)
    n = 256 * 37
    wq = weight_bytes(gtype, 1, n, rng, random_bytes=True).reshape(-1)
    odt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[out]
    got = qmm.dequantize(gtype, to_dev(wq), n, out_dtype=odt)
    torch.cuda.synchronize()
    want = torch.from_numpy(O.dequantize(gtype, wq, n)).to(odt)  # torch's f32 -> f16 / bf16 casts round to nearest even
    assert torch.equal(got.cpu().view(torch.int16 if out != "f32" else torch.int32),
                       want.view(torch.int16 if out != "f32" else torch.int32))


@pytest.mark.parametrize("gtype", [O.Q4_0, O.Q5_0, O.Q5K])
def test_adjacent_get_rows(gtype):
    rng = np.random.default_rng(41 + gtype)
    rows, k = 50, 512
    wq = weight_bytes(gtype, rows, k, rng)
    ids = np.array([3, 0, 49, 3, 17], np.uint32)
    got = qmm.get_rows(gtype, to_dev(wq.reshape(-1)), to_dev(ids), k, wq.shape[1]).cpu().numpy()
    want = O.dequantize(gtype, wq, rows * k).reshape(rows, k)[ids]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("glu", [False, True])
def test_adjacent_moe_matvec(gtype, glu):
    """launch_mmvq_gguf_<t>_moe: routed pairs against the oracle's per-route matmul (and the GLU form)."""
    rng = np.random.default_rng(51 + gtype + 7 * glu)
    E, n, k, tokens, topk = 4, 96, 512, 3, 2
    wg = weight_bytes(gtype, E * n, k, rng).reshape(E, -1)
    wu = weight_bytes(gtype, E * n, k, rng).reshape(E, -1)
    x = acts(rng, tokens, k)
    ids = np.array([[0, 3], [2, 2], [1, 0]], np.uint32)
    vy, kp = qmm.quantize_decode(gtype, to_dev(x))
    out = qmm.mmvq_moe(gtype, to_dev(wg), to_dev(wu) if glu else None, wg.shape[1], vy, to_dev(ids.reshape(-1)), k,
                       n, kp, topk, tokens * topk, 0)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(tokens, topk, n)
    g = O.indexed_moe(gtype, wg, E, n, k, x[:, None, :], ids)
    if glu:
        u = O.indexed_moe(gtype, wu, E, n, k, x[:, None, :], ids)
        want = g / (1 + np.exp(-g.astype(np.float64))) * u  # SiLU(gate) * up
        assert_parity(got, want, rel=1e-4, what=f"moe glu type {gtype}")
    else:
        assert_parity(got, g, what=f"moe type {gtype}")


@pytest.mark.parametrize("gtype", [O.Q4_0, O.Q5_0, O.Q5K])
@pytest.mark.parametrize("xdim1", [1, 2])
def test_adjacent_indexed_moe(gtype, xdim1):
    rng = np.random.default_rng(61 + gtype + xdim1)
    E, n, k, batch, topk = 3, 64, 768 if gtype == O.Q5K else 160, 4, 2
    w = weight_bytes(gtype, E * n, k, rng).reshape(E, -1)
    x = acts(rng, batch * xdim1, k).reshape(batch, xdim1, k)
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    got = qmm.indexed_moe(gtype, to_dev(w), to_dev(x), to_dev(ids), n).cpu().numpy()
    want = O.indexed_moe(gtype, w, E, n, k, x, ids)
    assert_parity(got, want, what=f"indexed type {gtype} xdim1={xdim1}")


# Rows of more than two 64-value units per lane at one or two columns: the types whose wide rows are split over two waves
# (Q4_K, Q8_0, Q4_0, Q5_0, IQ4_XS) and the two that keep one wave per row (Q6_K, Q5_K); odd and single-row counts
# (a pair with no row), 224 units (a partly idle second half), 256 (every lane full), 192 (three units per lane), and
# the ninth column of b = 9 (a one-column pass after a full one); the same at two columns (b = 2, and the last two
# of b = 10).
WIDE_SHAPES = [(37, 14336, 1), (1, 14336, 1), (64, 16384, 1), (33, 12288, 1), (3, 14336, 9), (29, 12288, 2),
               (37, 14336, 2), (64, 16384, 2), (5, 14336, 10)]


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q8_0, O.Q4_0, O.Q5_0, O.IQ4XS, O.Q6K, O.Q5K])
@pytest.mark.parametrize("shape", range(len(WIDE_SHAPES)))
def test_wide_rows_at_one_column(gtype, shape):
    n, k, b = WIDE_SHAPES[shape]
    rng = np.random.default_rng(500 + 10 * gtype + shape)
    wq = weight_bytes(gtype, n, k, rng)
    x = acts(rng, b, k)
    x[:, ::64] *= 30.0
    got, want, aq = run_matvec(gtype, wq, x, n)
    assert_parity(got, want, terms(gtype, aq, wq, b, n, k), what=f"type {gtype} n={n} k={k} b={b}")


# Wide rows of at least 4,096 (two workgroups of 8 rows for every CU) at one column take the four-wave form
# (k_mmvq_p4): 224 units (a half-idle fourth wave), 192 (an idle fourth wave), 132 (a mostly idle third wave), and a
# ragged last workgroup (4,100 and 4,099 rows).
P4_SHAPES = [(4100, 14336), (4096, 12288), (4099, 8448)]


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q8_0, O.Q4_0, O.Q5_0, O.IQ4XS, O.Q6K, O.Q5K])
@pytest.mark.parametrize("shape", range(len(P4_SHAPES)))
def test_wide_rows_four_waves(gtype, shape):
    n, k = P4_SHAPES[shape]
    rng = np.random.default_rng(1500 + 10 * gtype + shape)
    wq = weight_bytes(gtype, n, k, rng, random_bytes=True)
    x = acts(rng, 1, k)
    got, want, _ = run_matvec(gtype, wq, x, n)
    assert_parity(got, want, what=f"type {gtype} n={n} k={k}")


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q4_0])
@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_wide_rows_half_outputs(gtype, out):
    rng = np.random.default_rng(900 + gtype)
    n, k = 37, 14336
    wq = weight_bytes(gtype, n, k, rng, random_bytes=True)
    x = acts(rng, 1, k)
    odt = {"f16": torch.float16, "bf16": torch.bfloat16}[out]
    got, want, _ = run_matvec(gtype, wq, x, n, out_dtype=odt)
    # the f32 result rounded once to the output type: the north-star bound plus half an ulp of each value
    ulp = 2.0 ** -8 if out == "bf16" else 2.0 ** -11
    want = np.asarray(want, np.float64)
    err = np.abs(np.asarray(got, np.float64) - want)
    assert np.all(err <= 1e-3 * np.abs(want).max() + ulp * np.abs(want)), f"type {gtype} {out}"


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4_0, O.Q5_0])
@pytest.mark.parametrize("shape", [0, 3, 4, 5, 7, 8])
def test_wide_rows_reference_entries(gtype, shape):
    """The same wide rows through the reference-named entries over Q8_1 slots (unit_*_s: per-256 f32 scales of the
    activation), against the oracle's matmul over Q8_K activations."""
    n, k, b = WIDE_SHAPES[shape]
    rng = np.random.default_rng(700 + 10 * gtype + shape)
    wq = weight_bytes(gtype, n, k, rng)
    x = acts(rng, b, k)
    x[:, ::64] *= 30.0
    got = qmm.qmatmul_decode(gtype, to_dev(wq.reshape(-1)), to_dev(x), n, q8_1=True).cpu().numpy()
    assert_parity(got, O.matmul_q8k_act(gtype, x, wq, n), what=f"type {gtype} n={n} k={k} b={b}")
