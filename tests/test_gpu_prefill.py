"""GPU parity of the prefill path through the C ABI: the tile-layout Q8_K / Q8_0 quantizers (bit-exact; the Q8_K
tiles, launch_mmq_quantize_q8_1_*, fit the reference's MMQ scratch of M * k_padded / 128 * 144 + 128 * 144 bytes) and the
int8-MFMA matmul for Q4_K / Q6_K / Q8_0 and, on the Q8_0 kernel, Q4_0 / Q5_0 (max rel. error <= 1e-3 against the
oracle's CPU QMatMul)."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, terms, tiles_to_blocks, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


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
    got = tiles_to_blocks(y.cpu().numpy(), m, kp, at == O.Q8K)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m,k", [(5, 256), (130, 1024), (3, 300), (64, 4096)])
def test_q8k_tile_quantizer_is_bit_exact(m, k):
    """launch_mmq_quantize_q8k: the Q8_K quantization of the reference-named tiles, with exact f16 sums of 16."""
    rng = np.random.default_rng(m * 5 + k)
    x = acts(rng, m, k)
    y, kp = qmm.quantize_prefill(O.Q4K, to_dev(x), q8k=True)
    xp = np.zeros((m, kp), np.float32)
    xp[:, :k] = x
    got = tiles_to_blocks(y.cpu().numpy(), m, kp, True, s16=True)
    assert np.array_equal(got, O.quantize(O.Q8K, xp).reshape(-1))
    y1, _ = qmm.quantize_prefill(O.Q4K, to_dev(x))
    assert np.array_equal(y.cpu().numpy()[: m * kp // 256 * 260], y1.cpu().numpy()[: m * kp // 256 * 260])


def test_prefill_quantizer_row_gather():
    rng = np.random.default_rng(3)
    x = acts(rng, 10, 512)
    ids = np.array([7, 7, 0, 9, 3], dtype=np.int32)
    y, kp = qmm.quantize_prefill(O.Q4K, to_dev(x), ids=to_dev(ids))
    want = O.quantize(O.Q8K, x[ids]).reshape(-1)
    assert np.array_equal(tiles_to_blocks(y.cpu().numpy(), 5, kp, True), want)


CASES = [
    # (gtype, m, n, k)
    (O.Q4K, 40, 64, 512), (O.Q4K, 128, 128, 256), (O.Q4K, 130, 200, 1024), (O.Q4K, 1, 128, 4096),
    (O.Q4K, 512, 256, 4096), (O.Q4K, 17, 33, 2048),
    (O.Q6K, 40, 64, 512), (O.Q6K, 130, 200, 1024), (O.Q6K, 64, 96, 14336), (O.Q6K, 255, 129, 256),
    (O.Q8_0, 40, 64, 512), (O.Q8_0, 33, 48, 1056), (O.Q8_0, 130, 200, 1024), (O.Q8_0, 9, 32, 2688),
    (O.Q4_0, 40, 64, 512), (O.Q4_0, 33, 48, 1056), (O.Q4_0, 130, 200, 4096), (O.Q4_0, 9, 32, 2720),
    (O.Q5_0, 40, 64, 512), (O.Q5_0, 33, 48, 1056), (O.Q5_0, 130, 200, 4096), (O.Q5_0, 9, 32, 2720),
    # 32-value types with K a multiple of 256: the run-loading kernel, 32-row tiles with K split across
    # workgroups (partial planes summed in split order), 64-row tiles, a ragged last weight tile
    (O.Q8_0, 17, 300, 4096), (O.Q4_0, 20, 130, 2048), (O.Q5_0, 64, 257, 1280), (O.Q8_0, 300, 129, 768),
    # one superblock per row: every step of the ring past the first loads the same superblock again
    (O.Q8_0, 33, 64, 256), (O.Q4_0, 70, 96, 256),
    # Q5_K: the K-quant kernel with the fifth-bit plane (32-row tiles with split K, ragged edges)
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


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4_0, O.Q5_0])
def test_mmq_subnormal_block_scales(gtype):
    """The 32-value kernel's scale products (an f16 MFMA for Q4_0 / Q5_0) with f16 block scales in the subnormal range
    (below 6.1e-5) on both sides: activation rows of magnitude 1e-3 .. 1e-6 and weight rows of 1e-3 .. 1e-4 of the
    usual; rows whose every scale is subnormal must still match the CPU QMatMul to the relative bound."""
    m, n, k = 64, 96, 1024
    rng = np.random.default_rng(gtype + 77)
    w = weights(rng, n, k)
    w[::3] *= 1e-3
    w[1::5] *= 1e-4
    x = acts(rng, m, k)
    x[::2] *= 1e-3
    x[1::4] *= 1e-5
    x[3::8] *= 1e-6
    wq = O.quantize(gtype, w)
    want = O.matmul(gtype, x, wq, n)
    got = qmm.qmatmul_prefill(gtype, to_dev(wq), to_dev(x), n).cpu().numpy()
    assert np.count_nonzero(want) > 0.75 * want.size  # (scales below f16's range round to zero, in both)
    assert_parity(got, want, terms(gtype, x, wq, n), what=f"t{gtype} subnormal scales")


# (gtype, m, n, k): f16 / bf16 outputs of every prefill kernel -- the K-quant kernel (Q4_K, Q6_K, Q5_K), the pipelined
# 32-value kernel (Q8_0, Q4_0, Q5_0 with K a multiple of 256) and the simple Q8_0-layout kernel (K = 1056); the 17-row
# cases take split K, whose plane sum rounds to the output type once; Q6_K at 130 rows takes the 128-row tile with its
# weights staged in LDS
HALF_CASES = [(O.Q4K, 64, 128, 1024), (O.Q6K, 64, 128, 1024), (O.Q5K, 64, 128, 1024), (O.Q8_0, 64, 128, 1024),
              (O.Q4_0, 64, 128, 1024), (O.Q5_0, 64, 128, 1024), (O.Q8_0, 40, 96, 1056), (O.Q4_0, 40, 96, 1056),
              (O.Q5_0, 40, 96, 1056), (O.Q4K, 17, 300, 4096), (O.Q8_0, 17, 300, 4096), (O.Q6K, 130, 200, 1024)]


@pytest.mark.parametrize("out", ["f16", "bf16"])
@pytest.mark.parametrize("gtype,m,n,k", HALF_CASES)
def test_mmq_half_outputs(out, gtype, m, n, k):
    """The output is the f32 result rounded once to the half type: within the north-star bound plus half an ulp of
    the half type (2^-11 f16, 2^-8 bf16) of each value."""
    rng = np.random.default_rng(11 + gtype + m + k)
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, m, k)
    want = O.matmul(gtype, x, wq, n).astype(np.float64)
    tdt, ulp = {"f16": (torch.float16, 2.0 ** -11), "bf16": (torch.bfloat16, 2.0 ** -8)}[out]
    got = qmm.qmatmul_prefill(gtype, to_dev(wq), to_dev(x), n, out_dtype=tdt).float().cpu().numpy()
    err = np.abs(got - want)
    bound = 1e-3 * np.abs(want).max() + ulp * np.abs(want)
    assert np.all(err <= bound), f"{out} t{gtype} m{m} k{k}: worst excess {np.max(err - bound):.3e}"


# split K (the tile grid alone leaves compute units idle): Q4_K at 17 rows (4 splits), the Q6_K config shape (2), a
# 32-value type, an expert-grouped case
@pytest.mark.parametrize("gtype,m,n,k", [(O.Q4K, 17, 4096, 4096), (O.Q6K, 512, 4096, 14336), (O.Q8_0, 20, 4096, 4096),
                                         (O.Q5K, 17, 300, 4096)])
def test_split_k_is_deterministic(gtype, m, n, k):
    """Split-K partial sums are added in split order by a second kernel (no atomics), so two runs give the same bits;
    the result matches the oracle and, within rounding, the unsplit kernel (no fixup buffer)."""
    rng = np.random.default_rng(31 + gtype + m)
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, m, k)
    wd = to_dev(wq)
    y, _ = qmm.quantize_prefill(gtype, to_dev(x))
    a = qmm.mmq(gtype, wd, y, k, n, m).cpu().numpy()
    b = qmm.mmq(gtype, wd, y, k, n, m).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "split-K result differs between runs"
    one = qmm.mmq(gtype, wd, y, k, n, m, tmp_fixup=False).cpu().numpy()
    want = O.matmul(gtype, x, wq, n)
    assert_parity(a, want, what=f"split t{gtype} m{m}")
    assert_parity(one, want, what=f"unsplit t{gtype} m{m}")


def test_split_k_grouped_is_deterministic():
    rng = np.random.default_rng(77)
    E, n, k, tokens, topk = 4, 256, 4096, 24, 2  # 12 rows per expert: the tile route splits K over 4
    wq = O.quantize(O.Q8_0, weights(rng, E * n, k)).reshape(E, -1)
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = acts(rng, tokens, k)
    want = O.indexed_moe(O.Q8_0, wq, E, n, k, x[:, None], ids.astype(np.uint32)).reshape(tokens * topk, n)
    bounds, tok, src, counts, _ = qmm.moe_dispatch(to_dev(ids.reshape(-1)), E, topk)
    y, _ = qmm.quantize_prefill(O.Q8_0, to_dev(x), ids=src)
    outs = []
    for _ in range(2):
        out = torch.full((tokens * topk, n), float("nan"), device=DEV)
        qmm.mmq_moe(O.Q8_0, to_dev(wq), y, tok, bounds, E, k, n, tokens * topk, int(counts.max().item()), out)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert_parity(outs[0], want)


# (gtype, m, n, k): the K-quant kernel's tile shapes, split K, ragged edges and K not a multiple of 512
Q8K_CASES = [(O.Q4K, 40, 64, 512), (O.Q4K, 130, 200, 1024), (O.Q4K, 17, 300, 4096), (O.Q4K, 512, 256, 4096),
             (O.Q4K, 3, 33, 768), (O.Q5K, 40, 64, 512), (O.Q5K, 255, 129, 256), (O.Q5K, 17, 300, 4096)]


@pytest.mark.parametrize("gtype,m,n,k", Q8K_CASES)
def test_mmq_q8k_twin(gtype, m, n, k):
    """launch_mmq_gguf_{q4_k,q5_k}_q8k over `_q8k` tiles: the min term's per-superblock sums are exact integers on
    both activation forms (f16 sums of 16 here, the int16 sums of 32 split into two f16 halves on the reference
    names), so the output equals the reference-named entry's bit for bit, and the oracle's within the bound."""
    rng = np.random.default_rng(gtype * 77 + m + n + k)
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, m, k)
    x[:, ::64] *= 60.0
    wd, xd = to_dev(wq), to_dev(x)
    got = qmm.qmatmul_prefill(gtype, wd, xd, n, q8k=True).cpu().numpy()
    ref = qmm.qmatmul_prefill(gtype, wd, xd, n).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"t{gtype} m{m} n{n} k{k}"
    assert_parity(got, O.matmul(gtype, x, wq, n), terms(gtype, x, wq, n), what=f"t{gtype} m{m} n{n} k{k}")


@pytest.mark.parametrize("wtype", [O.Q4K, O.Q8_0])
@pytest.mark.parametrize("activation", [2, 0])
def test_glu_requantizer(wtype, activation):
    """launch_mmq_quantize_glu_q8_1_DS4_f32 / launch_mmq_quantize_glu_q8_0_f32: act(gate[r]) * up[r] for the gathered rows, quantized into the prefill
    layout.  ReLU (2) is exact in f32 (a select and one rounded product), so the blocks must equal the oracle's
    quantization of the same values byte for byte.  SiLU (0) goes through the device's expf: its blocks match those
    of the device-independent quantizer run on the same f32 products computed here, except where a product sits
    within a few ulps of a rounding step, and its values are within 1e-5 relative."""
    rng = np.random.default_rng(50 + wtype + activation)
    rows, k = 40, 1300
    gate = acts(rng, rows, k)
    up = acts(rng, rows, k)
    ids = rng.integers(0, rows, 33).astype(np.int32)
    y, kp = qmm.quantize_prefill_glu(wtype, to_dev(gate), to_dev(up), ids=to_dev(ids), activation=activation)
    g, u = gate[ids], up[ids]
    if activation == 2:
        h = np.where(g > 0, g, np.float32(0)) * u
    else:
        h = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32)
    hp = np.zeros((len(ids), kp), np.float32)
    hp[:, :k] = h
    at = O.ACT_TYPE[wtype]
    want = O.quantize(at, hp).reshape(-1)
    got = tiles_to_blocks(y.cpu().numpy(), len(ids), kp, at == O.Q8K)
    if wtype == O.Q4K:
        y16, _ = qmm.quantize_prefill_glu(wtype, to_dev(gate), to_dev(up), ids=to_dev(ids), activation=activation,
                                          q8k=True)
        assert np.array_equal(tiles_to_blocks(y16.cpu().numpy(), len(ids), kp, True, s16=True), got)
    if activation == 2:
        assert np.array_equal(got, want)
    else:
        deq_got = O.dequantize(at, got, len(ids) * kp)
        deq_want = O.dequantize(at, want, len(ids) * kp)
        scale = np.abs(deq_want).max()
        assert np.max(np.abs(deq_got - deq_want)) <= 2e-2 * scale  # at most a unit of one block's step
        assert np.mean(got == want) > 0.99


@pytest.mark.parametrize("gtype,n,k", [(O.Q4K, 14336, 4096), (O.Q6K, 4096, 14336), (O.Q8_0, 14336, 4096),
                                       (O.Q5K, 14336, 4096)])
def test_mmq_config_shapes(gtype, n, k):
    """[512, K] activations, every output checked against the oracle."""
    rng = np.random.default_rng(20261203 + gtype)
    m = 512
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, m, k)
    got = qmm.qmatmul_prefill(gtype, to_dev(wq), to_dev(x), n).cpu().numpy()
    want = O.matmul(gtype, x, wq, n)
    r = assert_parity(got, want, what=f"t{gtype}")
    print(f"type {gtype} [{m},{k}]x[{n},{k}]: max rel err {r:.2e}")


def iq4xs_weight(rng, n, k):
    """IQ4_XS weight bytes: random blocks (every byte pattern is a valid block; the reference has no IQ4_XS
    quantizer on this path), f16 scales near 0.002 of both signs."""
    return O.random_blocks(O.IQ4XS, n * k, rng, 0.002).reshape(n, -1)


# IQ4_XS on the K-quant kernel: 32-, 64- and 128-row activation tiles, split K (17 rows), ragged weight tiles, the
# FFN-down shape
IQ4XS_CASES = [(40, 64, 512), (130, 200, 1024), (17, 300, 4096), (255, 129, 256), (512, 256, 4096), (64, 96, 14336),
               (1, 128, 2048)]


@pytest.mark.parametrize("m,n,k", IQ4XS_CASES)
def test_mmq_iq4_xs_matches_the_cpu_qmatmul(m, n, k):
    rng = np.random.default_rng(23000 + m + n + k)
    wq = iq4xs_weight(rng, n, k)
    x = acts(rng, m, k)
    x[:, ::64] *= 60.0
    want = O.matmul(O.IQ4XS, x, wq, n)
    got = qmm.qmatmul_prefill(O.IQ4XS, to_dev(wq), to_dev(x), n).cpu().numpy()
    assert_parity(got, want, terms(O.IQ4XS, x, wq, n), what=f"iq4_xs m{m} n{n} k{k}")


@pytest.mark.parametrize("out", ["f16", "bf16"])
@pytest.mark.parametrize("m", [64, 130])  # (130: the 128-row tile, weights staged in LDS)
def test_mmq_iq4_xs_half_outputs(out, m):
    rng = np.random.default_rng(29 + m)
    n, k = 128, 1024
    wq = iq4xs_weight(rng, n, k)
    x = acts(rng, m, k)
    want = O.matmul(O.IQ4XS, x, wq, n).astype(np.float64)
    tdt, ulp = {"f16": (torch.float16, 2.0 ** -11), "bf16": (torch.bfloat16, 2.0 ** -8)}[out]
    got = qmm.qmatmul_prefill(O.IQ4XS, to_dev(wq), to_dev(x), n, out_dtype=tdt).float().cpu().numpy()
    assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max() + ulp * np.abs(want))


def test_mmq_iq4_xs_split_k_is_deterministic():
    rng = np.random.default_rng(37)
    m, n, k = 17, 4096, 4096
    wq = iq4xs_weight(rng, n, k)
    x = acts(rng, m, k)
    wd = to_dev(wq)
    y, _ = qmm.quantize_prefill(O.IQ4XS, to_dev(x))
    a = qmm.mmq(O.IQ4XS, wd, y, k, n, m).cpu().numpy()
    b = qmm.mmq(O.IQ4XS, wd, y, k, n, m).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert_parity(a, O.matmul(O.IQ4XS, x, wq, n), what="iq4_xs split")


def test_mmq_iq4_xs_rejects_misaligned_weights():
    rng = np.random.default_rng(41)
    wq = iq4xs_weight(rng, 32, 256)
    buf = torch.zeros(wq.size + 2, dtype=torch.uint8, device=DEV)
    buf[2:] = to_dev(wq.reshape(-1))
    y, _ = qmm.quantize_prefill(O.IQ4XS, to_dev(acts(rng, 40, 256)))
    with pytest.raises(qmm.QmmError, match="4-byte aligned"):
        qmm.mmq(O.IQ4XS, buf[2:], y, 256, 32, 40)


# Q6_K superblocks are 210 bytes, 2-byte aligned: the 64-row tile stages each row's superblock in LDS from the dword
# that holds its first byte.  Weights 2 bytes past a dword boundary, with an odd superblock count per row (rows
# alternately 0 and 2 bytes past a dword), against the oracle.
@pytest.mark.parametrize("m,n,k", [(130, 200, 768), (64, 129, 256), (512, 300, 1280), (100, 33, 2816)])
def test_mmq_q6_k_weights_2_bytes_past_a_dword(m, n, k):
    rng = np.random.default_rng(43 + m + n + k)
    wq = O.quantize(O.Q6K, weights(rng, n, k))
    x = acts(rng, m, k)
    buf = torch.zeros(wq.size + 2, dtype=torch.uint8, device=DEV)
    buf[2:] = to_dev(wq.reshape(-1))
    y, _ = qmm.quantize_prefill(O.Q6K, to_dev(x))
    got = qmm.mmq(O.Q6K, buf[2:], y, k, n, m).cpu().numpy()
    assert_parity(got, O.matmul(O.Q6K, x, wq, n), terms(O.Q6K, x, wq, n), what=f"q6_k +2 m{m} n{n} k{k}")
