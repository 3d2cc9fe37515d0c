"""GPU parity of the decode path through the C ABI: activation quantizers (bit-exact with the oracle) and the
Q8_0 / Q4_K / Q6_K matvec (max rel. error <= 1e-3 against the oracle's CPU QMatMul on the same bytes).  The
super-block types read Q8_1 slots (launch_mmvq_gguf_quantize_q8_1_*, 36 bytes per 32 values as the reference sizes
them, holding BlockQ8K::from_float's d and qs); Q8_0 reads Q8_0 blocks through its _q8_0 entries, or Q8_1 slots through
the reference-named ones (then checked against the oracle's matmul over Q8_K activations)."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, decode_act_blocks, patterned, terms, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def special_rows(rng, m, k):
    x = acts(rng, m, k)
    if k >= 512:
        x[0, 256:512] = 0.0                        # an all-zero block
        x[-1, 3], x[-1, 70] = -5.0, 5.0             # tied maxima of opposite signs: the first sets the sign
        x[-1, 1] = 7.0 if m > 1 else x[-1, 1]
    return x


@pytest.mark.parametrize("k", [256, 300, 4096, 14336])
@pytest.mark.parametrize("src", ["f32", "f16", "bf16"])
def test_q8_1_decode_quantizer_is_bit_exact(k, src):
    """launch_mmvq_gguf_quantize_q8_1_<src> into the reference's scratch (rows * pad(k, 512) / 32 * 36 bytes) with a
    guard region behind it: each slot holds BlockQ8K::from_float's d and qs, the int16 sums of each 32 values and a
    zero tail; the padding to k_padded quantizes as zeros; nothing is written past the scratch."""
    rng = np.random.default_rng(100 + k)
    x = special_rows(rng, 5, k)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[src]
    xt = to_dev(x).to(tdt)
    x_in = xt.float().cpu().numpy()  # the reference widens f16/bf16 to f32 before quantizing
    kp = qmm.pad_to(k, 512)
    size = 5 * kp // 32 * 36
    buf = torch.full((size + 4096,), 0xA5, dtype=torch.uint8, device=DEV)
    vy, kp2 = qmm.quantize_decode(qmm.Q4K, xt, out=buf)
    assert kp2 == kp
    got = buf.cpu().numpy()
    assert np.all(got[size:] == 0xA5), "written past the reference's scratch size"
    xp = np.zeros((5, kp), np.float32)
    xp[:, :k] = x_in
    want = O.quantize(O.Q8K, xp).reshape(-1)
    assert np.array_equal(decode_act_blocks(O.Q4K, got[:size], 5, kp), want)


@pytest.mark.parametrize("k", [32, 96, 4096, 1056])
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_q8_0_decode_quantizer_is_bit_exact(k, src):
    rng = np.random.default_rng(200 + k)
    x = acts(rng, 3, k)
    x[0, :32] = 0.0
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[src]
    xt = to_dev(x).to(tdt)
    vy, kp = qmm.quantize_decode(qmm.Q8_0, xt)
    xp = np.zeros((3, kp), np.float32)
    xp[:, :k] = xt.float().cpu().numpy()
    assert np.array_equal(vy.cpu().numpy(), O.quantize(O.Q8_0, xp).reshape(-1))


def special_value_row(k=2048):
    """NaN (a whole 32-value block, a single value, a whole 256-value block), an infinity, tiny normal values for which
    -127 / max overflows (saturated quantization) and negative zeros."""
    x = np.random.default_rng(9).standard_normal((2, k)).astype(np.float32)
    x[0, 0:32] = np.nan
    x[0, 40] = np.nan
    x[0, 256:512] = np.nan
    x[0, 512 + 7] = np.inf
    x[0, 768:1024] *= np.float32(1e-37)
    x[0, 1024:1280] = -0.0
    x[1, 300] = -np.inf
    return x


@pytest.mark.parametrize("qt", ["q8k", "q8_0"])
def test_decode_quantizers_on_special_values(qt):
    """The Q8_K slot quantizer and the Q8_0 block quantizer against the oracle, byte for byte, on NaN, infinite,
    overflowing and zero blocks (a block of NaNs: d = 0, as the reference's fold from 0 gives it)."""
    x = special_value_row()
    k = x.shape[1]
    if qt == "q8k":
        vy, kp = qmm.quantize_decode(qmm.Q4K, to_dev(x))
        xp = np.zeros((2, kp), np.float32)
        xp[:, :k] = x
        got = decode_act_blocks(O.Q4K, vy.cpu().numpy(), 2, kp)
        assert np.array_equal(got.view(np.uint8), O.quantize(O.Q8K, xp).reshape(-1).view(np.uint8))
    else:
        vy, kp = qmm.quantize_decode(qmm.Q8_0, to_dev(x))
        assert np.array_equal(vy.cpu().numpy(), O.quantize(O.Q8_0, x).reshape(-1))


def test_q8_0_quantizer_on_the_reference_known_answer_blocks():
    import test_oracle as T
    x = np.stack(T.reference_test_blocks()).reshape(1, -1)
    vy, kp = qmm.quantize_decode(qmm.Q8_0, to_dev(x))
    assert np.array_equal(vy.cpu().numpy(), O.quantize(O.Q8_0, x).reshape(-1))


CASES = [
    # (gtype, n, k, b)
    (O.Q4K, 256, 512, 1), (O.Q4K, 300, 1024, 3), (O.Q4K, 64, 4096, 4), (O.Q4K, 96, 14336, 2),
    (O.Q4K, 257, 2048, 8), (O.Q4K, 100, 4096, 16), (O.Q4K, 33, 256, 11),
    (O.Q6K, 256, 512, 1), (O.Q6K, 300, 1024, 4), (O.Q6K, 40, 14336, 1), (O.Q6K, 77, 4096, 9), (O.Q6K, 5, 768, 16),
    (O.Q8_0, 256, 512, 1), (O.Q8_0, 300, 1024, 4), (O.Q8_0, 48, 1056, 3), (O.Q8_0, 64, 4096, 8),
    (O.Q8_0, 31, 96, 2), (O.Q8_0, 17, 2688, 16),
]


@pytest.mark.parametrize("gtype,n,k,b", CASES)
def test_mmvq_matches_the_cpu_qmatmul(gtype, n, k, b):
    rng = np.random.default_rng(1000 * gtype + n + k + b)
    w = weights(rng, n, k)
    x = acts(rng, b, k)
    x[:, ::64] *= 60.0  # outliers: one scale per block far off (quantized/mod.rs:1775-1850)
    wq = O.quantize(gtype, w)
    want = O.matmul(gtype, x, wq, n)
    got = qmm.qmatmul_decode(gtype, to_dev(wq), to_dev(x), n).cpu().numpy()
    assert_parity(got, want, terms(gtype, x, wq, n), what=f"t{gtype} n{n} k{k} b{b}")


@pytest.mark.parametrize("n,k,b", [(256, 512, 1), (300, 1024, 4), (48, 1056, 3), (17, 2688, 16), (64, 14336, 2)])
def test_q8_0_reference_entries_over_q8_1_slots(n, k, b):
    """The reference's own sequence for a Q8_0 weight: launch_mmvq_gguf_quantize_q8_1_f32 then
    launch_mmvq_gguf_q8_0_f32_plain with stride_col_y = k_padded / 32.  The activation is Q8_K (one f32 scale per
    256 values), so the result is the CPU QMatMul's arithmetic over Q8_K activations (oracle matmul_q8k_act)."""
    rng = np.random.default_rng(3000 + n + k + b)
    wq = O.quantize(O.Q8_0, weights(rng, n, k))
    x = acts(rng, b, k)
    x[:, ::64] *= 60.0
    got = qmm.qmatmul_decode(O.Q8_0, to_dev(wq), to_dev(x), n, q8_1=True).cpu().numpy()
    assert_parity(got, O.matmul_q8k_act(O.Q8_0, x, wq, n), terms(O.Q8_0, x, wq, n), what=f"n{n} k{k} b{b}")


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0])
def test_mmvq_patterned_fixture(gtype):
    n, k = 64, 512
    w = patterned(n * k, 1).reshape(n, k)
    x = patterned(3 * k, 2).reshape(3, k)
    wq = O.quantize(gtype, w)
    got = qmm.qmatmul_decode(gtype, to_dev(wq), to_dev(x), n).cpu().numpy()
    assert_parity(got, O.matmul(gtype, x, wq, n), terms(gtype, x, wq, n))


@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_mmvq_half_outputs(out):
    rng = np.random.default_rng(7)
    n, k = 128, 1024
    wq = O.quantize(O.Q4K, weights(rng, n, k))
    x = acts(rng, 2, k)
    want = O.matmul(O.Q4K, x, wq, n)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[out]
    vy, kp = qmm.quantize_decode(O.Q4K, to_dev(x))
    got = qmm.mmvq(O.Q4K, to_dev(wq), vy, k, n, 2, kp, out_dtype=tdt).float().cpu().numpy()
    # the f32 result rounded once to the half type: the north-star bound plus half an ulp of each value
    ulp = {"f16": 2.0 ** -11, "bf16": 2.0 ** -8}[out]
    assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max() + ulp * np.abs(want))


def test_mmvq_config_shape_q4k_14336x4096():
    """Q4_K 14336x4096 from N(0, 0.02), activation [1, 4096] ~ N(0, 1); also b = 4 and 16."""
    rng = np.random.default_rng(20261201)
    n, k = 14336, 4096
    w = weights(rng, n, k)
    wq = O.quantize(O.Q4K, w)
    wd = to_dev(wq)
    for b in (1, 4, 16):
        x = acts(rng, b, k)
        want = O.matmul(O.Q4K, x, wq, n)
        got = qmm.qmatmul_decode(O.Q4K, wd, to_dev(x), n).cpu().numpy()
        r = assert_parity(got, want, what=f"b={b}")
        print(f"Q4_K 14336x4096 b={b}: max rel err {r:.2e}")


def test_mmvq_config_shape_q8_0_4096():
    """Q8_0 4096x4096 from N(0, 0.02), activation [1, 4096]."""
    rng = np.random.default_rng(20261202)
    n = k = 4096
    wq = O.quantize(O.Q8_0, weights(rng, n, k))
    x = acts(rng, 1, k)
    got = qmm.qmatmul_decode(O.Q8_0, to_dev(wq), to_dev(x), n).cpu().numpy()
    assert_parity(got, O.matmul(O.Q8_0, x, wq, n))


def test_row_stride_and_dst_stride():
    rng = np.random.default_rng(9)
    n, k = 50, 512
    wq = O.quantize(O.Q6K, weights(rng, n, k))
    x = acts(rng, 3, k)
    vy, kp = qmm.quantize_decode(O.Q6K, to_dev(x), kp=1024)  # padded activation rows
    out = torch.full((3, 64), 123.0, device=DEV)
    qmm.mmvq(O.Q6K, to_dev(wq), vy, k, n, 3, kp, out=out, stride_col_dst=64)
    got = out.cpu().numpy()
    assert_parity(got[:, :n], O.matmul(O.Q6K, x, wq, n))
    assert np.all(got[:, n:] == 123.0)  # nothing written past nrows

