"""GPU parity of launch_mmvq_gguf_<t>_<dt>_quantize_plain, the decode matvec that quantizes its own f32
activations: bit-identical outputs to the two-launch sequence (decode quantizer, then the plain matvec), parity
with the oracle's CPU QMatMul, and its argument checks."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def rows(rng, b, k):
    x = acts(rng, b, k)
    x[:, ::64] *= 60.0
    if k >= 512:
        x[0, 256:512] = 0.0                 # an all-zero Q8_K block
        x[-1, 3], x[-1, 70] = -5.0, 5.0      # tied maxima of opposite signs
        x[-1, 1] = 7.0 if b > 1 else x[-1, 1]
    return x


CASES = [
    (O.Q4K, 300, 256, 1), (O.Q4K, 257, 1024, 2), (O.Q4K, 14336, 4096, 1), (O.Q4K, 100, 4096, 2),
    (O.Q6K, 300, 512, 1), (O.Q6K, 77, 4096, 2), (O.Q6K, 5, 768, 1),
    (O.Q8_0, 256, 512, 1), (O.Q8_0, 48, 1088, 2), (O.Q8_0, 4096, 4096, 1), (O.Q8_0, 31, 64, 2),
]


@pytest.mark.parametrize("gtype,n,k,b", CASES)
def test_same_bits_as_the_two_launches_and_oracle_parity(gtype, n, k, b):
    rng = np.random.default_rng(31 * gtype + n + k + b)
    wq = O.quantize(gtype, weights(rng, n, k))
    x = rows(rng, b, k)
    wd, xd = to_dev(wq), to_dev(x)
    vy, kp = qmm.quantize_decode(gtype, xd)
    two = qmm.mmvq(gtype, wd, vy, k, n, b, kp).cpu().numpy()
    one = qmm.mmvq_quantize(gtype, wd, xd, n).cpu().numpy()
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32)), f"t{gtype} n{n} k{k} b{b}"
    assert_parity(one, O.matmul(gtype, x, wq, n), what=f"t{gtype} n{n} k{k} b{b}")


@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_half_outputs_match_the_two_launches(out):
    rng = np.random.default_rng(5)
    n, k = 333, 2048
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[out]
    wd = to_dev(O.quantize(O.Q4K, weights(rng, n, k)))
    xd = to_dev(rows(rng, 2, k))
    vy, kp = qmm.quantize_decode(O.Q4K, xd)
    two = qmm.mmvq(O.Q4K, wd, vy, k, n, 2, kp, out_dtype=tdt)
    one = qmm.mmvq_quantize(O.Q4K, wd, xd, n, out_dtype=tdt)
    assert torch.equal(one, two)


def test_strided_unaligned_rows():
    """Rows 1040 floats apart and a base 4 bytes past 16-byte alignment: the scalar load path."""
    rng = np.random.default_rng(6)
    n, k = 200, 1024
    wq = O.quantize(O.Q6K, weights(rng, n, k))
    big = to_dev(rng.standard_normal((2, 1040)).astype(np.float32))
    xd = big[:, 1:1 + k]
    assert xd.data_ptr() % 16 == 4 and xd.stride(0) == 1040
    one = qmm.mmvq_quantize(O.Q6K, to_dev(wq), xd, n).cpu().numpy()
    x = xd.cpu().numpy()
    vy, kp = qmm.quantize_decode(O.Q6K, xd.contiguous())
    two = qmm.mmvq(O.Q6K, to_dev(wq), vy, k, n, 2, kp).cpu().numpy()
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))
    assert_parity(one, O.matmul(O.Q6K, x, wq, n))


def wide_row(rng, k):
    """One row over k > 4096 values with the blocks the per-lane quantizer must get right: a zero Q8_K block, tied
    maxima of opposite signs in different lanes (the first in index order wins) both ways round and within one lane,
    tied maxima of one sign, a block whose maximum sits in its last value."""
    x = acts(rng, 1, k)
    x[0, ::64] *= 60.0
    x[0, 256:512] = 0.0
    x[0, 512 + 3], x[0, 512 + 16] = 900.0, -900.0        # Q6_K: lane 0 before lane 1; Q4_K / Q8_0: one lane
    x[0, 768 + 200], x[0, 768 + 40] = 900.0, -900.0      # the negative one first, in another quarter
    x[0, 1024 + 130], x[0, 1024 + 131] = -900.0, 900.0   # adjacent, one lane
    x[0, 1280 + 7], x[0, 1280 + 250] = 900.0, 900.0
    x[0, 1536 + 255] = -900.0
    x[0, k - 256 + 64], x[0, k - 256 + 192] = 900.0, -900.0
    return x


WIDE = [(O.Q6K, 4096, 14336), (O.Q6K, 37, 4352), (O.Q6K, 1000, 16384), (O.Q4K, 4096, 14336), (O.Q4K, 203, 8192),
        (O.Q8_0, 4096, 14336), (O.Q8_0, 77, 4160), (O.Q8_0, 16, 16384)]


def same_kernel_as_two_launches(n, k):
    """The wide one-launch form is the four-wave matvec; the plain matvec takes that kernel itself for rows of 129 to
    256 units when the rows give every CU two workgroups of 8 rows, and then the bits match."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return 128 < k // 64 <= 256 and (n + 7) // 8 >= 2 * cus


@pytest.mark.parametrize("gtype,n,k", WIDE)
def test_wide_rows_one_column(gtype, n, k):
    """Above 4096 values at one column each lane quantizes its own unit in registers: parity with the oracle, the
    same bits as the two launches where the matvec is the same kernel, and the same bits call after call."""
    rng = np.random.default_rng(17 * gtype + n + k)
    wq = O.quantize(gtype, weights(rng, n, k))
    x = wide_row(rng, k)
    wd, xd = to_dev(wq), to_dev(x)
    one = qmm.mmvq_quantize(gtype, wd, xd, n).cpu().numpy()
    assert_parity(one, O.matmul(gtype, x, wq, n), what=f"t{gtype} n{n} k{k}")
    vy, kp = qmm.quantize_decode(gtype, xd)
    two = qmm.mmvq(gtype, wd, vy, k, n, 1, kp).cpu().numpy()
    if same_kernel_as_two_launches(n, k):
        assert np.array_equal(one.view(np.uint32), two.view(np.uint32)), f"t{gtype} n{n} k{k}"
    else:
        assert_parity(two, O.matmul(gtype, x, wq, n), what=f"two launches t{gtype} n{n} k{k}")
    again = qmm.mmvq_quantize(gtype, wd, xd, n).cpu().numpy()
    assert np.array_equal(again.view(np.uint32), one.view(np.uint32))


SPECIAL = {
    "nan": lambda x, r: (x.__setitem__((0, 2048 + 5), np.nan), x.__setitem__((0, slice(2304, 2560)), np.nan)),
    "inf_both_signs": lambda x, r: (x.__setitem__((0, 2560 + 100), np.inf), x.__setitem__((0, 2560 + 20), -np.inf)),
    "inf": lambda x, r: x.__setitem__((0, 2816 + 33), -np.inf),
    "tiny": lambda x, r: x.__setitem__((0, slice(3072, 3328)), r.standard_normal(256).astype(np.float32) * 1e-39),
    "smallest": lambda x, r: x.__setitem__((0, slice(3328, 3584)), np.float32(1e-45)),
    "negative_zero": lambda x, r: x.__setitem__((0, slice(3584, 3840)), -0.0),
}


@pytest.mark.parametrize("gtype", [O.Q6K, O.Q4K, O.Q8_0])
def test_wide_rows_special_values(gtype):
    """NaN (never the maximum, quantized to 0), infinities (tied of both signs, and alone), blocks of values so
    small that -127 / max overflows (saturated quantization), negative zeros: the same bits as the two launches,
    each case in a row of its own (an infinity makes every output NaN)."""
    rng = np.random.default_rng(23 + gtype)
    n, k = 4096, 14336
    assert same_kernel_as_two_launches(n, k)
    wd = to_dev(O.quantize(gtype, weights(rng, n, k)))
    for name, plant in SPECIAL.items():
        x = wide_row(rng, k)
        plant(x, rng)
        xd = to_dev(x)
        vy, kp = qmm.quantize_decode(gtype, xd)
        two = qmm.mmvq(gtype, wd, vy, k, n, 1, kp).cpu().numpy()
        one = qmm.mmvq_quantize(gtype, wd, xd, n).cpu().numpy()
        assert np.array_equal(one.view(np.uint32), two.view(np.uint32)), f"t{gtype} {name}"


@pytest.mark.parametrize("gtype,k,b", [(O.Q4K, 8192, 2), (O.Q6K, 16640, 1), (O.Q4K, 1024, 3), (O.Q8_0, 1056, 1)])
def test_rejected_shapes_launch_nothing(gtype, k, b):
    rng = np.random.default_rng(7)
    n = 16
    wd = to_dev(O.quantize(gtype, weights(rng, n, k)))
    out = torch.full((b, n), 5.0, device=DEV)
    with pytest.raises(qmm.QmmError):
        qmm.mmvq_quantize(gtype, wd, to_dev(acts(rng, b, k)), n, out=out)
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())


# ------------------------------------------------------------------------------------------------ several weights

QK = {O.Q4K: 4096, O.Q6K: 2048, O.Q8_0: 1024}


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("b", [1, 2])
@pytest.mark.parametrize("activation", [0, 2])
def test_fused_glu_quantize_same_bits_as_two_launches(gtype, b, activation):
    """launch_mmvq_gguf_<t>_f32_fused_glu_quantize: the bits of the decode quantizer followed by _fused_glu, and the
    oracle's act(gate) * up within the north-star bound."""
    rng = np.random.default_rng(300 + gtype + b + activation)
    n, k = 300, QK[gtype]
    wg, wu = O.quantize(gtype, weights(rng, n, k)), O.quantize(gtype, weights(rng, n, k))
    x = rows(rng, b, k)
    xd = to_dev(x)
    got = qmm.mmvq_fused_glu_quantize(gtype, to_dev(wg), to_dev(wu), xd, n, activation).cpu().numpy()
    vy, kp = qmm.quantize_decode(gtype, xd)
    two = qmm.mmvq_fused_glu(gtype, to_dev(wg), to_dev(wu), vy, k, n, b, kp, activation=activation).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), two.view(np.uint32))
    g = O.matmul(gtype, x, wg, n).astype(np.float64)
    u = O.matmul(gtype, x, wu, n).astype(np.float64)
    f = (lambda v: v / (1 + np.exp(-v))) if activation == 0 else (lambda v: np.maximum(v, 0))
    assert_parity(got, f(g) * u)


@pytest.mark.parametrize("gtype,vtype", [(O.Q4K, O.Q4K), (O.Q6K, O.Q6K), (O.Q8_0, O.Q8_0), (O.Q4K, O.Q6K)])
@pytest.mark.parametrize("b", [1, 2])
@pytest.mark.parametrize("ns", [(4096, 1024, 1024), (128, 0, 48), (0, 0, 64), (200, 33, 0)])
def test_fused_qkv_quantize(gtype, vtype, b, ns):
    """launch_mmvq_gguf_<t>_f32_fused_qkv_quantize (and the Q4_K / Q6_K mix): each output the bits of the decode
    quantizer followed by that weight's plain matvec (an empty projection is left out), and the oracle's."""
    rng = np.random.default_rng(400 + gtype + vtype + b + sum(ns))
    k = QK[gtype] if gtype == vtype else 4096
    types = (gtype, gtype, vtype)
    ws = [O.quantize(t, weights(rng, max(n, 1), k)) for t, n in zip(types, ns)]
    x = rows(rng, b, k)
    xd = to_dev(x)
    outs = qmm.mmvq_fused_qkv_quantize(gtype, *(to_dev(w) for w in ws), xd, *ns, vtype=vtype)
    for t, w, n, got in zip(types, ws, ns, outs):
        if n == 0:
            continue
        vy, kp = qmm.quantize_decode(t, xd)
        two = qmm.mmvq(t, to_dev(w), vy, k, n, b, kp).cpu().numpy()
        g = got.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), two.view(np.uint32)), f"type {t} n={n}"
        assert_parity(g, O.matmul(t, x, w, n), what=f"type {t} n={n}")


def test_fused_quantize_rejects_bad_shapes():
    w = torch.zeros(144 * 64, dtype=torch.uint8, device=DEV)
    x = torch.zeros((3, 256), device=DEV)
    with pytest.raises(qmm.QmmError, match="b_size"):
        qmm.mmvq_fused_glu_quantize(O.Q4K, w, w, x, 4)
    x = torch.zeros((1, 8192), device=DEV)
    with pytest.raises(qmm.QmmError, match="4096"):
        qmm.mmvq_fused_qkv_quantize(O.Q4K, w, w, w, x, 1, 1, 1)
