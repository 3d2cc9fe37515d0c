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


@pytest.mark.parametrize("gtype,k,b", [(O.Q4K, 8192, 1), (O.Q4K, 1024, 3), (O.Q8_0, 1056, 1)])
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
