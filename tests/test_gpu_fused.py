"""GPU parity of the fused decode forms through the C ABI: launch_mmvq_gguf_<t>_<dt>_fused_glu (act(gate) * up of
one quantized activation) and _fused_qkv (three projections of one activation in one launch), against the oracle's
CPU QMatMul of each projection (max rel. error <= 1e-3; the GLU's activation applied to the oracle's f32 output)."""
import math

import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, terms, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ERF = np.vectorize(math.erf)
ACTS = {  # GluActivation (inference-quant/kernels/cuda/glu_activation.cuh)
    0: lambda v: v / (1.0 + np.exp(-v)),
    1: lambda v: 0.5 * v * (1.0 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3))),
    2: lambda v: np.maximum(v, 0.0),
    3: lambda v: 0.5 * v * (1.0 + ERF(v / math.sqrt(2.0))),
    4: lambda v: 1.0 / (1.0 + np.exp(-v)),
}
KS = {O.Q8_0: 512, O.Q4K: 512, O.Q6K: 768}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("b", [1, 2, 3, 4, 16])
def test_fused_glu(gtype, b):
    rng = np.random.default_rng(gtype * 10 + b)
    n, k = 200, KS[gtype]
    wg, wu = O.quantize(gtype, weights(rng, n, k)), O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, b, k)
    g = O.matmul(gtype, x, wg, n).astype(np.float64)
    u = O.matmul(gtype, x, wu, n).astype(np.float64)
    vy, kp = qmm.quantize_decode(gtype, dev(x))
    for act, f in ACTS.items():
        got = qmm.mmvq_fused_glu(gtype, dev(wg), dev(wu), vy, k, n, b, kp, activation=act).cpu().numpy()
        assert_parity(got, f(g) * u, what=f"t{gtype} b{b} act{act}")


def test_fused_glu_half_output():
    rng = np.random.default_rng(3)
    gtype, n, k, b = O.Q4K, 96, 512, 4
    wg, wu = O.quantize(gtype, weights(rng, n, k)), O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, b, k)
    want = ACTS[0](O.matmul(gtype, x, wg, n).astype(np.float64)) * O.matmul(gtype, x, wu, n)
    vy, kp = qmm.quantize_decode(gtype, dev(x))
    got = qmm.mmvq_fused_glu(gtype, dev(wg), dev(wu), vy, k, n, b, kp, out_dtype=torch.float16).float().cpu().numpy()
    # act(gate) * up in f32, rounded once to f16: the north-star bound plus half an f16 ulp of each value
    assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max() + 2.0 ** -11 * np.abs(want))


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("b", [1, 2, 4, 16])
def test_fused_qkv(gtype, b):
    rng = np.random.default_rng(gtype * 100 + b)
    k = KS[gtype]
    ns = (128, 32, 48)
    ws = [O.quantize(gtype, weights(rng, n, k)) for n in ns]
    x = acts(rng, b, k)
    vy, kp = qmm.quantize_decode(gtype, dev(x))
    outs = qmm.mmvq_fused_qkv(gtype, *(dev(w) for w in ws), vy, k, *ns, b, kp)
    for w, n, got, name in zip(ws, ns, outs, "qkv"):
        want = O.matmul(gtype, x, w, n)
        assert_parity(got.cpu().numpy(), want, terms(gtype, x, w, n), what=f"t{gtype} b{b} {name}")
