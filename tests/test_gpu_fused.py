"""GPU parity of the fused decode forms through the C ABI: launch_mmvq_gguf_<t>_<dt>_fused_glu (act(gate) * up of
one quantized activation) and _fused_qkv (three projections of one activation in one launch), for every weight type
the library serves, against the oracle's CPU QMatMul of each projection (max rel. error <= 1e-3; the GLU's activation
applied to the oracle's f32 output).  The 32-value types run both activation forms: their _q8_0 entries over Q8_0
blocks (the CPU QMatMul's own arithmetic) and the reference-named entries over Q8_1 slots (oracle matmul_q8k_act)."""
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
KS = {O.Q8_0: 512, O.Q4K: 512, O.Q6K: 768, O.Q4_0: 512, O.Q5_0: 544, O.Q5K: 512, O.IQ4XS: 768}
TYPES = [O.Q8_0, O.Q4K, O.Q6K, O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS]
# (weight type, q8_1): every type with its default activation, and the 32-value types on the reference names too
FORMS = [(t, None) for t in TYPES] + [(t, True) for t in (O.Q8_0, O.Q4_0, O.Q5_0)]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def wbytes(rng, gtype, n, k):
    if gtype == O.IQ4XS:  # no quantizer on this path: random blocks (every byte pattern is a valid block)
        return O.random_blocks(O.IQ4XS, n * k, rng, 0.002).reshape(n, -1)
    return O.quantize(gtype, weights(rng, n, k))


def cpu(gtype, x, w, n, q8_1):
    if q8_1 and gtype in (O.Q8_0, O.Q4_0, O.Q5_0):
        return O.matmul_q8k_act(gtype, x, w, n)
    return O.matmul(gtype, x, w, n)


@pytest.mark.parametrize("gtype,q8_1", FORMS)
@pytest.mark.parametrize("b", [1, 2, 3, 4, 16])
def test_fused_glu(gtype, q8_1, b):
    rng = np.random.default_rng(gtype * 10 + b)
    n, k = 200, KS[gtype]
    wg, wu = wbytes(rng, gtype, n, k), wbytes(rng, gtype, n, k)
    x = acts(rng, b, k)
    g = cpu(gtype, x, wg, n, q8_1).astype(np.float64)
    u = cpu(gtype, x, wu, n, q8_1).astype(np.float64)
    vy, kp = qmm.quantize_decode(gtype, dev(x), q8_1=q8_1)
    for act, f in ACTS.items():
        got = qmm.mmvq_fused_glu(gtype, dev(wg), dev(wu), vy, k, n, b, kp, activation=act, q8_1=q8_1).cpu().numpy()
        assert_parity(got, f(g) * u, what=f"t{gtype} q8_1={q8_1} b{b} act{act}")


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


@pytest.mark.parametrize("gtype,b", [(O.Q4K, 1), (O.Q4K, 2), (O.Q4K, 3), (O.Q6K, 1), (O.Q8_0, 1), (O.Q8_0, 5),
                                     (O.Q4_0, 2), (O.Q5K, 1)])
def test_fused_glu_wide_rows(gtype, b):
    """Hidden 18432 (K > 16384): rows of more than 256 units per wave take the looping kernel; every unit counts."""
    rng = np.random.default_rng(70 + gtype + b)
    n, k = 40, 18432
    wg, wu = wbytes(rng, gtype, n, k), wbytes(rng, gtype, n, k)
    x = acts(rng, b, k)
    g = O.matmul(gtype, x, wg, n).astype(np.float64)
    u = O.matmul(gtype, x, wu, n).astype(np.float64)
    vy, kp = qmm.quantize_decode(gtype, dev(x))
    got = qmm.mmvq_fused_glu(gtype, dev(wg), dev(wu), vy, k, n, b, kp, activation=0).cpu().numpy()
    assert_parity(got, ACTS[0](g) * u, what=f"t{gtype} b{b} K={k}")
    outs = qmm.mmvq_fused_qkv(gtype, dev(wg), dev(wu), dev(wg), vy, k, n, n, n, b, kp)
    assert_parity(outs[0].cpu().numpy(), g, what="qkv q")
    assert_parity(outs[1].cpu().numpy(), u, what="qkv k")


@pytest.mark.parametrize("gtype,q8_1", FORMS)
@pytest.mark.parametrize("b", [1, 2, 4, 16])
def test_fused_qkv(gtype, q8_1, b):
    rng = np.random.default_rng(gtype * 100 + b)
    k = KS[gtype]
    ns = (128, 32, 48)
    ws = [wbytes(rng, gtype, n, k) for n in ns]
    x = acts(rng, b, k)
    vy, kp = qmm.quantize_decode(gtype, dev(x), q8_1=q8_1)
    outs = qmm.mmvq_fused_qkv(gtype, *(dev(w) for w in ws), vy, k, *ns, b, kp, q8_1=q8_1)
    for w, n, got, name in zip(ws, ns, outs, "qkv"):
        want = cpu(gtype, x, w, n, q8_1)
        assert_parity(got.cpu().numpy(), want, terms(gtype, x, w, n), what=f"t{gtype} q8_1={q8_1} b{b} {name}")


@pytest.mark.parametrize("b", [1, 2, 8])
def test_fused_qkv_llama3_shapes(b):
    """Llama-3-8B attention projections: q 4096 x 4096, k and v 1024 x 4096, Q4_K, one launch."""
    rng = np.random.default_rng(20261204 + b)
    k = 4096
    ns = (4096, 1024, 1024)
    ws = [O.quantize(O.Q4K, weights(rng, n, k)) for n in ns]
    x = acts(rng, b, k)
    vy, kp = qmm.quantize_decode(O.Q4K, dev(x))
    outs = qmm.mmvq_fused_qkv(O.Q4K, *(dev(w) for w in ws), vy, k, *ns, b, kp)
    for w, n, got, name in zip(ws, ns, outs, "qkv"):
        assert_parity(got.cpu().numpy(), O.matmul(O.Q4K, x, w, n), what=f"llama3 b{b} {name}")
