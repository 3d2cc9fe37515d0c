"""GPU parity of the dense GLU routes of the host layer (fast_mmq.rs:717-899): QMatMul::down_from_glu (the GLU applied
inside the activation quantization, then the prefill matmul) and fused_ffn (gate and up over one activation
quantization, then down), through the C API (qmm_qmatmul_down_from_glu, qmm_fused_ffn), against the oracle's CPU
QMatMul chain: gate = x W_g^T, up = x W_u^T, mid = act(gate) * up in f32, out = mid W_d^T.  Tolerance: the north
star's max relative error 1e-3.  With ReLU the GPU's act(gate) * up is the same f32 value as the oracle's, so its
requantization is byte-identical and every element also meets the 1e-5 * sum|terms| bound."""
import ctypes

import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, terms, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def act(kind, v):
    """glu_activation.cuh: 0 SiLU, 1 GELU (tanh form), 2 ReLU, 3 GELU (erf form), 4 sigmoid -- in float64"""
    from math import erf
    v = np.asarray(v, np.float64)
    if kind == 0:
        return v / (1.0 + np.exp(-v))
    if kind == 1:
        return 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
    if kind == 2:
        return np.maximum(v, 0.0)
    if kind == 3:
        return 0.5 * v * (1.0 + np.vectorize(erf)(v / np.sqrt(2.0)))
    return 1.0 / (1.0 + np.exp(-v))


class Weights:
    """QTensor handles on the GPU for oracle-quantized weights."""

    def __init__(self):
        self.H = qmm.host()
        self.handles = []

    def add(self, gtype, wq, n, k):
        h = ctypes.c_void_p()
        rc = self.H.qmm_qtensor_from_data(gtype, wq.ctypes.data, wq.size, 1, n, k, 0, ctypes.byref(h))
        assert rc == 0, self.H.qmm_host_last_error()
        self.handles.append(h)
        return h

    def close(self):
        for h in self.handles:
            self.H.qmm_qtensor_free(h)


def host_fns():
    H = qmm.host()
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    H.qmm_qmatmul_down_from_glu.argtypes = [vp, vp, vp, i64, i32, vp, vp]
    H.qmm_fused_ffn.argtypes = [vp, vp, vp, vp, i64, i32, vp, vp]
    return H


# (weight type, rows, N, K): the K-quant kernel with 32/64/128-row tiles, split K, a 32-value type, the adjacent types
DOWN_CASES = [(O.Q4K, 40, 256, 1024), (O.Q6K, 130, 200, 2816), (O.Q8_0, 17, 300, 1024), (O.Q4_0, 64, 128, 512),
              (O.Q5K, 3, 96, 768), (O.Q6K, 1, 64, 256)]


@pytest.mark.parametrize("activation", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("gtype,m,n,k", DOWN_CASES)
def test_down_from_glu_matches_the_oracle(gtype, m, n, k, activation):
    rng = np.random.default_rng(500 + gtype * 7 + m + activation)
    wq = O.quantize(gtype, weights(rng, n, k))
    gate, up = acts(rng, m, k), acts(rng, m, k)
    if activation == 2:
        mid = np.maximum(gate, np.float32(0.0)) * up  # exact in f32, as on the GPU
    else:
        mid = (act(activation, gate) * up).astype(np.float32)
    want = O.matmul(gtype, mid, wq, n)
    H = host_fns()
    W = Weights()
    try:
        h = W.add(gtype, wq, n, k)
        out = torch.full((m, n), float("nan"), device="cuda")
        gd, ud = dev(gate), dev(up)  # (held: a temporary's memory could be handed to the next one)
        rc = H.qmm_qmatmul_down_from_glu(h, gd.data_ptr(), ud.data_ptr(), m, activation, out.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
        assert rc == 0, H.qmm_host_last_error()
        torch.cuda.synchronize()
    finally:
        W.close()
    got = out.cpu().numpy()
    assert_parity(got, want, terms(gtype, mid, wq, n) if activation == 2 else None,
                  what=f"down_from_glu t{gtype} m{m} act{activation}")


def ffn_case(rng, gt, dt, hidden, inter):
    return (O.quantize(gt, weights(rng, inter, hidden)), O.quantize(gt, weights(rng, inter, hidden)),
            O.quantize(dt, weights(rng, hidden, inter)))


def run_ffn(gt, dt, wg, wu, wd, x, hidden, inter, activation):
    H = host_fns()
    W = Weights()
    rows = x.shape[0]
    try:
        hg, hu = W.add(gt, wg, inter, hidden), W.add(gt, wu, inter, hidden)
        hd = W.add(dt, wd, hidden, inter)
        out = torch.full((rows, hidden), float("nan"), device="cuda")
        xd = dev(x)
        rc = H.qmm_fused_ffn(hg, hu, hd, xd.data_ptr(), rows, activation, out.data_ptr(),
                             torch.cuda.current_stream().cuda_stream)
        assert rc == 0, H.qmm_host_last_error()
        torch.cuda.synchronize()
    finally:
        W.close()
    return out.cpu().numpy()


def oracle_ffn(gt, dt, wg, wu, wd, x, hidden, inter, activation):
    g = O.matmul(gt, x, wg, inter)
    u = O.matmul(gt, x, wu, inter)
    mid = (act(activation, g) * u).astype(np.float32)
    return O.matmul(dt, mid, wd, hidden)


# rows <= 16 take the fused-GLU matvec, above the two prefill matmuls and down_from_glu
@pytest.mark.parametrize("rows", [1, 8, 16, 17, 64])
@pytest.mark.parametrize("gt,dt", [(O.Q4K, O.Q6K), (O.Q8_0, O.Q8_0), (O.Q6K, O.Q4K)])
def test_fused_ffn_matches_the_oracle(gt, dt, rows):
    """A Q4_K_M-style FFN (Q4_K gate/up, Q6_K down) and two other mixes at hidden 1024, inter 2816, SiLU."""
    rng = np.random.default_rng(900 + rows + gt)
    hidden, inter = 1024, 2816
    wg, wu, wd = ffn_case(rng, gt, dt, hidden, inter)
    x = acts(rng, rows, hidden)
    got = run_ffn(gt, dt, wg, wu, wd, x, hidden, inter, 0)
    assert_parity(got, oracle_ffn(gt, dt, wg, wu, wd, x, hidden, inter, 0), what=f"fused_ffn rows={rows}")


@pytest.mark.parametrize("rows", [4, 32])
def test_fused_ffn_llama3_shape(rows):
    """Config 4's FFN at its real shape: Q4_K gate/up 14336x4096, Q6_K down 4096x14336, SiLU."""
    rng = np.random.default_rng(77 + rows)
    hidden, inter = 4096, 14336
    wg, wu, wd = ffn_case(rng, O.Q4K, O.Q6K, hidden, inter)
    x = acts(rng, rows, hidden)
    got = run_ffn(O.Q4K, O.Q6K, wg, wu, wd, x, hidden, inter, 0)
    assert_parity(got, oracle_ffn(O.Q4K, O.Q6K, wg, wu, wd, x, hidden, inter, 0), what=f"llama3 ffn rows={rows}")


def test_fused_ffn_rejects_mismatched_weights():
    rng = np.random.default_rng(3)
    wg = O.quantize(O.Q4K, weights(rng, 512, 256))
    wd = O.quantize(O.Q6K, weights(rng, 512, 256))  # [512, 256]: not [hidden=256, inter=512]
    H = host_fns()
    W = Weights()
    try:
        hg, hu, hd = W.add(O.Q4K, wg, 512, 256), W.add(O.Q4K, wg, 512, 256), W.add(O.Q6K, wd, 512, 256)
        x = dev(acts(rng, 2, 256))
        out = torch.empty((2, 256), device="cuda")
        rc = H.qmm_fused_ffn(hg, hu, hd, x.data_ptr(), 2, 0, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        assert rc != 0 and b"down must be" in H.qmm_host_last_error()
    finally:
        W.close()
