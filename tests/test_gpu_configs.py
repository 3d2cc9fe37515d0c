"""GPU parity at the benchmark configurations' real shapes, through the same launches the bench times and through the
host QMatMul / MoE block, against the oracle's CPU QMatMul on every output.

Config 4: the Llama-3-8B linear stack (Q4_K q 4096x4096, k 1024x4096, o 4096x4096, gate/up 14336x4096; Q6_K v
1024x4096, down 4096x14336) at decode batch 1, 8 and 32 (the reference's quantized_llama.rs:25-68 projections; route
thresholds gguf/mod.rs:434-452).  Config 5: the Mixtral-shaped MoE, 8 Q4_K experts of gate/up 14336x4096 and down
4096x14336, 64 tokens top-2 from softmax(N(0,1) logits) (inference-nn/src/moe/experts/backends.rs:2175-2402).
Weights come from the oracle's restatement of the reference quantizer, activations are N(0,1); tolerance is the north
star's max relative error 1e-3 against the oracle (fp32 accumulation)."""
import ctypes

import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

STACK = [("q", O.Q4K, 4096, 4096), ("k", O.Q4K, 1024, 4096), ("v", O.Q6K, 1024, 4096), ("o", O.Q4K, 4096, 4096),
         ("gate", O.Q4K, 14336, 4096), ("up", O.Q4K, 14336, 4096), ("down", O.Q6K, 4096, 14336)]
F32 = 0  # GgmlDType::F32


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def silu(v):
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


@pytest.fixture(scope="module")
def stack():
    rng = np.random.default_rng(20261204)
    ws = {name: O.quantize(t, weights(rng, n, k)) for name, t, n, k in STACK}
    return ws, {name: dev(w) for name, w in ws.items()}


@pytest.mark.parametrize("b", [1, 2, 8, 24, 32])
def test_llama3_stack_projections_as_the_bench_runs_them(stack, b):
    """Each projection of one layer through the launch sequence bench.py's stack workload times, on QMatMul's route:
    the decode quantizer once per input and the matvec up to 32 rows (gate and up as one fused-GLU launch, SiLU),
    except the Q6_K down projection (K = 14336), which takes the prefill quantizer and matmul above 16 rows; at
    b <= 2, q / k / v in one launch and o and gate / up each in one, all three quantizing their own inputs."""
    ws, wd = stack
    rng = np.random.default_rng(40 + b)
    x = {"attn": acts(rng, b, 4096), "o": acts(rng, b, 4096), "ffn": acts(rng, b, 4096), "down": acts(rng, b, 14336)}
    group = {"q": "attn", "k": "attn", "v": "attn", "o": "o", "gate": "ffn", "up": "ffn", "down": "down"}
    spec = {name: (t, n, k) for name, t, n, k in STACK}
    want = {name: O.matmul(t, x[group[name]], ws[name], n) for name, (t, n, k) in spec.items()}
    xd = {g: dev(v) for g, v in x.items()}
    dec_of = {"attn": b <= 32, "o": b <= 32, "ffn": b <= 32, "down": b <= 16}
    bufs = {g: (qmm.quantize_decode(O.Q4K, v) if dec_of[g] else qmm.quantize_prefill(O.Q4K, v)) for g, v in xd.items()}
    if b <= 2:
        outs = qmm.mmvq_fused_qkv_quantize(O.Q4K, wd["q"], wd["k"], wd["v"], xd["attn"], 4096, 1024, 1024, vtype=O.Q6K)
        for name, got in zip("qkv", outs):
            assert_parity(got.cpu().numpy(), want[name], what=f"b={b} one-launch {name}")
        got = qmm.mmvq_fused_glu_quantize(O.Q4K, wd["gate"], wd["up"], xd["ffn"], 14336, activation=0).cpu().numpy()
        assert_parity(got, silu(want["gate"]) * want["up"], what=f"b={b} one-launch gate/up")
    for name in ("q", "k", "v", "o", "down"):
        t, n, k = spec[name]
        vy, kp = bufs[group[name]]
        decode = dec_of[group[name]]
        if decode and name == "o" and b <= 2:
            got = qmm.mmvq_quantize(t, wd[name], xd["o"], n)
        elif decode:
            got = qmm.mmvq(t, wd[name], vy, k, n, b, kp)
        else:
            got = qmm.mmq(t, wd[name], vy, k, n, b)
        assert_parity(got.cpu().numpy(), want[name], what=f"b={b} {name}")
    t, n, k = spec["gate"]
    vy, kp = bufs["ffn"]
    if dec_of["ffn"]:
        got = qmm.mmvq_fused_glu(t, wd["gate"], wd["up"], vy, k, n, b, kp, activation=0).cpu().numpy()
        assert_parity(got, silu(want["gate"]) * want["up"], what=f"b={b} fused gate/up")
    else:
        for name in ("gate", "up"):
            got = qmm.mmq(t, wd[name], vy, k, n, b).cpu().numpy()
            assert_parity(got, want[name], what=f"b={b} {name}")


@pytest.mark.parametrize("b", [1, 8, 24, 32, 40])
def test_llama3_stack_through_qmatmul_forward(stack, b):
    """The same projections through the host operator QMatMul::forward (qmm_qmatmul_forward), which picks the route
    for the row count itself."""
    ws, _ = stack
    H = qmm.host()
    rng = np.random.default_rng(80 + b)
    for name, t, n, k in STACK:
        w = ws[name]
        h = ctypes.c_void_p()
        rc = H.qmm_qtensor_from_data(t, w.ctypes.data, w.size, 1, n, k, 0, ctypes.byref(h))
        assert rc == 0, H.qmm_host_last_error()
        try:
            x = acts(rng, b, k)
            xd = dev(x)
            out = torch.full((b, n), float("nan"), dtype=torch.float32, device="cuda")
            rc = H.qmm_qmatmul_forward(h, xd.data_ptr(), F32, b, out.data_ptr(),
                                       torch.cuda.current_stream().cuda_stream)
            assert rc == 0, H.qmm_host_last_error()
            torch.cuda.synchronize()
        finally:
            H.qmm_qtensor_free(h)
        assert_parity(out.cpu().numpy(), O.matmul(t, x, w, n), what=f"QMatMul b={b} {name}")


# ------------------------------------------------------------------------------------------------ config 5

E, HIDDEN, INTER, TOKENS, TOPK = 8, 4096, 14336, 64, 2


def routing(rng, tokens, n_experts, topk):
    """top-k of softmax(logits), ties to the lower expert, weights renormalised (the Mixtral convention)"""
    logits = rng.standard_normal((tokens, n_experts)).astype(np.float32)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, ids, 1)
    return ids.astype(np.int32), (w / w.sum(1, keepdims=True)).astype(np.float32)


@pytest.fixture(scope="module")
def mixtral():
    """Eight distinct experts per projection: expert e is the quantized base weight with its rows rotated by 97 e
    (every row is a valid Q4_K row, and each expert differs at every row position)."""
    rng = np.random.default_rng(20261205)
    mats = []
    for rows, cols in ((INTER, HIDDEN), (INTER, HIDDEN), (HIDDEN, INTER)):
        base = O.quantize(O.Q4K, weights(rng, rows, cols))
        mats.append(np.ascontiguousarray(np.stack([np.roll(base, 97 * e, axis=0) for e in range(E)])))
    ids, w = routing(rng, TOKENS, E, TOPK)
    x = acts(rng, TOKENS, HIDDEN)
    return mats, ids, w, x


def test_mixtral_moe_grouped_projections(mixtral):
    """Each projection through dispatch -> gathered prefill quantization -> expert-grouped matmul
    (launch_mmq_gguf_q4_k_moe, and launch_mmq_gguf_q4_k_moe_q8k over `_q8k` tiles, the form the MoE block's grouped route
    runs) against the oracle's matmul per route at full shape; the down projection takes the oracle's own
    SiLU(gate) * up intermediate."""
    mats, ids, w, x = mixtral
    u32 = ids.astype(np.uint32)
    g = O.indexed_moe(O.Q4K, mats[0].reshape(E, -1), E, INTER, HIDDEN, x[:, None], u32).reshape(-1, INTER)
    u = O.indexed_moe(O.Q4K, mats[1].reshape(E, -1), E, INTER, HIDDEN, x[:, None], u32).reshape(-1, INTER)
    mid = (silu(g) * u).astype(np.float32)
    d = O.indexed_moe(O.Q4K, mats[2].reshape(E, -1), E, HIDDEN, INTER, mid.reshape(TOKENS, TOPK, INTER),
                      u32).reshape(-1, HIDDEN)
    bounds, tok, src, counts, _ = qmm.moe_dispatch(dev(ids.reshape(-1)), E, TOPK)
    ncols_max = int(counts.max().item())
    routes = TOKENS * TOPK
    for name, m, xin, rows_src, n, k, want in (
            ("gate", mats[0], x, src, INTER, HIDDEN, g), ("up", mats[1], x, src, INTER, HIDDEN, u),
            ("down", mats[2], mid, tok, HIDDEN, INTER, d)):
        y, _ = qmm.quantize_prefill(O.Q4K, dev(xin), ids=rows_src)
        out = torch.full((routes, n), float("nan"), device="cuda")
        md = dev(m)
        qmm.mmq_moe(O.Q4K, md, y, tok, bounds, E, k, n, routes, ncols_max, out)
        assert_parity(out.cpu().numpy(), want, what=f"grouped {name}")
        # the `_q8k` entry the host route takes, held to the oracle and to itself run again (the down projection splits
        # K in two here, summed in split order)
        y16, _ = qmm.quantize_prefill(O.Q4K, dev(xin), ids=rows_src, q8k=True)
        o1, o2 = (torch.full((routes, n), float("nan"), device="cuda") for _ in range(2))
        qmm.mmq_moe(O.Q4K, md, y16, tok, bounds, E, k, n, routes, ncols_max, o1, q8k=True)
        qmm.mmq_moe(O.Q4K, md, y16, tok, bounds, E, k, n, routes, ncols_max, o2, q8k=True)
        a = o1.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), o2.cpu().numpy().view(np.uint32)), f"grouped {name} (q8k) repeat"
        assert_parity(a, want, what=f"grouped {name} (q8k)")


@pytest.mark.parametrize("tokens", [TOKENS, 8])
def test_mixtral_moe_block(mixtral, tokens):
    """The host MoE block (qmm_moe_forward): out[t] = sum_s w[t, s] down_e(SiLU(gate_e(x_t)) up_e(x_t)), at 64 tokens on
    the grouped prefill route (what the bench times) and at 8 on the indexed decode route, against the oracle's
    per-route matmuls and weighted reduce.  The intermediate is requantized to Q8_K on both sides from f32 values whose
    summation order differs, so a value can land on the other side of a rounding step; the bound stays the north
    star's."""
    mats, ids, w, x = mixtral
    ids, w, x = ids[:tokens], w[:tokens], x[:tokens]
    H = qmm.host()
    handles = []
    try:
        for m, (rows, cols) in zip(mats, ((INTER, HIDDEN), (INTER, HIDDEN), (HIDDEN, INTER))):
            h = ctypes.c_void_p()
            rc = H.qmm_qtensor_from_data(O.Q4K, m.ctypes.data, m.size, E, rows, cols, 0, ctypes.byref(h))
            assert rc == 0, H.qmm_host_last_error()
            handles.append(h)
        moe = ctypes.c_void_p()
        assert H.qmm_moe_new(handles[0], handles[1], handles[2], 0, ctypes.byref(moe)) == 0, H.qmm_host_last_error()
        out = torch.full((tokens, HIDDEN), float("nan"), dtype=torch.float32, device="cuda")
        xd, idd, wd = dev(x), dev(ids), dev(w)
        rc = H.qmm_moe_forward(moe, xd.data_ptr(), tokens, idd.data_ptr(), wd.data_ptr(), TOPK, out.data_ptr(),
                               torch.cuda.current_stream().cuda_stream, 0)
        assert rc == 0, H.qmm_host_last_error()
        torch.cuda.synchronize()
        H.qmm_moe_free(moe)
        got = out.cpu().numpy()
    finally:
        for h in handles:
            H.qmm_qtensor_free(h)
    u32 = ids.astype(np.uint32)
    g = O.indexed_moe(O.Q4K, mats[0].reshape(E, -1), E, INTER, HIDDEN, x[:, None], u32)
    u = O.indexed_moe(O.Q4K, mats[1].reshape(E, -1), E, INTER, HIDDEN, x[:, None], u32)
    mid = (silu(g) * u).astype(np.float32)
    routes = O.indexed_moe(O.Q4K, mats[2].reshape(E, -1), E, HIDDEN, INTER, mid, u32)
    assert_parity(got, O.moe_weighted_reduce(routes, w), what=f"MoE block tokens={tokens}")
