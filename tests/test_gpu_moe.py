"""GPU parity of the MoE paths through the C ABI: the expert-indexed matvec (op-level gather_forward and the
fused gate/up decode form), the dispatch tables, the expert-grouped prefill matmul and the weighted reduce."""
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


def experts(rng, gtype, E, n, k):
    if gtype == O.IQ4XS:  # no quantizer on this path: random blocks (every byte pattern is a valid block)
        return O.random_blocks(O.IQ4XS, E * n * k, rng, 0.002).reshape(E, -1)
    w = weights(rng, E * n, k)
    return O.quantize(gtype, w).reshape(E, -1)


def routing(rng, tokens, E, topk):
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, ids, 1)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return ids.astype(np.int32), w


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("xdim1", [1, 2])
def test_indexed_moe_matches_the_oracle(gtype, xdim1):
    rng = np.random.default_rng(gtype + xdim1)
    E, n, k, batch, topk = 4, 96, 512, 5, 2
    wq = experts(rng, gtype, E, n, k)
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    x = acts(rng, batch * xdim1, k).reshape(batch, xdim1, k)
    want = O.indexed_moe(gtype, wq, E, n, k, x, ids)
    got = qmm.indexed_moe(gtype, to_dev(wq), to_dev(x), to_dev(ids), n).cpu().numpy()
    assert_parity(got, want)


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K])
def test_moe_decode_fused_glu(gtype):
    rng = np.random.default_rng(5)
    E, inter, hidden, tokens, topk = 4, 128, 512, 3, 2
    gate = experts(rng, gtype, E, inter, hidden)
    up = experts(rng, gtype, E, inter, hidden)
    ids = rng.integers(0, E, (tokens, topk)).astype(np.uint32)
    x = acts(rng, tokens, hidden)
    g = O.indexed_moe(gtype, gate, E, inter, hidden, x[:, None], ids).reshape(-1, inter)
    u = O.indexed_moe(gtype, up, E, inter, hidden, x[:, None], ids).reshape(-1, inter)
    vy, kp = qmm.quantize_decode(gtype, to_dev(x))
    stride = gate.shape[1]
    for act, f in ((0, lambda v: v / (1 + np.exp(-v))), (2, lambda v: np.maximum(v, 0))):
        got = qmm.mmvq_moe(gtype, to_dev(gate), to_dev(up), stride, vy, to_dev(ids.reshape(-1)), hidden, inter, kp,
                           topk, tokens * topk, activation=act).cpu().numpy()
        assert_parity(got, f(g.astype(np.float64)) * u)
    got = qmm.mmvq_moe(gtype, to_dev(gate), None, stride, vy, to_dev(ids.reshape(-1)), hidden, inter, kp, topk,
                       tokens * topk).cpu().numpy()
    assert_parity(got, g)


def test_moe_dispatch_groups_routes_by_expert():
    rng = np.random.default_rng(6)
    E, tokens, topk = 8, 64, 2
    ids, _ = routing(rng, tokens, E, topk)
    bounds, tok, src, counts, cursors = qmm.moe_dispatch(to_dev(ids.reshape(-1)), E, topk)
    wb, _, _ = O.moe_dispatch(ids, E, topk)
    b, t, s = bounds.cpu().numpy(), tok.cpu().numpy(), src.cpu().numpy()
    assert np.array_equal(b, wb)
    assert np.array_equal(counts.cpu().numpy(), np.diff(wb))
    assert np.array_equal(cursors.cpu().numpy(), wb[1:])
    flat = ids.reshape(-1)
    for e in range(E):
        seg = t[b[e]:b[e + 1]]
        assert np.all(flat[seg] == e)
        assert np.array_equal(s[b[e]:b[e + 1]], seg // topk)
    assert np.array_equal(np.sort(t), np.arange(tokens * topk))


def test_moe_dispatch_many_experts_and_empty():
    rng = np.random.default_rng(7)
    E, tokens, topk = 1500, 700, 3
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(tokens)]).astype(np.int32)
    bounds, tok, src, _, _ = qmm.moe_dispatch(to_dev(ids.reshape(-1)), E, topk)
    assert np.array_equal(bounds.cpu().numpy(), O.moe_dispatch(ids, E, topk)[0])
    b0, _, _, c0, _ = qmm.moe_dispatch(torch.zeros(0, dtype=torch.int32, device=DEV), 4, 2)
    assert np.all(b0.cpu().numpy() == 0) and np.all(c0.cpu().numpy() == 0)


def skewed_routing(rng, tokens, E, topk):
    """Expert 0 on every token (more than 32 rows), experts 0..E/2 only: the rest receive none."""
    ids = np.zeros((tokens, topk), dtype=np.int32)
    for t in range(tokens):
        ids[t, 1:] = rng.choice(np.arange(1, E // 2 + 1), topk - 1, replace=False)
    return ids


# 64 tokens x top-2 over 8 experts (16 rows each on average) and the skewed case take the few-row route of the
# K-quant grouped matmul; 400 tokens (100 rows per expert) take the 128-row tile route.
@pytest.mark.parametrize("case", ["uniform64", "skewed64", "uniform400"])
@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0, O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS])
def test_grouped_prefill_matches_the_oracle(gtype, case):
    rng = np.random.default_rng(8 + gtype)
    E, n, k, topk = 8, 160, 1024, 2
    tokens = 400 if case == "uniform400" else 64
    if case == "uniform400":
        k = 512
    wq = experts(rng, gtype, E, n, k)
    ids = skewed_routing(rng, tokens, E, topk) if case == "skewed64" else routing(rng, tokens, E, topk)[0]
    x = acts(rng, tokens, k)
    want = O.indexed_moe(gtype, wq, E, n, k, x[:, None], ids.astype(np.uint32)).reshape(tokens * topk, n)
    bounds, tok, src, counts, _ = qmm.moe_dispatch(to_dev(ids.reshape(-1)), E, topk)
    y, kp = qmm.quantize_prefill(gtype, to_dev(x), ids=src)
    out = torch.full((tokens * topk, n), float("nan"), device=DEV)
    ncols_max = int(counts.max().item())
    qmm.mmq_moe(gtype, to_dev(wq), y, tok, bounds, E, k, n, tokens * topk, ncols_max, out)
    assert_parity(out.cpu().numpy(), want)
    if gtype in (O.Q4K, O.Q5K):
        # launch_mmq_gguf_<t>_moe_q8k over `_q8k` tiles: the min term's sums are exact integers on both tile forms,
        # so the same bits
        y16, _ = qmm.quantize_prefill(gtype, to_dev(x), ids=src, q8k=True)
        out16 = torch.full((tokens * topk, n), float("nan"), device=DEV)
        qmm.mmq_moe(gtype, to_dev(wq), y16, tok, bounds, E, k, n, tokens * topk, ncols_max, out16, q8k=True)
        assert np.array_equal(out16.cpu().numpy().view(np.uint32), out.cpu().numpy().view(np.uint32)), case


# Q6_K experts of an odd row count with an odd superblock count per row: every other expert starts 2 bytes past a
# dword (the 64-row tile stages superblocks in LDS from the dword holding their first byte); 200 tokens take the
# 64-row tiles, 24 the 32-row ones.
@pytest.mark.parametrize("tokens", [24, 200])
def test_grouped_q6_k_experts_2_bytes_past_a_dword(tokens):
    rng = np.random.default_rng(17 + tokens)
    E, n, k, topk = 4, 129, 768, 2
    wq = experts(rng, O.Q6K, E, n, k)
    ids = routing(rng, tokens, E, topk)[0]
    x = acts(rng, tokens, k)
    want = O.indexed_moe(O.Q6K, wq, E, n, k, x[:, None], ids.astype(np.uint32)).reshape(tokens * topk, n)
    bounds, tok, src, counts, _ = qmm.moe_dispatch(to_dev(ids.reshape(-1)), E, topk)
    y, kp = qmm.quantize_prefill(O.Q6K, to_dev(x), ids=src)
    out = torch.full((tokens * topk, n), float("nan"), device=DEV)
    qmm.mmq_moe(O.Q6K, to_dev(wq), y, tok, bounds, E, k, n, tokens * topk, int(counts.max().item()), out)
    assert_parity(out.cpu().numpy(), want)


@pytest.mark.parametrize("kind", ["f32", "bf16_out", "f16_in", "bf16_in"])
def test_weighted_reduce(kind):
    rng = np.random.default_rng(9)
    tokens, topk, hidden = 37, 3, 300
    inp = rng.standard_normal((tokens, topk, hidden)).astype(np.float32)
    w = rng.random((tokens, topk)).astype(np.float32)
    w[4, 2] = 0.0
    inp[4, 2] = np.nan  # never read
    want = O.moe_weighted_reduce(inp, w)
    t = to_dev(inp)
    if kind == "f16_in":
        t = t.half()
    elif kind == "bf16_in":
        t = t.bfloat16()
    got = qmm.moe_weighted_reduce(t, to_dev(w), out_dtype=torch.bfloat16 if kind == "bf16_out" else None)
    tol = 1e-6 if kind == "f32" else 2e-2
    np.testing.assert_allclose(got.float().cpu().numpy(), want, rtol=tol, atol=tol)


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("tokens,topk", [(1, 2), (5, 4), (8, 8)])
def test_moe_down_with_weighted_sum(gtype, tokens, topk):
    """launch_mmvq_gguf_<t>_moe_wsum equals the two launches it replaces (the down projection per route, then the
    weighted reduce), and both match the oracle's per-route matmul and reduce; zero-weight routes drop out."""
    rng = np.random.default_rng(100 * gtype + 10 * tokens + topk)
    E, hidden, inter = 8, 256, 512 if gtype != O.Q8_0 else 160
    down = experts(rng, gtype, E, hidden, inter)
    ids, w = routing(rng, tokens, E, topk)
    w[0, -1] = 0.0  # a route that contributes nothing
    mid = acts(rng, tokens * topk, inter)
    vy, kp = qmm.quantize_decode(gtype, to_dev(mid))
    ids_d, w_d = to_dev(ids.astype(np.uint32).reshape(-1)), to_dev(w.reshape(-1))
    got = qmm.mmvq_moe_wsum(gtype, to_dev(down), down.shape[1], vy, ids_d, w_d, inter, hidden, kp, tokens,
                            topk).cpu().numpy()
    per_route = qmm.mmvq_moe(gtype, to_dev(down), None, down.shape[1], vy, ids_d, inter, hidden, kp, 1,
                             tokens * topk)
    two = qmm.moe_weighted_reduce(per_route.reshape(tokens, topk, hidden), w_d).cpu().numpy()
    np.testing.assert_allclose(got, two, rtol=1e-6, atol=1e-6 * np.abs(two).max())
    routes = O.indexed_moe(gtype, down, E, hidden, inter, mid.reshape(tokens, topk, inter),
                           ids.astype(np.uint32)).reshape(tokens, topk, hidden)
    assert_parity(got, O.moe_weighted_reduce(routes, w), what=f"moe wsum type {gtype}")


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("tokens,grouped", [(3, 0), (8, 0), (3, 1), (40, 0)])
def test_moe_experts_block(gtype, tokens, grouped):
    """The host MoE block (qmm_moe_forward): out[t] = sum_s w[t, s] * down_e(SiLU(gate_e(x_t)) * up_e(x_t)), on the
    indexed decode route (the down projection with the weighted sum folded in) and the grouped prefill route,
    against the oracle's matmuls per route and its weighted reduce."""
    import ctypes
    rng = np.random.default_rng(7 * gtype + tokens + 100 * grouped)
    E, hidden, inter, topk = 4, 256, 512, 2
    mats = [experts(rng, gtype, E, inter, hidden), experts(rng, gtype, E, inter, hidden),
            experts(rng, gtype, E, hidden, inter)]
    H = qmm.host()
    handles = []
    try:
        for m, (rows, cols) in zip(mats, ((inter, hidden), (inter, hidden), (hidden, inter))):
            h = ctypes.c_void_p()
            rc = H.qmm_qtensor_from_data(gtype, m.ctypes.data, m.size, E, rows, cols, 0, ctypes.byref(h))
            assert rc == 0, H.qmm_host_last_error()
            handles.append(h)
        moe = ctypes.c_void_p()
        assert H.qmm_moe_new(handles[0], handles[1], handles[2], 0, ctypes.byref(moe)) == 0, H.qmm_host_last_error()
        ids, w = routing(rng, tokens, E, topk)
        x = acts(rng, tokens, hidden)
        out = torch.empty((tokens, hidden), dtype=torch.float32, device=DEV)
        xd, idd, wd = to_dev(x), to_dev(ids), to_dev(w)
        rc = H.qmm_moe_forward(moe, xd.data_ptr(), tokens, idd.data_ptr(), wd.data_ptr(), topk, out.data_ptr(),
                               torch.cuda.current_stream().cuda_stream, grouped)
        assert rc == 0, H.qmm_host_last_error()
        torch.cuda.synchronize()
        H.qmm_moe_free(moe)
        got = out.cpu().numpy()
    finally:
        for h in handles:
            H.qmm_qtensor_free(h)
    u32 = ids.astype(np.uint32)
    g = O.indexed_moe(gtype, mats[0], E, inter, hidden, x[:, None], u32).astype(np.float64)
    u = O.indexed_moe(gtype, mats[1], E, inter, hidden, x[:, None], u32).astype(np.float64)
    mid = (g / (1 + np.exp(-g)) * u).astype(np.float32)
    routes = O.indexed_moe(gtype, mats[2], E, hidden, inter, mid, u32)
    # the intermediate is rounded to f32 by different exp implementations before its Q8 requantization: a value may
    # land on the other side of a rounding step, which moves the output far less than the north-star bound
    assert_parity(got, O.moe_weighted_reduce(routes, w), what=f"moe block type {gtype} tokens={tokens}")
