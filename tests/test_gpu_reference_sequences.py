"""The reference's own call sequences replayed through the C ABI, unchanged: the entry names, arguments, scratch sizes
and strides its Rust callers use, with a guard region behind every scratch buffer (nothing may be written past the
size the reference allocates), against the oracle.

  fast_mmvq::plain (fast_mmvq.rs:534-650): launch_mmvq_gguf_quantize_q8_1_<src>(x, vy, k, k_padded = pad(k, 512),
      b) into b * k_padded / 32 * 36 bytes, then launch_mmvq_gguf_<t>_<dst>_plain(w, vy, dst, k, n,
      stride_col_y = k_padded / 32, n, b);
  gguf/cuda.rs:196-498: launch_indexed_moe_forward_<t>_q8_1 over the same quantizer's rows;
  gguf/cuda.rs:1355-1520: launch_moe_gemv_fused_gate_up_<t>_q8_1, then launch_moe_gemv_down_aggregate_<t>_q8_1 into a
      zeroed buffer;
  fast_mmq (fast_mmq.rs:446-715): launch_mmq_quantize_q8_1_{D4,DS4,D2S6}(x, NULL, vy, type_x, k, k, 0, 0,
      k_padded = pad(k, 512), M, 1, 1) into M * k_padded / 128 * 144 + 128 * 144 bytes, then launch_mmq_gguf_<t>;
      the GLU form launch_mmq_quantize_glu_q8_1_<L>[_f32] before the down projection.

The super-block types' results are their CPU QMatMul's (oracle matmul); the 32-value types (Q8_0, Q4_0, Q5_0) read
Q8_K activations through these names, so theirs are the oracle's matmul_q8k_act.  Bound: max rel. error <= 1e-3."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
GUARD = 4096
B32 = (O.Q8_0, O.Q4_0, O.Q5_0)
TYPES = [O.Q8_0, O.Q4K, O.Q6K, O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS]
MOE_TYPES = [O.Q8_0, O.Q4K, O.Q6K, O.Q4_0, O.Q5_0, O.Q5K]
SRC = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
TYPE_X = {"f32": 0, "f16": 1, "bf16": 30}


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def wbytes(rng, gtype, n, k):
    if gtype == O.IQ4XS:  # no quantizer on this path: random blocks (every byte pattern is a valid block)
        return O.random_blocks(O.IQ4XS, n * k, rng, 0.002).reshape(n, -1)
    return O.quantize(gtype, weights(rng, n, k))


def cpu(gtype, x, w, n):
    """The CPU result the reference-named entries reproduce."""
    return O.matmul_q8k_act(gtype, x, w, n) if gtype in B32 else O.matmul(gtype, x, w, n)


def guarded(nbytes):
    buf = torch.full((nbytes + GUARD,), 0xA5, dtype=torch.uint8, device=DEV)
    return buf


def assert_guard(buf, nbytes, what):
    tail = buf[nbytes:].cpu().numpy()
    assert np.all(tail == 0xA5), f"{what}: written past the reference's {nbytes}-byte scratch"


def decode_quantize(x, k):
    """launch_mmvq_gguf_quantize_q8_1_<src> as fast_mmvq::plain calls it; returns (scratch, k_padded, scratch bytes)."""
    b = x.shape[0]
    kp = qmm.pad_to(k, 512)
    nbytes = b * kp // 32 * 36
    vy = guarded(nbytes)
    src = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[x.dtype]
    getattr(qmm.lib(), f"launch_mmvq_gguf_quantize_q8_1_{src}")(qmm._ptr(x), qmm._ptr(vy), k, kp, b, qmm._stream())
    qmm.check()
    return vy, kp, nbytes


def kcase(gtype):
    # K not a multiple of 512, so k_padded > K and the padding is quantized as zeros
    return 1312 if gtype in B32 else 1280


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("src,dst", [("f32", "f32"), ("f16", "f16"), ("bf16", "bf16"), ("bf16", "f32")])
def test_fast_mmvq_plain_sequence(gtype, src, dst):
    rng = np.random.default_rng(500 + gtype * 7 + len(src) + len(dst))
    n, k = 300, kcase(gtype)
    wq = wbytes(rng, gtype, n, k)
    wd = to_dev(wq)
    for b in ((1, 5, 16, 32) if gtype in (O.Q4K, O.Q6K) else (1, 5, 16)):
        x = acts(rng, b, k)
        x[:, ::64] *= 40.0
        xt = to_dev(x).to(SRC[src])
        vy, kp, nbytes = decode_quantize(xt, k)
        out = torch.empty((b, n), dtype=SRC[dst], device=DEV)
        getattr(qmm.lib(), f"launch_mmvq_gguf_{qmm.tname(gtype)}_{dst}_plain")(
            qmm._ptr(wd), qmm._ptr(vy), qmm._ptr(out), k, n, kp // 32, n, b, qmm._stream())
        qmm.check()
        assert_guard(vy, nbytes, "quantize_q8_1")
        want = cpu(gtype, xt.float().cpu().numpy(), wq, n)
        got = out.float().cpu().numpy()
        if dst == "f32":
            assert_parity(got, want, what=f"t{gtype} {src}->{dst} b{b}")
        else:  # the f32 result rounded once to the half type
            ulp = 2.0 ** -8 if dst == "bf16" else 2.0 ** -11
            assert np.all(np.abs(got - want) <= 1e-3 * np.abs(want).max() + ulp * np.abs(want)), f"t{gtype} b{b}"


@pytest.mark.parametrize("gtype", MOE_TYPES)
@pytest.mark.parametrize("xdim1", [1, 2])
def test_indexed_moe_forward_sequence(gtype, xdim1):
    """gguf/cuda.rs:196-498: quantize the [batch * input_dim1, k] input with kx_padded = pad(k, 512), then
    launch_indexed_moe_forward_<t>_q8_1(w, vy, ids, out, n, k, batch, topk, k_padded, input_dim1)."""
    rng = np.random.default_rng(600 + gtype + xdim1)
    E, n, k, batch, topk = 4, 96, kcase(gtype), 5, 2
    wq = np.stack([wbytes(rng, gtype, n, k).reshape(-1) for _ in range(E)])
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    x = acts(rng, batch * xdim1, k)
    vy, kp, nbytes = decode_quantize(to_dev(x), k)
    out = torch.full((batch * topk, n), float("nan"), device=DEV)
    wd, idd = to_dev(wq), to_dev(ids)  # held until the launch has run
    getattr(qmm.lib(), f"launch_indexed_moe_forward_{qmm.MOE_TYPE[gtype]}_q8_1")(
        qmm._ptr(wd), qmm._ptr(vy), qmm._ptr(idd), qmm._ptr(out), n, k, batch, topk, kp, xdim1, qmm._stream())
    qmm.check()
    assert_guard(vy, nbytes, "quantize_q8_1")
    want = np.zeros((batch * topk, n), np.float32)
    for b in range(batch):
        for s in range(topk):
            row = b * xdim1 + (0 if xdim1 == 1 else s)
            want[b * topk + s] = cpu(gtype, x[row: row + 1], wq[ids[b, s]], n)[0]
    assert_parity(out.cpu().numpy(), want, what=f"t{gtype} xdim1={xdim1}")


def gelu_tanh(v):
    return 0.5 * v * (1.0 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3)))


def silu(v):
    return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("gtype", MOE_TYPES)
@pytest.mark.parametrize("act_type", [0, 1])
def test_moe_gemv_fused_decode_sequence(gtype, act_type):
    """indexed_moe_fused_decode (gguf/cuda.rs:1355-1520): the hidden state quantized with k_padded = pad(hidden, 512);
    launch_moe_gemv_fused_gate_up_<t>_q8_1 -> [batch * topk, inter] f32 (act_type 0 GELU-tanh, else SiLU); that
    quantized with pad(inter, 512); launch_moe_gemv_down_aggregate_<t>_q8_1 adds each token's weighted routes into
    the output buffer."""
    rng = np.random.default_rng(700 + gtype * 3 + act_type)
    E, hidden, inter, batch, topk = 4, kcase(gtype), 256 if gtype not in B32 else 288, 3, 2
    gate = np.stack([wbytes(rng, gtype, inter, hidden).reshape(-1) for _ in range(E)])
    up = np.stack([wbytes(rng, gtype, inter, hidden).reshape(-1) for _ in range(E)])
    down = np.stack([wbytes(rng, gtype, hidden, inter).reshape(-1) for _ in range(E)])
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(batch)]).astype(np.uint32)
    tw = rng.random((batch, topk)).astype(np.float32)
    tw[1, 1] = 0.0  # a route of weight zero contributes nothing
    x = acts(rng, batch, hidden)
    L = qmm.lib()
    t = qmm.MOE_TYPE[gtype]

    # device copies held until the launches have run (a temporary freed at once could be reused by the next copy)
    gd, ud, dd, idd, twd = (to_dev(a) for a in (gate, up, down, ids.reshape(-1), tw.reshape(-1)))
    vy, kp, nbytes = decode_quantize(to_dev(x), hidden)
    h = torch.full((batch * topk, inter), float("nan"), device=DEV)
    getattr(L, f"launch_moe_gemv_fused_gate_up_{t}_q8_1")(
        qmm._ptr(gd), qmm._ptr(ud), qmm._ptr(vy), qmm._ptr(idd), qmm._ptr(h), inter, hidden, batch, topk, kp, act_type,
        qmm._stream())
    qmm.check()
    assert_guard(vy, nbytes, "quantize_q8_1 (hidden)")
    act = gelu_tanh if act_type == 0 else silu
    want_h = np.zeros((batch * topk, inter), np.float64)
    for b in range(batch):
        for s in range(topk):
            e = ids[b, s]
            g = cpu(gtype, x[b: b + 1], gate[e], inter)[0].astype(np.float64)
            u = cpu(gtype, x[b: b + 1], up[e], inter)[0].astype(np.float64)
            want_h[b * topk + s] = act(g) * u
    got_h = h.cpu().numpy()
    assert_parity(got_h, want_h, what=f"gate_up t{gtype} act{act_type}")

    vh, kp2, nbytes2 = decode_quantize(h, inter)
    init = rng.standard_normal((batch, hidden)).astype(np.float32)
    for start in (np.zeros_like(init), init):
        out = to_dev(start)
        getattr(L, f"launch_moe_gemv_down_aggregate_{t}_q8_1")(
            qmm._ptr(dd), qmm._ptr(vh), qmm._ptr(idd), qmm._ptr(twd), qmm._ptr(out), hidden, inter, batch, topk, kp2,
            qmm._stream())
        qmm.check()
        assert_guard(vh, nbytes2, "quantize_q8_1 (intermediate)")
        want = np.zeros((batch, hidden), np.float64)
        for b in range(batch):
            for s in range(topk):
                p = b * topk + s
                want[b] += tw[b, s] * cpu(gtype, got_h[p: p + 1], down[ids[b, s]], hidden)[0]
        got = out.cpu().numpy().astype(np.float64) - start
        assert_parity(got, want, rel=2e-3, what=f"down_aggregate t{gtype}")


def mmq_scratch_bytes(m, kp):
    return m * kp // 128 * 144 + 128 * 144  # fast_mmq.rs: workspace_main + workspace_extra


def mmq_launch(gtype, w, vy, out, k, n, m):
    fx, nsm = qmm.fixup(w.device)
    type_dst = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 30}[out.dtype]
    getattr(qmm.lib(), f"launch_mmq_gguf_{qmm.tname(gtype)}")(
        qmm._ptr(fx), qmm._ptr(w), qmm._ptr(vy), qmm._ptr(out), k, n, m, k // O.BLOCK_SIZE[gtype], n, 0, nsm,
        160 * 1024, 64, type_dst, qmm._stream())
    qmm.check()


@pytest.mark.parametrize("gtype", TYPES)
@pytest.mark.parametrize("layout,src", [("D4", "f32"), ("DS4", "bf16"), ("D2S6", "f16")])
def test_fast_mmq_sequence(gtype, layout, src):
    """M = 40 and 130 rows; K = 1280 (a multiple of 256 but not of 512, so k_padded = K + 256) and, for the 32-value
    types, K = 1312 (not a multiple of 256: their kernel over single 32-value blocks)."""
    rng = np.random.default_rng(800 + gtype * 5 + len(layout))
    n = 200
    for m, k in ((40, kcase(gtype)), (130, 1280)):
        wq = wbytes(rng, gtype, n, k)
        x = acts(rng, m, k)
        x[:, ::64] *= 40.0
        xt = to_dev(x).to(SRC[src])
        kp = qmm.pad_to(qmm.pad_to(k, 512), 128)
        nbytes = mmq_scratch_bytes(m, kp)
        vy = guarded(nbytes)
        getattr(qmm.lib(), f"launch_mmq_quantize_q8_1_{layout}")(
            qmm._ptr(xt), None, qmm._ptr(vy), TYPE_X[src], k, k, 0, 0, kp, m, 1, 1, qmm._stream())
        qmm.check()
        out = torch.full((m, n), float("nan"), dtype=SRC[src], device=DEV)
        mmq_launch(gtype, to_dev(wq), vy, out, k, n, m)
        assert_guard(vy, nbytes, f"mmq_quantize_q8_1_{layout}")
        want = cpu(gtype, xt.float().cpu().numpy(), wq, n)
        got = out.float().cpu().numpy()
        ulp = {"f32": 0.0, "f16": 2.0 ** -11, "bf16": 2.0 ** -8}[src]
        err = np.abs(got - want)
        assert np.all(err <= 1e-3 * np.abs(want).max() + ulp * np.abs(want)), f"t{gtype} {layout} {src} m{m} k{k}"


def glu_host(g, u, activation, src):
    """The reference's mmq_glu_product on the host: f32 act(gate) * up, or, for f16 / bf16 inputs, act(gate) rounded
    to the input type, times up, rounded again."""
    g64 = g.astype(np.float64)
    a = {0: silu, 2: lambda v: np.maximum(v, 0.0)}[activation](g64).astype(np.float32)
    if src == "f32":
        return a * u
    dt = torch.float16 if src == "f16" else torch.bfloat16
    a = torch.from_numpy(a).to(dt).float().numpy()
    return torch.from_numpy(a * u).to(dt).float().numpy()


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K, O.Q8_0, O.Q5_0])
@pytest.mark.parametrize("form,src", [("_f32", "f32"), ("", "bf16"), ("", "f16")])
def test_fast_mmq_down_from_glu_sequence(gtype, form, src):
    """fast_mmq::down_from_glu (fast_mmq.rs:545-600): launch_mmq_quantize_glu_q8_1_<L>[_f32](gate, up, NULL, vy,
    [type_x,] k, k, k_padded, M, activation) then launch_mmq_gguf_<t> of the down weight.  ReLU: the products are
    exact, so the result is the oracle's down projection of the host-computed GLU values."""
    rng = np.random.default_rng(900 + gtype + len(src))
    m, n, k = 48, 160, kcase(gtype)
    wq = wbytes(rng, gtype, n, k)
    gate = to_dev(acts(rng, m, k)).to(SRC[src])
    up = to_dev(acts(rng, m, k)).to(SRC[src])
    kp = qmm.pad_to(k, 512)
    nbytes = mmq_scratch_bytes(m, kp)
    vy = guarded(nbytes)
    L = qmm.lib()
    if form == "_f32":
        L.launch_mmq_quantize_glu_q8_1_DS4_f32(qmm._ptr(gate), qmm._ptr(up), None, qmm._ptr(vy), k, k, kp, m, 2,
                                               qmm._stream())
    else:
        L.launch_mmq_quantize_glu_q8_1_D4(qmm._ptr(gate), qmm._ptr(up), None, qmm._ptr(vy), TYPE_X[src], k, k, kp, m,
                                          2, qmm._stream())
    qmm.check()
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    mmq_launch(gtype, to_dev(wq), vy, out, k, n, m)
    assert_guard(vy, nbytes, "mmq_quantize_glu_q8_1")
    h = glu_host(gate.float().cpu().numpy(), up.float().cpu().numpy(), 2, src)
    assert_parity(out.cpu().numpy(), cpu(gtype, h, wq, n), what=f"t{gtype} {src}")


@pytest.mark.parametrize("row_bytes,rows,n", [(144 * 16, 10, 7), (210, 5, 9), (34, 100, 70000), (4000, 3000, 3)])
def test_gather_rows_u8(row_bytes, rows, n):
    """launch_gather_rows_u8 (gguf/ffi.rs:591-599, raw.rs:405): dst row i = src row ids[i], bytes copied as they are;
    an id past the source rows gives a zero row."""
    rng = np.random.default_rng(row_bytes + rows + n)
    src = rng.integers(0, 256, (rows, row_bytes), dtype=np.uint8)
    ids = rng.integers(0, rows, n).astype(np.uint32)
    ids[-1] = rows + 3  # out of range
    out = torch.full((n, row_bytes), 0x5A, dtype=torch.uint8, device=DEV)
    qmm.gather_rows_u8(to_dev(src), to_dev(ids), row_bytes, rows, out=out)
    got = out.cpu().numpy()
    want = np.zeros((n, row_bytes), np.uint8)
    want[:-1] = src[ids[:-1]]
    assert np.array_equal(got, want)
