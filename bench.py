#!/usr/bin/env python3
"""Benchmark of the GGUF quantized-linear hot path on one MI355X ("Q4_K bs=1 matvec GB/s (% of
HBM peak); prefill int8 TOPS at M=512").

One step = one pass of the hot path over one batch of synthetic input, with every input resident in HBM:
  headline: activation f32 [1, 4096] -> Q8_K values -> Q4_K 14336x4096 matvec -> f32 [1, 14336]
  in one launch, launch_mmvq_gguf_q4_k_f32_quantize_plain, whose output is bit-identical to the reference's two
  launches (launch_mmvq_gguf_quantize_q8_1_f32 + launch_mmvq_gguf_q4_k_f32_plain, fast_mmvq::plain); the two-launch
  step and its matvec alone are reported in "extra".  Weights rotate over 16 copies (528 MB > the 256 MB
  Infinity Cache), so every step streams its weight from HBM.  K steps are captured in one HIP graph and
  replayed once between a synchronize on both sides; `value` = algorithmic bytes per step / time per step.
Extra lines in "extra": Q4_K decode at b = 4 and 16, Q8_0 4096^2 decode, the M = 512 prefill (Q4_K and Q6_K,
int8 TOPS), the Llama-3-8B linear stack (tokens/s) and the 8-expert MoE (64 tokens, top-2).
`roofline` is the step's one kernel, `cpu_baseline` the reference's x86 CPU QMatMul route (oracle/x86.c, a C restatement of the
reference's) on the box's host cores over a bounded sample.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "inference.rs_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA, published (POP/s)
SEED = 20261201

Q8_0, Q4K, Q6K = 8, 12, 14
Q4_0, Q5_0, Q5K, IQ4XS = 2, 6, 13, 23
BS = {Q8_0: 32, Q4K: 256, Q6K: 256, Q4_0: 32, Q5_0: 32, Q5K: 256, IQ4XS: 256}
TS = {Q8_0: 34, Q4K: 144, Q6K: 210, Q4_0: 18, Q5_0: 22, Q5K: 176, IQ4XS: 136}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------------ data

_host = None


def host_lib():
    global _host
    if _host is None:
        import qmm
        _host = ctypes.CDLL(qmm.HOST_LIB_PATH)
        _host.qmm_quantize_cpu.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        _host.qmm_host_last_error.restype = ctypes.c_char_p
        for n in ("qmm_qtensor_from_data",):
            getattr(_host, n).argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
        _host.qmm_moe_new.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
        _host.qmm_moe_forward.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_int]
        _host.qmm_qtensor_device_ptr.argtypes = [ctypes.c_void_p]
        _host.qmm_qtensor_device_ptr.restype = ctypes.c_void_p
    return _host


def quantized_weight(gtype, n, k, seed):
    """N(0, 0.02) f32 weights quantized on the host by the library's QTensor quantizer (IQ4_XS, which has no
    quantizer in the reference: random indices and scale codes under f16 scales of 0.002)."""
    rng = np.random.default_rng(seed)
    if gtype == IQ4XS:
        raw = rng.integers(0, 256, n * k // 256 * 136, dtype=np.uint8)
        d = (rng.uniform(0.5, 1.5, n * k // 256) * 0.002).astype(np.float16).view(np.uint8).reshape(-1, 2)
        raw.reshape(-1, 136)[:, :2] = d
        return raw
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    out = np.empty(n * k // BS[gtype] * TS[gtype], dtype=np.uint8)
    rc = host_lib().qmm_quantize_cpu(gtype, w.ctypes.data, w.size, out.ctypes.data)
    if rc != 0:
        raise RuntimeError(host_lib().qmm_host_last_error().decode())
    return out


def device_copies(torch, data, copies):
    t = torch.from_numpy(data).cuda()
    return [t] + [t.clone() for _ in range(copies - 1)]


# ------------------------------------------------------------------------------------------------ timing

EAGER = False  # --eager: launch every step directly (for counter collection, which wants plain dispatches)


def graph_time(torch, fn, steps, warmup):
    """Capture `steps` calls of fn(i) in one HIP graph and replay it once between synchronizes; the same for
    `warmup` calls first (untimed).  Returns seconds for the timed replay."""
    if EAGER:
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            fn(i)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / 1e3
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(3):
            fn(i)  # eager: sizes workspaces, loads code objects
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    if warmup > 0:
        gw = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gw):
            for i in range(warmup):
                fn(i)
        gw.replay()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


# ------------------------------------------------------------------------------------------------ workloads

def decode_workload(torch, qmm, gtype, n, k, b, copies, steps, warmup, seed):
    """The reference's decode step as two launches: launch_mmvq_gguf_quantize_* (f32 activation -> Q8 blocks) and
    launch_mmvq_gguf_<t>_f32_plain (the matvec), with the matvec alone timed in a second graph; for b <= 2 and
    k <= 4096, or b = 1 and k <= 16384, also the same step as one launch, launch_mmvq_gguf_<t>_f32_quantize_plain
    (bit-identical output)."""
    wq = quantized_weight(gtype, n, k, seed)
    ws = device_copies(torch, wq, copies)
    rng = np.random.default_rng(seed + 1)
    x = torch.from_numpy(rng.standard_normal((b, k), dtype=np.float32)).cuda()
    vy, kp = qmm.quantize_decode(gtype, x)
    out = torch.empty((b, n), dtype=torch.float32, device="cuda")

    def step(i):
        qmm.quantize_decode(gtype, x, kp=kp, out=vy)
        qmm.mmvq(gtype, ws[i % copies], vy, k, n, b, kp, out=out)

    def matvec_only(i):
        qmm.mmvq(gtype, ws[i % copies], vy, k, n, b, kp, out=out)

    def one_launch(i):
        qmm.mmvq_quantize(gtype, ws[i % copies], x, n, out=out)

    t = graph_time(torch, step, steps, warmup)
    y = out.cpu().numpy()
    t_kernel = graph_time(torch, matvec_only, steps, warmup)
    w_bytes = wq.size
    act_q_bytes = qmm.act_bytes(gtype, b, kp)
    step_bytes = w_bytes + b * k * 4 + b * n * 4            # f32 activation in, f32 out
    # what the matvec itself must move: weights, the Q8 activation blocks, the f32 outputs
    kernel_bytes = w_bytes + act_q_bytes + b * n * 4
    r = {
        "seconds": t, "ms_per_step": t / steps * 1e3, "gb_s": step_bytes / (t / steps) / 1e9,
        "step_bytes": step_bytes, "kernel_us": t_kernel / steps * 1e6,
        "kernel_gb_s": kernel_bytes / (t_kernel / steps) / 1e9, "kernel_bytes": kernel_bytes,
        "weights": wq, "x": x.cpu().numpy(), "y": y,
    }
    if (b <= 2 and k <= 4096 or b == 1 and k <= 16384) and gtype in (Q8_0, Q4K, Q6K):
        t1 = graph_time(torch, one_launch, steps, warmup)
        if not np.array_equal(out.cpu().numpy().view(np.uint32), y.view(np.uint32)):
            raise RuntimeError("one-launch decode differs from the two-launch result")
        r["one_launch"] = {"ms_per_step": t1 / steps * 1e3, "gb_s": step_bytes / (t1 / steps) / 1e9,
                           "kernel_us": t1 / steps * 1e6}
    return r


def prefill_workload(torch, qmm, gtype, n, k, m, copies, steps, warmup, seed):
    wq = quantized_weight(gtype, n, k, seed)
    ws = device_copies(torch, wq, copies)
    rng = np.random.default_rng(seed + 1)
    x = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).cuda()
    # QMatMul::forward's prefill route: Q4_K and Q5_K read the `_q8k` tiles (launch_mmq_quantize_q8k and the _q8k
    # entries), Q6_K the Q8_K tiles, the 32-value types the Q8_0 tiles
    q8k = gtype in (Q4K, Q5K)
    y, kp = qmm.quantize_prefill(gtype, x, q8k=q8k)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")

    def step(i):
        qmm.quantize_prefill(gtype, x, out=y, q8k=q8k)
        qmm.mmq(gtype, ws[i % copies], y, k, n, m, out=out, q8k=q8k)

    def mmq_only(i):
        qmm.mmq(gtype, ws[i % copies], y, k, n, m, out=out, q8k=q8k)

    t = graph_time(torch, step, steps, warmup)
    tk = graph_time(torch, mmq_only, steps, warmup)
    ops = 2.0 * m * n * k
    return {"ms_per_step": t / steps * 1e3, "tops": ops / (t / steps) / 1e12, "kernel_us": tk / steps * 1e6,
            "kernel_tops": ops / (tk / steps) / 1e12, "ops": ops,
            "frac_int8_peak": ops / (tk / steps) / 1e12 / INT8_PEAK_TOPS}


def stack_workload(torch, qmm, batches, steps, warmup, seed):
    """Llama-3-8B linears, Q4_K for q/k/o/gate/up and Q6_K for v/down, 32 layers; one weight per shape is
    quantized and its bytes copied to every layer (distinct HBM copies, so every step streams 4.44 GB).
    Per layer, as the reference's decode path runs them: the attention input is quantized once and q, k, v read
    that one activation; o and down quantize their own inputs; gate and up are one fused-GLU launch
    (launch_mmvq_gguf_q4_k_f32_fused_glu) over their shared input.  At b <= 2 the launches that can quantize their
    own f32 input do: q, k and v in one launch (launch_mmvq_gguf_q4_k_q6_k_f32_fused_qkv_quantize), o
    (launch_mmvq_gguf_q4_k_f32_quantize_plain) and gate / up (launch_mmvq_gguf_q4_k_f32_fused_glu_quantize), with the
    same output bits as their two-launch forms; the down projection (K = 14336) quantizes its own input at b = 1
    (launch_mmvq_gguf_q6_k_f32_quantize_plain, the same bits as its two launches) and keeps its quantizer at b = 2.
    Each input
    takes QMatMul's route: the decode launcher up to 32 rows, except the Q6_K down projection (K = 14336) above 16
    rows, which takes the prefill matmul; one quantized activation per distinct input.  The inputs are synthetic, one
    per projection group."""
    shapes = [("q", Q4K, 4096, 4096), ("k", Q4K, 1024, 4096), ("v", Q6K, 1024, 4096), ("o", Q4K, 4096, 4096),
              ("gate", Q4K, 14336, 4096), ("up", Q4K, 14336, 4096), ("down", Q6K, 4096, 14336)]
    layers = 32
    base = {name: quantized_weight(t, n, k, seed + i) for i, (name, t, n, k) in enumerate(shapes)}
    dev = {name: [torch.from_numpy(base[name]).cuda() for _ in range(layers)] for name, _, _, _ in shapes}
    total_bytes = sum(base[name].size for name, _, _, _ in shapes) * layers
    res = {"weight_bytes_per_step": total_bytes,
           "launches_per_layer": "decode b = 1: q/k/v in one launch, o, gate/up and down each in one, all four "
                                 "quantizing their input = 4; b = 2: the same with down quantize + matvec = 5; "
                                 "b 3..16: 4 quantize + 6 = 10; b 17..32: the same with down on the prefill matmul "
                                 "= 10"}
    import qmm as Q
    for b in batches:
        rng = np.random.default_rng(seed + 100 + b)
        xs = {g: torch.from_numpy(rng.standard_normal((b, kk), dtype=np.float32)).cuda()
              for g, kk in (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 14336))}
        outs = {name: torch.empty((b, n), dtype=torch.float32, device="cuda") for name, _, n, _ in shapes}
        # QMatMul's route (QMatMul::max_decode_rows): the decode launcher up to 32 rows for Q4_K and for Q6_K with
        # K <= 8192, up to 16 for the Q6_K down projection (K = 14336); the prefill matmul above
        dec_of = {"attn": b <= 32, "o": b <= 32, "ffn": b <= 32, "down": b <= 16}
        # all seven types here quantize activations to Q8_K, so one buffer per input serves every projection on it
        bufs = {g: (Q.quantize_decode(Q4K, x) if dec_of[g] else Q.quantize_prefill(Q4K, x)) for g, x in xs.items()}
        group = {"q": "attn", "k": "attn", "v": "attn", "o": "o", "gate": "ffn", "up": "ffn", "down": "down"}
        kdim = {name: k for name, _, _, k in shapes}
        tdim = {name: t for name, t, _, _ in shapes}
        ndim = {name: n for name, _, n, _ in shapes}

        one_launch = b <= 2  # q/k/v, o and gate/up quantize their own f32 inputs

        def step(i):
            for layer in range(layers):
                for g, x in xs.items():
                    vy, kp = bufs[g]
                    if one_launch and (g != "down" or b == 1):
                        continue
                    if dec_of[g]:
                        Q.quantize_decode(Q4K, x, kp=kp, out=vy)
                    else:
                        Q.quantize_prefill(Q4K, x, out=vy)
                if one_launch:
                    Q.mmvq_fused_qkv_quantize(Q4K, dev["q"][layer], dev["k"][layer], dev["v"][layer], xs["attn"],
                                              4096, 1024, 1024, outs=(outs["q"], outs["k"], outs["v"]), vtype=Q6K)
                    Q.mmvq_quantize(Q4K, dev["o"][layer], xs["o"], 4096, out=outs["o"])
                    Q.mmvq_fused_glu_quantize(Q4K, dev["gate"][layer], dev["up"][layer], xs["ffn"], 14336,
                                              out=outs["gate"])
                    if b == 1:
                        Q.mmvq_quantize(Q6K, dev["down"][layer], xs["down"], 4096, out=outs["down"])
                    else:
                        vy, kp = bufs["down"]
                        Q.mmvq(Q6K, dev["down"][layer], vy, 14336, 4096, b, kp, out=outs["down"])
                    continue
                for name in ("q", "k", "v", "o", "gate", "down"):
                    vy, kp = bufs[group[name]]
                    t, n, k = tdim[name], ndim[name], kdim[name]
                    decode = dec_of[group[name]]
                    if decode and name == "gate":
                        Q.mmvq_fused_glu(Q4K, dev["gate"][layer], dev["up"][layer], vy, k, n, b, kp,
                                         out=outs["gate"])
                    elif decode:
                        Q.mmvq(t, dev[name][layer], vy, k, n, b, kp, out=outs[name])
                    else:
                        Q.mmq(t, dev[name][layer], vy, k, n, b, out=outs[name])
                        if name == "gate":
                            Q.mmq(Q4K, dev["up"][layer], vy, k, n, b, out=outs["up"])

        st = max(2, steps // 50)
        t = graph_time(torch, step, st, 1)
        per = t / st
        res[f"b{b}"] = {"ms_per_step": per * 1e3, "tokens_per_s": b / per,
                        "gb_s": total_bytes / per / 1e9, "frac_hbm_peak": total_bytes / per / 1e9 / HBM_PEAK_GBS}
    return res


def moe_workload(torch, qmm, steps, warmup, seed, tokens=64, force_grouped=False):
    """8 experts, gate/up Q4_K 14336x4096 and down Q4_K 4096x14336; `tokens` tokens, top-2 from softmax(N(0,1)
    logits) (Mixtral renormalisation): the grouped prefill path of the MoE experts block at 64 tokens, the indexed
    decode path (gate/up GLU matvec, then down with the weighted sum folded in) at 8 or fewer."""
    E, hidden, inter, topk = 8, 4096, 14336, 2
    H = host_lib()
    gate = quantized_weight(Q4K, inter, hidden, seed)
    up = quantized_weight(Q4K, inter, hidden, seed + 1)
    down = quantized_weight(Q4K, hidden, inter, seed + 2)
    handles = []
    for data, rows, cols in ((gate, inter, hidden), (up, inter, hidden), (down, hidden, inter)):
        stack = np.concatenate([data] * E)
        h = ctypes.c_void_p()
        if H.qmm_qtensor_from_data(Q4K, stack.ctypes.data, stack.size, E, rows, cols, 0, ctypes.byref(h)) != 0:
            raise RuntimeError(H.qmm_host_last_error().decode())
        handles.append(h)
    moe = ctypes.c_void_p()
    if H.qmm_moe_new(handles[0], handles[1], handles[2], 0, ctypes.byref(moe)) != 0:
        raise RuntimeError(H.qmm_host_last_error().decode())
    rng = np.random.default_rng(seed + 3)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :topk].astype(np.int32)
    w = np.take_along_axis(p, ids, 1)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((tokens, hidden), dtype=np.float32)).cuda()
    ids_d, w_d = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    out = torch.empty((tokens, hidden), dtype=torch.float32, device="cuda")

    def step(i):
        rc = H.qmm_moe_forward(moe, x.data_ptr(), tokens, ids_d.data_ptr(), w_d.data_ptr(), topk, out.data_ptr(),
                               torch.cuda.current_stream().cuda_stream, 1 if force_grouped else 0)
        if rc != 0:
            raise RuntimeError(H.qmm_host_last_error().decode())

    st = max(20, steps // 10)
    t = graph_time(torch, step, st, 2)
    per = t / st
    # weight bytes the step must read: every expert at 64 tokens; at decode sizes only the experts routed to
    wbytes = 3 * len(np.unique(ids)) * gate.size
    ops = 2.0 * tokens * topk * 3 * inter * hidden
    return {"ms_per_step": per * 1e3, "weight_bytes": wbytes, "gb_s": wbytes / per / 1e9,
            "frac_hbm_peak": wbytes / per / 1e9 / HBM_PEAK_GBS, "tops": ops / per / 1e12}


def read_floor_workload(torch, qmm, steps, warmup, seed):
    """The HBM read floor for the headline: one launch streaming 33,030,144 bytes (the Q4_K 14336x4096 weight) over 16
    rotating copies, as qmm_hbm_read_probe's grid-stride walk (depth x per-CU workgroups swept) and as walks over Q4_K
    rows (the decode units' loads, contiguous chunks, contiguous chunks plus headers; 1 or 2 rows in flight per wave);
    the best grid-stride time is the floor a one-launch decode step can reach."""
    nbytes = 33030144
    copies = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(16)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(16 * cus * 256, dtype=torch.int32, device="cuda")
    res = {"bytes": nbytes, "copies": 16}
    L = qmm.bench_lib()

    def run(pattern, per_cu, depth):
        def fn(i):
            rc = L.qmm_hbm_read_probe(qmm._ptr(copies[i % 16]), nbytes, pattern, per_cu, depth, qmm._ptr(out),
                                      qmm._stream())
            if rc != 0:
                raise RuntimeError(qmm.last_error())
        return graph_time(torch, fn, steps, warmup) / steps

    best = None
    for per_cu in (1, 2, 4, 8):
        for depth in (1, 2, 4, 8):
            t = run(0, per_cu, depth)
            res[f"stride_wg{per_cu}_d{depth}_us"] = t * 1e6
            if best is None or t < best[0]:
                best = (t, f"stride wg{per_cu} d{depth}")
    rows = None
    for pattern, name in ((1, "units"), (2, "contig"), (3, "contig_hdr")):
        for per_cu in (2, 4, 8):
            for depth in (1, 2):
                t = run(pattern, per_cu, depth)
                res[f"rows_{name}_wg{per_cu}_d{depth}_us"] = t * 1e6
                if pattern == 1 and (rows is None or t < rows):
                    rows = t
    res["floor_us"] = best[0] * 1e6
    res["floor_gb_s"] = nbytes / best[0] / 1e9
    res["floor_form"] = best[1]
    res["matvec_rows_gb_s"] = nbytes / rows / 1e9
    return res


def peaks_workload(torch, qmm, steps, warmup, seed):
    """What this box measures against the published peaks (8.0 TB/s HBM, 5.0 POP/s dense int8), with the probes of
    libqmmbench.so:
      copy        one grid-stride 16-byte copy of 1 GB (bytes read + written per second), best of a small sweep of
                  workgroups per CU and loads in flight;
      read_sizes  one launch streaming 33, 66, 132, 264 and 528 MB (the grid-stride read at its best shape), each
                  rotated over copies totalling more than 256 MB (the Infinity Cache); a least-squares line
                  t = t0 + bytes / B gives the fixed cost of a launch (t0) and the asymptotic read rate (B);
      int8_mfma   every wave of 2 workgroups per CU issuing four independent v_mfma_i32_32x32x32_i8 chains."""
    B = qmm.bench_lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(16 * cus * 256, dtype=torch.int32, device="cuda")
    res = {}

    def timed(fn, st, wu):
        return graph_time(torch, fn, st, wu) / st

    # copy: 1 GB, two buffer pairs alternated
    nb = 1 << 30
    bufs = [torch.empty(nb, dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(4)]
    best = None
    for per_cu in (2, 4, 8):
        for depth in (1, 2, 4):
            def fn(i, per_cu=per_cu, depth=depth):
                src, dst = (bufs[0], bufs[1]) if i % 2 == 0 else (bufs[2], bufs[3])
                if B.qmm_bench_copy(qmm._ptr(src), qmm._ptr(dst), nb, per_cu, depth, qmm._stream()) != 0:
                    raise RuntimeError(qmm.last_error())
            t = timed(fn, 20, 4)
            if best is None or t < best[0]:
                best = (t, per_cu, depth)
    res["copy"] = {"bytes_read_plus_written": 2 * nb, "us": best[0] * 1e6, "gb_s": 2 * nb / best[0] / 1e9,
                   "form": f"wg{best[1]} d{best[2]}"}
    del bufs

    # one-launch reads at five sizes (grid-stride read, best of 2 / 4 / 8 workgroups per CU at 4 loads in flight)
    pts = []
    for mb in (33, 66, 132, 264, 528):
        nbytes = mb * 1000 * 1000 // 16 * 16
        ncop = max(2, -(-300 * 1000 * 1000 // nbytes))
        cps = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(ncop)]
        tb = None
        for per_cu in (2, 4, 8):
            def fn(i, per_cu=per_cu):
                if B.qmm_hbm_read_probe(qmm._ptr(cps[i % ncop]), nbytes, 0, per_cu, 4, qmm._ptr(out),
                                        qmm._stream()) != 0:
                    raise RuntimeError(qmm.last_error())
            st = max(8, min(steps // 4, int(2e10 // nbytes)))
            t = timed(fn, st, max(2, st // 10))
            tb = t if tb is None else min(tb, t)
        pts.append((nbytes, tb))
        res[f"read_{mb}mb"] = {"bytes": nbytes, "copies": ncop, "us": tb * 1e6, "gb_s": nbytes / tb / 1e9}
        del cps
    xs = np.array([p[0] for p in pts], dtype=np.float64)
    ts = np.array([p[1] for p in pts], dtype=np.float64)
    slope, t0 = np.polyfit(xs, ts, 1)
    res["read_fit"] = {"launch_us": t0 * 1e6, "asymptotic_gb_s": 1.0 / slope / 1e9,
                       "note": "least-squares t = launch_us + bytes / asymptotic rate over the five one-launch reads"}

    # dense int8 MFMA
    iters = 4096
    ops = [0.0]

    def mf(i):
        ops[0] = B.qmm_bench_mfma_i8(2, iters, qmm._ptr(out), qmm._stream())
        if ops[0] <= 0:
            raise RuntimeError(qmm.last_error())
    t = timed(mf, 10, 2)
    res["int8_mfma"] = {"ops_per_launch": ops[0], "us": t * 1e6, "tops": ops[0] / t / 1e12,
                        "form": "2 workgroups x 4 waves per CU, 4 independent v_mfma_i32_32x32x32_i8 chains per wave"}
    res["summary"] = {"hbm_copy_gb_s": res["copy"]["gb_s"], "hbm_read_asymptotic_gb_s": res["read_fit"]["asymptotic_gb_s"],
                      "read_launch_us": res["read_fit"]["launch_us"], "int8_mfma_tops": res["int8_mfma"]["tops"]}
    return res


# ------------------------------------------------------------------------------------------------ CPU baseline

def _timed(fn, seconds, min_reps):
    fn(0)
    reps, t0 = 0, time.perf_counter()
    while True:
        fn(reps)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= min_reps:
            return el / reps, reps, el


def cpu_baseline(wq, n, k, seconds=10.0):
    """The reference's CPU QMatMul on this box's host, as the reference runs it on x86-64: repacked 16-row tiles
    with vpdpbusd at the level repack_x86::level() picks (AVX-512 VNNI / AVX-VNNI / AVX2), AMX for Q4_K at
    m >= 32 where the CPU has it, threads = physical cores (oracle/x86.c, a C restatement of repack_x86.rs /
    avx.rs).  Headline: Q4_K 14336x4096 at b = 1 over 8 rotating weight copies for about `seconds`.  Also, for
    about a third of that each: config 1 (Q8_0 4096x4096, m = 1, 32 rotating copies), the Q4_K prefill at
    M = 512, and the scalar vec_dot_unopt restatement (oracle/oracle.c) on the headline."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    cores = O.x86_physical_cores()
    rng = np.random.default_rng(SEED + 7)
    x = rng.standard_normal((1, k), dtype=np.float32)
    step_bytes = wq.size + k * 4 + n * 4

    ws = [O.X86Weight(O.Q4K, wq if i == 0 else wq.copy(), n, k) for i in range(8)]
    out = np.zeros((1, n), np.float32)
    paths = set()
    per, reps, el = _timed(lambda i: paths.add(ws[i % 8].matmul(x, cores, out)[1]), seconds, 8)
    head_path = "/".join(sorted(paths))
    del ws

    extra = {}
    # config 1: Q8_0 4096x4096 QMatMul at m = 1 (17.8 MB per weight; 32 copies, 570 MB, beyond any host L3)
    w8 = quantized_weight(Q8_0, 4096, 4096, SEED + 5)
    x8 = rng.standard_normal((1, 4096), dtype=np.float32)
    w8s = [O.X86Weight(O.Q8_0, w8 if i == 0 else w8.copy(), 4096, 4096) for i in range(32)]
    o8 = np.zeros((1, 4096), np.float32)
    p8 = set()
    t8, r8, e8 = _timed(lambda i: p8.add(w8s[i % 32].matmul(x8, cores, o8)[1]), seconds / 3, 32)
    del w8s
    b8 = w8.size + 4096 * 8
    extra["q8_0_4096x4096_m1"] = {"ms_per_step": t8 * 1e3, "gb_s": b8 / t8 / 1e9, "path": "/".join(sorted(p8)),
                                  "sample": f"{r8} calls in {e8:.1f} s, 32 rotating copies"}
    # Q4_K prefill, M = 512 (the weight stays resident: compute-bound on the CPU)
    xp = rng.standard_normal((512, k), dtype=np.float32)
    wp = O.X86Weight(O.Q4K, wq, n, k)
    op = np.zeros((512, n), np.float32)
    pp = set()
    tp, rp, ep = _timed(lambda i: pp.add(wp.matmul(xp, cores, op)[1]), seconds / 3, 2)
    del wp
    extra["q4_k_prefill_m512"] = {"ms_per_step": tp * 1e3, "tops": 2 * 512 * n * k / tp / 1e12,
                                  "path": "/".join(sorted(pp)), "sample": f"{rp} calls in {ep:.1f} s"}
    # the scalar restatement (k_quants.rs vec_dot_unopt + matmul), same headline workload
    copies = [wq] + [wq.copy() for _ in range(7)]
    ts, rs, es = _timed(lambda i: O.matmul(O.Q4K, x, copies[i % 8], n, cores), seconds / 3, 8)
    extra["scalar_vec_dot_unopt_headline"] = {"ms_per_step": ts * 1e3, "gb_s": step_bytes / ts / 1e9,
                                              "sample": f"{rs} calls in {es:.1f} s, 8 rotating copies"}
    return {"value": step_bytes / per / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "variant": f"x86 repacked path ({head_path})",
            "sample": f"{reps} Q4_K 14336x4096 b=1 QMatMul calls (quantize + {head_path}, 8 rotating weight "
                      f"copies) in {el:.1f} s; oracle/x86.c, a restatement of repack_x86.rs at the level "
                      f"repack_x86::level() picks; host CPU: {O.x86_describe()}, {cores} physical cores",
            "ms_per_step": per * 1e3, "extra": extra}


# ------------------------------------------------------------------------------------------------ main

EXTRA_NAMES = {"q4_k_decode_b4", "q4_k_decode_b16", "q8_0_decode_4096", "q4_k_prefill_m512", "q6_k_prefill_m512",
               "llama3_8b_linear_stack", "moe_8x_q4_k_64tok_top2", "q4_0_decode", "q5_0_decode", "q5_k_decode",
               "iq4_xs_decode", "q6_k_decode", "moe_8x_q4_k_4tok_top2", "q4_0_prefill_m512", "q8_0_prefill_m512",
               "q5_0_prefill_m512", "q5_k_prefill_m512", "iq4_xs_prefill_m512", "read_floor", "peaks"}


def decode_summary(r):
    d = {key: r[key] for key in ("ms_per_step", "gb_s", "kernel_us", "kernel_gb_s")}
    if "one_launch" in r:
        d["one_launch"] = r["one_launch"]
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--quick", action="store_true", help="headline only: no extra workloads, no CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="no HIP graphs: one dispatch per launch (for rocprofv3 --pmc)")
    ap.add_argument("--only", choices=sorted(EXTRA_NAMES), default=None, nargs="+",
                    help="run only these extra workloads (no headline, no CPU baseline) and print their JSON")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="only copy MB megabytes device-to-device 20 times (the known-size kernel that scales HBM "
                         "counters), then exit")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Decode and prefill would shard by output rows with no exchange.", file=sys.stderr)
        sys.exit(2)

    import torch
    import qmm
    qmm.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        sys.exit(1)
    if args.calibrate_copy:
        nbytes = args.calibrate_copy * 1000 * 1000
        a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(20):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": nbytes, "copies": 20}))
        return
    log(f"device: {torch.cuda.get_device_name(0)}; library {qmm.build_id()}")

    n, k = 14336, 4096
    extra_runs = {
        "q4_k_decode_b4": lambda: decode_summary(decode_workload(torch, qmm, Q4K, n, k, 4, 16, args.steps // 2,
                                                                 args.warmup // 2, SEED)),
        "q4_k_decode_b16": lambda: decode_summary(decode_workload(torch, qmm, Q4K, n, k, 16, 16, args.steps // 2,
                                                                  args.warmup // 2, SEED)),
        "q8_0_decode_4096": lambda: decode_summary(decode_workload(torch, qmm, Q8_0, 4096, 4096, 1, 32, args.steps,
                                                                   args.warmup, SEED + 5)),
        "q4_k_prefill_m512": lambda: prefill_workload(torch, qmm, Q4K, 14336, 4096, 512, 10,
                                                      max(20, args.steps // 20), 5, SEED + 9),
        "q6_k_prefill_m512": lambda: prefill_workload(torch, qmm, Q6K, 4096, 14336, 512, 8,
                                                      max(20, args.steps // 20), 5, SEED + 11),
        "llama3_8b_linear_stack": lambda: stack_workload(torch, qmm, (1, 8, 32), args.steps, args.warmup, SEED + 20),
        "moe_8x_q4_k_64tok_top2": lambda: moe_workload(torch, qmm, args.steps // 10, 2, SEED + 30),
        "moe_8x_q4_k_4tok_top2": lambda: moe_workload(torch, qmm, args.steps // 10, 2, SEED + 31, tokens=4),
        "q4_0_prefill_m512": lambda: prefill_workload(torch, qmm, Q4_0, 14336, 4096, 512, 10,
                                                      max(20, args.steps // 20), 5, SEED + 45),
        "q8_0_prefill_m512": lambda: prefill_workload(torch, qmm, Q8_0, 14336, 4096, 512, 10,
                                                      max(20, args.steps // 20), 5, SEED + 46),
        "q5_0_prefill_m512": lambda: prefill_workload(torch, qmm, Q5_0, 14336, 4096, 512, 10,
                                                      max(20, args.steps // 20), 5, SEED + 47),
        "q5_k_prefill_m512": lambda: prefill_workload(torch, qmm, Q5K, 14336, 4096, 512, 10,
                                                      max(20, args.steps // 20), 5, SEED + 48),
        "iq4_xs_prefill_m512": lambda: prefill_workload(torch, qmm, IQ4XS, 14336, 4096, 512, 10,
                                                        max(20, args.steps // 20), 5, SEED + 49),
        # the other weight types at the headline shape, b = 1: the two-launch step and the matvec alone
        "q6_k_decode": lambda: decode_summary(decode_workload(torch, qmm, Q6K, n, k, 1, 12, args.steps // 2,
                                                              args.warmup // 2, SEED + 40)),
        "q4_0_decode": lambda: decode_summary(decode_workload(torch, qmm, Q4_0, n, k, 1, 16, args.steps // 2,
                                                              args.warmup // 2, SEED + 41)),
        "q5_0_decode": lambda: decode_summary(decode_workload(torch, qmm, Q5_0, n, k, 1, 16, args.steps // 2,
                                                              args.warmup // 2, SEED + 42)),
        "q5_k_decode": lambda: decode_summary(decode_workload(torch, qmm, Q5K, n, k, 1, 16, args.steps // 2,
                                                              args.warmup // 2, SEED + 43)),
        "iq4_xs_decode": lambda: decode_summary(decode_workload(torch, qmm, IQ4XS, n, k, 1, 16, args.steps // 2,
                                                                args.warmup // 2, SEED + 44)),
        "read_floor": lambda: read_floor_workload(torch, qmm, args.steps // 4, args.warmup // 4, SEED),
        "peaks": lambda: peaks_workload(torch, qmm, args.steps, args.warmup, SEED),
    }
    assert set(extra_runs) == EXTRA_NAMES
    if args.only:
        res = {}
        for name in args.only:
            log(f"only: {name}")
            res[name] = extra_runs[name]()
        print(json.dumps(res), flush=True)
        return

    log("headline: Q4_K 14336x4096 decode b=1")
    head = decode_workload(torch, qmm, Q4K, n, k, 1, 16, args.steps, args.warmup, SEED)
    one = head["one_launch"]
    log(f"  one launch {one['ms_per_step'] * 1e3:.2f} us/step, {one['gb_s']:.0f} GB/s; two launches "
        f"{head['ms_per_step'] * 1e3:.2f} us/step; plain matvec {head['kernel_us']:.2f} us")

    extra = {"q4_k_decode_b1_two_launch": {
        "ms_per_step": head["ms_per_step"], "gb_s": head["gb_s"],
        "step": "launch_mmvq_gguf_quantize_q8_1_f32 + launch_mmvq_gguf_q4_k_f32_plain",
        "matvec": {"kernel": "k_mmvq_p<unit_q4k_s, out_f32, 1, 1, true>", "kernel_us": head["kernel_us"],
                   "gb_s": head["kernel_gb_s"], "algorithmic_bytes": head["kernel_bytes"],
                   "frac_hbm_peak": head["kernel_gb_s"] / HBM_PEAK_GBS}}}
    if not args.quick:
        for name, run in extra_runs.items():
            log(name)
            extra[name] = run()

    base = None
    if not args.quick:
        log("CPU baseline (the reference's x86 route, oracle/x86.c)")
        base = cpu_baseline(head["weights"], n, k, args.cpu_seconds)

    # the step is one launch: its kernel moves the step's bytes (weights, f32 activation, f32 output)
    kb = head["step_bytes"]
    achieved = one["gb_s"]
    traffic = None
    tpath = os.path.join(REPO, "profiles", "traffic_q4_k_decode_14336x4096_b1.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    line = {
        "metric": "Q4_K bs=1 matvec GB/s (% of HBM peak); prefill int8 TOPS at M=512",
        "value": round(one["gb_s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(one["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: weights N(0,0.02) quantized by the library's QTensor quantizer, activations N(0,1), "
                f"seed {SEED}; 16 weight copies rotated (528 MB)",
        "config": {"workload": "q4_k_decode_14336x4096_b1", "weight": "Q4_K 14336x4096", "batch": 1,
                   "activation": "f32 [1,4096] -> Q8_K values (in the reference's Q8_1 scratch layout)",
                   "frac_hbm_peak": round(one["gb_s"] / HBM_PEAK_GBS, 4),
                   "step": "launch_mmvq_gguf_q4_k_f32_quantize_plain (quantize + matvec in one launch, the same "
                           "bits as the reference's two launches), HIP graph of K steps"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k_mmvq_pq<unit_q4k, out_f32, 1, 1, true, 8, 2>", "kernel_us": round(one["kernel_us"], 3),
                     "algorithmic_bytes": kb},
        "cpu_baseline": base,
        "extra": extra,
    }
    if "q4_k_prefill_m512" in extra:
        line["prefill_int8_tops_m512"] = round(extra["q4_k_prefill_m512"]["kernel_tops"], 1)
    if "peaks" in extra:
        pk = extra["peaks"]["summary"]
        line["measured_peaks"] = pk
        line["roofline"]["frac_of_measured_read"] = round(achieved / pk["hbm_read_asymptotic_gb_s"], 4)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
