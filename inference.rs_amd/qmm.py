"""Python front end of libinferencequant.so (the C ABI in include/inferencequant.h).

Device buffers and streams come from PyTorch (ROCm build): tensors' data pointers and
``torch.cuda.current_stream().cuda_stream`` are handed to the C ABI through ctypes.  Every launcher
is asynchronous on that stream.  There is no fallback: if the library is missing this module raises.

The helpers below mirror how inference.rs's Rust host drives the same symbols
(crates/inference-quant/src/gguf/fast_mmvq.rs:477-665 for decode, fast_mmq.rs:604-715 for prefill,
gguf/cuda.rs:259-625 for the MoE paths).
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "lib", "libinferencequant.so")
HOST_LIB_PATH = os.path.join(HERE, "lib", "libinferencequant_host.so")
BENCH_LIB_PATH = os.path.join(HERE, "lib", "libqmmbench.so")
HEADERS = [os.path.join(REPO, "include", "inferencequant.h"), os.path.join(REPO, "include", "qmm_host.h")]

# GGUF type ids (crates/inference-tensor/src/quantized/mod.rs:582-603) and block geometry
F32, F16, Q8_0, Q4K, Q6K, Q8K, BF16 = 0, 1, 8, 12, 14, 15, 30
# the adjacent types served by the decode matvec and the dequantizers (IQ4_XS: inference-quant gguf/kernel.rs:141)
Q4_0, Q5_0, Q5K, IQ4XS = 2, 6, 13, 23
BLOCK_SIZE = {Q8_0: 32, Q4K: 256, Q6K: 256, Q8K: 256, Q4_0: 32, Q5_0: 32, Q5K: 256, IQ4XS: 256}
TYPE_SIZE = {Q8_0: 34, Q4K: 144, Q6K: 210, Q8K: 292, Q4_0: 18, Q5_0: 22, Q5K: 176, IQ4XS: 136}
ACT_TYPE = {Q8_0: Q8_0, Q4K: Q8K, Q6K: Q8K, Q4_0: Q8_0, Q5_0: Q8_0, Q5K: Q8K, IQ4XS: Q8K}
TYPE_NAME = {Q8_0: "q8_0", Q4K: "q4_k", Q6K: "q6_k"}
ADJ_TYPE_NAME = {Q4_0: "q4_0", Q5_0: "q5_0", Q5K: "q5_k", IQ4XS: "iq4_xs"}
# the reference's type names in the indexed / fused MoE symbols (gguf/ffi.rs:60-224, 280-440)
MOE_TYPE = {Q8_0: "q8_0", Q4K: "q4k", Q6K: "q6k", Q4_0: "q4_0", Q5_0: "q5_0", Q5K: "q5k"}
B32 = (Q8_0, Q4_0, Q5_0)  # the 32-value types: their CPU dot products take Q8_0 activation blocks

# Activation layouts (include/inferencequant.h).  q8_1=True: the reference-named quantizers and entries (Q8_K in the
# reference's Q8_1-sized buffers: 36 bytes per 32 values for decode, 276 per 256 for prefill), every weight type.
# q8_1=False: the 32-value types' _q8_0 entries over Q8_0 blocks.  The default (None) is what the C++ host layer uses:
# Q8_1 slots for the super-block types, Q8_0 blocks for the 32-value types -- each the CPU QMatMul's own quantization.


def _q8_1(wtype: int, q8_1) -> bool:
    return (wtype not in B32) if q8_1 is None else bool(q8_1)


def _sfx(wtype: int, q8_1) -> str:
    """Entry-name suffix: the _q8_0 twin for a 32-value type over Q8_0 blocks."""
    return "" if _q8_1(wtype, q8_1) else "_q8_0"


def tname(wtype: int) -> str:
    return TYPE_NAME.get(wtype) or ADJ_TYPE_NAME[wtype]

_lib = None


class QmmError(RuntimeError):
    pass


def build(force: bool = True) -> None:
    """Compile the kernel and host libraries in-tree (hipcc --offload-arch=gfx950)."""
    cmd = ["make", "-s", "-C", HERE, "-j8"]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)


def declared_symbols(header: str | None = None) -> list[str]:
    """Every function and object the C headers declare, after macro expansion (gcc -E)."""
    names: list[str] = []
    for h in ([header] if header else HEADERS):
        if not os.path.exists(h):
            continue
        out = subprocess.run(["gcc", "-E", "-P", "-x", "c", "-I", os.path.join(REPO, "include"), h],
                             check=True, capture_output=True, text=True).stdout
        own = out[out.find("extern") if "extern" in out else 0:]
        for m in re.finditer(r"\b((?:launch|qmm|inference|moe_router)_\w+)\s*(?:\(|\[)", own):
            if m.group(1) not in names:
                names.append(m.group(1))
    return names


def lib() -> ctypes.CDLL:
    """Load libinferencequant.so (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QmmError(f"{LIB_PATH} is missing: run `make -C {HERE}` (or __graft_entry__.build())")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_CTYPE_RET = {"void": None, "int": ctypes.c_int, "double": ctypes.c_double}


def _ctype_of(decl: str):
    """ctypes type of one C parameter declaration (type plus name) of the ABI headers."""
    if "*" in decl:
        return ctypes.c_void_p
    words = decl.replace("const", " ").split()
    base = " ".join(words[:-1]) if len(words) > 1 else words[0]
    return {"int64_t": ctypes.c_int64, "uint32_t": ctypes.c_uint32, "int32_t": ctypes.c_int32, "int": ctypes.c_int,
            "bool": ctypes.c_bool, "_Bool": ctypes.c_bool, "float": ctypes.c_float,
            "double": ctypes.c_double}[base]


def prototypes(header: str | None = None) -> dict:
    """name -> (restype, argtypes) of every function the C header declares (after macro expansion, gcc -E)."""
    h = header or HEADERS[0]
    out = subprocess.run(["gcc", "-E", "-P", "-x", "c", "-I", os.path.join(REPO, "include"), h], check=True,
                         capture_output=True, text=True).stdout
    protos = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b((?:launch|qmm|moe_router)_\w+)\s*\(([^()]*)\)\s*;", out):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        ret_words = ret.replace("const", " ").split()
        if "*" in ret:
            restype = ctypes.c_char_p if "char" in ret_words else ctypes.c_void_p
        else:
            restype = _CTYPE_RET[ret_words[-1]]
        argtypes = [] if args in ("", "void") else [_ctype_of(a) for a in args.split(",")]
        protos[name] = (restype, argtypes)
    return protos


def _declare(L: ctypes.CDLL) -> None:
    for name, (restype, argtypes) in prototypes().items():
        f = getattr(L, name)
        f.restype = restype
        f.argtypes = argtypes


def last_error() -> str:
    return lib().qmm_last_error().decode()


def check() -> None:
    """Raise if the last launcher on this thread recorded an error (then clear it)."""
    msg = last_error()
    if msg:
        lib().qmm_clear_error()
        raise QmmError(msg)


_bench = None


def bench_lib() -> ctypes.CDLL:
    """Load libqmmbench.so, bench.py's measurement probes (HBM read floor, copy rate, int8 MFMA rate)."""
    global _bench
    if _bench is None:
        lib()
        if not os.path.exists(BENCH_LIB_PATH):
            raise QmmError(f"{BENCH_LIB_PATH} is missing: run `make -C {HERE}`")
        B = ctypes.CDLL(BENCH_LIB_PATH)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        B.qmm_hbm_read_probe.argtypes = [vp, i64, i32, i32, i32, vp, vp]
        B.qmm_hbm_read_probe.restype = i32
        B.qmm_bench_copy.argtypes = [vp, vp, i64, i32, i32, vp]
        B.qmm_bench_copy.restype = i32
        B.qmm_bench_mfma_i8.argtypes = [i32, i32, vp, vp]
        B.qmm_bench_mfma_i8.restype = ctypes.c_double
        _bench = B
    return _bench


def build_id() -> str:
    arr = ctypes.c_char.in_dll(lib(), "inference_kernel_build_id")
    return ctypes.cast(ctypes.addressof(arr), ctypes.c_char_p).value.decode()


# ------------------------------------------------------------------------------------------------ torch helpers

def _torch():
    import torch
    return torch


def _stream():
    return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def pad_to(k: int, m: int) -> int:
    return (k + m - 1) // m * m


def act_bytes(wtype: int, rows: int, kp: int, q8_1=None) -> int:
    """Bytes of `rows` decode activation rows of kp values: Q8_1-slot rows (36 per 32 values) or Q8_0 blocks."""
    return rows * kp // 32 * (36 if _q8_1(wtype, q8_1) else 34)


_DT = {}


def _src_name(x) -> str:
    torch = _torch()
    return {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[x.dtype]


def quantize_decode(wtype: int, x, kp: int | None = None, out=None, q8_1=None):
    """Quantize activation rows x [rows, k] (f32/f16/bf16, on the GPU) for wtype's decode entries:
    launch_mmvq_gguf_quantize_q8_1_<src> (Q8_1 slots; kp defaults to pad(k, 512) as the reference's fast_mmvq
    pads) or launch_mmvq_gguf_quantize_q8_0_<src> (Q8_0 blocks, kp = pad(k, 32)).  Returns (uint8 tensor, kp)."""
    torch = _torch()
    rows, k = x.shape
    slots = _q8_1(wtype, q8_1)
    kp = kp or pad_to(k, 512 if slots else 32)
    if out is None:
        out = torch.empty(act_bytes(wtype, rows, kp, q8_1), dtype=torch.uint8, device=x.device)
    blk = "q8_1" if slots else "q8_0"
    getattr(lib(), f"launch_mmvq_gguf_quantize_{blk}_{_src_name(x)}")(_ptr(x), _ptr(out), k, kp, rows, _stream())
    check()
    return out, kp


def _oname(t) -> str:
    torch = _torch()
    return {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[t.dtype]


def mmvq(wtype: int, w, vy, k: int, n: int, b: int, kp: int, out_dtype=None, out=None, stride_col_dst=None,
         q8_1=None):
    """Decode matvec: dst [b, n] = Q(y) . W^T through launch_mmvq_gguf_<t>_<dtype>_plain (or _plain_q8_0);
    stride_col_y = kp / 32 as the reference passes it."""
    torch = _torch()
    out_dtype = out_dtype or torch.float32
    if out is None:
        out = torch.empty((b, stride_col_dst or n), dtype=out_dtype, device=w.device)
    getattr(lib(), f"launch_mmvq_gguf_{tname(wtype)}_{_oname(out)}_plain{_sfx(wtype, q8_1)}")(
        _ptr(w), _ptr(vy), _ptr(out), k, n, kp // 32, stride_col_dst or n, b, _stream())
    check()
    return out


def mmvq_quantize(wtype: int, w, x, n: int, out_dtype=None, out=None):
    """Decode matvec from f32 activations x [b, k] (b <= 2 and k <= 4096, or b = 1 and k <= 16384), quantized
    inside the launch: launch_mmvq_gguf_<t>_<dtype>_quantize_plain."""
    torch = _torch()
    b, k = x.shape
    if out is None:
        out = torch.empty((b, n), dtype=out_dtype or torch.float32, device=w.device)
    oname = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[out.dtype]
    getattr(lib(), f"launch_mmvq_gguf_{TYPE_NAME[wtype]}_{oname}_quantize_plain")(
        _ptr(w), _ptr(x), _ptr(out), k, n, x.stride(0), out.stride(0), b, _stream())
    check()
    return out


def mmvq_fused_glu_quantize(wtype: int, w_gate, w_up, x, n: int, activation: int = 0, out_dtype=None, out=None):
    """act(W_gate . Q(x)) * (W_up . Q(x)) for f32 x [b, k] (b <= 2, k <= 4096), quantized inside the launch:
    launch_mmvq_gguf_<t>_<dtype>_fused_glu_quantize."""
    torch = _torch()
    b, k = x.shape
    if out is None:
        out = torch.empty((b, n), dtype=out_dtype or torch.float32, device=w_gate.device)
    getattr(lib(), f"launch_mmvq_gguf_{TYPE_NAME[wtype]}_{_oname(out)}_fused_glu_quantize")(
        _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(out), k, n, x.stride(0), out.stride(0), b, activation, _stream())
    check()
    return out


def mmvq_fused_qkv_quantize(wtype: int, wq, wk, wv, x, nq: int, nk: int, nv: int, out_dtype=None, outs=None,
                            vtype=None):
    """(q, k, v) = W . Q(x) for f32 x [b, k] (b <= 2, k <= 4096), quantized inside the launch:
    launch_mmvq_gguf_<t>_<dtype>_fused_qkv_quantize, or with vtype = Q6K for Q4_K q / k,
    launch_mmvq_gguf_q4_k_q6_k_f32_fused_qkv_quantize."""
    torch = _torch()
    b, k = x.shape
    if outs is None:
        dt = out_dtype or torch.float32
        outs = tuple(torch.empty((b, n), dtype=dt, device=x.device) for n in (nq, nk, nv))
    if vtype is not None and vtype != wtype:
        name = f"launch_mmvq_gguf_{TYPE_NAME[wtype]}_{TYPE_NAME[vtype]}_{_oname(outs[0])}_fused_qkv_quantize"
    else:
        name = f"launch_mmvq_gguf_{TYPE_NAME[wtype]}_{_oname(outs[0])}_fused_qkv_quantize"
    getattr(lib(), name)(_ptr(wq), _ptr(wk), _ptr(wv), _ptr(x), _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]), k, nq,
                         nk, nv, x.stride(0), b, _stream())
    check()
    return outs


def mmvq_fused_glu(wtype: int, w_gate, w_up, vy, k: int, n: int, b: int, kp: int, activation: int = 0,
                   out_dtype=None, out=None, q8_1=None):
    """dst [b, n] = act(Q(y) . W_gate^T) * (Q(y) . W_up^T) through launch_mmvq_gguf_<t>_<dtype>_fused_glu."""
    torch = _torch()
    if out is None:
        out = torch.empty((b, n), dtype=out_dtype or torch.float32, device=w_gate.device)
    getattr(lib(), f"launch_mmvq_gguf_{tname(wtype)}_{_oname(out)}_fused_glu{_sfx(wtype, q8_1)}")(
        _ptr(w_gate), _ptr(w_up), _ptr(vy), _ptr(out), k, n, kp // 32, out.shape[1], b, activation, _stream())
    check()
    return out


def mmvq_fused_qkv(wtype: int, wq, wk, wv, vy, k: int, nq: int, nk: int, nv: int, b: int, kp: int, out_dtype=None,
                   outs=None, q8_1=None):
    """(q [b, nq], k [b, nk], v [b, nv]) through one launch_mmvq_gguf_<t>_<dtype>_fused_qkv."""
    torch = _torch()
    if outs is None:
        dt = out_dtype or torch.float32
        outs = tuple(torch.empty((b, n), dtype=dt, device=wq.device) for n in (nq, nk, nv))
    getattr(lib(), f"launch_mmvq_gguf_{tname(wtype)}_{_oname(outs[0])}_fused_qkv{_sfx(wtype, q8_1)}")(
        _ptr(wq), _ptr(wk), _ptr(wv), _ptr(vy), _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]), k, nq, nk, nv,
        kp // 32, b, _stream())
    check()
    return outs


def tc_scratch_bytes(k: int, rows: int) -> int:
    """The reference's tensor-core activation scratch: (k / 32) * 288 bytes per 8-row half
    (crates/inference-quant/src/gguf/fast_mmvq.rs:92-93, 1903-1908)."""
    return k // 32 * (32 * 8 + 8 * 2 + 8 * 2) * ((rows + 7) // 8)


def tc_quantize(x, out=None):
    """x [rows, k] (k a multiple of 256) -> the tensor-core entries' layout (rows of k / 256 blocks {f32 d; i8 qs[256]})
    through launch_mmvq_tc_quantize_<src>; out defaults to the reference's scratch size."""
    torch = _torch()
    rows, k = x.shape
    if out is None:
        out = torch.empty(tc_scratch_bytes(k, rows), dtype=torch.uint8, device=x.device)
    getattr(lib(), f"launch_mmvq_tc_quantize_{_src_name(x)}")(_ptr(x), _ptr(out), k, rows, _stream())
    check()
    return out


def mmvq_tc(wtype: int, w, vy, k: int, n: int, b: int, cfg: int = 0, out_dtype=None, out=None):
    """dst [b, n] through launch_mmvq_tc_gguf_<t>_<dtype>_plain over tc_quantize's layout."""
    torch = _torch()
    if out is None:
        out = torch.empty((b, n), dtype=out_dtype or torch.float32, device=w.device)
    oname = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[out.dtype]
    getattr(lib(), f"launch_mmvq_tc_gguf_{TYPE_NAME[wtype]}_{oname}_plain")(
        _ptr(w), _ptr(vy), _ptr(out), k, n, out.stride(0), b, cfg, _stream())
    check()
    return out


def qmatmul_decode(wtype: int, w, x, n: int, out_dtype=None, q8_1=None):
    """x [b, k] -> [b, n]: quantize then matvec (the two launches fast_mmvq::plain makes)."""
    vy, kp = quantize_decode(wtype, x, q8_1=q8_1)
    return mmvq(wtype, w, vy, x.shape[1], n, x.shape[0], kp, out_dtype=out_dtype, q8_1=q8_1)


def mmvq_moe(wtype: int, w_gate, w_up, expert_stride: int, vy, ids, k: int, n: int, kp: int, y_div: int,
             n_pairs: int, activation: int = 0, out=None, q8_1=None):
    torch = _torch()
    if out is None:
        out = torch.empty((n_pairs, n), dtype=torch.float32, device=w_gate.device)
    getattr(lib(), f"launch_mmvq_gguf_{tname(wtype)}_moe{_sfx(wtype, q8_1)}")(
        _ptr(w_gate), _ptr(w_up), expert_stride, _ptr(vy), _ptr(ids), _ptr(out), k, n, kp // 32, y_div, n_pairs,
        activation, 1, _stream())
    check()
    return out


def mmvq_moe_wsum(wtype: int, w, expert_stride: int, vy, ids, weights, k: int, n: int, kp: int, n_tokens: int,
                  topk: int, out=None, q8_1=None):
    """MoE down projection with the weighted sum over each token's routes: launch_mmvq_gguf_<t>_moe_wsum.
    vy: n_tokens * topk activation rows; ids u32 and weights f32 [n_tokens, topk] -> out [n_tokens, n] f32."""
    torch = _torch()
    if out is None:
        out = torch.empty((n_tokens, n), dtype=torch.float32, device=w.device)
    getattr(lib(), f"launch_mmvq_gguf_{tname(wtype)}_moe_wsum{_sfx(wtype, q8_1)}")(
        _ptr(w), expert_stride, _ptr(vy), _ptr(ids), _ptr(weights), _ptr(out), k, n, kp // 32, n_tokens, topk,
        _stream())
    check()
    return out


def indexed_moe(wtype: int, w, x, ids, n: int, out=None, q8_1=None):
    """The op-level gather_forward: x [batch, xdim1, k] f32, ids [batch, topk] u32 -> [batch, topk, n], through
    launch_indexed_moe_forward_<t>_q8_1 (or _q8_0)."""
    torch = _torch()
    batch, xdim1, k = x.shape
    topk = ids.shape[1]
    vy, kp = quantize_decode(wtype, x.reshape(batch * xdim1, k), q8_1=q8_1)
    if out is None:
        out = torch.zeros((batch, topk, n), dtype=torch.float32, device=x.device)
    act = "q8_1" if _q8_1(wtype, q8_1) else "q8_0"
    getattr(lib(), f"launch_indexed_moe_forward_{MOE_TYPE[wtype]}_{act}")(
        _ptr(w), _ptr(vy), _ptr(ids), _ptr(out), n, k, batch, topk, kp, xdim1, _stream())
    check()
    return out


def moe_gemv_gate_up(wtype: int, w_gate, w_up, vy, ids, n: int, k: int, batch: int, topk: int, kp: int,
                     act_type: int = 1, out=None):
    """launch_moe_gemv_fused_gate_up_<t>_q8_1: vy = batch Q8_1-slot rows of kp values; out [batch * topk, n] f32 =
    act(W_gate[e] . x_b) * (W_up[e] . x_b), act_type 0 GELU (tanh), else SiLU."""
    torch = _torch()
    if out is None:
        out = torch.empty((batch * topk, n), dtype=torch.float32, device=w_gate.device)
    getattr(lib(), f"launch_moe_gemv_fused_gate_up_{MOE_TYPE[wtype]}_q8_1")(
        _ptr(w_gate), _ptr(w_up), _ptr(vy), _ptr(ids), _ptr(out), n, k, batch, topk, kp, act_type, _stream())
    check()
    return out


def moe_gemv_down_aggregate(wtype: int, w, vy, ids, weights, n: int, k: int, batch: int, topk: int, kp: int, out):
    """launch_moe_gemv_down_aggregate_<t>_q8_1: vy = batch * topk Q8_1-slot rows of kp values; out [batch, n] f32
    += sum over slots of weights * (W[e] . x_p)."""
    getattr(lib(), f"launch_moe_gemv_down_aggregate_{MOE_TYPE[wtype]}_q8_1")(
        _ptr(w), _ptr(vy), _ptr(ids), _ptr(weights), _ptr(out), n, k, batch, topk, kp, _stream())
    check()
    return out


def gather_rows_u8(src, ids, row_bytes: int, rows: int, out=None):
    """launch_gather_rows_u8: out [len(ids), row_bytes] uint8 = rows ids of src (zeros for an id >= rows)."""
    torch = _torch()
    if out is None:
        out = torch.empty((ids.numel(), row_bytes), dtype=torch.uint8, device=src.device)
    lib().launch_gather_rows_u8(_ptr(src), _ptr(ids), _ptr(out), row_bytes, rows, ids.numel(), _stream())
    check()
    return out


def moe_dispatch(topk_ids, n_experts: int, topk: int):
    torch = _torch()
    total = topk_ids.numel()
    dev = topk_ids.device
    bounds = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    tok = torch.empty(max(total, 1), dtype=torch.int32, device=dev)
    src = torch.empty(max(total, 1), dtype=torch.int32, device=dev)
    counts = torch.empty(n_experts, dtype=torch.int32, device=dev)
    cursors = torch.empty(n_experts, dtype=torch.int32, device=dev)
    lib().launch_moe_dispatch(_ptr(topk_ids), _ptr(bounds), _ptr(tok), _ptr(src), total, n_experts, topk,
                              _ptr(counts), _ptr(cursors), _stream())
    check()
    return bounds, tok[:total], src[:total], counts, cursors


def moe_weighted_reduce(inp, weights, out_dtype=None):
    torch = _torch()
    tokens, topk, hidden = inp.shape
    if inp.dtype == torch.float32:
        suffix = "_bf16" if out_dtype == torch.bfloat16 else ""
        odt = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
    elif inp.dtype == torch.float16:
        suffix, odt = "_f16_input", torch.float16
    else:
        suffix, odt = "_bf16_input", torch.bfloat16
    out = torch.empty((tokens, hidden), dtype=odt, device=inp.device)
    rc = getattr(lib(), f"launch_moe_weighted_reduce_flat{suffix}")(_ptr(inp), _ptr(weights), _ptr(out), tokens,
                                                                    hidden, topk, _stream())
    check()
    if rc != 0:
        raise QmmError(f"moe_weighted_reduce returned {rc}")
    return out


# ------------------------------------------------------------------------------------------------ prefill

def mmq_act_bytes(wtype: int, rows: int, kp: int, q8_1=None, q8k=False) -> int:
    return rows * kp // 256 * (292 if q8k else 276 if _q8_1(wtype, q8_1) else 272)


def quantize_prefill(wtype: int, x, ids=None, rows: int | None = None, out=None, q8_1=None, q8k=False):
    """Quantize x [rows, k] (or the rows ids selects) into wtype's prefill tile layout: launch_mmq_quantize_q8_1_DS4
    (Q8_K tiles), launch_mmq_quantize_q8_0, or with q8k launch_mmq_quantize_q8k (the `_q8k` tiles of the Q4_K / Q5_K
    _q8k entries).  Returns (uint8 tensor, kp)."""
    torch = _torch()
    k = x.shape[-1]
    kp = pad_to(k, 256)
    ne1 = rows if rows is not None else (ids.numel() if ids is not None else x.shape[0])
    if out is None:
        out = torch.empty(max(mmq_act_bytes(wtype, ne1, kp, q8_1, q8k), 1), dtype=torch.uint8, device=x.device)
    type_x = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[x.dtype]
    name = "q8k" if q8k else "q8_1_DS4" if _q8_1(wtype, q8_1) else "q8_0"
    getattr(lib(), f"launch_mmq_quantize_{name}")(_ptr(x), _ptr(ids), _ptr(out), type_x, k, x.stride(0),
                                                  x.stride(0) * x.shape[0], x.stride(0) * x.shape[0], kp, ne1, 1, 1,
                                                  _stream())
    check()
    return out, kp


_fixups = {}


def fixup(device):
    """(buffer, nsm): the split-K fixup workspace the reference hands every MMQ launch (tmp_fixup, sized
    nsm * 128 * 128 f32 in fast_mmq.rs:442-444), one per device, with the device's CU count as nsm."""
    torch = _torch()
    idx = torch.device(device).index or 0
    if idx not in _fixups:
        nsm = torch.cuda.get_device_properties(idx).multi_processor_count
        _fixups[idx] = (torch.empty(nsm * 128 * 128 * 4, dtype=torch.uint8, device=f"cuda:{idx}"), nsm)
    return _fixups[idx]


def quantize_prefill_glu(wtype: int, gate, up, ids=None, activation: int = 0, out=None, q8_1=None, q8k=False):
    """act(gate[r]) * up[r] for r = ids[i] (or i), [rows, k] inputs, quantized into the prefill tile layout through
    launch_mmq_quantize_glu_q8_1_DS4_f32 (f32 inputs) / launch_mmq_quantize_glu_q8_1_DS4 (f16 / bf16 inputs),
    launch_mmq_quantize_glu_q8_0_f32, or with q8k launch_mmq_quantize_glu_q8k_f32.  Returns (uint8 tensor, kp)."""
    torch = _torch()
    k = gate.shape[-1]
    kp = pad_to(k, 256)
    ne1 = ids.numel() if ids is not None else gate.shape[0]
    if out is None:
        out = torch.empty(max(mmq_act_bytes(wtype, ne1, kp, q8_1, q8k), 1), dtype=torch.uint8, device=gate.device)
    if q8k:
        lib().launch_mmq_quantize_glu_q8k_f32(_ptr(gate), _ptr(up), _ptr(ids), _ptr(out), k, gate.stride(0), kp, ne1,
                                              activation, _stream())
    elif not _q8_1(wtype, q8_1):
        lib().launch_mmq_quantize_glu_q8_0_f32(_ptr(gate), _ptr(up), _ptr(ids), _ptr(out), k, gate.stride(0), kp, ne1,
                                               activation, _stream())
    elif gate.dtype == torch.float32:
        lib().launch_mmq_quantize_glu_q8_1_DS4_f32(_ptr(gate), _ptr(up), _ptr(ids), _ptr(out), k, gate.stride(0), kp,
                                                   ne1, activation, _stream())
    else:
        type_x = {torch.float16: F16, torch.bfloat16: BF16}[gate.dtype]
        lib().launch_mmq_quantize_glu_q8_1_DS4(_ptr(gate), _ptr(up), _ptr(ids), _ptr(out), type_x, k, gate.stride(0),
                                               kp, ne1, activation, _stream())
    check()
    return out, kp


def mmq(wtype: int, w, y, k: int, n: int, m: int, out_dtype=None, out=None, tmp_fixup=True, q8_1=None, q8k=False):
    """Prefill matmul: dst [m, n] through launch_mmq_gguf_<t> (or _q8_0, or with q8k the Q4_K / Q5_K _q8k entries over
    `_q8k` tiles).  tmp_fixup=False passes no fixup buffer (no split-K)."""
    torch = _torch()
    out_dtype = out_dtype or torch.float32
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=w.device)
    type_dst = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[out.dtype]
    fx, nsm = fixup(w.device) if tmp_fixup else (None, 256)
    getattr(lib(), f"launch_mmq_gguf_{tname(wtype)}{'_q8k' if q8k else _sfx(wtype, q8_1)}")(
        _ptr(fx), _ptr(w), _ptr(y), _ptr(out), k, n, m, k // BLOCK_SIZE[wtype], n, 0, nsm, 160 * 1024, 64, type_dst,
        _stream())
    check()
    return out


def qmatmul_prefill(wtype: int, w, x, n: int, out_dtype=None, q8_1=None, q8k=False):
    y, _ = quantize_prefill(wtype, x, q8_1=q8_1, q8k=q8k)
    return mmq(wtype, w, y, x.shape[1], n, x.shape[0], out_dtype=out_dtype, q8_1=q8_1, q8k=q8k)


def mmq_moe(wtype: int, w, y, ids_dst, expert_bounds, n_experts: int, k: int, n: int, ncols_dst: int,
            ncols_max: int, out, tmp_fixup=True, q8_1=None, q8k=False):
    """Expert-grouped prefill matmul through launch_mmq_gguf_<t>_moe (or _q8_0, or with q8k the Q4_K / Q5_K
    _moe_q8k entries over `_q8k` tiles)."""
    fx, nsm = fixup(w.device) if tmp_fixup else (None, 256)
    getattr(lib(), f"launch_mmq_gguf_{tname(wtype)}_moe{'_q8k' if q8k else _sfx(wtype, q8_1)}")(
        _ptr(fx), _ptr(w), _ptr(y), _ptr(ids_dst), _ptr(expert_bounds), _ptr(out), k, n, ncols_dst,
        k // BLOCK_SIZE[wtype], n, n_experts, ncols_max, 0, nsm, 160 * 1024, 64, _stream())
    check()
    return out


# ------------------------------------------------------------------------------------------------ dequantization

def dequantize(wtype: int, w, n: int, out_dtype=None, out=None):
    """The n values of the blocks in w (a uint8 tensor) as f32 / f16 / bf16: launch_dequantize_<t>_<dtype>."""
    torch = _torch()
    if out is None:
        out = torch.empty(n, dtype=out_dtype or torch.float32, device=w.device)
    oname = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[out.dtype]
    if wtype == IQ4XS:  # the reference's (nrows, ncols) form
        getattr(lib(), f"launch_dequantize_iq4_xs_{oname}")(_ptr(w), _ptr(out), 1, n, _stream())
    else:
        getattr(lib(), f"launch_dequantize_{TYPE_NAME.get(wtype) or ADJ_TYPE_NAME[wtype]}_{oname}")(
            _ptr(w), _ptr(out), n, _stream())
    check()
    return out


def get_rows(wtype: int, w, ids, ne00: int, nb01: int, out=None):
    """Embedding gather: out [len(ids), ne00] f32 = rows ids of the block matrix w (rows nb01 bytes apart)."""
    torch = _torch()
    if out is None:
        out = torch.empty((ids.numel(), ne00), dtype=torch.float32, device=w.device)
    getattr(lib(), f"launch_get_rows_{TYPE_NAME.get(wtype) or ADJ_TYPE_NAME[wtype]}")(
        _ptr(w), _ptr(ids), _ptr(out), ne00, nb01, ids.numel(), _stream())
    check()
    return out


def router_topk(logits, top_k: int, score_mode: int = 1, weight_mode: int = 0, renormalize: bool = True,
                bias=None, expert_scale=None, clamp=None, norm_min: float = 0.0, output_scale: float = 1.0):
    """moe_router_topk_<dtype>: logits [rows, experts] (f32 / bf16 / f16) -> (weights f32, ids int32) [rows, k]."""
    torch = _torch()
    rows, n = logits.shape
    w = torch.empty((rows, top_k), dtype=torch.float32, device=logits.device)
    ids = torch.empty((rows, top_k), dtype=torch.int32, device=logits.device)
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[logits.dtype]
    f = getattr(lib(), f"moe_router_topk_{name}")
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 5 + [ctypes.c_bool] * 2 + [ctypes.c_float] * 4 + \
        [ctypes.c_int64]
    lo, hi = clamp if clamp is not None else (0.0, 0.0)
    f(_ptr(logits), _ptr(w), _ptr(ids), _ptr(bias), _ptr(expert_scale), rows, n, top_k, score_mode, weight_mode,
      renormalize, clamp is not None, lo, hi, norm_min, output_scale, _torch().cuda.current_stream().cuda_stream)
    check()
    return w, ids


def q8_0_exact(w, x, n: int, out=None):
    """x [b, k] (f32 or bf16, b <= 8) -> [b, n] in x's dtype against a Q8_0 weight, activations unquantized:
    launch_mmvq_gguf_q8_0_<dtype>_exact."""
    torch = _torch()
    b, k = x.shape
    if out is None:
        out = torch.empty((b, n), dtype=x.dtype, device=x.device)
    oname = {torch.float32: "f32", torch.bfloat16: "bf16"}[x.dtype]
    getattr(lib(), f"launch_mmvq_gguf_q8_0_{oname}_exact")(_ptr(w), _ptr(x), _ptr(out), k, n, b, _stream())
    check()
    return out


# ------------------------------------------------------------------------------------------------ GGUF files (host)

_host = None


def host() -> ctypes.CDLL:
    """Load libinferencequant_host.so (the QTensor / QMatMul / GGUF host layer, include/qmm_host.h)."""
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB_PATH):
            raise QmmError(f"{HOST_LIB_PATH} is missing: run `make -C {HERE}`")
        H = ctypes.CDLL(HOST_LIB_PATH)
        vp, i32, i64, u32, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64
        cp = ctypes.c_char_p
        H.qmm_host_last_error.restype = cp
        H.qmm_gguf_open.argtypes = [cp, i32, ctypes.POINTER(vp)]
        H.qmm_gguf_close.argtypes = [vp]
        H.qmm_gguf_version.argtypes = [vp]
        H.qmm_gguf_tensor_data_offset.argtypes = [vp]
        H.qmm_gguf_tensor_data_offset.restype = u64
        H.qmm_gguf_tensor_count.argtypes = [vp]
        H.qmm_gguf_tensor_count.restype = i64
        H.qmm_gguf_tensor_info.argtypes = [vp, i64, cp, i64, ctypes.POINTER(u32), ctypes.POINTER(i64),
                                           ctypes.POINTER(i32), ctypes.POINTER(u64)]
        H.qmm_gguf_metadata_count.argtypes = [vp]
        H.qmm_gguf_metadata_count.restype = i64
        H.qmm_gguf_metadata_key.argtypes = [vp, i64, cp, i64]
        H.qmm_gguf_metadata_type.argtypes = [vp, cp]
        H.qmm_gguf_metadata_u64.argtypes = [vp, cp, ctypes.POINTER(u64)]
        H.qmm_gguf_metadata_i64.argtypes = [vp, cp, ctypes.POINTER(i64)]
        H.qmm_gguf_metadata_f64.argtypes = [vp, cp, ctypes.POINTER(ctypes.c_double)]
        H.qmm_gguf_metadata_string.argtypes = [vp, cp, cp, i64, ctypes.POINTER(i64)]
        H.qmm_gguf_metadata_array.argtypes = [vp, cp, ctypes.POINTER(i64), ctypes.POINTER(i32)]
        H.qmm_gguf_large_array.argtypes = [vp, cp, u64, u64, vp, i64]
        H.qmm_gguf_load_tensor.argtypes = [vp, cp, i32, ctypes.POINTER(vp)]
        H.qmm_gguf_peek_architecture.argtypes = [cp, cp, i64]
        H.qmm_gguf_write.argtypes = [cp, u64, vp, i64, i64, ctypes.POINTER(cp), ctypes.POINTER(vp)]
        H.qmm_qtensor_from_data.argtypes = [u32, vp, i64, i64, i64, i64, i32, ctypes.POINTER(vp)]
        H.qmm_qtensor_free.argtypes = [vp]
        H.qmm_qtensor_device_ptr.argtypes = [vp]
        H.qmm_qtensor_device_ptr.restype = vp
        H.qmm_qtensor_storage_bytes.argtypes = [vp]
        H.qmm_qtensor_storage_bytes.restype = i64
        H.qmm_qmatmul_forward.argtypes = [vp, vp, u32, i64, vp, vp]
        H.qmm_moe_new.argtypes = [vp, vp, vp, i32, ctypes.POINTER(vp)]
        H.qmm_moe_free.argtypes = [vp]
        H.qmm_moe_forward.argtypes = [vp, vp, i64, vp, vp, i64, vp, vp, i32]
        _host = H
    return _host


def _host_check(rc: int) -> None:
    if rc != 0:
        raise QmmError(host().qmm_host_last_error().decode())


class GgufFile:
    """A GGUF file read by the host layer's Content::read (qmm_gguf_open); tensors load into QTensor handles."""

    def __init__(self, path: str, summary: bool = False):
        H = host()
        self._h = ctypes.c_void_p()
        _host_check(H.qmm_gguf_open(path.encode(), int(summary), ctypes.byref(self._h)))

    def close(self) -> None:
        if self._h:
            host().qmm_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        self.close()

    @property
    def version(self) -> int:
        return host().qmm_gguf_version(self._h)

    @property
    def tensor_data_offset(self) -> int:
        return host().qmm_gguf_tensor_data_offset(self._h)

    def tensors(self) -> list:
        """[(name, ggml type id, dims outermost first, offset)] in the file's table order."""
        H = host()
        out = []
        for i in range(H.qmm_gguf_tensor_count(self._h)):
            name = ctypes.create_string_buffer(4096)
            dt, nd, off = ctypes.c_uint32(), ctypes.c_int(), ctypes.c_uint64()
            dims = (ctypes.c_int64 * 8)()
            _host_check(H.qmm_gguf_tensor_info(self._h, i, name, 4096, ctypes.byref(dt), dims, ctypes.byref(nd),
                                               ctypes.byref(off)))
            out.append((name.value.decode(), dt.value, [dims[d] for d in range(nd.value)], off.value))
        return out

    def keys(self) -> list:
        H = host()
        out = []
        for i in range(H.qmm_gguf_metadata_count(self._h)):
            b = ctypes.create_string_buffer(4096)
            _host_check(H.qmm_gguf_metadata_key(self._h, i, b, 4096))
            out.append(b.value.decode())
        return out

    def value_type(self, key: str) -> int:
        return host().qmm_gguf_metadata_type(self._h, key.encode())

    def u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        _host_check(host().qmm_gguf_metadata_u64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def i64(self, key: str) -> int:
        v = ctypes.c_int64()
        _host_check(host().qmm_gguf_metadata_i64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def f64(self, key: str) -> float:
        v = ctypes.c_double()
        _host_check(host().qmm_gguf_metadata_f64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def string(self, key: str) -> str:
        n = ctypes.c_int64()
        _host_check(host().qmm_gguf_metadata_string(self._h, key.encode(), None, 0, ctypes.byref(n)))
        b = ctypes.create_string_buffer(n.value + 1)
        _host_check(host().qmm_gguf_metadata_string(self._h, key.encode(), b, n.value + 1, ctypes.byref(n)))
        return b.raw[:n.value].decode("utf-8", "replace")

    def array(self, key: str):
        n, t = ctypes.c_int64(), ctypes.c_int()
        _host_check(host().qmm_gguf_metadata_array(self._h, key.encode(), ctypes.byref(n), ctypes.byref(t)))
        return n.value, t.value

    def large_array(self, key: str, begin: int, end: int, elem_size: int) -> bytes:
        buf = ctypes.create_string_buffer(max(1, (end - begin) * elem_size))
        _host_check(host().qmm_gguf_large_array(self._h, key.encode(), begin, end, buf, len(buf)))
        return buf.raw[:(end - begin) * elem_size]

    def load_tensor(self, name: str, device_ordinal: int = -1) -> ctypes.c_void_p:
        """A qmm_qtensor handle (free with host().qmm_qtensor_free) on the CPU or HIP device device_ordinal."""
        t = ctypes.c_void_p()
        _host_check(host().qmm_gguf_load_tensor(self._h, name.encode(), device_ordinal, ctypes.byref(t)))
        return t


def gguf_write(path: str, kv_count: int, kv_bytes: bytes, tensors: list) -> None:
    """qmm_gguf_write: tensors = [(name, qmm_qtensor handle)], the metadata already serialized."""
    names = (ctypes.c_char_p * max(1, len(tensors)))(*[n.encode() for n, _ in tensors])
    handles = (ctypes.c_void_p * max(1, len(tensors)))(*[h.value if hasattr(h, "value") else h for _, h in tensors])
    kv = ctypes.create_string_buffer(kv_bytes, max(1, len(kv_bytes)))
    _host_check(host().qmm_gguf_write(path.encode(), kv_count, kv, len(kv_bytes), len(tensors), names, handles))
