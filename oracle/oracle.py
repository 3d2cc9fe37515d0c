"""TEST INFRASTRUCTURE ONLY: ctypes front end of the C oracle (oracle.c).

The checker for the HIP library.  Only tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this module.  It restates
inference.rs's CPU QMatMul (crates/inference-tensor/src/quantized/k_quants.rs);
each C function cites the lines it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

# GGUF type ids (crates/inference-tensor/src/quantized/mod.rs:582-603; IQ4_XS: inference-quant/src/gguf/kernel.rs:141)
Q8_0, Q4K, Q6K, Q8K = 8, 12, 14, 15
Q4_0, Q5_0, Q5K, IQ4XS = 2, 6, 13, 23

# block layouts (k_quants.rs:152-223), as numpy structured dtypes
BLOCK_DTYPES = {
    Q8_0: np.dtype([("d", "<u2"), ("qs", "i1", 32)]),
    Q4K: np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qs", "u1", 128)]),
    Q6K: np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")]),
    Q8K: np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)]),
    Q4_0: np.dtype([("d", "<u2"), ("qs", "u1", 16)]),
    Q5_0: np.dtype([("d", "<u2"), ("qh", "u1", 4), ("qs", "u1", 16)]),
    Q5K: np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qh", "u1", 32), ("qs", "u1", 128)]),
    IQ4XS: np.dtype([("d", "<u2"), ("scales_h", "<u2"), ("scales_l", "u1", 4), ("qs", "u1", 128)]),
}
BLOCK_SIZE = {Q8_0: 32, Q4K: 256, Q6K: 256, Q8K: 256, Q4_0: 32, Q5_0: 32, Q5K: 256, IQ4XS: 256}
TYPE_SIZE = {t: d.itemsize for t, d in BLOCK_DTYPES.items()}
ACT_TYPE = {Q8_0: Q8_0, Q4K: Q8K, Q6K: Q8K, Q4_0: Q8_0, Q5_0: Q8_0, Q5K: Q8K, IQ4XS: Q8K}
# the IQ4_NL value table (crates/inference-quant/src/gguf/raw.rs:13-15)
KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int8)
VEC_DOT = {Q8_0: "oracle_vec_dot_q8_0_q8_0", Q4K: "oracle_vec_dot_q4k_q8k", Q6K: "oracle_vec_dot_q6k_q8k",
           Q4_0: "oracle_vec_dot_q4_0_q8_0", Q5_0: "oracle_vec_dot_q5_0_q8_0", Q5K: "oracle_vec_dot_q5k_q8k",
           IQ4XS: "oracle_vec_dot_iq4xs_q8k"}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_quantize_block32.argtypes = [vp, vp]
        L.oracle_quantize_block32.restype = ctypes.c_float
        L.oracle_quantize.argtypes = [ctypes.c_int, vp, i64, vp]
        L.oracle_dequantize.argtypes = [ctypes.c_int, vp, i64, vp]
        L.oracle_matmul.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, ctypes.c_int]
        L.oracle_matmul_preq.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, ctypes.c_int]
        L.oracle_matmul_q8k_act.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, ctypes.c_int]
        L.oracle_indexed_moe.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, i64, i64, i64, vp, vp, ctypes.c_int]
        L.oracle_moe_dispatch.argtypes = [vp, i32, i32, i32, vp, vp, vp]
        L.oracle_moe_weighted_reduce.argtypes = [vp, vp, vp, i32, i32, i32]
        for name in VEC_DOT.values():
            getattr(L, name).argtypes = [i64, vp, vp]
            getattr(L, name).restype = ctypes.c_float
        L.oracle_x86_select.argtypes = [ctypes.c_int, i64, i64, i64]
        L.oracle_x86_prepare.argtypes = [ctypes.c_int, vp, i64, i64]
        L.oracle_x86_prepare.restype = vp
        L.oracle_x86_release.argtypes = [vp]
        L.oracle_x86_matmul.argtypes = [vp, i64, vp, vp, ctypes.c_int]
        L.oracle_x86_describe.argtypes = [ctypes.c_char_p, ctypes.c_int]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32_to_f16_bits(x: float) -> int:
    return int(lib().oracle_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(int(h)))


def quantize_block32(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape == (32,)
    qs = np.zeros(32, dtype=np.int8)
    d = lib().oracle_quantize_block32(_p(x), _p(qs))
    return np.float32(d), qs


def quantize(gtype: int, x: np.ndarray) -> np.ndarray:
    """Quantize a float32 array (last dim a multiple of the block size) into a uint8 byte array of blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    bs = BLOCK_SIZE[gtype]
    assert x.shape[-1] % bs == 0
    out = np.zeros(n // bs * TYPE_SIZE[gtype], dtype=np.uint8)
    rc = lib().oracle_quantize(gtype, _p(x), n, _p(out))
    assert rc == 0
    return out.reshape(x.shape[:-1] + (x.shape[-1] // bs * TYPE_SIZE[gtype],))


def random_blocks(gtype: int, n_values: int, rng: np.random.Generator, scale: float = 0.01) -> np.ndarray:
    """Random bytes of n_values / block-size blocks of gtype with finite f16 scales near `scale` (every byte pattern of
    the quantized fields is a valid block); for a type without a quantizer (IQ4_XS) and for edge patterns."""
    nb = n_values // BLOCK_SIZE[gtype]
    raw = rng.integers(0, 256, nb * TYPE_SIZE[gtype], dtype=np.uint8)
    b = raw.view(BLOCK_DTYPES[gtype])
    for f in ("d", "dmin"):
        if f in b.dtype.names:
            b[f] = (rng.uniform(0.5, 1.5, nb) * scale * rng.choice([-1, 1], nb)).astype(np.float16).view(np.uint16)
    return raw


def blocks(gtype: int, data: np.ndarray) -> np.ndarray:
    """View quantized bytes as structured blocks."""
    return np.ascontiguousarray(data).reshape(-1).view(BLOCK_DTYPES[gtype])


def dequantize(gtype: int, data: np.ndarray, n: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    y = np.zeros(n, dtype=np.float32)
    lib().oracle_dequantize(gtype, _p(data), n, _p(y))
    return y


def vec_dot(gtype: int, k: int, w_row: np.ndarray, a_row: np.ndarray) -> float:
    name = VEC_DOT[gtype]
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    a_row = np.ascontiguousarray(a_row, dtype=np.uint8)
    return float(getattr(lib(), name)(k, _p(w_row), _p(a_row)))


def matmul(gtype: int, x: np.ndarray, w: np.ndarray, n: int, threads: int = 0) -> np.ndarray:
    """The reference CPU QMatMul: x [m, k] f32 against quantized weight bytes of n rows -> [m, n] f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert w.size == n * k // BLOCK_SIZE[gtype] * TYPE_SIZE[gtype]
    dst = np.zeros((m, n), dtype=np.float32)
    rc = lib().oracle_matmul(gtype, m, k, n, _p(x), _p(w), _p(dst), threads)
    assert rc == 0
    return dst


def matmul_q8k_act(gtype: int, x: np.ndarray, w: np.ndarray, n: int, threads: int = 0) -> np.ndarray:
    """The arithmetic of the library's reference-named entries (oracle.h oracle_matmul_q8k_act): Q8_K activations for
    every weight type; for the super-block types the same as matmul()."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert w.size == n * k // BLOCK_SIZE[gtype] * TYPE_SIZE[gtype]
    dst = np.zeros((m, n), dtype=np.float32)
    rc = lib().oracle_matmul_q8k_act(gtype, m, k, n, _p(x), _p(w), _p(dst), threads)
    assert rc == 0
    return dst


def matmul_preq(gtype: int, a_q: np.ndarray, m: int, k: int, w: np.ndarray, n: int, threads: int = 0) -> np.ndarray:
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    dst = np.zeros((m, n), dtype=np.float32)
    rc = lib().oracle_matmul_preq(gtype, m, k, n, _p(a_q), _p(w), _p(dst), threads)
    assert rc == 0
    return dst


def indexed_moe(gtype: int, w: np.ndarray, n_experts: int, n: int, k: int, x: np.ndarray, ids: np.ndarray,
                threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    batch, xdim1, kk = x.shape
    assert kk == k
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    topk = ids.shape[1]
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.zeros((batch, topk, n), dtype=np.float32)
    rc = lib().oracle_indexed_moe(gtype, n_experts, n, k, _p(w), _p(x), batch, xdim1, topk, _p(ids), _p(y), threads)
    assert rc == 0, "bad expert id or shape"
    return y


def moe_dispatch(topk_ids: np.ndarray, n_experts: int, topk: int):
    ids = np.ascontiguousarray(topk_ids, dtype=np.int32).reshape(-1)
    total = ids.size
    bounds = np.zeros(n_experts + 1, dtype=np.int32)
    tok = np.zeros(total, dtype=np.int32)
    src = np.zeros(total, dtype=np.int32)
    rc = lib().oracle_moe_dispatch(_p(ids), total, n_experts, topk, _p(bounds), _p(tok), _p(src))
    assert rc == 0
    return bounds, tok, src


def moe_weighted_reduce(inp: np.ndarray, weights: np.ndarray) -> np.ndarray:
    inp = np.ascontiguousarray(inp, dtype=np.float32)
    tokens, topk, hidden = inp.shape
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    out = np.zeros((tokens, hidden), dtype=np.float32)
    lib().oracle_moe_weighted_reduce(_p(inp), _p(weights), _p(out), tokens, hidden, topk)
    return out


def router_topk(logits: np.ndarray, top_k: int, score_mode: int, weight_mode: int, renormalize: bool,
                bias: np.ndarray | None = None, expert_scale: np.ndarray | None = None, clamp=None,
                norm_min: float = 0.0, output_scale: float = 1.0):
    """The MoE router (crates/inference-nn/kernels/cuda/sort.cu:1455-1610, the same steps as the op of
    crates/inference-nn/src/ops/moe_router.rs:50-79), per row in float32:
    raw = logit (clamped; NaN -> -inf); score = raw / softmax(raw) / sigmoid(raw) (1490-1494);
    selection = score + bias (NaN -> -inf, 1496-1508); top_k rounds of the largest selection, ties to the lower
    expert (1510-1574); weight = score / raw then a softmax over the picks / sigmoid(raw) (1558-1580);
    renormalize by max(sum, norm_min) (1582-1596); times output_scale * expert_scale[id] (1598-1608).
    Returns (weights [rows, top_k] f32, ids [rows, top_k] u32)."""
    f = np.float32
    lg = np.asarray(logits, dtype=f)
    rows, n = lg.shape
    W = np.zeros((rows, top_k), f)
    I = np.zeros((rows, top_k), np.uint32)
    for r in range(rows):
        raw = lg[r].copy()
        if clamp is not None:
            raw = np.fmin(np.fmax(raw, f(clamp[0])), f(clamp[1]))  # fmaxf / fminf: a NaN yields the bound
        raw[np.isnan(raw)] = -np.inf
        with np.errstate(over="ignore", invalid="ignore"):
            if score_mode == 1:
                e = np.exp(raw - raw.max(), dtype=f)
                score = e * (f(1) / e.sum(dtype=f))
            elif score_mode == 2:
                score = f(1) / (f(1) + np.exp(-raw, dtype=f))
            else:
                score = raw.copy()
        sel = score + bias.astype(f) if bias is not None else score.copy()
        sel[np.isnan(sel)] = -np.inf
        picks = []
        for _ in range(top_k):
            best = max(range(n), key=lambda e: (sel[e], -e))
            picks.append(best)
            sel[best] = -np.inf
        if weight_mode == 1:
            w = np.array([raw[e] for e in picks], f)
            w = np.exp(w - w.max(), dtype=f)
            w = w * (f(1) / w.sum(dtype=f))
        elif weight_mode == 2:
            w = np.array([f(1) / (f(1) + np.exp(-raw[e], dtype=f)) for e in picks], f)
        else:
            w = np.array([score[e] for e in picks], f)
        if renormalize:
            w = w * (f(1) / max(w.sum(dtype=f), f(norm_min)))
        sc = np.full(top_k, f(output_scale), f)
        if expert_scale is not None:
            sc = sc * np.asarray(expert_scale, f)[picks]
        W[r] = w * sc
        I[r] = picks
    return W, I


# ------------------------------------------------------------------ the reference's x86 CPU path (x86.c)

X86_PATHS = {1: "amx", 2: "tiles", 3: "compact_avx2", 4: "scalar"}


def x86_level() -> int:
    """repack_x86::level(): 0 none, 1 AVX2, 2 AVX-VNNI, 3 AVX-512 VNNI (the reference's MISTRALRS_FORCE_AVX2 /
    MISTRALRS_FORCE_AVXVNNI environment switches are read on every call)."""
    return int(lib().oracle_x86_level())


def x86_amx() -> bool:
    return bool(lib().oracle_x86_amx())


def x86_physical_cores() -> int:
    return int(lib().oracle_x86_physical_cores())


def x86_describe() -> str:
    buf = ctypes.create_string_buffer(512)
    lib().oracle_x86_describe(buf, 512)
    return buf.value.decode(errors="replace")


class X86Weight:
    """A quantized weight prepared as the reference's CPU QMatMul caches it on x86 (tiles, AMX tiles)."""

    def __init__(self, gtype: int, w: np.ndarray, n: int, k: int):
        self.w = np.ascontiguousarray(w, dtype=np.uint8)  # the handle points into these bytes
        assert self.w.size == n * k // BLOCK_SIZE[gtype] * TYPE_SIZE[gtype]
        self.gtype, self.n, self.k = gtype, n, k
        self.h = lib().oracle_x86_prepare(gtype, _p(self.w), n, k)
        assert self.h, f"type {gtype} has no x86 path"

    def matmul(self, x: np.ndarray, threads: int = 0, out: np.ndarray | None = None):
        """x [m, k] f32 -> ([m, n] f32, path name)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.shape
        assert k == self.k
        dst = out if out is not None else np.zeros((m, self.n), dtype=np.float32)
        path = lib().oracle_x86_matmul(self.h, m, _p(x), _p(dst), threads)
        assert path > 0
        return dst, X86_PATHS[path]

    def __del__(self):
        if getattr(self, "h", None):
            lib().oracle_x86_release(self.h)
            self.h = None
