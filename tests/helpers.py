"""Shared data generators and parity checks for the GPU tests (seeded; the oracle is the checker)."""
import numpy as np

import oracle as O


def weights(rng, n, k, sigma=0.02):
    return (rng.standard_normal((n, k)) * sigma).astype(np.float32)


def acts(rng, m, k):
    return rng.standard_normal((m, k)).astype(np.float32)


def patterned(n, salt=0):
    """The reference's deterministic fixture pattern (fast_mmq.rs:1580-1804): ((i*37 + salt*19) % 211)/105 - 1."""
    i = np.arange(n, dtype=np.int64)
    return (((i * 37 + salt * 19) % 211) / 105.0 - 1.0).astype(np.float32)


def terms(gtype, x, wq, n):
    """Per-output sum of |dequantized activation * dequantized weight| (the scale of the rounding error)."""
    import test_oracle as T
    m, k = x.shape
    a = T.NP_DEQUANT[O.ACT_TYPE[gtype]](O.quantize(O.ACT_TYPE[gtype], x)).reshape(m, k)
    w = T.NP_DEQUANT[gtype](wq).reshape(n, k)
    return np.abs(a) @ np.abs(w).T


def assert_parity(got, want, term=None, rel=1e-3, term_tol=1e-5, what=""):
    """max|got - want| <= rel * max|want| (fp32 accumulation, identical integer dots);
    and, per element, |got - want| <= term_tol * sum|terms| (only the f32 summation order differs)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), what
    err = np.max(np.abs(got - want)) if got.size else 0.0
    scale = max(np.max(np.abs(want)) if want.size else 0.0, 1e-30)
    assert err <= rel * scale, f"{what}: max|d|={err:.3e} max|ref|={scale:.3e} rel={err / scale:.3e}"
    if term is not None:
        bad = np.abs(got - want) > term_tol * term + 1e-30
        assert not bad.any(), f"{what}: {bad.sum()} elements beyond {term_tol} * sum|terms|"
    return err / scale


# ------------------------------------------------------------------------------------------------ activation layouts

# A Q8_1 slot, the super-block activation of the reference-named decode entries: f32 d, int8 qs[256], int16 sums of
# each 32 values, 12 zero bytes (288 bytes per 256 values, the reference's 36 per 32)
SLOT = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("s32", "<i2", 8), ("pad", "u1", 12)])
assert SLOT.itemsize == 288


def _q8k(d, qs):
    """Q8_K blocks (the oracle's BlockQ8K bytes) from d [n] and qs [n, 256]; the per-16 sums follow from qs."""
    out = np.zeros(d.shape, O.BLOCK_DTYPES[O.Q8K])
    out["d"], out["qs"] = d, qs
    out["bsums"] = qs.astype(np.int32).reshape(-1, 16, 16).sum(-1)
    return out


def _check_s32(qs, s32, what):
    want = qs.astype(np.int32).reshape(-1, 8, 32).sum(-1)
    assert np.array_equal(np.asarray(s32, np.int32).reshape(-1, 8), want), f"{what}: per-32 sums"


def slots_to_q8k(buf):
    """Q8_1-slot bytes -> the oracle's Q8_K block bytes, after checking each slot's per-32 sums and zero tail."""
    s = np.ascontiguousarray(buf).reshape(-1).view(SLOT)
    _check_s32(s["qs"], s["s32"], "slot")
    assert not s["pad"].any(), "slot tail not zero"
    return _q8k(s["d"], s["qs"]).view(np.uint8).reshape(-1)


def decode_act_blocks(gtype, buf, m, kp, k=None, q8_1=None):
    """The decode activation bytes a quantizer wrote for wtype `gtype` (m rows of kp values) as the oracle's block
    bytes for the first k values of each row: Q8_K blocks from Q8_1 slots, Q8_0 blocks as they are."""
    import qmm
    k = kp if k is None else k
    raw = np.ascontiguousarray(buf).reshape(-1)
    if qmm._q8_1(gtype, q8_1):
        blk = slots_to_q8k(raw[: m * kp // 256 * 288]).reshape(m, kp // 256, 292)
        return np.ascontiguousarray(blk[:, : -(-k // 256)]).reshape(-1)
    return np.ascontiguousarray(raw[: m * kp // 32 * 34].reshape(m, kp // 32, 34)[:, : -(-k // 32)]).reshape(-1)


def tiles_to_blocks(buf, rows, kp, q8k, s16=False):
    """Prefill tile bytes -> the oracle's block bytes [rows, kp / block]: Q8_K tiles (qs [nsb][rows][256] | f32 d
    [nsb][rows] | int16 per-32 sums [nsb][rows][8], 276 bytes per 256 values; the sums are checked), with s16 the
    `_q8k` tiles (the same qs and d, then f16 per-16 sums [nsb][rows][16], 292 per 256; the sums are checked), or
    Q8_0 tiles (qs | f16 d [nsb][rows][8], 272 per 256)."""
    nsb = kp // 256
    b = np.ascontiguousarray(buf).reshape(-1)[: rows * nsb * (292 if s16 else 276 if q8k else 272)]
    qs = b[: nsb * rows * 256].view(np.int8).reshape(nsb, rows, 256).transpose(1, 0, 2).reshape(-1, 256)
    if q8k or s16:
        d = b[nsb * rows * 256: nsb * rows * 260].view(np.float32).reshape(nsb, rows).T.reshape(-1)
        if s16:
            # sums of 16 int8 lie within +-2048, where f16 holds every integer: they must be exact
            h = b[nsb * rows * 260:].view(np.float16).reshape(nsb, rows, 16).transpose(1, 0, 2).reshape(-1, 16)
            want = qs.reshape(-1, 16, 16).astype(np.int32).sum(axis=2)
            assert np.array_equal(h.astype(np.float32), want.astype(np.float32)), "tile f16 sums of 16"
        else:
            s32 = b[nsb * rows * 260:].view(np.int16).reshape(nsb, rows, 8).transpose(1, 0, 2)
            _check_s32(qs, s32, "tile")
        return _q8k(d, qs).view(np.uint8).reshape(-1)
    d8 = b[nsb * rows * 256:].view(np.uint16).reshape(nsb, rows, 8)
    out = np.zeros((rows, nsb * 8), dtype=O.BLOCK_DTYPES[O.Q8_0])
    out["d"] = d8.transpose(1, 0, 2).reshape(rows, nsb * 8)
    out["qs"] = qs.reshape(rows, nsb * 8, 32)
    return out.view(np.uint8).reshape(-1)
