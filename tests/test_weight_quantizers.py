"""Pins of the oracle's K-quant weight quantizers: Q4_K, Q5_K and Q6_K blocks from f32 values (oracle/oracle.c,
restating k_quants.rs:1930-2001, 2235-2334, 2577-2646 and the searches of utils.rs:135-361 as Quantizer::LlamaCpp
builds them, every product rounded before it is added).  No reference build, golden vector or importable
implementation of these exists here, so four checks of different kinds hold them:

1. exact grids: values d sc q - dmin m with power-of-two d, dmin and integer sc, m, q (each sub-block reaching both
   ends of its level range) are what the format represents exactly; the quantizer must find that representation: the
   stored d and dmin are the f16 powers of two, the unpacked 6-bit (Q6_K: 8-bit) scales and the levels are the integers
   the values were built from, and dequantization gives the values back bit for bit;
2. the searches re-derived in float64 from what they compute: the affine least-squares fit of make_qkx2_quants over the
   min-max levels and the 21 (Q4_K) / 16 (Q5_K) candidate scales, and the scale of make_qx_quants maximising
   (sum w x l)^2 / sum w l^2 over the plain and 18 nudged scales, each candidate's levels rounded from the scaled
   values; the oracle's levels must be the float64 optimum wherever the optimum wins by a clear margin;
3. a second, separate float32 reading of utils.rs / k_quants.rs in numpy (which never fuses a product into a sum): the
   blocks must be byte-identical -- this catches a slip of transcription or of rounding (a fused multiply-add) in
   either reading, not a misreading they share, which 1 and 2 are for;
4. planted mistakes: the oracle rebuilt with each of eight deliberate mistakes (ORACLE_PLANT, oracle.c) must fail at
   least one of the checks above.
"""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as O

f32 = np.float32
MAGIC = f32(12582912.0)  # 1.5 * 2^23
HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_C = os.path.join(os.path.dirname(HERE), "oracle", "oracle.c")


# ------------------------------------------------------------------------------------------------ library handles

def bind(path):
    L = ctypes.CDLL(path)
    vp = ctypes.c_void_p
    L.oracle_quantize.argtypes = [ctypes.c_int, vp, ctypes.c_int64, vp]
    L.oracle_dequantize.argtypes = [ctypes.c_int, vp, ctypes.c_int64, vp]
    L.oracle_make_qkx2_quants.argtypes = [ctypes.c_int, vp, vp, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                          ctypes.c_int, vp, vp]
    L.oracle_make_qkx2_quants.restype = ctypes.c_float
    L.oracle_make_qx_quants.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, ctypes.c_int]
    L.oracle_make_qx_quants.restype = ctypes.c_float
    return L


def quantize(L, gtype, x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(x.size // 256 * O.TYPE_SIZE[gtype], np.uint8)
    assert L.oracle_quantize(gtype, x.ctypes.data, x.size, out.ctypes.data) == 0
    return out


def dequantize(L, gtype, q, n):
    y = np.zeros(n, np.float32)
    L.oracle_dequantize(gtype, np.ascontiguousarray(q).ctypes.data, n, y.ctypes.data)
    return y


def qkx2(L, nmax, x, w, rmin, rdelta, nstep):
    x, w = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32)
    l = np.zeros(32, np.uint8)
    neg_min = ctypes.c_float()
    s = L.oracle_make_qkx2_quants(nmax, x.ctypes.data, w.ctypes.data, rmin, rdelta, nstep, 0, l.ctypes.data,
                                  ctypes.byref(neg_min))
    return f32(s), f32(neg_min.value), l.astype(np.int64)


def qx(L, x, nmax=32, rmse_type=1):
    x = np.ascontiguousarray(x, np.float32)
    ls = np.zeros(x.size, np.int8)
    s = L.oracle_make_qx_quants(x.size, nmax, x.ctypes.data, ls.ctypes.data, rmse_type)
    return f32(s), ls.astype(np.int64)


@pytest.fixture(scope="module")
def lib():
    return bind(O.LIB_PATH)


# ------------------------------------------------------------------------------------------------ field decoders

def f16_bits(v):
    return int(np.float16(v).view(np.uint16))


def k4_scales(scales):
    """the 6-bit (scale, min) pairs of the 12 packed bytes: the GGUF K-quant header layout (get_scale_min_k4)"""
    q = [int(b) for b in scales]
    sc, mn = [], []
    for j in range(8):
        if j < 4:
            sc.append(q[j] & 63)
            mn.append(q[j + 4] & 63)
        else:
            sc.append((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4))
            mn.append((q[j + 4] >> 4) | ((q[j] >> 6) << 4))
    return np.array(sc), np.array(mn)


def q4k_levels(blk):
    """levels 0..15 of the 256 values: qs[32 c + l] holds value 64 c + l (low nibble) and 64 c + 32 + l (high)"""
    qs = blk["qs"].astype(np.int64).reshape(4, 32)
    return np.stack([qs & 15, qs >> 4], 1).reshape(256)


def q5k_levels(blk):
    lo = q4k_levels(blk)
    qh = blk["qh"].astype(np.int64)
    hi = np.stack([(qh >> (2 * c)) & 1 for c in range(4)] + [(qh >> (2 * c + 1)) & 1 for c in range(4)], 0)
    # sub-block 2c takes bit 2c, sub-block 2c + 1 bit 2c + 1
    order = [0, 4, 1, 5, 2, 6, 3, 7]
    return lo + 16 * np.concatenate([hi[order[j]] for j in range(8)])


def q6k_levels(blk):
    """levels 0..63: for half h, ql[64 h + l] / ql[64 h + 32 + l] low / high nibbles, qh[32 h + l] 2-bit fields"""
    ql = blk["ql"].astype(np.int64)
    qh = blk["qh"].astype(np.int64)
    out = np.zeros(256, np.int64)
    for h in range(2):
        for l in range(32):
            a, b, c = ql[64 * h + l], ql[64 * h + 32 + l], qh[32 * h + l]
            out[128 * h + l] = (a & 15) | ((c & 3) << 4)
            out[128 * h + 32 + l] = (b & 15) | (((c >> 2) & 3) << 4)
            out[128 * h + 64 + l] = (a >> 4) | (((c >> 4) & 3) << 4)
            out[128 * h + 96 + l] = (b >> 4) | (((c >> 6) & 3) << 4)
    return out


# ------------------------------------------------------------------------------------------------ 1. exact grids

def grid_blocks_affine(rng, nb, nmax):
    """Q4_K / Q5_K blocks on their exact grid: value = sc_j q D - m_j Dmin, D and Dmin powers of two, one sub-block at
    each of sc = 63 and m = 63 (so the block's d and dmin come out as D and Dmin), every sub-block holding levels 0 and
    nmax and at least six distinct levels."""
    xs, want = [], []
    for _ in range(nb):
        D, Dm = 2.0 ** -int(rng.integers(6, 15)), 2.0 ** -int(rng.integers(6, 15))
        sc = rng.integers(1, 64, 8)
        m = rng.integers(0, 64, 8)
        sc[rng.integers(8)] = 63
        m[rng.integers(8)] = 63
        q = rng.integers(0, nmax + 1, (8, 32))
        for j in range(8):
            p = rng.permutation(32)
            q[j, p[0]], q[j, p[1]] = 0, nmax
            q[j, p[2:6]] = rng.choice(np.arange(1, nmax), 4, replace=False)
        x = (sc[:, None] * q * D - m[:, None] * Dm).astype(np.float64)
        assert np.array_equal(x.astype(np.float32).astype(np.float64), x)  # exact in f32
        xs.append(x.reshape(256))
        want.append((D, Dm, sc, m, q.reshape(256)))
    return np.array(xs, np.float32), want


def check_exact_grid_affine(L, gtype, seed=1):
    nmax = 15 if gtype == O.Q4K else 31
    rng = np.random.default_rng(seed)
    x, want = grid_blocks_affine(rng, 150, nmax)
    q = quantize(L, gtype, x)
    blocks = q.view(O.BLOCK_DTYPES[gtype])
    for b, (D, Dm, sc, m, lv) in zip(blocks, want):
        assert int(b["d"]) == f16_bits(D) and int(b["dmin"]) == f16_bits(Dm)
        s, mm = k4_scales(b["scales"])
        assert np.array_equal(s, sc) and np.array_equal(mm, m)
        assert np.array_equal(q4k_levels(b) if gtype == O.Q4K else q5k_levels(b), lv)
    y = dequantize(L, gtype, q, x.size)
    assert np.array_equal(y, x.reshape(-1))


def grid_blocks_q6k(rng, nb):
    """Q6_K blocks on their exact grid: value = sc_j (q - 32) D over 16-value groups, D a power of two, one group at
    sc = -128 (whose scale is then the block's largest, setting d = D), the others at nonzero |sc| <= 127; every
    group holds level 0 (its one value of largest magnitude) and several odd levels."""
    xs, want = [], []
    for _ in range(nb):
        D = 2.0 ** -int(rng.integers(8, 20))
        sc = rng.integers(1, 128, 16) * rng.choice([-1, 1], 16)
        sc[rng.integers(16)] = -128
        q = rng.integers(1, 64, (16, 16))
        for j in range(16):
            p = rng.permutation(16)
            q[j, p[0]] = 0
            q[j, p[1:4]] = 2 * rng.integers(0, 32, 3) + 1
        x = (sc[:, None] * (q - 32) * D).astype(np.float64)
        assert np.array_equal(x.astype(np.float32).astype(np.float64), x)
        xs.append(x.reshape(256))
        want.append((D, sc, q.reshape(256)))
    return np.array(xs, np.float32), want


def check_exact_grid_q6k(L, seed=2):
    rng = np.random.default_rng(seed)
    x, want = grid_blocks_q6k(rng, 150)
    q = quantize(L, O.Q6K, x)
    for b, (D, sc, lv) in zip(q.view(O.BLOCK_DTYPES[O.Q6K]), want):
        assert int(b["d"]) == f16_bits(D)
        assert np.array_equal(b["scales"].astype(np.int64), sc)
        assert np.array_equal(q6k_levels(b), lv)
    assert np.array_equal(dequantize(L, O.Q6K, q, x.size), x.reshape(-1))


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q5K])
def test_affine_k_quants_find_exact_grids(lib, gtype):
    check_exact_grid_affine(lib, gtype)


def test_q6k_finds_exact_grids(lib):
    check_exact_grid_q6k(lib)


# ------------------------------------------------------------------------------------------------ 2. float64 searches

def levels(v64, x32, iscale32, near):
    """rint of the float64 scaled values v64; a value exactly at a half-integer -- where the search's own scale puts
    an extreme value, e.g. 14.5 (max - min) / (max - min) -- is a tie that the algorithm settles by how its f32
    product rounds, so there the f32 product iscale32 * x32 is rounded as the reference rounds it (ties to even).
    A value within 1e-4 of a half-integer but not on it is one that f32 and float64 may round apart: near[0] counts
    them."""
    L = np.rint(v64)
    dist = np.abs(v64 - np.floor(v64) - 0.5)
    tie = dist < 1e-6
    near[0] += int(np.count_nonzero((dist >= 1e-6) & (dist < 1e-4)))
    if tie.any():
        L[tie] = nearest_int(f32(iscale32) * np.asarray(x32, np.float32))[tie]
    return L


def qkx2_f64(x, w, nmax, rmin, rdelta, nstep):
    """make_qkx2_quants from what it computes, in float64: levels of the min-max fit, then of each scale
    (rmin + rdelta is + nmax) / (max - min) applied to x - min; each candidate after the first refit by weighted
    least squares (scale, min) with the min held at or below 0; a candidate whose weighted squared error beats the
    best so far becomes the best, and its refit min is the `min` the later candidates scale from (as the reference's
    loop updates it).  Returns (levels, scale, min, margin, near): margin = the relative gap between the winner's error
    and the closest other candidate's, near = the scaled values that f32 and float64 may round apart."""
    x32 = np.asarray(x, np.float32)
    x, w = x.astype(np.float64), w.astype(np.float64)
    lo, hi = min(x.min(), 0.0), x.max()
    r32 = f32(f32(hi) - f32(lo))
    iscale = nmax / (hi - lo)
    near = [0]
    L0 = np.clip(levels(iscale * (x - lo), x32 - f32(lo), f32(nmax) / r32, near), 0, nmax)
    cands = [(np.sum(w * ((hi - lo) / nmax * L0 + lo - x) ** 2), L0, (hi - lo) / nmax, lo)]
    best = 0
    mn_cur, mn_cur32 = lo, f32(lo)
    for i in range(nstep + 1):
        iscale = (rmin + rdelta * i + nmax) / (hi - mn_cur)
        isc32 = f32(f32(f32(f32(rdelta) * f32(i)) + f32(rmin)) + f32(nmax)) / f32(f32(hi) - mn_cur32)
        Lc = np.clip(levels(iscale * (x - mn_cur), x32 - mn_cur32, isc32, near), 0, nmax)
        sw, sl, sl2, sx, sxl = w.sum(), (w * Lc).sum(), (w * Lc * Lc).sum(), (w * x).sum(), (w * Lc * x).sum()
        det = sw * sl2 - sl * sl
        if det <= 0:
            continue
        s = (sw * sxl - sx * sl) / det
        mn = (sl2 * sx - sl * sxl) / det
        if mn > 0:
            mn, s = 0.0, sxl / sl2
        cands.append((np.sum(w * (s * Lc + mn - x) ** 2), Lc, s, mn))
        if cands[-1][0] < cands[best][0]:
            best = len(cands) - 1
            # the reference carries the f32 refit min on; its float64 value is the one computed here, to f32
            mn_cur, mn_cur32 = mn, f32(mn)
    e = cands[best][0]
    others = [c[0] for i, c in enumerate(cands) if i != best and not np.array_equal(c[1], cands[best][1])]
    margin = (min(others) - e) / max(e, 1e-300) if others else np.inf
    return cands[best][1].astype(np.int64), cands[best][2], cands[best][3], margin, near[0]


def qx_f64(x, nmax):
    """make_qx_quants (rmse_type 1: weights x^2) from what it computes, in float64: for the plain scale -nmax / max
    and the 18 nudges -(nmax + 0.1 is) / max, is = +-1..9, levels l = clamp(rint(iscale x), -nmax, nmax - 1); the
    first candidate with the largest (sum w x l)^2 / sum w l^2 wins and the scale is sum w x l / sum w l^2.
    Returns (levels, scale, margin)."""
    x32 = np.asarray(x, np.float32)
    x = x.astype(np.float64)
    w = x * x
    mx = x[np.argmax(np.abs(x))]
    cands = []
    near = [0]
    for i in [0] + [i for i in range(-9, 10) if i != 0]:
        isc32 = f32(f32(-nmax) / f32(mx)) if i == 0 else f32(-f32(f32(f32(0.1) * f32(i)) + f32(nmax)) / f32(mx))
        Lc = np.clip(levels(-(nmax + 0.1 * i) / mx * x, x32, isc32, near), -nmax, nmax - 1)
        sl2 = (w * Lc * Lc).sum()
        if sl2 <= 0:
            continue
        slx = (w * x * Lc).sum()
        cands.append((slx * slx / sl2, Lc, slx / sl2))
    best = 0
    for c in range(1, len(cands)):
        if cands[c][0] > cands[best][0]:
            best = c
    # the residual error of a candidate is sum w x^2 minus its score: the margin compares residuals
    total = np.sum(w * x * x)
    e = total - cands[best][0]
    others = [total - c[0] for c in cands if not np.array_equal(c[1], cands[best][1])]
    margin = (min(others) - e) / max(e, 1e-300) if others else np.inf
    return cands[best][1].astype(np.int64), cands[best][2], margin, near[0]


def check_qkx2_f64(L, nmax, rmin, rdelta, nstep, seed=3, n=400):
    """The reference computes its least-squares refits in f32, where sum_l2 sum_x - sum_l sum_xl cancels, so its
    comparison of two candidates whose errors are within a fraction of a percent can go either way.  Hence: the
    oracle's fit (levels, scale, min) is never more than 2% worse in float64 error than the float64 optimum, and where
    the optimum wins by more than 0.1%, the oracle's levels are the optimum's in at least 95% of the cases."""
    rng = np.random.default_rng(seed)
    compared = agree = 0
    for t in range(n):
        x = (rng.standard_normal(32) * 0.02 + (0.01 if t % 3 == 0 else 0.0)).astype(np.float32)
        w = (np.sqrt(np.mean(x.astype(np.float64) ** 2)) + np.abs(x)).astype(np.float32)
        Lw, sw, mw, margin, near = qkx2_f64(x, w, nmax, rmin, rdelta, nstep)
        if near:
            continue
        s, neg_min, l = qkx2(L, nmax, x, w, rmin, rdelta, nstep)
        x64, w64 = x.astype(np.float64), w.astype(np.float64)
        e_best = np.sum(w64 * (sw * Lw + mw - x64) ** 2)
        e_got = np.sum(w64 * (float(s) * l - float(neg_min) - x64) ** 2)
        assert e_got <= e_best * 1.02 + 1e-18, f"case {t}: error {e_got:.4e} against the optimum's {e_best:.4e}"
        if margin > 1e-3:
            compared += 1
            agree += bool(np.array_equal(l, Lw))
    assert compared > n // 3 and agree >= 0.95 * compared, (compared, agree)


def check_qx_f64(L, seed=4, n=400):
    """make_qx_quants compares (sum w x l)^2 / sum w l^2 between candidates in f32; the scores of candidates whose
    residuals differ by a fraction of a percent differ by about 1e-6 relative, near f32's resolution, so that choice
    can go either way.  Hence: the oracle's fit is never more than 2% worse in float64 residual than the float64
    optimum, and where the optimum's residual wins by more than 0.1%, its levels are the optimum's in at least 95% of
    the cases, with the scale within 1e-4 there."""
    rng = np.random.default_rng(seed)
    compared = agree = 0
    for t in range(n):
        x = (rng.standard_normal(16) * 0.02).astype(np.float32)
        if t % 4 == 0:
            x[rng.integers(16)] *= 6.0  # an outlier sets the max
        Lw, sw, margin, near = qx_f64(x, 32)
        if near:
            continue
        s, ls = qx(L, x)
        x64 = x.astype(np.float64)
        w = x64 * x64
        e_best = np.sum(w * (sw * Lw - x64) ** 2)
        e_got = np.sum(w * (float(s) * (ls - 32) - x64) ** 2)
        assert e_got <= e_best * 1.02 + 1e-30, f"case {t}: residual {e_got:.4e} against the optimum's {e_best:.4e}"
        if margin > 1e-3:
            compared += 1
            if np.array_equal(ls - 32, Lw):
                agree += 1
                assert abs(float(s) - sw) <= 1e-4 * abs(sw)
    assert compared > n // 3 and agree >= 0.95 * compared, (compared, agree)


@pytest.mark.parametrize("nmax,rmin,nstep", [(15, -1.0, 20), (31, -0.5, 15)])
def test_qkx2_search_is_its_float64_optimum(lib, nmax, rmin, nstep):
    check_qkx2_f64(lib, nmax, rmin, 0.1, nstep)


def test_qx_search_is_its_float64_optimum(lib):
    check_qx_f64(lib)


# ------------------------------------------------------------------------------------------------ 3. float32 reading

def nearest_int(v):
    """utils.rs:32-35: add 1.5 * 2^23 in f32 and read the low mantissa bits (ties to even)"""
    t = (np.asarray(v, np.float32) + MAGIC).astype(np.float32)
    return (t.view(np.uint32) & np.uint32(0x007FFFFF)).astype(np.int64) - 0x00400000


def fold(terms):
    """0 + t0 + t1 + ... in f32, in order along the last axis (add.accumulate is sequential), for every row at once"""
    return np.add.accumulate(np.asarray(terms, np.float32), axis=-1, dtype=np.float32)[..., -1]


def col(v):
    return np.asarray(v, np.float32)[:, None]


def np_qkx2(nmax, X, W, rmin, rdelta, nstep):
    """make_qkx2_quants (utils.rs:268-361), Quantizer::LlamaCpp (every a * b + c rounds the product first), for the
    rows of X [B, 32] with weights W at once: returns scale [B], -min [B], levels [B, 32]"""
    X, W = np.asarray(X, np.float32), np.asarray(W, np.float32)
    mn, mx = X.min(1), X.max(1)
    sum_w, sum_x = fold(W), fold(W * X)
    mn = np.where(mn > 0, f32(0), mn).astype(np.float32)
    flat = mx == mn
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        iscale = (f32(nmax) / (mx - mn)).astype(np.float32)
        scale = (f32(1) / iscale).astype(np.float32)
        l = np.clip(nearest_int(col(iscale) * (X - col(mn))), 0, nmax)
        diff = (col(scale) * l.astype(np.float32) + col(mn)) - X
        best = fold(W * (diff * diff))
        for i in range(nstep + 1):
            c = f32(f32(f32(f32(rdelta) * f32(i)) + f32(rmin)) + f32(nmax))
            isc = (c / (mx - mn)).astype(np.float32)
            la = np.clip(nearest_int(col(isc) * (X - col(mn))), 0, nmax)
            lf = la.astype(np.float32)
            wl = W * lf
            sum_l, sum_l2, sum_xl = fold(wl), fold(wl * lf), fold(wl * X)
            d = (sum_w * sum_l2 - sum_l * sum_l).astype(np.float32)
            this_scale = (-(sum_x * sum_l - sum_w * sum_xl) / d).astype(np.float32)
            this_min = ((sum_l2 * sum_x - sum_l * sum_xl) / d).astype(np.float32)
            pos = this_min > 0
            this_scale = np.where(pos, sum_xl / sum_l2, this_scale).astype(np.float32)
            this_min = np.where(pos, f32(0), this_min).astype(np.float32)
            diff = (col(this_scale) * lf + col(this_min)) - X
            cur = fold(W * (diff * diff))
            upd = (d > 0) & (cur < best) & ~flat
            l = np.where(upd[:, None], la, l)
            best, scale, mn = np.where(upd, cur, best), np.where(upd, this_scale, scale), np.where(upd, this_min, mn)
    l = np.where(flat[:, None], 0, l)
    scale = np.where(flat, f32(0), scale).astype(np.float32)
    return scale, (-mn).astype(np.float32), l


def np_qx(X, nmax=32):
    """make_qx_quants (utils.rs:135-264) with rmse_type 1, no importance weights, Quantizer::LlamaCpp, for the rows
    of X [B, n] at once: returns scale [B], levels [B, n] (offset by nmax)"""
    X = np.asarray(X, np.float32)
    ax = np.abs(X)
    zero = ax.max(1) < f32(1e-15)
    mx = X[np.arange(len(X)), np.argmax(ax, 1)]  # the first value of largest magnitude
    W = X * X
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        quant = lambda isc: np.clip(nearest_int(col(isc) * X), -nmax, nmax - 1)

        def sums(isc):
            lf = quant(isc).astype(np.float32)
            return fold((W * X) * lf), fold((W * lf) * lf)

        iscale = (f32(-nmax) / mx).astype(np.float32)
        sumlx, suml2 = sums(iscale)
        ls = nmax + quant(iscale)
        scale = np.where(suml2 != 0, sumlx / suml2, f32(0)).astype(np.float32)
        best = (scale * sumlx).astype(np.float32)
        for i in range(-9, 10):
            if i == 0:
                continue
            isc = (-(f32(f32(0.1) * f32(i)) + f32(nmax)) / mx).astype(np.float32)
            sumlx, suml2 = sums(isc)
            upd = (suml2 > 0) & ((sumlx * sumlx) > (best * suml2))
            ls = np.where(upd[:, None], nmax + quant(isc), ls)
            scale = np.where(upd, sumlx / suml2, scale).astype(np.float32)
            best = np.where(upd, scale * sumlx, best).astype(np.float32)
    return np.where(zero, f32(0), scale), np.where(zero[:, None], 0, ls)


def qkx2_weights(X):
    """k_quants.rs:302-305: each 32-value row's RMS plus each |x|"""
    av = np.sqrt((fold(X * X) / f32(32)).astype(np.float32)).astype(np.float32)
    return (col(av) + np.abs(X)).astype(np.float32)


def running_max(v):
    """fold(0.0, |max, v| v.max(max)) over the columns; a zero sub-block's min is -0.0, and on a +-0 tie the
    accumulator (+0.0) stays, as ggml's `if (v > max) max = v` keeps it: an all-zero block stores dmin = +0 (no value
    depends on that sign)"""
    acc = np.zeros(len(v), np.float32)
    for j in range(v.shape[1]):
        acc = np.where(v[:, j] > acc, v[:, j], acc)
    return acc


def np_affine_blocks(x, nmax, rmin, nstep):
    """Q4_K (nmax 15, k_quants.rs:1950-2013) / Q5_K (nmax 31, k_quants.rs:2255-2334) blocks of x [B, 256], plain path:
    returns d, dmin (f16), the 6-bit scales and mins [B, 8], the levels [B, 256]"""
    x = np.asarray(x, np.float32)
    B = len(x)
    sub = x.reshape(B * 8, 32)
    scales, mins, l = np_qkx2(nmax, sub, qkx2_weights(sub), rmin, 0.1, nstep)
    scales, mins, l = scales.reshape(B, 8), mins.reshape(B, 8), l.reshape(B, 256)
    max_scale, max_min = running_max(scales), running_max(mins)
    with np.errstate(divide="ignore"):
        inv_scale = np.where(max_scale > 0, f32(63) / max_scale, f32(0)).astype(np.float32)
        inv_min = np.where(max_min > 0, f32(63) / max_min, f32(0)).astype(np.float32)
    ls = np.minimum(nearest_int(col(inv_scale) * scales), 63) & 0xFF
    lm = np.minimum(nearest_int(col(inv_min) * mins), 63) & 0xFF
    d = (max_scale / f32(63)).astype(np.float16)
    dmin = (max_min / f32(63)).astype(np.float16)
    sd = (col(d.astype(np.float32)) * (ls & 63).astype(np.float32)).astype(np.float32)
    dm = (col(dmin.astype(np.float32)) * (lm & 63).astype(np.float32)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = ((x.reshape(B, 8, 32) + dm[:, :, None]) / sd[:, :, None]).astype(np.float32)
        req = np.clip(nearest_int(v), 0, nmax).reshape(B, 256)
    keep = np.repeat(sd == 0, 32, axis=1)
    return d, dmin, ls & 63, lm & 63, np.where(keep, l, req)


def np_q6k_blocks(x):
    """Q6_K blocks of x [B, 256] (k_quants.rs:2590-2646, no imatrix): returns d (f16), scales [B, 16] (i8), levels"""
    x = np.asarray(x, np.float32)
    B = len(x)
    scales, l = np_qx(x.reshape(B * 16, 16))
    scales, l = scales.reshape(B, 16), l.reshape(B, 256)
    max_scale, max_abs = np.zeros(B, np.float32), np.zeros(B, np.float32)
    for j in range(16):  # the first scale of largest magnitude
        up = np.abs(scales[:, j]) > max_abs
        max_abs, max_scale = np.where(up, np.abs(scales[:, j]), max_abs), np.where(up, scales[:, j], max_scale)
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = (f32(-128) / max_scale).astype(np.float32)
        d = (f32(1) / iscale).astype(np.float32).astype(np.float16)
        sc = np.minimum(nearest_int(col(iscale) * scales), 127).astype(np.int8)
        dd = (col(d.astype(np.float32)) * sc.astype(np.float32)).astype(np.float32)
        v = (x.reshape(B, 16, 16) / dd[:, :, None]).astype(np.float32)
        req = (np.clip(nearest_int(v), -32, 31) + 32).reshape(B, 256)
    keep = np.repeat(dd == 0, 16, axis=1)
    return d, sc, np.where(keep, l, req)


def bit_level_inputs(seed, nb):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((nb, 256)) * 0.02).astype(np.float32)
    x[1] = 0.0                                  # a zero block
    x[2, :32] = 0.0125                          # a flat positive sub-block (min clamped to 0)
    x[3, 32:64] = -0.0125                       # a flat negative sub-block
    x[4] *= 1e-4                                # tiny values
    x[5, 7] = 0.4                               # an outlier
    x[6] = np.abs(x[6])                         # positive values only
    x[7::11] += 0.01                            # rows with a positive offset (the refit min often clamps to 0)
    return x


def check_bit_level(L, gtype, seed=5, nb=8000):
    """every block byte-identical to the numpy reading: d, dmin, the unpacked scales and mins, the levels"""
    x = bit_level_inputs(seed, nb)
    got = quantize(L, gtype, x).view(O.BLOCK_DTYPES[gtype])
    if gtype == O.Q6K:
        d, sc, lvl = np_q6k_blocks(x)
        bad = (got["d"] != d.view(np.uint16)) | (got["scales"] != sc).any(1)
        bad |= np.array([not np.array_equal(q6k_levels(got[i]), lvl[i]) for i in range(nb)])
    else:
        nmax, rmin, nstep = (15, -1.0, 20) if gtype == O.Q4K else (31, -0.5, 15)
        d, dmin, ls, lm, lvl = np_affine_blocks(x, nmax, rmin, nstep)
        bad = (got["d"] != d.view(np.uint16)) | (got["dmin"] != dmin.view(np.uint16))
        dec = [k4_scales(got[i]["scales"]) for i in range(nb)]
        bad |= np.array([not (np.array_equal(dec[i][0], ls[i]) and np.array_equal(dec[i][1], lm[i])) for i in range(nb)])
        lev = q4k_levels if gtype == O.Q4K else q5k_levels
        bad |= np.array([not np.array_equal(lev(got[i]), lvl[i]) for i in range(nb)])
    assert not bad.any(), f"{int(bad.sum())} of {nb} blocks differ, first {np.nonzero(bad)[0][:5]}"


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q5K, O.Q6K])
def test_blocks_match_a_separate_float32_reading(lib, gtype):
    check_bit_level(lib, gtype)


# ------------------------------------------------------------------------------------------------ 4. planted mistakes

CHECKS = {
    "grid_q4k": lambda L: check_exact_grid_affine(L, O.Q4K),
    "grid_q5k": lambda L: check_exact_grid_affine(L, O.Q5K),
    "grid_q6k": lambda L: check_exact_grid_q6k(L),
    "f64_q4k": lambda L: check_qkx2_f64(L, 15, -1.0, 0.1, 20, n=150),
    "f64_q5k": lambda L: check_qkx2_f64(L, 31, -0.5, 0.1, 15, n=150),
    "f64_qx": lambda L: check_qx_f64(L, n=150),
    "bits_q4k": lambda L: check_bit_level(L, O.Q4K),
    "bits_q5k": lambda L: check_bit_level(L, O.Q5K),
    "bits_q6k": lambda L: check_bit_level(L, O.Q6K),
}
# the plants of oracle.c and the checks that bear on the code each one touches
PLANTS = {
    1: ["bits_q4k", "bits_q5k", "f64_q4k"],   # fused multiply-adds in make_qkx2_quants
    2: ["grid_q4k", "bits_q4k"],              # Q4_K search from rmin -0.5
    3: ["grid_q4k", "bits_q4k"],              # Q4_K dmin = max_min / 64
    4: ["f64_qx", "grid_q6k", "bits_q6k"],    # make_qx_quants candidates around nmax - 1
    5: ["grid_q6k", "bits_q6k"],              # Q6_K scales by -127 / max_scale
    6: ["grid_q5k", "bits_q5k"],              # Q5_K 20 search steps
    7: ["f64_q4k", "f64_q5k", "bits_q4k"],    # absolute error as the score
    8: ["f64_q4k", "bits_q4k", "bits_q5k"],   # a positive min refit by sum_xl / sum_l
}


@pytest.fixture(scope="module")
def planted_dir(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is needed to build the planted oracles")
    return tmp_path_factory.mktemp("planted")


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_every_planted_mistake_is_caught(planted_dir, plant):
    so = str(planted_dir / f"liboracle_plant{plant}.so")
    subprocess.run(["gcc", "-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
                    f"-DORACLE_PLANT={plant}", "-shared", "-o", so, ORACLE_C, "-lm"], check=True)
    L = bind(so)
    caught = []
    for name in PLANTS[plant]:
        try:
            CHECKS[name](L)
        except AssertionError:
            caught.append(name)
    assert caught, f"plant {plant} passed every check it should fail: {PLANTS[plant]}"
