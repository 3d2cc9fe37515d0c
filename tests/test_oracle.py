"""CPU tests that pin the oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (a dropped term,
a wrong sign or index, a transposed operand, half-to-even instead of half-away
rounding) fails it.  Reference citations are inference.rs file:line.
"""
import numpy as np
import pytest

import oracle as O


def round_half_away(v32: np.ndarray) -> np.ndarray:
    """Rust's f32::round computed in float64, where |v| + 0.5 is exact for float32 inputs."""
    v = v32.astype(np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


# ---------------------------------------------------------------- f16 (half 2.7.1 f16::from_f32 / to_f32 = IEEE RNE)

def test_f16_decode_matches_numpy_on_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([O.f16_bits_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    w = want[::7]
    both_nan = np.isnan(got) & np.isnan(w)
    assert np.array_equal(got[~both_nan].view(np.uint32), w[~both_nan].view(np.uint32))


def test_f16_encode_matches_numpy_round_to_nearest_even():
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 4000).astype(np.float32),
        # exact halfway points between neighbouring f16 values (ties to even), subnormal range and overflow edge
        (np.arange(1, 2048, dtype=np.float32) + np.float32(0.5)),
        np.float32(2.0 ** -24) * np.arange(0, 64, dtype=np.float32) * np.float32(0.75),
        np.array([65504.0, 65519.0, 65520.0, 1e9, -0.0, 0.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8], dtype=np.float32),
    ])
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_bits(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- quantize_block32 (quantized/mod.rs:1650-1686 cases)

def reference_test_blocks():
    """The blocks of quantized/mod.rs:1660-1677: 64 pseudo-random blocks, a tie block with max 127, a zero block."""
    blocks = []
    for b in range(64):
        blocks.append(np.array([(((b * 32 + i) * 2654435761 % 1000) - 500.0) / 37.0 for i in range(32)],
                               dtype=np.float32))
    tie = np.array([127.0 if i == 0 else (i - 16.0) + (0.5 if i % 2 == 0 else 0.49999997) for i in range(32)],
                   dtype=np.float32)
    blocks.append(tie)
    blocks.append(np.zeros(32, dtype=np.float32))
    return blocks


def test_quantize_block32_known_answers():
    for x in reference_test_blocks():
        d, qs = O.quantize_block32(x)
        amax = np.float32(np.max(np.abs(x)))
        want_d = np.float32(amax / np.float32(127.0))
        want_id = np.float32(np.float32(1.0) / want_d) if want_d != 0 else np.float32(0.0)
        want_q = round_half_away(x * want_id).astype(np.int8)
        assert d.view(np.uint32) == want_d.view(np.uint32)
        assert np.array_equal(qs, want_q)


def test_quantize_block32_ties_round_away_from_zero():
    x = reference_test_blocks()[64]
    d, qs = O.quantize_block32(x)
    assert d == np.float32(1.0)  # max 127: each value is its own quant
    want = round_half_away(x).astype(np.int8)
    assert np.array_equal(qs, want)
    # the block discriminates: ties to even (numpy's rint) would give other quants
    assert not np.array_equal(qs, np.rint(x).astype(np.int8))


def test_q8_0_rows_store_f16_scales():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    q = O.blocks(O.Q8_0, O.quantize(O.Q8_0, x))
    for b, blk in enumerate(q):
        xb = x.reshape(-1, 32)[b]
        d, qs = O.quantize_block32(xb)
        assert blk["d"] == np.float32(d).astype(np.float16).view(np.uint16)
        assert np.array_equal(blk["qs"], qs)


# ---------------------------------------------------------------- Q8_K activation quantizer (k_quants.rs:2721-2760)

def q8k_expected(x):
    amax_i = int(np.argmax(np.abs(x)))  # numpy argmax: the first of the maxima
    mx = x[amax_i]
    if np.abs(mx) == 0:
        return np.float32(0.0), np.zeros(256, np.int8), np.zeros(16, np.int16)
    iscale = np.float32(np.float32(-127.0) / mx)
    q = np.clip(round_half_away(iscale * x), -128, 127).astype(np.int8)
    bs = q.reshape(16, 16).astype(np.int32).sum(axis=1).astype(np.int16)
    return np.float32(np.float32(1.0) / iscale), q, bs


@pytest.mark.parametrize("case", ["random", "zero", "tied_opposite_signs", "tied_same", "tiny", "outlier"])
def test_q8k_closed_form(case):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256).astype(np.float32)
    if case == "zero":
        x[:] = 0
    elif case == "tied_opposite_signs":
        x = np.clip(x, -2, 2)
        x[5], x[77] = -3.0, 3.0  # the first maximal |x| (negative) sets the sign of the scale
    elif case == "tied_same":
        x = np.clip(x, -2, 2)
        x[9], x[200] = 3.0, 3.0
    elif case == "tiny":
        x *= np.float32(1e-30)
    elif case == "outlier":
        x[123] = 1e4
    blk = O.blocks(O.Q8K, O.quantize(O.Q8K, x))[0]
    d, q, bs = q8k_expected(x)
    assert blk["d"].view(np.uint32) == d.view(np.uint32)
    assert np.array_equal(blk["qs"], q)
    assert np.array_equal(blk["bsums"], bs)
    if case == "tied_opposite_signs":
        assert blk["qs"][5] == -127 and blk["qs"][77] == 127
    if case != "zero":
        assert np.max(np.abs(blk["qs"].astype(np.int32))) == 127  # the maximum maps to -127 exactly


# ---------------------------------------------------------------- Q4_K / Q6_K weight quantizers: invariants

def _q4k_fields(blk):
    sc = blk["scales"].astype(np.int32)
    s = np.zeros(8, np.int32)
    m = np.zeros(8, np.int32)
    for j in range(8):  # utils.rs:119-129
        if j < 4:
            s[j], m[j] = sc[j] & 63, sc[j + 4] & 63
        else:
            s[j] = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)
            m[j] = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
    return s, m


def np_dequant_q4k(data):
    """Independent vectorised dequantizer (k_quants.rs:2096-2123 layout: qs[32c+l] low = 64c+l, high = 64c+32+l)."""
    out = []
    for blk in O.blocks(O.Q4K, data):
        d = np.float32(np.uint16(blk["d"]).view(np.float16))
        dmin = np.float32(np.uint16(blk["dmin"]).view(np.float16))
        s, m = _q4k_fields(blk)
        qs = blk["qs"].reshape(4, 32)
        vals = np.empty(256, np.float64)
        for c in range(4):
            lo, hi = qs[c] & 0xF, qs[c] >> 4
            vals[64 * c:64 * c + 32] = np.float64(d) * s[2 * c] * lo - np.float64(dmin) * m[2 * c]
            vals[64 * c + 32:64 * c + 64] = np.float64(d) * s[2 * c + 1] * hi - np.float64(dmin) * m[2 * c + 1]
        out.append(vals)
    return np.concatenate(out)


def np_dequant_q6k(data):
    """Independent dequantizer for Q6_K (k_quants.rs:2634-2644 packing, 2649-2680)."""
    out = []
    for blk in O.blocks(O.Q6K, data):
        d = np.float64(np.uint16(blk["d"]).view(np.float16))
        vals = np.empty(256, np.float64)
        for h in range(2):
            ql = blk["ql"][64 * h:64 * h + 64].astype(np.int32)
            qh = blk["qh"][32 * h:32 * h + 32].astype(np.int32)
            for q, (lo_src, shift_lo, hbit) in enumerate([(ql[:32], 0, 0), (ql[32:], 0, 2), (ql[:32], 4, 4),
                                                           (ql[32:], 4, 6)]):
                v = ((lo_src >> shift_lo) & 0xF) | (((qh >> hbit) & 3) << 4)
                idx = 128 * h + 32 * q + np.arange(32)
                vals[idx] = d * blk["scales"][idx // 16].astype(np.float64) * (v - 32)
        out.append(vals)
    return np.concatenate(out)


def np_dequant_q8_0(data):
    b = O.blocks(O.Q8_0, data)
    d = b["d"].view(np.float16).astype(np.float64)
    return (b["qs"].astype(np.float64) * d[:, None]).reshape(-1)


def np_dequant_q8k(data):
    b = O.blocks(O.Q8K, data)
    return (b["qs"].astype(np.float64) * b["d"].astype(np.float64)[:, None]).reshape(-1)


def _f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def np_dequant_q4_0(data):
    """Q4_0 (k_quants.rs:116-120, 313-330): qs[j] low nibble = value j, high nibble = value j + 16, minus 8."""
    b = O.blocks(O.Q4_0, data)
    q = np.concatenate([b["qs"] & 0xF, b["qs"] >> 4], axis=1).astype(np.float64) - 8
    return (q * _f16(b["d"])[:, None]).reshape(-1)


def np_dequant_q5_0(data):
    """Q5_0 (k_quants.rs:133-138, 720-743): the fifth bit of value i is bit i of the little-endian qh word."""
    b = O.blocks(O.Q5_0, data)
    qh = b["qh"].copy().view("<u4")[:, 0]
    bits = (qh[:, None] >> np.arange(32, dtype=np.uint32)) & 1
    q = np.concatenate([b["qs"] & 0xF, b["qs"] >> 4], axis=1).astype(np.int64) + 16 * bits - 16
    return (q.astype(np.float64) * _f16(b["d"])[:, None]).reshape(-1)


def np_dequant_q5k(data):
    """Q5_K (k_quants.rs:200-206, 2433-2467): Q4_K's fields; bit 2c (2c + 1) of qh[l] adds 16 to value 64c + l
    (64c + 32 + l)."""
    out = []
    for blk in O.blocks(O.Q5K, data):
        d, dmin = _f16(blk["d"]), _f16(blk["dmin"])
        s, m = _q4k_fields(blk)
        qs = blk["qs"].reshape(4, 32).astype(np.int64)
        qh = blk["qh"].astype(np.int64)
        vals = np.empty(256, np.float64)
        for c in range(4):
            lo = (qs[c] & 0xF) + 16 * ((qh >> (2 * c)) & 1)
            hi = (qs[c] >> 4) + 16 * ((qh >> (2 * c + 1)) & 1)
            vals[64 * c:64 * c + 32] = d * s[2 * c] * lo - dmin * m[2 * c]
            vals[64 * c + 32:64 * c + 64] = d * s[2 * c + 1] * hi - dmin * m[2 * c + 1]
        out.append(vals)
    return np.concatenate(out)


def np_dequant_iq4xs(data):
    """IQ4_XS (crates/inference-quant/src/gguf/raw.rs:794-808): sub-block ib's 6-bit scale is nibble ib of scales_l
    plus bits 2ib..2ib+1 of scales_h, minus 32; values index the IQ4_NL table."""
    out = []
    for blk in O.blocks(O.IQ4XS, data):
        d = _f16(blk["d"])
        lo_nib = np.stack([blk["scales_l"] & 0xF, blk["scales_l"] >> 4], axis=1).reshape(8).astype(np.int64)
        hi = (int(blk["scales_h"]) >> (2 * np.arange(8))) & 3
        ls = lo_nib | (hi << 4)
        qs = blk["qs"].reshape(8, 16)
        idx = np.concatenate([qs & 0xF, qs >> 4], axis=1)
        out.append((d * (ls - 32)[:, None] * O.KVALUES_IQ4NL[idx].astype(np.float64)).reshape(-1))
    return np.concatenate(out)


NP_DEQUANT = {O.Q4K: np_dequant_q4k, O.Q6K: np_dequant_q6k, O.Q8_0: np_dequant_q8_0, O.Q8K: np_dequant_q8k,
              O.Q4_0: np_dequant_q4_0, O.Q5_0: np_dequant_q5_0, O.Q5K: np_dequant_q5k, O.IQ4XS: np_dequant_iq4xs}


def weight_bytes(gtype, w, rng):
    """Quantized bytes of w, or random blocks of its size for a type the reference has no quantizer for."""
    if gtype == O.IQ4XS:
        return O.random_blocks(gtype, w.size, rng, 0.002).reshape(w.shape[0], -1)
    return O.quantize(gtype, w)


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q8K, O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS])
def test_dequantize_matches_independent_decoder(gtype):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((4, 512)) * 0.02).astype(np.float32)
    q = weight_bytes(gtype, x, rng)
    got = O.dequantize(gtype, q, x.size).astype(np.float64)
    want = NP_DEQUANT[gtype](q)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("gtype,tol", [(O.Q8_0, 0.006), (O.Q4K, 0.12), (O.Q6K, 0.03), (O.Q8K, 0.012), (O.Q4_0, 0.12),
                                      (O.Q5_0, 0.06), (O.Q5K, 0.06)])
def test_quantize_round_trip_error(gtype, tol):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    y = O.dequantize(gtype, O.quantize(gtype, x), x.size).reshape(x.shape)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < tol, rel


def test_q4k_weight_invariants():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    b = O.blocks(O.Q4K, O.quantize(O.Q4K, x))
    for blk in b:
        s, m = _q4k_fields(blk)
        assert s.max() == 63  # the largest sub-block scale sets d = max/63 and quantizes to 63
        assert (s >= 0).all() and (m >= 0).all() and (s <= 63).all() and (m <= 63).all()
        assert np.uint16(blk["d"]).view(np.float16) > 0


def test_q6k_weight_invariants():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    b = O.blocks(O.Q6K, O.quantize(O.Q6K, x))
    for blk in b:
        sc = blk["scales"].astype(np.int32)
        assert np.max(np.abs(sc)) >= 127  # the largest |scale| maps to -128 (or 127 after the min)
        assert np.uint16(blk["d"]).view(np.float16) != 0


def test_q4_0_and_q5_0_quantize_exact_grids_exactly():
    """Values on the quantization grid (d a power of two, the block's extreme at the grid's negative end) come back
    as the very integers they were built from (k_quants.rs:380-418, 681-717)."""
    rng = np.random.default_rng(14)
    for gtype, levels, off in ((O.Q4_0, 16, 8), (O.Q5_0, 32, 16)):
        q = rng.integers(0, levels, (6, 32))
        q[:, 5] = 0                       # max |x| = off * d at a negative value: d = max / -off exactly
        q[:, 6:][q[:, 6:] == 0] = 1       # and the first such value is the only one
        d = 2.0 ** -rng.integers(3, 9, 6)
        x = ((q - off) * d[:, None] * -1.0).astype(np.float32) * -1.0
        got = O.blocks(gtype, O.quantize(gtype, x.reshape(1, -1)))
        assert np.array_equal(_f16(got["d"]), d)
        vals = np.concatenate([got["qs"] & 0xF, got["qs"] >> 4], axis=1).astype(np.int64)
        if gtype == O.Q5_0:
            qh = got["qh"].copy().view("<u4")[:, 0]
            vals += 16 * ((qh[:, None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int64)
        assert np.array_equal(vals, q)


def test_q4_0_and_q5_0_quantizer_clamps_the_positive_end():
    """The value of largest magnitude sets d = max / -8 (-16); a positive extreme lands on q = 0 and the other sign's
    values saturate at 15 (31), the `min` of the reference's cast."""
    x = np.zeros(32, np.float32)
    x[0], x[1] = 1.0, -1.0      # tie: the first (positive) wins, d = -1/8
    b = O.blocks(O.Q4_0, O.quantize(O.Q4_0, x[None]))[0]
    assert _f16(b["d"]) == -0.125 and (b["qs"][0] & 0xF) == 0 and (b["qs"][1] & 0xF) == 15
    b = O.blocks(O.Q5_0, O.quantize(O.Q5_0, x[None]))[0]
    assert _f16(b["d"]) == -1 / 16 and (b["qs"][0] & 0xF) == 0 and (b["qs"][1] & 0xF) == 15
    assert b["qh"].copy().view("<u4")[0] & 0b11 == 0b10  # value 1 = 31 has its fifth bit, value 0 = 0 not
    z = O.blocks(O.Q5_0, O.quantize(O.Q5_0, np.zeros((1, 32), np.float32)))[0]
    # 0 / -16 = -0.0, so d is f16 -0; id = 0 and every value (0 * 0 + 16.5) -> 16: low nibble 0, fifth bit set
    assert z["d"] == 0x8000 and (z["qs"] == 0x00).all()
    assert z["qh"].copy().view("<u4")[0] == 0xFFFFFFFF


def test_q5k_is_q4k_plus_the_fifth_bit():
    """A Q5_K block with qh = 0 dequantizes exactly as the Q4_K block of the same header and nibbles (pinned above),
    and each qh bit adds 16 * d * scale to its value."""
    rng = np.random.default_rng(15)
    raw = O.random_blocks(O.Q5K, 4 * 256, rng)
    b = O.blocks(O.Q5K, raw)
    q4 = np.zeros(4, O.BLOCK_DTYPES[O.Q4K])
    for f in ("d", "dmin", "scales", "qs"):
        q4[f] = b[f]
    b0 = b.copy()
    b0["qh"] = 0
    assert np.array_equal(O.dequantize(O.Q5K, b0.view(np.uint8), 1024).view(np.uint32),
                          O.dequantize(O.Q4K, q4.view(np.uint8), 1024).view(np.uint32))
    full = O.dequantize(O.Q5K, raw, 1024).astype(np.float64)
    zero = O.dequantize(O.Q5K, b0.view(np.uint8), 1024).astype(np.float64)
    for i, blk in enumerate(b):
        s, _ = _q4k_fields(blk)
        for c in range(4):
            for half in range(2):
                bit = (blk["qh"].astype(np.int64) >> (2 * c + half)) & 1
                idx = 256 * i + 64 * c + 32 * half + np.arange(32)
                step = _f16(blk["d"]) * s[2 * c + half] * 16
                np.testing.assert_allclose(full[idx] - zero[idx], bit * step, rtol=1e-6, atol=1e-6 * abs(step) + 1e-30)


def test_q5k_weight_invariants():
    rng = np.random.default_rng(16)
    x = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    b = O.blocks(O.Q5K, O.quantize(O.Q5K, x))
    for blk in b:
        s, m = _q4k_fields(blk)
        assert s.max() == 63 and (m <= 63).all() and _f16(blk["d"]) > 0


def test_iq4xs_closed_form():
    """A hand-built IQ4_XS block: d = 0.5, sub-block ib's scale code 32 + ib + 1 (so ls - 32 = ib + 1; codes above 15
    use scales_h), value j of sub-block ib = index (j + ib) % 16 of the IQ4_NL table."""
    blk = np.zeros(1, O.BLOCK_DTYPES[O.IQ4XS])
    blk["d"] = np.float16(0.5).view(np.uint16)
    codes = 33 + np.arange(8)
    sl = np.zeros(4, np.uint8)
    sh = 0
    for ib, c in enumerate(codes):
        sl[ib // 2] |= (c & 0xF) << (4 * (ib % 2))
        sh |= (int(c) >> 4) << (2 * ib)
    blk["scales_l"], blk["scales_h"] = sl, sh
    idx = (np.arange(32)[None, :] + np.arange(8)[:, None]) % 16
    blk["qs"] = (idx[:, :16] | (idx[:, 16:] << 4)).reshape(-1)
    got = O.dequantize(O.IQ4XS, blk.view(np.uint8), 256).reshape(8, 32)
    want = 0.5 * (np.arange(8) + 1)[:, None] * O.KVALUES_IQ4NL[idx]
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q4_0, O.Q5_0, O.Q5K])
def test_tensor_quantizes_to_its_rows_quantized_alone(gtype):
    """quantized/mod.rs:1720-1765: a whole tensor's bytes equal its rows quantized one at a time."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((40, 2048)).astype(np.float32)
    whole = O.quantize(gtype, x)
    rows = np.stack([O.quantize(gtype, x[r:r + 1])[0] for r in range(x.shape[0])])
    assert np.array_equal(whole, rows)


# ---------------------------------------------------------------- vec_dot / matmul against float64 brute force

def brute(gtype, x, wq, n):
    """float64 sum of dequantized weight times dequantized (Q8_K or Q8_0) activation."""
    m, k = x.shape
    aq = O.quantize(O.ACT_TYPE[gtype], x)
    a = NP_DEQUANT[O.ACT_TYPE[gtype]](aq).reshape(m, k)
    w = NP_DEQUANT[gtype](wq).reshape(n, k)
    return a @ w.T, np.abs(a) @ np.abs(w).T


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS])
@pytest.mark.parametrize("k", [256, 512, 1024, 4096])
def test_matmul_matches_float64_brute_force(gtype, k):
    rng = np.random.default_rng(9 + k)
    n, m = 24, 3
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, ::64] *= 60.0  # the outlier pattern of quantized/mod.rs:1775-1850
    wq = weight_bytes(gtype, w, rng)
    got = O.matmul(gtype, x, wq, n)
    want, terms = brute(gtype, x, wq, n)
    assert np.all(np.abs(got - want) <= 1e-5 * terms + 1e-12)


def test_brute_force_check_catches_a_planted_min_sign_error():
    """The check above is sensitive: a Q4_K dequantizer with the min added instead of subtracted fails it."""
    rng = np.random.default_rng(10)
    k, n = 512, 8
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, k)).astype(np.float32)
    wq = O.quantize(O.Q4K, w)
    got = O.matmul(O.Q4K, x, wq, n)
    aq = O.quantize(O.Q8K, x)
    a = np_dequant_q8k(aq).reshape(2, k)
    planted = []
    for blk in O.blocks(O.Q4K, wq):
        d = np.float64(np.uint16(blk["d"]).view(np.float16))
        dmin = np.float64(np.uint16(blk["dmin"]).view(np.float16))
        s, m = _q4k_fields(blk)
        qs = blk["qs"].reshape(4, 32)
        v = np.empty(256)
        for c in range(4):
            v[64 * c:64 * c + 32] = d * s[2 * c] * (qs[c] & 0xF) + dmin * m[2 * c]
            v[64 * c + 32:64 * c + 64] = d * s[2 * c + 1] * (qs[c] >> 4) + dmin * m[2 * c + 1]
        planted.append(v)
    wrong = a @ np.concatenate(planted).reshape(n, k).T
    _, terms = brute(O.Q4K, x, wq, n)
    assert not np.all(np.abs(got - wrong) <= 1e-5 * terms + 1e-12)


@pytest.mark.parametrize("gtype", [O.Q4_0, O.Q5_0, O.Q4K, O.Q6K, O.Q8_0, O.Q5K])
def test_quantized_matmuls_match_their_dequantized_weights(gtype):
    """quantized/mod.rs:1882-1918: Frobenius relative error < 0.02 against the f32 matmul of the dequantized weight."""
    rng = np.random.default_rng(11)
    K, N = 512, 48
    w = rng.standard_normal((N, K)).astype(np.float32)
    wq = O.quantize(gtype, w)
    dense = O.dequantize(gtype, wq, w.size).reshape(N, K)
    for m in (1, 3, 9, 33):
        x = rng.standard_normal((m, K)).astype(np.float32)
        got = O.matmul(gtype, x, wq, N)
        want = x @ dense.T
        assert np.linalg.norm(got - want) < 0.02 * np.linalg.norm(want)


def test_vec_dot_is_the_matmul_entry():
    rng = np.random.default_rng(12)
    k, n = 1024, 5
    for gtype in (O.Q4K, O.Q6K, O.Q8_0, O.Q4_0, O.Q5_0, O.Q5K, O.IQ4XS):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((1, k)).astype(np.float32)
        wq = weight_bytes(gtype, w, rng)
        aq = O.quantize(O.ACT_TYPE[gtype], x)
        mm = O.matmul(gtype, x, wq, n)
        for c in range(n):
            assert O.vec_dot(gtype, k, wq[c], aq[0]) == mm[0, c]


# ---------------------------------------------------------------- MoE (gguf/mod.rs:573-608; moe_dispatch.cu)

def test_indexed_moe_is_a_matmul_per_route():
    rng = np.random.default_rng(13)
    E, n, k, batch, topk = 3, 16, 512, 4, 2
    w = (rng.standard_normal((E, n, k)) * 0.02).astype(np.float32)
    wq = O.quantize(O.Q4K, w.reshape(E * n, k)).reshape(E, -1)
    ids = rng.integers(0, E, (batch, topk)).astype(np.uint32)
    for xdim1 in (1, topk):
        x = rng.standard_normal((batch, xdim1, k)).astype(np.float32)
        y = O.indexed_moe(O.Q4K, wq, E, n, k, x, ids)
        for b in range(batch):
            for s in range(topk):
                xr = x[b, 0 if xdim1 == 1 else s][None]
                want = O.matmul(O.Q4K, xr, wq[ids[b, s]], n)[0]
                assert np.array_equal(y[b, s], want)


def test_moe_dispatch_and_reduce():
    rng = np.random.default_rng(14)
    E, tokens, topk = 8, 64, 2
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(tokens)]).astype(np.int32)
    bounds, tok, src = O.moe_dispatch(ids, E, topk)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    assert np.array_equal(np.diff(bounds), counts) and bounds[0] == 0 and bounds[-1] == tokens * topk
    for e in range(E):
        routes = tok[bounds[e]:bounds[e + 1]]
        assert np.all(ids.reshape(-1)[routes] == e)
        assert np.array_equal(src[bounds[e]:bounds[e + 1]], routes // topk)
    assert np.array_equal(np.sort(tok), np.arange(tokens * topk))
    inp = rng.standard_normal((tokens, topk, 32)).astype(np.float32)
    wts = rng.random((tokens, topk)).astype(np.float32)
    wts[3, 1] = 0.0
    inp[3, 1] = np.nan  # a parked route with zero weight is never read
    out = O.moe_weighted_reduce(inp, wts)
    inp2 = inp.copy()
    inp2[3, 1] = 0
    want = (inp2.astype(np.float64) * wts[:, :, None]).sum(axis=1)
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------------------------- MoE router oracle

def test_router_oracle_softmax_top2_closed_form():
    # Mixtral's convention: softmax over the experts, the two largest, renormalised to sum to one
    logits = np.array([[0.5, 2.0, -1.0, 1.0, 2.0]], np.float32)  # a tie at 2.0: expert 1 before expert 4
    w, ids = O.router_topk(logits, 2, 1, 0, True)
    assert ids.tolist() == [[1, 4]]
    assert np.allclose(w, [[0.5, 0.5]], rtol=1e-6)
    w, ids = O.router_topk(logits, 3, 1, 0, False)
    p = np.exp(logits[0] - logits[0].max())
    p /= p.sum()
    assert ids.tolist() == [[1, 4, 3]] and np.allclose(w[0], p[[1, 4, 3]], rtol=1e-6)


def test_router_oracle_matches_a_stable_argsort_and_the_weight_modes():
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((20, 64)).astype(np.float32)
    bias = rng.standard_normal(64).astype(np.float32)
    for score_mode in (0, 1, 2):
        w, ids = O.router_topk(logits, 6, score_mode, 0, False, bias=bias)
        x = logits.astype(np.float64)
        score = {0: x, 1: np.exp(x - x.max(1, keepdims=True)) / np.exp(x - x.max(1, keepdims=True)).sum(1, keepdims=True),
                 2: 1 / (1 + np.exp(-x))}[score_mode]
        want_ids = np.argsort(-(score + bias), axis=1, kind="stable")[:, :6]
        assert np.array_equal(ids, want_ids)
        # the bias only selects: the weights are the unbiased scores
        assert np.allclose(w, np.take_along_axis(score, want_ids, 1), rtol=2e-6, atol=1e-7)
    w, ids = O.router_topk(logits, 4, 0, 1, False)  # weight mode 1: a softmax over the picked raw logits
    r = np.take_along_axis(logits.astype(np.float64), ids.astype(np.int64), 1)
    assert np.allclose(w, np.exp(r - r.max(1, keepdims=True)) / np.exp(r - r.max(1, keepdims=True)).sum(1, keepdims=True),
                       rtol=2e-6)
    w2, _ = O.router_topk(logits, 4, 0, 2, True, expert_scale=np.full(64, 2.0, np.float32), output_scale=0.5)
    s = 1 / (1 + np.exp(-r))
    assert np.allclose(w2, s / s.sum(1, keepdims=True), rtol=2e-6)  # 0.5 * 2.0 = 1


def test_router_oracle_nan_and_clamp():
    logits = np.array([[np.nan, 1.0, 3.0, 2.0]], np.float32)
    _, ids = O.router_topk(logits, 3, 0, 0, False)
    assert ids.tolist() == [[2, 3, 1]]  # NaN is -inf: picked last
    w, ids = O.router_topk(logits, 3, 0, 0, False, clamp=(0.5, 1.5))
    # 3 and 2 clamp to 1.5 (ties to the lower index); the clamp takes NaN to its lower bound, as fmaxf does
    assert ids.tolist() == [[2, 3, 1]] and w.tolist() == [[1.5, 1.5, 1.0]]
    _, ids = O.router_topk(logits, 4, 0, 0, False, clamp=(1.25, 1.5))
    assert ids.tolist() == [[2, 3, 0, 1]]  # NaN -> 1.25, 1.0 -> 1.25: a tie, the lower index first
