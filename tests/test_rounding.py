"""The activation quantizers' round-and-saturate (round_sat_i8 in inference.rs_amd/csrc/common.h) rounds half away
from zero as trunc(p + copysign(0.5 - 2^-25, p)), the add in f32 with rounding to nearest even.  This checks that
identity for every non-negative f32 below 256 (the sign is symmetric, and from 128 up the saturation decides)
against the exact round-half-up of the value in double, as the reference's f32::round gives it
(k_quants.rs:2746-2750, quantized/mod.rs:50)."""
import numpy as np


def test_round_half_away_identity_every_f32_below_256():
    h = np.float32(0.49999997)
    assert float(h) == 0.5 - 2.0 ** -25
    end = int(np.float32(256.0).view(np.uint32))
    step = 1 << 25
    bad = 0
    for lo in range(0, end, step):
        p = np.arange(lo, min(lo + step, end), dtype=np.uint32).view(np.float32)
        fast = np.trunc(p + h)                      # f32 add, then truncation (the conversion)
        exact = np.floor(p.astype(np.float64) + 0.5)  # half away from zero for p >= 0, exact in double
        bad += int(np.count_nonzero(fast.astype(np.float64) != exact))
    assert bad == 0


def test_saturation_and_specials():
    h = np.float32(0.49999997)

    def fast(p):
        p = np.float32(p)
        if p != p:
            return 0
        t = np.float32(p + np.copysign(h, p))
        return int(min(max(np.trunc(t), -128.0), 127.0))  # truncating conversion, then the clamp

    def rust(p):
        if p != p:
            return 0
        r = np.floor(abs(float(p)) + 0.5) * (1 if p >= 0 else -1)
        return int(min(max(r, -128), 127))

    for p in [0.0, -0.0, 0.5, -0.5, 0.49999997, -0.49999997, 1.5, -1.5, 2.5, -2.5, 126.5, 127.4, 127.5, -127.5,
              -128.4, -128.5, -128.6, 1e30, -1e30, np.inf, -np.inf, np.nan, 1e-45, -1e-45]:
        assert fast(p) == rust(p), p
