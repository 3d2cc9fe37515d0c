// CPU block quantizers behind QTensor::quantize (crates/inference-tensor/src/quantized/mod.rs:391-413:
// weights are quantized on the host and then uploaded).  Same bytes as the reference's llama.cpp-style
// quantizer (Quantizer::LlamaCpp): products are rounded before every sum, so this file is compiled with
// -ffp-contract=off.
//   Q8_0  k_quants.rs:923-949 + quantized/mod.rs:41-56
//   Q8_K  k_quants.rs:2721-2760
//   Q4_K  k_quants.rs:1930-2001 (no imatrix) with utils.rs:268-361 (make_qkx2_quants)
//   Q6_K  k_quants.rs:2590-2646 (no imatrix) with utils.rs:135-264 (make_qx_quants)
//   Q5_K  k_quants.rs:2256-2334 (no imatrix): Q4_K's fit with 31 levels and Q5K_SEARCH, fifth bits in qh
//   Q4_0  k_quants.rs:380-418;  Q5_0  k_quants.rs:681-717
#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>

#include "qtensor.h"

namespace inference_rs_amd {
namespace cpu {
namespace {

inline uint32_t bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

// round to nearest, ties to even, by the 1.5 * 2^23 add (utils.rs:3-4, 32-35)
inline int32_t nearest_int(float v) {
  volatile float t = v + 12582912.0f;
  return static_cast<int32_t>(bits(t) & 0x007fffffu) - 0x00400000;
}

inline int32_t nearest_int_mul(float a, float b) {
  volatile float p = a * b;  // rounded before the magic add (utils.rs:70-73, LlamaCpp)
  return nearest_int(p);
}

inline int8_t as_i8(float v) {  // Rust `f32 as i8`
  if (std::isnan(v)) return 0;
  return static_cast<int8_t>(std::min(127.0f, std::max(-128.0f, v)));
}

template <int N>
struct Fit {
  std::array<uint8_t, N> l;
  float scale, neg_min;
};

// make_qkx2_quants: affine fit of x (32 values) onto 0..nmax under weights w, from the min/max fit and
// nstep + 1 candidate scales rmin + rdelta * is (utils.rs:268-361)
Fit<32> qkx2(const float *x, const float *w, int nmax, float rmin, float rdelta, int nstep) {
  Fit<32> f{};
  float lo = x[0], hi = x[0], sw = w[0], sx = w[0] * x[0];
  for (int i = 1; i < 32; ++i) {
    lo = std::fmin(lo, x[i]);
    hi = std::fmax(hi, x[i]);
    sw += w[i];
    sx = w[i] * x[i] + sx;
  }
  lo = lo > 0.0f ? 0.0f : lo;
  if (hi == lo) {
    f.l.fill(0);
    f.scale = 0.0f;
    f.neg_min = -lo;
    return f;
  }
  float iscale = static_cast<float>(nmax) / (hi - lo);
  float scale = 1.0f / iscale, mn = lo, best = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const int32_t q = std::clamp(nearest_int_mul(iscale, x[i] - lo), 0, nmax);
    f.l[i] = static_cast<uint8_t>(q);
    const float diff = scale * static_cast<float>(q) + lo - x[i];
    best = w[i] * (diff * diff) + best;
  }
  std::array<int32_t, 32> cand;
  // the search keeps shifting by the best min found so far, as the reference's `min` does
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rdelta * static_cast<float>(is) + rmin + static_cast<float>(nmax)) / (hi - mn);
    float s_l = 0.0f, s_l2 = 0.0f, s_xl = 0.0f;
    for (int i = 0; i < 32; ++i) {
      cand[i] = std::clamp(nearest_int_mul(iscale, x[i] - mn), 0, nmax);
      const float lf = static_cast<float>(cand[i]);
      const float wl = w[i] * lf;
      s_l += wl;
      s_l2 = wl * lf + s_l2;
      s_xl = wl * x[i] + s_xl;
    }
    const float det = sw * s_l2 - s_l * s_l;
    if (!(det > 0.0f)) continue;
    float this_scale = (sw * s_xl - sx * s_l) / det;
    float this_min = (s_l2 * sx - s_l * s_xl) / det;
    if (this_min > 0.0f) {
      this_min = 0.0f;
      this_scale = s_xl / s_l2;
    }
    float err = 0.0f;
    for (int i = 0; i < 32; ++i) {
      const float diff = this_scale * static_cast<float>(cand[i]) + this_min - x[i];
      err = w[i] * (diff * diff) + err;
    }
    if (err < best) {
      for (int i = 0; i < 32; ++i) f.l[i] = static_cast<uint8_t>(cand[i]);
      best = err;
      scale = this_scale;
      mn = this_min;
    }
  }
  f.scale = scale;
  f.neg_min = -mn;
  return f;
}

// make_qx_quants with rmse_type 1 (weights x^2) over 16 values into -32..31 (utils.rs:135-264)
float qx16(const float *x, int8_t *ls) {
  constexpr int nmax = 32;
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 16; ++i)
    if (std::fabs(x[i]) > amax) {
      amax = std::fabs(x[i]);
      mx = x[i];
    }
  if (amax < 1e-15f) {
    std::memset(ls, 0, 16);
    return 0.0f;
  }
  auto level = [&](float is, float v) { return std::clamp(nearest_int_mul(is, v), -nmax, nmax - 1); };
  auto fit = [&](float is, float &slx, float &sl2) {
    slx = 0.0f;
    sl2 = 0.0f;
    for (int i = 0; i < 16; ++i) {
      const float q = static_cast<float>(level(is, x[i]));
      const float w = x[i] * x[i];
      slx = (w * x[i]) * q + slx;
      sl2 = (w * q) * q + sl2;
    }
  };
  float iscale = -static_cast<float>(nmax) / mx;
  float slx, sl2;
  fit(iscale, slx, sl2);
  for (int i = 0; i < 16; ++i) ls[i] = static_cast<int8_t>(nmax + level(iscale, x[i]));
  float scale = sl2 != 0.0f ? slx / sl2 : 0.0f;
  float best = scale * slx;
  for (int is = -9; is <= 9; ++is) {
    if (is == 0) continue;
    iscale = -(0.1f * static_cast<float>(is) + static_cast<float>(nmax)) / mx;
    fit(iscale, slx, sl2);
    if (sl2 > 0.0f && slx * slx > best * sl2) {
      for (int i = 0; i < 16; ++i) ls[i] = static_cast<int8_t>(nmax + level(iscale, x[i]));
      scale = slx / sl2;
      best = scale * slx;
    }
  }
  return scale;
}

// The shared part of Q4_K and Q5_K: per-sub-block affine fits onto 0..nmax, 6-bit scales and mins packed into
// scales[12] (the inverse of get_scale_min_k4, k_quants.rs:1979-1990), f16 d / dmin, and the final levels L
// re-quantized against the stored scales.
template <int NMAX>
void kquant_levels(const float *x, float rmin, int nstep, uint16_t &d16, uint16_t &dmin16, uint8_t scales[12],
                   std::array<uint8_t, 256> &L) {
  std::array<float, 8> sc{}, mn{};
  for (int j = 0; j < 8; ++j) {
    const float *xs = x + 32 * j;
    float ss = 0.0f;
    for (int i = 0; i < 32; ++i) ss = ss + xs[i] * xs[i];
    const float rms = std::sqrt(ss / 32.0f);
    float w[32];
    for (int i = 0; i < 32; ++i) w[i] = rms + std::fabs(xs[i]);  // qkx2_weights, k_quants.rs:302-305
    const Fit<32> f = qkx2(xs, w, NMAX, rmin, 0.1f, nstep);
    std::copy(f.l.begin(), f.l.end(), L.begin() + 32 * j);
    sc[j] = f.scale;
    mn[j] = f.neg_min;
  }
  float max_sc = 0.0f, max_mn = 0.0f;
  for (int j = 0; j < 8; ++j) {
    max_sc = std::fmax(sc[j], max_sc);
    max_mn = std::fmax(mn[j], max_mn);
  }
  const float inv_sc = max_sc > 0.0f ? 63.0f / max_sc : 0.0f;
  const float inv_mn = max_mn > 0.0f ? 63.0f / max_mn : 0.0f;
  std::array<uint8_t, 8> ls, lm;
  for (int j = 0; j < 8; ++j) {
    ls[j] = static_cast<uint8_t>(std::min(nearest_int_mul(inv_sc, sc[j]), 63));
    lm[j] = static_cast<uint8_t>(std::min(nearest_int_mul(inv_mn, mn[j]), 63));
  }
  for (int j = 0; j < 4; ++j) {
    scales[j] = static_cast<uint8_t>(ls[j] | ((ls[j + 4] >> 4) << 6));
    scales[j + 4] = static_cast<uint8_t>(lm[j] | ((lm[j + 4] >> 4) << 6));
    scales[j + 8] = static_cast<uint8_t>((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
  }
  d16 = f32_to_f16(max_sc / 63.0f);
  dmin16 = f32_to_f16(max_mn / 63.0f);
  const float d = f16_to_f32(d16), dmin = f16_to_f32(dmin16);
  for (int j = 0; j < 8; ++j) {
    const int s = j < 4 ? (scales[j] & 63) : ((scales[j + 4] & 0xF) | ((scales[j - 4] >> 6) << 4));
    const int m = j < 4 ? (scales[j + 4] & 63) : ((scales[j + 4] >> 4) | ((scales[j] >> 6) << 4));
    const float dj = d * static_cast<float>(s);
    if (dj == 0.0f) continue;  // keeps the fit's levels
    const float dm = dmin * static_cast<float>(m);
    for (int i = 0; i < 32; ++i)
      L[32 * j + i] = static_cast<uint8_t>(std::clamp(nearest_int((x[32 * j + i] + dm) / dj), 0, NMAX));
  }
}

void q4k_block(const float *x, qmm_block_q4k &b) {
  std::array<uint8_t, 256> L{};
  std::memset(&b, 0, sizeof b);
  kquant_levels<15>(x, -1.0f, 20, b.d, b.dmin, b.scales, L);  // Q4K_SEARCH, k_quants.rs:248-253
  for (int c = 0; c < 4; ++c)
    for (int l = 0; l < 32; ++l) b.qs[32 * c + l] = static_cast<uint8_t>(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

void q5k_block(const float *x, qmm_block_q5k &b) {
  std::array<uint8_t, 256> L{};
  std::memset(&b, 0, sizeof b);
  kquant_levels<31>(x, -0.5f, 15, b.d, b.dmin, b.scales, L);  // Q5K_SEARCH, k_quants.rs:254-259
  for (int c = 0; c < 4; ++c)
    for (int l = 0; l < 32; ++l) {
      const uint8_t lo = L[64 * c + l], hi = L[64 * c + 32 + l];
      b.qs[32 * c + l] = static_cast<uint8_t>((lo & 15) | ((hi & 15) << 4));
      b.qh[l] |= static_cast<uint8_t>(((lo >> 4) << (2 * c)) | ((hi >> 4) << (2 * c + 1)));
    }
}

// Q4_0 / Q5_0: d = (the signed value of largest magnitude, first on a tie) / -levels/2, q = clamp(x / d + off + 0.5)
// truncated (Rust's saturating casts)
float absmax_signed32(const float *x) {
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 32; ++i)
    if (amax < std::fabs(x[i])) {
      amax = std::fabs(x[i]);
      mx = x[i];
    }
  return mx;
}

void q4_0_block(const float *x, qmm_block_q4_0 &b) {
  const float d = absmax_signed32(x) / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  b.d = f32_to_f16(d);
  auto q = [&](float v) {  // (v * id + 8.5) as u8, then min 15
    const float t = v * id + 8.5f;
    const int u = std::isnan(t) || t <= 0.0f ? 0 : t >= 255.0f ? 255 : static_cast<int>(t);
    return static_cast<uint8_t>(std::min(u, 15));
  };
  for (int j = 0; j < 16; ++j) b.qs[j] = static_cast<uint8_t>(q(x[j]) | (q(x[16 + j]) << 4));
}

void q5_0_block(const float *x, qmm_block_q5_0 &b) {
  const float d = absmax_signed32(x) / -16.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  b.d = f32_to_f16(d);
  auto q = [&](float v) {  // ((v * id + 16.5) as i8).min(31) as u8
    return static_cast<uint8_t>(std::min<int>(as_i8(v * id + 16.5f), 31));
  };
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const uint8_t a = q(x[j]), c = q(x[16 + j]);
    b.qs[j] = static_cast<uint8_t>((a & 15) | ((c & 15) << 4));
    qh |= static_cast<uint32_t>((a >> 4) & 1) << j;
    qh |= static_cast<uint32_t>((c >> 4) & 1) << (16 + j);
  }
  std::memcpy(b.qh, &qh, 4);
}

void q6k_block(const float *x, qmm_block_q6k &b) {
  std::array<int8_t, 256> L{};
  std::array<float, 16> sc{};
  float max_abs = 0.0f, max_sc = 0.0f;
  for (int g = 0; g < 16; ++g) {
    sc[g] = qx16(x + 16 * g, L.data() + 16 * g);
    if (std::fabs(sc[g]) > max_abs) {
      max_abs = std::fabs(sc[g]);
      max_sc = sc[g];
    }
  }
  const float iscale = -128.0f / max_sc;
  b.d = f32_to_f16(1.0f / iscale);
  for (int g = 0; g < 16; ++g) b.scales[g] = static_cast<int8_t>(std::min(nearest_int_mul(iscale, sc[g]), 127));
  const float d = f16_to_f32(b.d);
  for (int g = 0; g < 16; ++g) {
    const float dg = d * static_cast<float>(b.scales[g]);
    if (dg == 0.0f) continue;
    for (int i = 0; i < 16; ++i)
      L[16 * g + i] = static_cast<int8_t>(std::clamp(nearest_int(x[16 * g + i] / dg), -32, 31) + 32);
  }
  // ql: low nibbles of values (l, l+64) and (l+32, l+96); qh: their top two bits (k_quants.rs:2634-2644)
  for (int h = 0; h < 2; ++h)
    for (int i = 0; i < 32; ++i) {
      const int base = 128 * h + i;
      const uint8_t q1 = L[base], q2 = L[base + 32], q3 = L[base + 64], q4 = L[base + 96];
      b.ql[64 * h + i] = static_cast<uint8_t>((q1 & 0xF) | ((q3 & 0xF) << 4));
      b.ql[64 * h + 32 + i] = static_cast<uint8_t>((q2 & 0xF) | ((q4 & 0xF) << 4));
      b.qh[32 * h + i] = static_cast<uint8_t>((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
}

void q8_0_block(const float *x, qmm_block_q8_0 &b) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[i]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int i = 0; i < 32; ++i) b.qs[i] = as_i8(std::round(x[i] * id));
  b.d = f32_to_f16(d);
}

void q8k_block(const float *x, qmm_block_q8k &b) {
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 256; ++i)
    if (amax < std::fabs(x[i])) {
      amax = std::fabs(x[i]);
      mx = x[i];
    }
  if (amax == 0.0f) {
    std::memset(&b, 0, sizeof b);
    return;
  }
  const float iscale = -127.0f / mx;
  for (int i = 0; i < 256; ++i) b.qs[i] = as_i8(std::round(iscale * x[i]));
  for (int g = 0; g < 16; ++g) {
    int s = 0;
    for (int i = 0; i < 16; ++i) s += b.qs[16 * g + i];
    b.bsums[g] = static_cast<int16_t>(s);
  }
  b.d = 1.0f / iscale;
}

template <class B, class F>
void for_blocks(const float *x, int64_t n, int bs, void *out, F fn) {
  B *y = static_cast<B *>(out);
  const int64_t nb = n / bs;
#pragma omp parallel for schedule(static) if (nb >= 64)
  for (int64_t i = 0; i < nb; ++i) fn(x + i * bs, y[i]);
}

}  // namespace

uint16_t f32_to_f16(float f) {
  // IEEE binary16, round to nearest even (the `half` crate's f16::from_f32)
  const uint32_t u = bits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u | ((a >> 13) & 0x3ffu) : 0u));
  if (a >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // rounds past 65504
  if (a < 0x38800000u) {                                               // below 2^-14: f16 subnormal
    if (a < 0x33000000u) return static_cast<uint16_t>(sign);           // at most 2^-25: to zero
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const int shift = 126 - static_cast<int>(a >> 23);  // 14..24
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return static_cast<uint16_t>(sign | r);
  }
  uint32_t r = ((a >> 13) - ((127u - 15u) << 10));
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return static_cast<uint16_t>(sign | r);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    const float v = std::ldexp(static_cast<float>(m), -24);
    return sign ? -v : v;
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

bool quantize(GgmlDType t, const float *x, int64_t n, void *out) {
  switch (t) {
    case GgmlDType::Q8_0:
      if (n % 32) return false;
      for_blocks<qmm_block_q8_0>(x, n, 32, out, q8_0_block);
      return true;
    case GgmlDType::Q4K:
      if (n % 256) return false;
      for_blocks<qmm_block_q4k>(x, n, 256, out, q4k_block);
      return true;
    case GgmlDType::Q6K:
      if (n % 256) return false;
      for_blocks<qmm_block_q6k>(x, n, 256, out, q6k_block);
      return true;
    case GgmlDType::Q8K:
      if (n % 256) return false;
      for_blocks<qmm_block_q8k>(x, n, 256, out, q8k_block);
      return true;
    case GgmlDType::Q5K:
      if (n % 256) return false;
      for_blocks<qmm_block_q5k>(x, n, 256, out, q5k_block);
      return true;
    case GgmlDType::Q4_0:
      if (n % 32) return false;
      for_blocks<qmm_block_q4_0>(x, n, 32, out, q4_0_block);
      return true;
    case GgmlDType::Q5_0:
      if (n % 32) return false;
      for_blocks<qmm_block_q5_0>(x, n, 32, out, q5_0_block);
      return true;
    default: return false;
  }
}

bool dequantize(GgmlDType t, const void *blocks, int64_t n, float *y) {
  switch (t) {
    case GgmlDType::Q8_0: {
      const auto *b = static_cast<const qmm_block_q8_0 *>(blocks);
      for (int64_t i = 0; i < n / 32; ++i) {
        const float d = f16_to_f32(b[i].d);
        for (int j = 0; j < 32; ++j) y[32 * i + j] = static_cast<float>(b[i].qs[j]) * d;
      }
      return true;
    }
    case GgmlDType::Q4K: {
      const auto *b = static_cast<const qmm_block_q4k *>(blocks);
      for (int64_t i = 0; i < n / 256; ++i) {
        const float d = f16_to_f32(b[i].d), dmin = f16_to_f32(b[i].dmin);
        for (int j = 0; j < 8; ++j) {
          const uint8_t *s = b[i].scales;
          const int sc = j < 4 ? (s[j] & 63) : ((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
          const int m = j < 4 ? (s[j + 4] & 63) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
          const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(m);
          const int c = j / 2, hi = j & 1;
          for (int l = 0; l < 32; ++l) {
            const uint8_t q = b[i].qs[32 * c + l];
            y[256 * i + 32 * j + l] = d1 * static_cast<float>(hi ? (q >> 4) : (q & 0xF)) - m1;
          }
        }
      }
      return true;
    }
    case GgmlDType::Q6K: {
      const auto *b = static_cast<const qmm_block_q6k *>(blocks);
      for (int64_t i = 0; i < n / 256; ++i) {
        const float d = f16_to_f32(b[i].d);
        for (int v = 0; v < 256; ++v) {
          const int h = v / 128, r = v % 128, q = r / 32, l = r % 32;
          const uint8_t lo = b[i].ql[64 * h + 32 * (q & 1) + l];
          const int nib = (q >> 1) ? (lo >> 4) : (lo & 0xF);
          const int hb = (b[i].qh[32 * h + l] >> (2 * q)) & 3;
          y[256 * i + v] = d * static_cast<float>(b[i].scales[v / 16]) * static_cast<float>((nib | (hb << 4)) - 32);
        }
      }
      return true;
    }
    case GgmlDType::Q8K: {
      const auto *b = static_cast<const qmm_block_q8k *>(blocks);
      for (int64_t i = 0; i < n / 256; ++i)
        for (int j = 0; j < 256; ++j) y[256 * i + j] = b[i].d * static_cast<float>(b[i].qs[j]);
      return true;
    }
    case GgmlDType::Q5K: {  // k_quants.rs:2433-2467
      const auto *b = static_cast<const qmm_block_q5k *>(blocks);
      for (int64_t i = 0; i < n / 256; ++i) {
        const float d = f16_to_f32(b[i].d), dmin = f16_to_f32(b[i].dmin);
        for (int j = 0; j < 8; ++j) {
          const uint8_t *s = b[i].scales;
          const int sc = j < 4 ? (s[j] & 63) : ((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
          const int m = j < 4 ? (s[j + 4] & 63) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
          const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(m);
          const int c = j / 2, hi = j & 1;
          for (int l = 0; l < 32; ++l) {
            const uint8_t q = b[i].qs[32 * c + l];
            const int v = (hi ? (q >> 4) : (q & 0xF)) + 16 * ((b[i].qh[l] >> j) & 1);
            y[256 * i + 32 * j + l] = d1 * static_cast<float>(v) - m1;
          }
        }
      }
      return true;
    }
    case GgmlDType::Q4_0:  // k_quants.rs:313-330
    case GgmlDType::Q5_0: {  // k_quants.rs:720-743
      const bool five = t == GgmlDType::Q5_0;
      const size_t bytes = five ? 22 : 18;
      const uint8_t *p = static_cast<const uint8_t *>(blocks);
      for (int64_t i = 0; i < n / 32; ++i, p += bytes) {
        uint16_t dh;
        std::memcpy(&dh, p, 2);
        const float d = f16_to_f32(dh);
        uint32_t qh = 0;
        if (five) std::memcpy(&qh, p + 2, 4);
        const uint8_t *qs = p + (five ? 6 : 2);
        for (int v = 0; v < 32; ++v) {
          int q = v < 16 ? (qs[v] & 0xF) : (qs[v - 16] >> 4);
          if (five) q |= static_cast<int>((qh >> v) & 1) << 4;
          y[32 * i + v] = static_cast<float>(q - (five ? 16 : 8)) * d;
        }
      }
      return true;
    }
    default: return false;
  }
}

}  // namespace cpu
}  // namespace inference_rs_amd
