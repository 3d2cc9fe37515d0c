// Shared device and host helpers for the gfx950 GGUF kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmm_blocks.h"

#define QMM_WAVE 64

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ host-side error reporting
void qmm_set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
// compute units of the current device (queried once per device)
int qmm_device_cus();

// Workgroups of kernel K with `threads` threads and `lds` bytes of dynamic LDS that one CU holds at once, queried
// once per kernel (every device of the process is taken to be alike); at least 1.
template <auto K>
int qmm_resident_per_cu(int threads, size_t lds) {
  static const int n = [&] {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, K, threads, lds) != hipSuccess || v < 1) v = 1;
    return v;
  }();
  return n;
}

// ------------------------------------------------------------------ scalar conversions (device)

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);  // exact
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32: round to nearest even
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __builtin_bit_cast(float, h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                             // round to nearest even
  return (uint16_t)(u >> 16);
}

// Rust's `p.round() as i8` (saturating, NaN -> 0) in four operations: round (half away from zero) is
// trunc(p + copysign(0.5 - 2^-25, p)) with the f32 add rounding to nearest even (equal for every f32 of magnitude
// below 256, checked exhaustively against floor(|p| + 0.5) in double; above 128 the saturation decides either way),
// the truncation is the hardware conversion v_cvt_i32_f32 (NaN -> 0, out of range -> the nearest int32), and the
// clamp to -128..127 one integer median of three.
__device__ __forceinline__ int32_t round_sat_i8(float p) {
#pragma clang fp contract(off)
  const float t = p + __builtin_copysignf(0.49999997f, p);
  int32_t i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(t));  // the hardware conversion: NaN -> 0, out of range saturates
  return i < -128 ? -128 : (i > 127 ? 127 : i);
}

// Element loads of the three activation dtypes.
// load4: the four values at p, p + 1, p + 2, p + 3 in one vector load (p aligned to four values)
struct in_f32 {
  typedef float T;
  static __device__ __forceinline__ float load(const float *p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void load4(const float *p, float v[4]) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 f = *(const f32x4 *)p;
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
};
struct in_f16 {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const uint16_t *p, int64_t i) { return f16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ void load4(const uint16_t *p, float v[4]) {
    const uint2 h = *(const uint2 *)p;
    v[0] = f16_bits_to_f32(h.x & 0xffffu), v[1] = f16_bits_to_f32(h.x >> 16);
    v[2] = f16_bits_to_f32(h.y & 0xffffu), v[3] = f16_bits_to_f32(h.y >> 16);
  }
};
struct in_bf16 {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const uint16_t *p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ void load4(const uint16_t *p, float v[4]) {
    const uint2 h = *(const uint2 *)p;
    v[0] = bf16_bits_to_f32(h.x & 0xffffu), v[1] = bf16_bits_to_f32(h.x >> 16);
    v[2] = bf16_bits_to_f32(h.y & 0xffffu), v[3] = bf16_bits_to_f32(h.y >> 16);
  }
};

// Output stores.
struct out_f32 {
  typedef float T;
  static __device__ __forceinline__ void store(float *p, int64_t i, float v) { p[i] = v; }
};
struct out_f16 {
  typedef uint16_t T;
  static __device__ __forceinline__ void store(uint16_t *p, int64_t i, float v) { p[i] = f32_to_f16_bits(v); }
};
struct out_bf16 {
  typedef uint16_t T;
  static __device__ __forceinline__ void store(uint16_t *p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
};

// ------------------------------------------------------------------ wave64 reductions


// Sum over the wave through DPP (no LDS round trips); the total lands in lane 63 (other lanes hold partial sums).
//   quad_perm [1,0,3,2], [2,3,0,1]: quad sums; row_half_mirror, row_mirror: 16-lane row sums;
//   row_bcast15 into rows 1, 3 and row_bcast31 into rows 2, 3: row 3 ends with the total.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf,
                                                                   false));
}
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  v = dpp_add<0x142, 0xa>(v);  // row_bcast15
  v = dpp_add<0x143, 0xc>(v);  // row_bcast31
  return v;
}

// Maximum of non-negative values over the wave with the same DPP pattern (0, what a lane outside a row_bcast
// mask reads, is the identity); every lane gets the result through lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                        0xf, false)));
}
// The same over unsigned values (0 is the identity)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
  return v > o ? v : o;
}
__device__ __forceinline__ float wave_max_nonneg(float v) {
  v = dpp_max<0xb1, 0xf>(v);
  v = dpp_max<0x4e, 0xf>(v);
  v = dpp_max<0x141, 0xf>(v);
  v = dpp_max<0x140, 0xf>(v);
  v = dpp_max<0x142, 0xa>(v);
  v = dpp_max<0x143, 0xc>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over each quad of lanes (xor 1, xor 2 through quad_perm); every lane of the quad gets it.
__device__ __forceinline__ int quad_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);
  return v + __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Bytes [shift, shift + 4) of the 8-byte little-endian pair (lo, hi), shift in 0..3.
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t shift) {
  return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// GLU activations, numbered as the reference's GluActivation (inference-quant/kernels/cuda/glu_activation.cuh):
// 0 SiLU, 1 GELU (tanh form), 2 ReLU, 3 GELU (erf form), 4 sigmoid
__device__ __forceinline__ float glu_act(int activation, float x) {
  switch (activation) {
    case 1: return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * (x * x * x))));
    case 2: return fmaxf(x, 0.0f);
    case 3: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    case 4: return 1.0f / (1.0f + expf(-x));
    default: return x / (1.0f + expf(-x));
  }
}
constexpr int kGluActivations = 5;

static inline int64_t qmm_ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
