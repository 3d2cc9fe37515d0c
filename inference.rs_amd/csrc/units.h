// Per-type "units" of the decode dot product: the slice of one weight row a lane owns, the matching slice
// of one activation row, and their dot product.  A row of K values is split into units that lanes of a
// wave stride over; every unit's integer dot is exact and is scaled to f32 once, so a lane's float work
// mirrors the reference's per-block scaling (k_quants.rs vec_dot_unopt) and only the order of the
// per-unit f32 sums differs.
//
//   Q4_K  unit = a quarter super-block (64 values, sub-blocks 2c and 2c+1): 16 B header + 32 B of nibbles
//         against 64 Q8_K values, their bsums and d.            (k_quants.rs:1848-1928)
//   Q6_K  unit = 64 values 128h + 32q + 16p + (0..15), q = 0..3: three 16 B slices of ql/qh, four int8 scales,
//         d; activations with the four matching bsums.           (k_quants.rs:2518-2575)
//   Q8_0  unit = two consecutive 34 B blocks (68 B, dword aligned when a row holds an even number of blocks)
//         against two Q8_0 activation blocks.                    (k_quants.rs:982-999)
//   Q4_0 / Q5_0  unit = a pair of 18 / 22 B blocks against two Q8_0 blocks (one block when rows hold an odd
//         number).                                               (k_quants.rs:432-449, 615-637)
//   Q5_K  unit = Q4_K's quarter super-block plus the 32 fifth-bit bytes.  (k_quants.rs:2145-2232)
//   IQ4_XS unit = two 32-value sub-blocks: 8 B header + 32 B of table indices.
//                                                   (inference-quant/src/gguf/cpu_dot.rs:416-440)
#pragma once

#include <initializer_list>

#include "common.h"

// No multiply is fused into an add here: each unit's f32 arithmetic is the same instructions in every kernel that
// inlines it, whatever the code around it, so the decode entries that share a unit give the same bits.
#pragma clang fp contract(off)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16 bytes from a 16-byte aligned address
__device__ __forceinline__ u32x4 ld_a16(const uint8_t *p) { return *(const u32x4 *)p; }

// 16 bytes from a 4-byte aligned address (global_load_dwordx4 needs dword alignment only)
__device__ __forceinline__ u32x4 ld_a4(const uint8_t *p) {
  u32x4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 4), 16);
  return v;
}
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)__builtin_assume_aligned(p, 4); }
__device__ __forceinline__ uint32_t ld16(const uint8_t *p) { return *(const uint16_t *)__builtin_assume_aligned(p, 2); }

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Buffer resource over [base, base + bytes) (gfx9 raw buffer, dword format): loads past the end return zero.
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, int64_t bytes) {
  const int n = bytes > 0x7ffffff0 ? 0x7ffffff0 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

// Where a unit's weight loads read: byte offsets o (>= -3) from the start of one weight row.
//   row_ptr  plain global loads from a row pointer
//   row_buf  raw buffer loads over the row; an empty buffer (a row past the end) reads zeros with no memory
//            traffic, so a persistent wave can request "the row after next" unconditionally
struct row_ptr {
  const uint8_t *p;
  __device__ __forceinline__ u32x4 a16(int o) const { return ld_a16(p + o); }
  __device__ __forceinline__ u32x4 a4x16(int o) const { return ld_a4(p + o); }
  __device__ __forceinline__ uint32_t x4(int o) const { return ld32(p + o); }
  __device__ __forceinline__ u32x2 x8(int o) const {
    u32x2 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p + o, 4), 8);
    return v;
  }
  __device__ __forceinline__ uint32_t x2(int o) const { return ld16(p + o); }
  __device__ __forceinline__ uint32_t mis(int o) const { return (uint32_t)((uintptr_t)(p + o) & 3); }
};
struct row_buf {
  rsrc_t r;
  uint32_t m;  // the row start's address mod 4: the buffer starts m bytes earlier, dword aligned
  __device__ __forceinline__ u32x4 a16(int o) const {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(o + (int)m), 0, 0);
  }
  __device__ __forceinline__ u32x4 a4x16(int o) const { return a16(o); }
  __device__ __forceinline__ uint32_t x4(int o) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (uint32_t)(o + (int)m), 0, 0);
  }
  __device__ __forceinline__ u32x2 x8(int o) const {
    return __builtin_amdgcn_raw_buffer_load_b64(r, (uint32_t)(o + (int)m), 0, 0);
  }
  __device__ __forceinline__ uint32_t x2(int o) const {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (uint32_t)(o + (int)m), 0, 0);
  }
  __device__ __forceinline__ uint32_t mis(int o) const { return (m + (uint32_t)o) & 3; }
};
// row: a wave-uniform pointer; bytes 0 for a row that does not exist
__device__ __forceinline__ row_buf make_row_buf(const uint8_t *row, int64_t bytes) {
  const uint32_t m = (uint32_t)((uintptr_t)row & 3);
  return {make_rsrc(row - m, bytes > 0 ? bytes + m : 0), m};
}

// Activations quantized by the lane that uses them (quantize_a, the one-launch decode over rows of more than 4096
// values): one lane, one 64-value unit, read as 16 float4 from a 16-byte aligned f32 row.
__device__ __forceinline__ void load_unit_f32(const float *x, const int (&off)[16], float (&v)[16][4]) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const f32x4 f = *(const f32x4 *)(x + off[j]);
    v[j][0] = f.x, v[j][1] = f.y, v[j][2] = f.z, v[j][3] = f.w;
  }
}

// One lane's share of one 256-value Q8_K block: v[j] holds values off[j] .. off[j] + 3 of the block (off increasing in
// j), and the block's four units sit on the four lanes of a quad, all of them live or none.  The block is quantized as
// BlockQ8K::from_float does it (crates/inference-tensor/src/quantized/k_quants.rs:2721-2760), with the standalone
// quantizer's single IEEE operations: m, the value of largest magnitude (the first in index order, which only matters
// when both signs reach the maximum: then the quad finds the first), iscale = -127 / m, q = round(iscale * x)
// saturated, d = 1 / iscale; a block whose maximum is 0 (or that holds no number) is zeros (iscale 0 makes every q 0:
// 0 * x is a zero or a NaN).  NaNs are never the maximum (fmaxf / fminf drop them).  Leaves the lane's int8 values in
// q (4 per dword, in v's order) and the sums of each four dwords in s16; returns d.
__device__ __forceinline__ float q8k_unit(const float (&v)[16][4], const int (&off)[16], uint32_t (&q)[16],
                                          int (&s16)[4]) {
#pragma clang fp contract(off)
  float hi = v[0][0], lo = v[0][0];
#pragma unroll
  for (int j = 0; j < 16; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) hi = fmaxf(hi, v[j][i]), lo = fminf(lo, v[j][i]);
  // the block's on its four lanes, on the bit patterns (as in q8k_waves): fabsf keeps a zero maximum +0, and a lane of
  // NaNs takes part as 0
  const float la = fabsf(fmaxf(hi, -lo));
  uint32_t mb = la == la ? __builtin_bit_cast(uint32_t, la) : 0u;
  mb = dpp_max_u32<0xb1, 0xf>(mb);
  mb = dpp_max_u32<0x4e, 0xf>(mb);
  const float amax = __builtin_bit_cast(float, mb);
  int sg = (hi == amax ? 1 : 0) | (-lo == amax ? 2 : 0);
  sg |= __builtin_amdgcn_update_dpp(0, sg, 0xb1, 0xf, 0xf, false);
  sg |= __builtin_amdgcn_update_dpp(0, sg, 0x4e, 0xf, 0xf, false);
  float m = sg == 2 ? -amax : amax;
  if (sg == 3) {  // uniform over the quad
    int key = 1024;  // 2 * index + sign of the lane's first value of magnitude amax
#pragma unroll
    for (int j = 15; j >= 0; j--)
#pragma unroll
      for (int i = 3; i >= 0; i--)
        if (fabsf(v[j][i]) == amax) key = 2 * (off[j] + i) + (v[j][i] < 0.0f ? 1 : 0);
    key = min(key, __builtin_amdgcn_update_dpp(0, key, 0xb1, 0xf, 0xf, false));
    key = min(key, __builtin_amdgcn_update_dpp(0, key, 0x4e, 0xf, 0xf, false));
    m = (key & 1) ? -amax : amax;
  }
  const bool nz = amax > 0.0f;
  const float iscale = nz ? -127.0f / m : 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) w |= (uint32_t)(round_sat_i8(iscale * v[j][i]) & 0xff) << (8 * i);
    q[j] = w;
  }
#pragma unroll
  for (int g = 0; g < 4; g++) {
    int s = 0;
#pragma unroll
    for (int j = 4 * g; j < 4 * g + 4; j++) s = sdot4((int)q[j], 0x01010101, s);
    s16[g] = s;
  }
  return nz ? 1.0f / iscale : 0.0f;
}

// One 32-value Q8_0 block held by one lane (quantize_block32 + the f16 scale, crates/inference-tensor/src/quantized/
// mod.rs:41-56, k_quants.rs:923-949, with the standalone quantizer's operations): v[0..8) are its values in order.
// Leaves the int8 values in q and returns the scale as the matvec reads it back (f16-rounded).
__device__ __forceinline__ float q8_0_unit_block(const float (*v)[4], uint32_t *q) {
#pragma clang fp contract(off)
  float amax = 0.0f;  // (the reference's fold(0, max(|v|)): a block of NaNs has d = 0)
#pragma unroll
  for (int j = 0; j < 8; j++)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j][0]), fabsf(v[j][1])), fmaxf(fabsf(v[j][2]), fabsf(v[j][3]))));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) w |= (uint32_t)(round_sat_i8(v[j][i] * id) & 0xff) << (8 * i);
    q[j] = w;
  }
  return f16_bits_to_f32(f32_to_f16_bits(d));
}

// ------------------------------------------------------------------------------------------------ Q4_K
struct unit_q4k {
  static constexpr int kType = QMM_TYPE_Q4K;
  static constexpr int kValuesPerUnit = 64;
  static constexpr int kActBlockBytes = 292;  // qmm_block_q8k
  static constexpr int kActBlockValues = 256;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 256 * 144; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 64); }

  struct W {
    u32x4 hdr, q0, q1;
  };
  struct A {
    uint32_t q[16];
    int b0, b1;
    float d;
  };

  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
    const int o = (u >> 2) * 144, c = u & 3;
    w.hdr = r.a16(o);
    w.q0 = r.a16(o + 16 + 32 * c);
    w.q1 = r.a16(o + 32 + 32 * c);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }

  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 2) * 292;
    const int c = u & 3;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const u32x4 v = ld_a4(p + 4 + 64 * c + 16 * i);
      a.q[4 * i + 0] = v.x;
      a.q[4 * i + 1] = v.y;
      a.q[4 * i + 2] = v.z;
      a.q[4 * i + 3] = v.w;
    }
    const uint32_t s01 = ld32(p + 260 + 8 * c), s23 = ld32(p + 264 + 8 * c);
    a.b0 = (int)(int16_t)(s01 & 0xffff) + (int)(int16_t)(s01 >> 16);
    a.b1 = (int)(int16_t)(s23 & 0xffff) + (int)(int16_t)(s23 >> 16);
    a.d = __builtin_bit_cast(float, ld32(p));
  }
  // the same registers from the f32 row x (16-byte aligned): values 64c .. 64c + 63 of block u / 4
  static __device__ __forceinline__ void quantize_a(const float *x, int u, A &a) {
    int off[16];
#pragma unroll
    for (int j = 0; j < 16; j++) off[j] = 64 * (u & 3) + 4 * j;
    float v[16][4];
    load_unit_f32(x + 256 * (int64_t)(u >> 2), off, v);
    int s[4];
    a.d = q8k_unit(v, off, a.q, s);
    a.b0 = s[0] + s[1];
    a.b1 = s[2] + s[3];
  }

  // 6-bit scales and mins of sub-blocks 2c, 2c+1 (get_scale_min_k4, quantized/utils.rs:119-129)
  static __device__ __forceinline__ void scales(const W &w, int c, int &sc0, int &sc1, int &m0, int &m1) {
    const int sh = 16 * (c & 1);
    const uint32_t Y = w.hdr.y >> sh, Z = w.hdr.z >> sh, Wd = w.hdr.w >> sh;
    if (c < 2) {
      sc0 = Y & 63;
      sc1 = (Y >> 8) & 63;
      m0 = Z & 63;
      m1 = (Z >> 8) & 63;
    } else {
      sc0 = (Wd & 15) | (((Y >> 6) & 3) << 4);
      sc1 = ((Wd >> 8) & 15) | (((Y >> 14) & 3) << 4);
      m0 = ((Wd >> 4) & 15) | (((Z >> 6) & 3) << 4);
      m1 = ((Wd >> 12) & 15) | (((Z >> 14) & 3) << 4);
    }
  }

  static __device__ __forceinline__ float dot(const W &w, const A &a, int u) {
    int sc0, sc1, m0, m1;
    scales(w, u & 3, sc0, sc1, m0, m1);
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      s0 = sdot4((int)(qw[k] & 0x0f0f0f0fu), (int)a.q[k], s0);
      s1 = sdot4((int)((qw[k] >> 4) & 0x0f0f0f0fu), (int)a.q[8 + k], s1);
    }
    const int i1 = sc0 * s0 + sc1 * s1;
    const int i2 = m0 * a.b0 + m1 * a.b1;
    const float d = f16_bits_to_f32(w.hdr.x & 0xffff), dmin = f16_bits_to_f32(w.hdr.x >> 16);
    return a.d * (d * (float)i1 - dmin * (float)i2);
  }
};

// ------------------------------------------------------------------------------------------------ Q6_K
struct unit_q6k {
  static constexpr int kType = QMM_TYPE_Q6K;
  static constexpr int kValuesPerUnit = 64;
  static constexpr int kActBlockBytes = 292;
  static constexpr int kActBlockValues = 256;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 256 * 210; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 64); }

  // Weight loads only fill registers; realignment and decoding happen in dot(), so a prefetched row does not
  // wait for its data when it is requested.
  struct W {
    u32x4 qa, qb, qh;      // the dwords covering 16 bytes at a 2-byte aligned address each
    uint32_t ea, eb, eh;   // and the dword after each
    uint32_t off;          // the unit's byte offset within those dwords: 0 or 2
    u32x2 sc;              // the dwords from the one holding the unit's first int8 scale (scales 8h .. 8h + 7)
    uint32_t se;           // and the dword holding the last when off = 2 (the second again when off = 0)
    uint32_t d;            // f16 bits
  };
  struct A {
    uint32_t q[16];
    int bs[4];
    float d;
  };

  static __device__ __forceinline__ void realign(const u32x4 &v, uint32_t e, uint32_t off, uint32_t out[4]) {
    out[0] = align_bytes(v.y, v.x, off);
    out[1] = align_bytes(v.z, v.y, off);
    out[2] = align_bytes(v.w, v.z, off);
    out[3] = align_bytes(e, v.w, off);
  }

  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
    const int sb = (u >> 2) * 210;
    const int h = (u >> 1) & 1, p = u & 1;
    w.off = r.mis(sb);
    const int a4 = sb - (int)w.off;
    w.qa = r.a4x16(a4 + 64 * h + 16 * p);
    w.ea = r.x4(a4 + 64 * h + 16 * p + 16);
    w.qb = r.a4x16(a4 + 64 * h + 32 + 16 * p);
    w.eb = r.x4(a4 + 64 * h + 32 + 16 * p + 16);
    w.qh = r.a4x16(a4 + 128 + 32 * h + 16 * p);
    w.eh = r.x4(a4 + 128 + 32 * h + 16 * p + 16);
    w.sc = r.x8(a4 + 192 + 8 * h);  // (8 scale bytes in 2 or 3 dwords: no dword past the block is read)
    w.se = r.x4(a4 + 192 + 8 * h + (w.off ? 8 : 4));
    w.d = r.x2(sb + 208);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }

  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p0 = row + (int64_t)(u >> 2) * 292;
    const int h = (u >> 1) & 1, p = u & 1;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4 v = ld_a4(p0 + 4 + 128 * h + 32 * q + 16 * p);
      a.q[4 * q + 0] = v.x;
      a.q[4 * q + 1] = v.y;
      a.q[4 * q + 2] = v.z;
      a.q[4 * q + 3] = v.w;
    }
    const u32x4 bs = ld_a4(p0 + 260 + 16 * h);  // bsums[8h .. 8h+8)
    const uint32_t bw[4] = {bs.x, bs.y, bs.z, bs.w};
#pragma unroll
    for (int q = 0; q < 4; q++) a.bs[q] = (int)(int16_t)(bw[q] >> (16 * p));  // bsums[8h + 2q + p]
    a.d = __builtin_bit_cast(float, ld32(p0));
  }
  // the same registers from the f32 row x (16-byte aligned)
  static __device__ __forceinline__ void quantize_a(const float *x, int u, A &a) {
    const int h = (u >> 1) & 1, p = u & 1;
    int off[16];
#pragma unroll
    for (int j = 0; j < 16; j++) off[j] = 128 * h + 32 * (j >> 2) + 16 * p + 4 * (j & 3);
    float v[16][4];
    load_unit_f32(x + 256 * (int64_t)(u >> 2), off, v);
    a.d = q8k_unit(v, off, a.q, a.bs);
  }

  static __device__ __forceinline__ float dot(const W &w, const A &a, int u) {
    uint32_t qa[4], qb[4], qh[4];
    realign(w.qa, w.ea, w.off, qa);
    realign(w.qb, w.eb, w.off, qb);
    realign(w.qh, w.eh, w.off, qh);
    const int p = u & 1;
    // scales 8h .. 8h + 7 as two dwords; scale q of this unit is byte 2q + p
    const uint32_t scw[2] = {align_bytes(w.sc.y, w.sc.x, w.off), align_bytes(w.se, w.sc.y, w.off)};
    int isum = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t *src = (q & 1) ? qb : qa;
      const int nsh = (q >> 1) * 4;
      int s = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t v = ((src[k] >> nsh) & 0x0f0f0f0fu) | (((qh[k] >> (2 * q)) & 0x03030303u) << 4);
        s = sdot4((int)v, (int)a.q[4 * q + k], s);
      }
      const int sc = (int)(int8_t)(scw[q >> 1] >> (16 * (q & 1) + 8 * p));
      isum += sc * (s - 32 * a.bs[q]);  // (q6 - 32) . q8 = q6 . q8 - 32 * bsum
    }
    return a.d * f16_bits_to_f32(w.d) * (float)isum;
  }
};

// ------------------------------------------------------------------------------------------------ Q8_0
// Fast path: rows of an even number of blocks, so every block pair starts dword aligned.
struct unit_q8_0 {
  static constexpr int kType = QMM_TYPE_Q8_0;
  static constexpr int kValuesPerUnit = 64;
  static constexpr int kActBlockBytes = 34;
  static constexpr int kActBlockValues = 32;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 32 * 34; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 64); }

  // activations: decoded at load (once per launch); weights: the 17 dwords of a block pair, decoded in dot()
  struct A {
    uint32_t qa[8], qb[8];
    float da, db;
  };
  struct W {
    uint32_t dw[17];
  };

  static __device__ __forceinline__ void load_raw(const uint8_t *p, uint32_t dw[17]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const u32x4 v = ld_a4(p + 16 * i);
      dw[4 * i] = v.x;
      dw[4 * i + 1] = v.y;
      dw[4 * i + 2] = v.z;
      dw[4 * i + 3] = v.w;
    }
    dw[16] = ld32(p + 64);
  }
  static __device__ __forceinline__ void decode(const uint32_t dw[17], A &a) {
    a.da = f16_bits_to_f32(dw[0] & 0xffff);
#pragma unroll
    for (int i = 0; i < 8; i++) a.qa[i] = align_bytes(dw[i + 1], dw[i], 2);
    a.db = f16_bits_to_f32(dw[8] >> 16);
#pragma unroll
    for (int i = 0; i < 8; i++) a.qb[i] = dw[9 + i];
  }

  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
    const int o = u * 68;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const u32x4 v = r.a4x16(o + 16 * i);
      w.dw[4 * i] = v.x;
      w.dw[4 * i + 1] = v.y;
      w.dw[4 * i + 2] = v.z;
      w.dw[4 * i + 3] = v.w;
    }
    w.dw[16] = r.x4(o + 64);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    uint32_t dw[17];
    load_raw(row + (int64_t)u * 68, dw);
    decode(dw, a);
  }
  // the same registers from the f32 row x (16-byte aligned): blocks 2u and 2u + 1
  static __device__ __forceinline__ void quantize_a(const float *x, int u, A &a) {
    int off[16];
#pragma unroll
    for (int j = 0; j < 16; j++) off[j] = 4 * j;
    float v[16][4];
    load_unit_f32(x + 64 * (int64_t)u, off, v);
    a.da = q8_0_unit_block(v, a.qa);
    a.db = q8_0_unit_block(v + 8, a.qb);
  }

  static __device__ __forceinline__ float dot(const W &wr, const A &a, int) {
    A w;
    decode(wr.dw, w);
    int sa = 0, sb = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      sa = sdot4((int)w.qa[i], (int)a.qa[i], sa);
      sb = sdot4((int)w.qb[i], (int)a.qb[i], sb);
    }
    // (sum_i as f32 * d_x) * d_y per block, k_quants.rs:997
    return (float)sa * w.da * a.da + (float)sb * w.db * a.db;
  }
};

// Q8_0 rows of an odd number of blocks: one block per unit, read with 16-bit loads (2-byte alignment).
struct unit_q8_0_odd {
  static constexpr int kType = QMM_TYPE_Q8_0;
  static constexpr int kValuesPerUnit = 32;
  static constexpr int kActBlockBytes = 34;
  static constexpr int kActBlockValues = 32;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 32 * 34; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 32); }

  struct A {
    uint32_t q[8];
    float d;
  };
  struct W {
    uint32_t h[17];  // the block's 17 16-bit words (weights: decoded in dot())
  };

  static __device__ __forceinline__ void load_raw(const uint8_t *p, uint32_t h[17]) {
#pragma unroll
    for (int i = 0; i < 17; i++) h[i] = ld16(p + 2 * i);
  }
  static __device__ __forceinline__ void decode(const uint32_t h[17], A &a) {
    a.d = f16_bits_to_f32(h[0]);
#pragma unroll
    for (int i = 0; i < 8; i++) a.q[i] = h[1 + 2 * i] | (h[2 + 2 * i] << 16);
  }
  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
#pragma unroll
    for (int i = 0; i < 17; i++) w.h[i] = r.x2(u * 34 + 2 * i);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    uint32_t h[17];
    load_raw(row + (int64_t)u * 34, h);
    decode(h, a);
  }
  static __device__ __forceinline__ float dot(const W &wr, const A &a, int) {
    A w;
    decode(wr.h, w);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = sdot4((int)w.q[i], (int)a.q[i], s);
    return (float)s * w.d * a.d;
  }
};

// ------------------------------------------------------------------------------------------------ Q4_0 / Q5_0
// The 32-value types with an offset (Q4_0: q - 8, k_quants.rs:432-449; Q5_0: q - 16, k_quants.rs:615-637) against
// Q8_0 activation blocks.  A block's integer dot is sum(q * a) - off * sum(a): the nibbles (and fifth bits) are
// dotted as unsigned bytes and the activation block's sum, taken once when the activation unit is loaded, removes
// the offset.  Scaling per block as the reference: (float)sumi * d_w * d_a.

// bits 0..3 of h moved to bit 4 of bytes 0..3
__device__ __forceinline__ uint32_t spread4_bit4(uint32_t h) { return ((h * 0x00204081u) & 0x01010101u) << 4; }

// sum(q * a) over one block: qs = the 16 nibble bytes as 4 dwords, qh = Q5_0's fifth bits (unused for Q4_0)
template <int T>
__device__ __forceinline__ int dot_b32(const uint32_t qs[4], uint32_t qh, const uint32_t a[8]) {
  int s = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    uint32_t lo = qs[k] & 0x0f0f0f0fu, hi = (qs[k] >> 4) & 0x0f0f0f0fu;
    if (T == QMM_TYPE_Q5_0) {
      lo |= spread4_bit4((qh >> (4 * k)) & 15u);
      hi |= spread4_bit4((qh >> (16 + 4 * k)) & 15u);
    }
    s = sdot4((int)lo, (int)a[k], s);
    s = sdot4((int)hi, (int)a[4 + k], s);
  }
  return s;
}

template <int T>
struct fmt_b32 {
  static constexpr int kOff = T == QMM_TYPE_Q5_0 ? 16 : 8;
  static constexpr int kBytes = T == QMM_TYPE_Q5_0 ? 22 : 18;
  static constexpr int kPairDwords = kBytes / 2;  // two blocks: 36 or 44 bytes
};

// Rows of an even number of blocks starting dword aligned: a unit is a block pair (64 values), read as dwords.
template <int T>
struct unit_b32 {
  using F = fmt_b32<T>;
  static constexpr int kType = T;
  static constexpr int kValuesPerUnit = 64;
  static constexpr int kActBlockBytes = 34;
  static constexpr int kActBlockValues = 32;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 32 * F::kBytes; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 64); }

  struct A {
    uint32_t qa[8], qb[8];
    float da, db;
    int sa, sb;  // sums of the two blocks' values
  };
  struct W {
    uint32_t dw[F::kPairDwords];
  };

  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
    const int o = u * (2 * F::kBytes);
#pragma unroll
    for (int i = 0; i + 4 <= F::kPairDwords; i += 4) {
      const u32x4 v = r.a4x16(o + 4 * i);
      w.dw[i] = v.x;
      w.dw[i + 1] = v.y;
      w.dw[i + 2] = v.z;
      w.dw[i + 3] = v.w;
    }
#pragma unroll
    for (int i = F::kPairDwords / 4 * 4; i < F::kPairDwords; i++) w.dw[i] = r.x4(o + 4 * i);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    typename unit_q8_0::A q;
    unit_q8_0::load_a(row, u, q);
    int sa = 0, sb = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      a.qa[i] = q.qa[i];
      a.qb[i] = q.qb[i];
      sa = sdot4((int)q.qa[i], 0x01010101, sa);
      sb = sdot4((int)q.qb[i], 0x01010101, sb);
    }
    a.da = q.da;
    a.db = q.db;
    a.sa = sa;
    a.sb = sb;
  }

  static __device__ __forceinline__ float dot(const W &w, const A &a, int) {
    uint32_t q0[4], q1[4], h0 = 0, h1 = 0;
    float d0, d1;
    if (T == QMM_TYPE_Q5_0) {
      // block 0: d bytes 0-1, qh 2-5, qs 6-21; block 1: d 22-23, qh 24-27, qs 28-43
      d0 = f16_bits_to_f32(w.dw[0] & 0xffff);
      h0 = align_bytes(w.dw[1], w.dw[0], 2);
#pragma unroll
      for (int i = 0; i < 4; i++) q0[i] = align_bytes(w.dw[i + 2], w.dw[i + 1], 2);
      d1 = f16_bits_to_f32(w.dw[5] >> 16);
      h1 = w.dw[6];
#pragma unroll
      for (int i = 0; i < 4; i++) q1[i] = w.dw[7 + i];
    } else {
      // block 0: d bytes 0-1, qs 2-17; block 1: d 18-19, qs 20-35
      d0 = f16_bits_to_f32(w.dw[0] & 0xffff);
#pragma unroll
      for (int i = 0; i < 4; i++) q0[i] = align_bytes(w.dw[i + 1], w.dw[i], 2);
      d1 = f16_bits_to_f32(w.dw[4] >> 16);
#pragma unroll
      for (int i = 0; i < 4; i++) q1[i] = w.dw[5 + i];
    }
    const int s0 = dot_b32<T>(q0, h0, a.qa) - F::kOff * a.sa;
    const int s1 = dot_b32<T>(q1, h1, a.qb) - F::kOff * a.sb;
    return (float)s0 * d0 * a.da + (float)s1 * d1 * a.db;
  }
};

// Any other row: one block per unit, read as 16-bit words (blocks are 2-byte aligned).
template <int T>
struct unit_b32_odd {
  using F = fmt_b32<T>;
  static constexpr int kType = T;
  static constexpr int kValuesPerUnit = 32;
  static constexpr int kActBlockBytes = 34;
  static constexpr int kActBlockValues = 32;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 32 * F::kBytes; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 32); }

  struct A {
    uint32_t q[8];
    float d;
    int s;
  };
  struct W {
    uint32_t h[F::kBytes / 2];
  };
  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
#pragma unroll
    for (int i = 0; i < F::kBytes / 2; i++) w.h[i] = r.x2(u * F::kBytes + 2 * i);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    typename unit_q8_0_odd::A q;
    unit_q8_0_odd::load_a(row, u, q);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      a.q[i] = q.q[i];
      s = sdot4((int)q.q[i], 0x01010101, s);
    }
    a.d = q.d;
    a.s = s;
  }
  static __device__ __forceinline__ float dot(const W &w, const A &a, int) {
    constexpr int o = T == QMM_TYPE_Q5_0 ? 3 : 1;  // first 16-bit word of qs
    uint32_t qs[4];
#pragma unroll
    for (int i = 0; i < 4; i++) qs[i] = w.h[o + 2 * i] | (w.h[o + 2 * i + 1] << 16);
    const uint32_t qh = T == QMM_TYPE_Q5_0 ? (w.h[1] | (w.h[2] << 16)) : 0u;
    const int s = dot_b32<T>(qs, qh, a.q) - F::kOff * a.s;
    return (float)s * f16_bits_to_f32(w.h[0]) * a.d;
  }
};

// ------------------------------------------------------------------------------------------------ Q5_K
// unit = a quarter super-block as for Q4_K (sub-blocks 2c, 2c+1) plus the 32 qh bytes, whose bits 2c and 2c + 1 are
// the two sub-blocks' fifth bits (k_quants.rs:2145-2232).  Super-blocks are 176 bytes, so 16-byte aligned rows stay
// aligned.
struct unit_q5k {
  static constexpr int kType = QMM_TYPE_Q5K;
  static constexpr int kValuesPerUnit = 64;
  static constexpr int kActBlockBytes = 292;
  static constexpr int kActBlockValues = 256;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 256 * 176; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 64); }

  struct W {
    u32x4 hdr, h0, h1, q0, q1;
  };
  using A = unit_q4k::A;

  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
    const int o = (u >> 2) * 176, c = u & 3;
    w.hdr = r.a16(o);
    w.h0 = r.a16(o + 16);
    w.h1 = r.a16(o + 32);
    w.q0 = r.a16(o + 48 + 32 * c);
    w.q1 = r.a16(o + 64 + 32 * c);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) { unit_q4k::load_a(row, u, a); }

  static __device__ __forceinline__ float dot(const W &w, const A &a, int u) {
    const int c = u & 3;
    int sc0, sc1, m0, m1;
    unit_q4k::W hw;
    hw.hdr = w.hdr;
    unit_q4k::scales(hw, c, sc0, sc1, m0, m1);
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    const uint32_t hb[8] = {w.h0.x, w.h0.y, w.h0.z, w.h0.w, w.h1.x, w.h1.y, w.h1.z, w.h1.w};
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t lo = (qw[k] & 0x0f0f0f0fu) | (((hb[k] >> (2 * c)) & 0x01010101u) << 4);
      const uint32_t hi = ((qw[k] >> 4) & 0x0f0f0f0fu) | (((hb[k] >> (2 * c + 1)) & 0x01010101u) << 4);
      s0 = sdot4((int)lo, (int)a.q[k], s0);
      s1 = sdot4((int)hi, (int)a.q[8 + k], s1);
    }
    const int i1 = sc0 * s0 + sc1 * s1;
    const int i2 = m0 * a.b0 + m1 * a.b1;
    const float d = f16_bits_to_f32(w.hdr.x & 0xffff), dmin = f16_bits_to_f32(w.hdr.x >> 16);
    return a.d * (d * (float)i1 - dmin * (float)i2);
  }
};

// ------------------------------------------------------------------------------------------------ IQ4_XS
// unit = sub-blocks 2c, 2c+1 of a 136-byte super-block: the 8-byte header and 32 bytes of table indices
// (crates/inference-quant/src/gguf/cpu_dot.rs:416-440).  Four indices at a time become table values with two
// byte permutes (entries 0-7 and 8-15) and a bitwise select on bit 3.
struct unit_iq4xs {
  static constexpr int kType = QMM_TYPE_IQ4_XS;
  static constexpr int kValuesPerUnit = 64;
  static constexpr int kActBlockBytes = 292;
  static constexpr int kActBlockValues = 256;
  static __host__ __device__ int64_t row_bytes(int64_t k) { return k / 256 * 136; }
  static __host__ __device__ int units(int64_t k) { return (int)(k / 64); }

  struct W {
    uint32_t h0, h1;  // d | scales_h << 16, scales_l
    u32x4 q0, q1;
  };
  using A = unit_q4k::A;

  template <class Src>
  static __device__ __forceinline__ void load_w(const Src &r, int u, W &w) {
    const int o = (u >> 2) * 136, c = u & 3;
    w.h0 = r.x4(o);
    w.h1 = r.x4(o + 4);
    w.q0 = r.a4x16(o + 8 + 32 * c);
    w.q1 = r.a4x16(o + 24 + 32 * c);
  }
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_w(row_ptr{row}, u, w); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) { unit_q4k::load_a(row, u, a); }

  // the IQ4_NL table (raw.rs:13-15) as int8 bytes: entries 0-3, 4-7, 8-11, 12-15
  static constexpr uint32_t kT0 = 0xBFAD9881u, kT1 = 0xF6EADDCFu, kT2 = 0x26190D01u, kT3 = 0x71594535u;

  // four 4-bit indices (one per byte) -> their table values
  static __device__ __forceinline__ uint32_t lookup(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kT1, kT0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kT3, kT2, sel);
    // byte selector 4 picks byte 0 of the first operand (0xff), selector 12 gives 0x00
    const uint32_t mask = __builtin_amdgcn_perm(0xffffffffu, 0u, (n & 0x08080808u) ^ 0x0c0c0c0cu);
    return (hi & mask) | (lo & ~mask);
  }

  static __device__ __forceinline__ float dot(const W &w, const A &a, int u) {
    const int c = u & 3;
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    int s[2] = {0, 0};
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t q = qw[4 * h + k];
        s[h] = sdot4((int)lookup(q & 0x0f0f0f0fu), (int)a.q[8 * h + k], s[h]);
        s[h] = sdot4((int)lookup((q >> 4) & 0x0f0f0f0fu), (int)a.q[8 * h + 4 + k], s[h]);
      }
    int ls[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int ib = 2 * c + h;
      ls[h] = (int)(((w.h1 >> (4 * ib)) & 15u) | (((w.h0 >> (16 + 2 * ib)) & 3u) << 4)) - 32;
    }
    // d = d_w * d_a, then d * (ls * sumi) per sub-block (cpu_dot.rs:426, 437)
    const float d = f16_bits_to_f32(w.h0 & 0xffff) * a.d;
    return d * (float)(ls[0] * s[0]) + d * (float)(ls[1] * s[1]);
  }
};

// ------------------------------------------------------------------------------------------------ tensor-core layout
// Activations of the tensor-core matvec entries (launch_mmvq_tc_quantize_*, launch_mmvq_tc_gguf_<t>_*_plain):
// Q8_K blocks without their bsums, {f32 d; int8 qs[256]}, 260 bytes per 256 values and rows K / 256 blocks apart,
// so b rows fit the reference's tensor-core scratch of 288 bytes per 256 values and 8-row half
// (crates/inference-quant/src/gguf/fast_mmvq.rs:92-93, 1903-1908).  The units sum the int8 values they need
// themselves (one v_dot4 against ones per 4 values, once per launch), so the integer dots are those of the
// decode layout.
__device__ __forceinline__ int byte_sum(const uint32_t *q, int n, int acc) {
  for (int i = 0; i < n; i++) acc = sdot4((int)q[i], 0x01010101, acc);
  return acc;
}

struct unit_q4k_tc : unit_q4k {
  static constexpr int kActBlockBytes = 260;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 2) * 260;
    const int c = u & 3;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const u32x4 v = ld_a4(p + 4 + 64 * c + 16 * i);
      a.q[4 * i + 0] = v.x;
      a.q[4 * i + 1] = v.y;
      a.q[4 * i + 2] = v.z;
      a.q[4 * i + 3] = v.w;
    }
    a.b0 = byte_sum(a.q, 8, 0);      // sub-block 2c: bsums[4c] + bsums[4c + 1]
    a.b1 = byte_sum(a.q + 8, 8, 0);  // sub-block 2c + 1
    a.d = __builtin_bit_cast(float, ld32(p));
  }
};

struct unit_q6k_tc : unit_q6k {
  static constexpr int kActBlockBytes = 260;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p0 = row + (int64_t)(u >> 2) * 260;
    const int h = (u >> 1) & 1, p = u & 1;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4 v = ld_a4(p0 + 4 + 128 * h + 32 * q + 16 * p);
      a.q[4 * q + 0] = v.x;
      a.q[4 * q + 1] = v.y;
      a.q[4 * q + 2] = v.z;
      a.q[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) a.bs[q] = byte_sum(a.q + 4 * q, 4, 0);  // bsums[8h + 2q + p]
    a.d = __builtin_bit_cast(float, ld32(p0));
  }
};

// ------------------------------------------------------------------------------------------------ Q8_1-slot layout
// Activations of the reference-named decode entries (launch_mmvq_gguf_quantize_q8_1_* and every matvec that reads
// them): the reference's Q8_1 scratch holds 36 bytes per 32 values (crates/inference-quant/src/gguf/fast_mmvq.rs:
// 17-18, 534-542), 288 per 256, and the quantizer cannot know which weight type will read it.  Each 256 values are
// one qmm_block_q8ks {f32 d; int8 qs[256]; int16 s32[8]; pad}: BlockQ8K::from_float's d and qs (bit-exact with the
// CPU quantizer of the K-quant types) and the sums of each 32 of the qs.  The super-block types read it as their CPU
// dot product does; the 32-value types (Q8_0, Q4_0, Q5_0), whose CPU dot products take Q8_0 blocks, read each 32
// values of it as a block with the scale d of its 256 (the per-block f32 scaling is unchanged).
constexpr int kSlotBytes = 288;

struct unit_q4k_s : unit_q4k {
  static constexpr int kActBlockBytes = kSlotBytes;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 2) * kSlotBytes;
    const int c = u & 3;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const u32x4 v = ld_a4(p + 4 + 64 * c + 16 * i);
      a.q[4 * i + 0] = v.x;
      a.q[4 * i + 1] = v.y;
      a.q[4 * i + 2] = v.z;
      a.q[4 * i + 3] = v.w;
    }
    const uint32_t s = ld32(p + 260 + 4 * c);  // sums of sub-blocks 2c, 2c + 1
    a.b0 = (int)(int16_t)(s & 0xffff);
    a.b1 = (int)(int16_t)(s >> 16);
    a.d = __builtin_bit_cast(float, ld32(p));
  }
};
struct unit_q5k_s : unit_q5k {
  static constexpr int kActBlockBytes = kSlotBytes;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) { unit_q4k_s::load_a(row, u, a); }
};
struct unit_iq4xs_s : unit_iq4xs {
  static constexpr int kActBlockBytes = kSlotBytes;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) { unit_q4k_s::load_a(row, u, a); }
};
// Q6_K's 16-value sums are not in the slot: the unit sums its int8 values itself (as the tensor-core unit does)
struct unit_q6k_s : unit_q6k {
  static constexpr int kActBlockBytes = kSlotBytes;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p0 = row + (int64_t)(u >> 2) * kSlotBytes;
    const int h = (u >> 1) & 1, p = u & 1;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4 v = ld_a4(p0 + 4 + 128 * h + 32 * q + 16 * p);
      a.q[4 * q + 0] = v.x;
      a.q[4 * q + 1] = v.y;
      a.q[4 * q + 2] = v.z;
      a.q[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) a.bs[q] = byte_sum(a.q + 4 * q, 4, 0);  // bsums[8h + 2q + p]
    a.d = __builtin_bit_cast(float, ld32(p0));
  }
};

// 32-value types: unit u (a block pair) is values 64 (u % 4) .. +64 of slot u / 4
struct unit_q8_0_s : unit_q8_0 {
  static constexpr int kActBlockBytes = kSlotBytes;
  static constexpr int kActBlockValues = 256;
  static __device__ __forceinline__ void load_qs(const uint8_t *p, uint32_t (&q)[8]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const u32x4 v = ld_a4(p + 16 * i);
      q[4 * i] = v.x, q[4 * i + 1] = v.y, q[4 * i + 2] = v.z, q[4 * i + 3] = v.w;
    }
  }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 2) * kSlotBytes;
    const int c = u & 3;
    load_qs(p + 4 + 64 * c, a.qa);
    load_qs(p + 36 + 64 * c, a.qb);
    a.da = a.db = __builtin_bit_cast(float, ld32(p));
  }
};
// one block per unit: values 32 (u % 8) .. +32 of slot u / 8
struct unit_q8_0_odd_s : unit_q8_0_odd {
  static constexpr int kActBlockBytes = kSlotBytes;
  static constexpr int kActBlockValues = 256;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 3) * kSlotBytes;
    unit_q8_0_s::load_qs(p + 4 + 32 * (u & 7), a.q);
    a.d = __builtin_bit_cast(float, ld32(p));
  }
};
template <int T>
struct unit_b32_s : unit_b32<T> {
  using A = typename unit_b32<T>::A;
  static constexpr int kActBlockBytes = kSlotBytes;
  static constexpr int kActBlockValues = 256;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 2) * kSlotBytes;
    const int c = u & 3;
    unit_q8_0_s::load_qs(p + 4 + 64 * c, a.qa);
    unit_q8_0_s::load_qs(p + 36 + 64 * c, a.qb);
    a.da = a.db = __builtin_bit_cast(float, ld32(p));
    const uint32_t s = ld32(p + 260 + 4 * c);  // sums of the two blocks
    a.sa = (int)(int16_t)(s & 0xffff);
    a.sb = (int)(int16_t)(s >> 16);
  }
};
template <int T>
struct unit_b32_odd_s : unit_b32_odd<T> {
  using A = typename unit_b32_odd<T>::A;
  static constexpr int kActBlockBytes = kSlotBytes;
  static constexpr int kActBlockValues = 256;
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    const uint8_t *p = row + (int64_t)(u >> 3) * kSlotBytes;
    unit_q8_0_s::load_qs(p + 4 + 32 * (u & 7), a.q);
    a.d = __builtin_bit_cast(float, ld32(p));
    a.s = (int)(int16_t)ld16(p + 260 + 2 * (u & 7));
  }
};

// ------------------------------------------------------------------------------------------------ unit choice

// activation layout of a decode launch
enum ActFmt { kActSlots = 0, kActQ8_0 = 1 };

constexpr bool is_b32(int t) { return t == QMM_TYPE_Q8_0 || t == QMM_TYPE_Q4_0 || t == QMM_TYPE_Q5_0; }

// The units of weight type T against layout F: `pairs` for rows the unit reads as block pairs (every row of the
// super-block types; 32-value rows of an even number of blocks, dword aligned), `odd` otherwise.
template <int T, int F>
struct decode_units;
template <> struct decode_units<QMM_TYPE_Q4K, kActSlots> { typedef unit_q4k_s pairs; typedef unit_q4k_s odd; };
template <> struct decode_units<QMM_TYPE_Q6K, kActSlots> { typedef unit_q6k_s pairs; typedef unit_q6k_s odd; };
template <> struct decode_units<QMM_TYPE_Q5K, kActSlots> { typedef unit_q5k_s pairs; typedef unit_q5k_s odd; };
template <> struct decode_units<QMM_TYPE_IQ4_XS, kActSlots> { typedef unit_iq4xs_s pairs; typedef unit_iq4xs_s odd; };
template <> struct decode_units<QMM_TYPE_Q8_0, kActSlots> { typedef unit_q8_0_s pairs; typedef unit_q8_0_odd_s odd; };
template <> struct decode_units<QMM_TYPE_Q8_0, kActQ8_0> { typedef unit_q8_0 pairs; typedef unit_q8_0_odd odd; };
template <> struct decode_units<QMM_TYPE_Q4_0, kActSlots> {
  typedef unit_b32_s<QMM_TYPE_Q4_0> pairs;
  typedef unit_b32_odd_s<QMM_TYPE_Q4_0> odd;
};
template <> struct decode_units<QMM_TYPE_Q4_0, kActQ8_0> {
  typedef unit_b32<QMM_TYPE_Q4_0> pairs;
  typedef unit_b32_odd<QMM_TYPE_Q4_0> odd;
};
template <> struct decode_units<QMM_TYPE_Q5_0, kActSlots> {
  typedef unit_b32_s<QMM_TYPE_Q5_0> pairs;
  typedef unit_b32_odd_s<QMM_TYPE_Q5_0> odd;
};
template <> struct decode_units<QMM_TYPE_Q5_0, kActQ8_0> {
  typedef unit_b32<QMM_TYPE_Q5_0> pairs;
  typedef unit_b32_odd<QMM_TYPE_Q5_0> odd;
};

// bytes of one activation row of stride_col_y blocks: 36-byte Q8_1 blocks (slots, 8 per 256 values) or 34-byte Q8_0
template <int F>
constexpr int64_t act_row_bytes(int stride_col_y) { return (int64_t)stride_col_y * (F == kActSlots ? 36 : 34); }

// Byte alignment the decode units need of a weight pointer: 16-byte loads for Q4_K / Q5_K, dword loads for IQ4_XS,
// 16-bit loads (or realigned dwords) for the rest.
constexpr uintptr_t weight_align(int type) {
  return type == QMM_TYPE_Q4K || type == QMM_TYPE_Q5K ? 16 : type == QMM_TYPE_IQ4_XS ? 4 : 2;
}

// Whether a 32-value row reads as block pairs: an even number of blocks per row, every weight pointer and row
// dword aligned, and (Q8_0 blocks) every activation pair too
template <int T, int F>
inline bool reads_pairs(int ncols_x, int stride_col_y, const void *vy, std::initializer_list<const void *> ws,
                 int64_t expert_stride = 0) {
  if (!is_b32(T)) return true;
  bool ok = ncols_x % 64 == 0 && expert_stride % 4 == 0;
  if (F == kActQ8_0) ok = ok && stride_col_y % 2 == 0 && (uintptr_t)vy % 4 == 0;
  for (const void *w : ws) ok = ok && (w == nullptr || (uintptr_t)w % 4 == 0);
  return ok;
}

#pragma clang fp contract(fast)
