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
#pragma once

#include "common.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) {
    const uint8_t *p = row + (int64_t)(u >> 2) * 144;
    const int c = u & 3;
    w.hdr = ld_a16(p);
    w.q0 = ld_a16(p + 16 + 32 * c);
    w.q1 = ld_a16(p + 32 + 32 * c);
  }

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
    uint32_t sc[4];        // 16-bit loads holding the four int8 scales
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

  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) {
    const uint8_t *sb = row + (int64_t)(u >> 2) * 210;
    const int h = (u >> 1) & 1, p = u & 1;
    w.off = (uint32_t)((uintptr_t)sb & 3);
    const uint8_t *a4 = sb - w.off;
    w.qa = ld_a4(a4 + 64 * h + 16 * p);
    w.ea = ld32(a4 + 64 * h + 16 * p + 16);
    w.qb = ld_a4(a4 + 64 * h + 32 + 16 * p);
    w.eb = ld32(a4 + 64 * h + 32 + 16 * p + 16);
    w.qh = ld_a4(a4 + 128 + 32 * h + 16 * p);
    w.eh = ld32(a4 + 128 + 32 * h + 16 * p + 16);
#pragma unroll
    for (int q = 0; q < 4; q++) w.sc[q] = ld16(sb + 192 + 8 * h + 2 * q);
    w.d = ld16(sb + 208);
  }

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

  static __device__ __forceinline__ float dot(const W &w, const A &a, int u) {
    uint32_t qa[4], qb[4], qh[4];
    realign(w.qa, w.ea, w.off, qa);
    realign(w.qb, w.eb, w.off, qb);
    realign(w.qh, w.eh, w.off, qh);
    const int p = u & 1;
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
      const int sc = (int)(int8_t)(w.sc[q] >> (8 * p));
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

  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_raw(row + (int64_t)u * 68, w.dw); }
  static __device__ __forceinline__ void load_a(const uint8_t *row, int u, A &a) {
    uint32_t dw[17];
    load_raw(row + (int64_t)u * 68, dw);
    decode(dw, a);
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
  static __device__ __forceinline__ void load_w(const uint8_t *row, int u, W &w) { load_raw(row + (int64_t)u * 34, w.h); }
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
