// Int8 MFMA operand builders shared by the prefill matmul and the skinny (few-row) matmul: the two int8 weight
// planes that fold the K-quant sub-block scales into the MFMA operand, the MFMA wrappers and the 32x32 output
// layout.  Exactness: Q4_K sc (6 bit) = 8 sh + sl, so sc * q4 = 8 (sh * q4) + (sl * q4) with both planes <= 105;
// Q6_K w = sc * (q6 - 32) in [-4064, 4096] (and IQ4_XS's (ls - 32) * kv in [-4064, 4032]) = 256 wh + wl with wh in
// [-16, 16] and wl in [-128, 127] (split256).  Each superblock's integer dot is exact in int32.
#pragma once

#include "common.h"
#include "units.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef short s2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }
__device__ __forceinline__ v16f mfma_f16(v8h a, v8h b, v16f c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }

__device__ __forceinline__ uint32_t mul_bytes(uint32_t v, uint32_t s) {
  // four byte lanes times a small factor; every product < 256 so no lane carries into the next
  const us2 r = __builtin_bit_cast(us2, v) * (us2){(unsigned short)s, (unsigned short)s};
  return __builtin_bit_cast(uint32_t, r);
}

// v_permlane32_swap_b32 (gfx950): lanes 32..63 of lo trade places with lanes 0..31 of hi, so that afterwards lo
// holds lane half 0's lo in both halves of each lane pair and hi lane half 1's hi (device pass only: the builtin
// needs the gfx950 target)
__device__ __forceinline__ void swap_lane_halves(uint32_t &lo, uint32_t &hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto r = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
  lo = r[0];
  hi = r[1];
#endif
}

// The two int8 planes of four weights w in [-4224, 4095]: lo and hi hold w + 128 of weights (0, 2) and (1, 3) in
// their 16-bit lanes.  w + 128 = 256 wh + (wl + 128): wh is the high byte of the lane, wl its low byte less 128
// (the low byte with its top bit flipped, as int8), so each plane is one byte permute.
// (v_perm_b32 (S0, S1, sel): byte k of the result is byte sel_k of the eight bytes S1 (0..3), S0 (4..7); sel 12 = 0)
__device__ __forceinline__ void split256(s2 lo, s2 hi, v4i &b1, v4i &b2, int i) {
  const uint32_t l = __builtin_bit_cast(uint32_t, lo), h = __builtin_bit_cast(uint32_t, hi);
  b2[i] = (int)(__builtin_amdgcn_perm(h, l, 0x06020400u) ^ 0x80808080u);  // low bytes of l.x, h.x, l.y, h.y
  b1[i] = (int)__builtin_amdgcn_perm(h, l, 0x07030501u);                  // their high bytes
}

// Q6_K values q6 = ql | qh << 4 of four bytes (ql's low nibbles, the 2-bit fields of qh at bit hsh (even) of each
// byte) as 16-bit lanes: *lo = bytes 0 and 2, *hi = bytes 1 and 3
__device__ __forceinline__ void q6_lanes(uint32_t ql, uint32_t qh, int hsh, s2 &lo, s2 &hi) {
  const uint32_t b = (hsh <= 4 ? qh << (4 - hsh) : qh >> (hsh - 4)) & 0x30303030u;
  const uint32_t v6 = (ql & 0x0f0f0f0fu) | b;
  lo = __builtin_bit_cast(s2, __builtin_amdgcn_perm(0u, v6, 0x0c020c00u));
  hi = __builtin_bit_cast(s2, __builtin_amdgcn_perm(0u, v6, 0x0c030c01u));
}

// The Q4_K / Q5_K min term sum_j m_j * S_j goes through an f16 MFMA, exact in f32.  The activation sums of 32 values
// S_j (int16, |S| <= 4064) are not exact in f16, so each is split as S = 64 h + l, l in [0, 63], h in [-64, 63],
// both exact, and the weight side carries (64 m_j, m_j).  The halves come from the f16 bit patterns of 1024 + v
// (0x6400 + v for 0 <= v < 1024) less 1024 in packed f16 arithmetic.  For one dword of two sums (S_a low, S_b high):
// hpair = (f16 h_a, f16 h_b), lpair = (f16 l_a, f16 l_b).  The A fragment of sub-blocks (a, b, c, d) is
// (h_a, h_b, l_a, l_b, h_c, h_d, l_c, l_d) and the B fragment (64 m_a, 64 m_b, m_a, m_b, 64 m_c, 64 m_d, m_c, m_d).
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void s32_split(uint32_t sums, uint32_t &hpair, uint32_t &lpair) {
  const s2 h = (__builtin_bit_cast(s2, sums) >> (s2){6, 6}) + (s2){0x6440, 0x6440};  // 0x6400 + (h + 64)
  const uint32_t l = (sums & 0x003f003fu) | 0x64006400u;                              // 0x6400 + l
  hpair = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, h) - (h2){(_Float16)1088.0f, (_Float16)1088.0f});
  lpair = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, l) - (h2){(_Float16)1024.0f, (_Float16)1024.0f});
}
// the A fragment of four sub-blocks from their two dwords of sums
__device__ __forceinline__ v8h min_frag(uint32_t s01, uint32_t s23) {
  uint32_t f[4];
  s32_split(s01, f[0], f[1]);
  s32_split(s23, f[2], f[3]);
  return __builtin_bit_cast(v8h, (u32x4){f[0], f[1], f[2], f[3]});
}

// Row of 32x32 output register r of lane group g (v_mfma 32x32 D layout): 8 (r / 4) + 4 g + r % 4
__device__ __forceinline__ int out_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// ------------------------------------------------------------------------------------------ weight policies

// Q4_K: per lane (weight row n, lane group g), per superblock: 16 B header + 4 x 16 B of nibbles
// (qs[32c + 16g .. +16], c = 0..3) -> sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles).
struct wq4k {
  static constexpr int kBytes = 144;
  static constexpr int kPlanes = 2;
  static constexpr int kShift = 3;  // I1 = 8 * plane1 + plane2
  static constexpr bool kMin = true;
  static constexpr bool kDma = true;  // prefill stages activations by DMA (see mmq.hip)
  static constexpr int kLoads = 5;    // load() issues five 16-byte loads
  // activation chunk (16 values) of MFMA step j for lane half g: values 32 j + 16 g .. +16
  static __device__ __forceinline__ int chunk(int j, int g) { return 2 * j + g; }
  struct Raw {
    u32x4 hdr, q[4];
  };
  // superblock sb of the row at byte offset `row` of the resource
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t row, uint32_t sb, int g, Raw &r) {
    const uint32_t o = row + sb * kBytes;
    r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 16 + 32 * c + 16 * g, 0, 0);
  }
  // the same bytes of one superblock already in LDS, as 16-byte pieces PS bytes apart: piece k holds bytes
  // 16 k .. +16 (off, the superblock's start within its first dword, is 0: Q4_K superblocks are 16-byte aligned)
  static constexpr bool kLdsWeights = true;
  static constexpr int kLwTM = 2;  // the activation tile (32 kLwTM rows per wave) that takes weights from LDS
  template <int PS>
  static __device__ __forceinline__ void load_lds(const uint8_t *p, uint32_t, int g, Raw &r) {
    r.hdr = *(const u32x4 *)p;
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = *(const u32x4 *)(p + PS * (1 + 2 * c + g));
  }
  struct Prep {
    float d, dmin;
    v8h bmin;
  };
  // 6-bit scale of sub-block j, get_scale_min_k4 (quantized/utils.rs:119-129); unpacked where it is used, so
  // the eight scales are not all live at once
  static __device__ __forceinline__ uint32_t scale(const Raw &r, int j) {
    const uint32_t s[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
    auto byte = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    return j < 4 ? byte(j) & 63 : (byte(j + 4) & 0xf) | ((byte(j - 4) >> 6) << 4);
  }
  // S16: the A operand is the f16 sums of 16 values (`_q8k` tiles): k = 8g + 2i + h holds sub-block 4g + i's min m
  // for both of its halves.  Otherwise the sums of 32 split as 64 h + l (min_frag's order): k = 8g + 4 (i / 2) + i % 2
  // holds 64 m, two further on m.  Sub-block 4g + i's 6-bit min is byte(4 + i) & 63 (g = 0) or
  // (byte(8 + i) >> 4) | ((byte(4 + i) >> 6) << 4) (g = 1).
  template <bool S16 = false>
  static __device__ __forceinline__ void prepare(const Raw &r, int g, Prep &p) {
    const uint32_t s[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
    auto byte = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    p.d = f16_bits_to_f32(r.hdr.x & 0xffff);
    p.dmin = f16_bits_to_f32(r.hdr.x >> 16);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = byte(4 + i) & 63, hi = (byte(8 + i) >> 4) | ((byte(4 + i) >> 6) << 4);
      const uint32_t m = g ? hi : lo;
      if constexpr (S16) {
        const _Float16 mh = (_Float16)(float)m;
        p.bmin[2 * i] = mh;
        p.bmin[2 * i + 1] = mh;
      } else {
        p.bmin[4 * (i >> 1) + (i & 1)] = (_Float16)(float)(64 * m);
        p.bmin[4 * (i >> 1) + (i & 1) + 2] = (_Float16)(float)m;
      }
    }
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int j, v4i &b1, v4i &b2) {
    (void)p;
    const u32x4 q = r.q[j >> 1];
    const uint32_t sc = scale(r, j), sh = sc >> 3, sl = sc & 7;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t nib = (j & 1) ? ((w[i] >> 4) & 0x0f0f0f0fu) : (w[i] & 0x0f0f0f0fu);
      b1[i] = (int)mul_bytes(nib, sh);
      b2[i] = (int)mul_bytes(nib, sl);
    }
  }
};

// Q5_K (k_quants.rs:200-206, 2145-2232): Q4_K's header and nibbles plus qh[32], whose bit j of byte l is the fifth
// bit of value l of sub-block j's low or high half (32 j + l for j's nibble half).  q5 = nib + 16 h, so
// sc * q5 = 8 (sh * nib) + (sl * nib) + 16 (h * sc): the two Q4_K planes plus a third, h * sc <= 63.
struct wq5k {
  static constexpr int kBytes = 176;
  static constexpr int kPlanes = 3;
  static constexpr int kShift = 3;
  static constexpr bool kMin = true;
  static constexpr bool kDma = true;
  static constexpr int kLoads = 6;  // header, this lane's 16 qh bytes, four 16-byte nibble chunks
#ifndef QMM_Q5K_LW
#define QMM_Q5K_LW 1
#endif
  static constexpr bool kLdsWeights = QMM_Q5K_LW;
  static constexpr int kLwTM = 1;  // (three planes: 32-row activation tiles only)
  // activation chunk (16 values) of MFMA step j for lane half g: values 32 j + 16 g .. +16
  static __device__ __forceinline__ int chunk(int j, int g) { return 2 * j + g; }
  struct Raw {
    u32x4 hdr, qh, q[4];
  };
  // the same bytes of one superblock already in LDS, as 16-byte pieces PS bytes apart (superblocks 16-byte aligned)
  template <int PS>
  static __device__ __forceinline__ void load_lds(const uint8_t *p, uint32_t, int g, Raw &r) {
    r.hdr = *(const u32x4 *)p;
    r.qh = *(const u32x4 *)(p + PS * (1 + g));
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = *(const u32x4 *)(p + PS * (3 + 2 * c + g));
  }
  typedef wq4k::Prep Prep;
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t row, uint32_t sb, int g, Raw &r) {
    const uint32_t o = row + sb * kBytes;
    r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
    r.qh = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 16 + 16 * g, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 48 + 32 * c + 16 * g, 0, 0);
  }
  template <bool S16 = false>
  static __device__ __forceinline__ void prepare(const Raw &r, int g, Prep &p) {
    wq4k::Raw h;
    h.hdr = r.hdr;
    wq4k::prepare<S16>(h, g, p);
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int j, v4i &b1, v4i &b2, v4i &b3) {
    (void)p;
    wq4k::Raw h;
    h.hdr = r.hdr;
    const u32x4 q = r.q[j >> 1];
    const uint32_t sc = wq4k::scale(h, j), sh = sc >> 3, sl = sc & 7;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w}, qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t nib = (j & 1) ? ((w[i] >> 4) & 0x0f0f0f0fu) : (w[i] & 0x0f0f0f0fu);
      b1[i] = (int)mul_bytes(nib, sh);
      b2[i] = (int)mul_bytes(nib, sl);
      b3[i] = (int)mul_bytes((qh[i] >> j) & 0x01010101u, sc);
    }
  }
};

// Q6_K: per lane, per superblock: ql[64h + 32p + 16g ..+16], qh[32h + 16g ..+16] (h, p in {0,1}), the 8 scales
// sc[2j + g] and d.  Chunk j (32 values 32j..32j+31) covers h = j / 4, q = j % 4, l = 16g + (0..15).
struct wq6k {
  static constexpr int kBytes = 210;
  static constexpr int kPlanes = 2;
  static constexpr int kShift = 8;  // I = 256 * wh + wl (split256)
  static constexpr bool kMin = false;
  static constexpr bool kDma = false;
  static constexpr int kLoads = 6;  // at least six loads (16-byte ones; the 4-byte ones may merge)
  static constexpr bool kLdsWeights = true;
#ifndef QMM_Q6K_LW_TM
#define QMM_Q6K_LW_TM 4
#endif
  static constexpr int kLwTM = QMM_Q6K_LW_TM;
  // activation chunk (16 values) of MFMA step j for lane half g: values 32 j + 16 g .. +16
  static __device__ __forceinline__ int chunk(int j, int g) { return 2 * j + g; }
  // 16 bytes at a 2-byte aligned offset, kept as the five dwords that cover them: realigned only when used, so a
  // prefetch does not wait for its data at issue time
  struct Chunk {
    u32x4 v;
    uint32_t e;
  };
  struct Raw {
    Chunk ql[2][2], qh[2], sc;
    uint32_t off;  // the block's byte offset within its first dword: 0 or 2
    uint32_t d;
  };
  static __device__ __forceinline__ void ld16(rsrc_t rs, uint32_t a4, uint32_t x, Chunk &c) {
    c.v = __builtin_amdgcn_raw_buffer_load_b128(rs, a4 + x, 0, 0);
    c.e = __builtin_amdgcn_raw_buffer_load_b32(rs, a4 + x + 16, 0, 0);
  }
  static __device__ __forceinline__ void words(const Chunk &c, uint32_t off, uint32_t out[4]) {
    out[0] = align_bytes(c.v.y, c.v.x, off);
    out[1] = align_bytes(c.v.z, c.v.y, off);
    out[2] = align_bytes(c.v.w, c.v.z, off);
    out[3] = align_bytes(c.e, c.v.w, off);
  }
  // superblock sb of the row at byte offset `row` of the resource (210-byte blocks are 2-byte aligned)
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t row, uint32_t sb, int g, Raw &r) {
    const uint32_t o = row + sb * kBytes, off = o & 3, a4 = o - off;
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int p = 0; p < 2; p++) ld16(rs, a4, 64 * h + 32 * p + 16 * g, r.ql[h][p]);
      ld16(rs, a4, 128 + 32 * h + 16 * g, r.qh[h]);
    }
    ld16(rs, a4, 192, r.sc);  // the fifth dword may end past the last row: it then reads as 0, unused
    r.off = off;
    r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, o + 208, 0, 0);
  }
  // The same bytes from LDS, where the 224 bytes from the dword holding the superblock's first byte lie as 16-byte
  // pieces PS bytes apart (piece k: bytes 16 k .. +16 of that window); off = the superblock's start in the window
  template <int PS>
  static __device__ __forceinline__ void lds16(const uint8_t *p, int k, Chunk &c) {
    c.v = *(const u32x4 *)(p + PS * k);
    c.e = *(const uint32_t *)(p + PS * (k + 1));
  }
  template <int PS>
  static __device__ __forceinline__ void load_lds(const uint8_t *p, uint32_t off, int g, Raw &r) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int q = 0; q < 2; q++) lds16<PS>(p, 4 * h + 2 * q + g, r.ql[h][q]);
      lds16<PS>(p, 8 + 2 * h + g, r.qh[h]);
    }
    lds16<PS>(p, 12, r.sc);
    r.off = off;
    r.d = *(const uint16_t *)(p + PS * 13 + off);
  }
  struct Prep {
    int sc[8];
    float d;
    float dmin;  // unused: Q6_K has no min term
    v8h bmin;
    uint32_t ql[2][2][4], qh[2][4];  // realigned
  };
  static __device__ __forceinline__ void prepare(const Raw &r, int g, Prep &p) {
    uint32_t sc[4];
    words(r.sc, r.off, sc);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int idx = 2 * j + g;  // scale of values 16 (2j + g) .. +16
      p.sc[j] = (int)(int8_t)((sc[idx >> 2] >> (8 * (idx & 3))) & 0xff);
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int q = 0; q < 2; q++) words(r.ql[h][q], r.off, p.ql[h][q]);
      words(r.qh[h], r.off, p.qh[h]);
    }
    p.d = f16_bits_to_f32(r.d);
    p.dmin = 0.0f;
    p.bmin = (v8h){};
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int j, v4i &b1, v4i &b2) {
    (void)r;
    const int h = j >> 2, q = j & 3;
    const uint32_t *ql = p.ql[h][q & 1];
    const int nsh = (q >> 1) * 4;
    const s2 sc2 = {(short)p.sc[j], (short)p.sc[j]};
    const s2 c2 = (s2){128, 128} - (s2){32, 32} * sc2;  // (q6 - 32) sc + 128 = q6 sc + c2
#pragma unroll
    for (int i = 0; i < 4; i++) {
      s2 lo, hi;
      q6_lanes(ql[i] >> nsh, p.qh[h][i], 2 * q, lo, hi);
      split256(lo * sc2 + c2, hi * sc2 + c2, b1, b2, i);  // w + 128
    }
  }
};

// IQ4_XS (gguf/cpu_dot.rs:416-440): 136-byte superblock {f16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128]}; sub-block
// ib holds qs[16 ib .. +16], values 0..15 in the low nibbles and 16..31 in the high ones, each value
// kvalues_iq4nl[q] (int8) times the sub-block scale ls - 32 in [-32, 31].  w = (ls - 32) * kv in [-4064, 4032] splits
// as Q6_K's: 64 wh + wl, wl in [0, 63], wh in [-64, 63].
// The scale is folded into every weight byte, so an MFMA step may mix sub-blocks across lane halves: lane half g
// loads qs[64 g .. +64] (sub-blocks 4g .. 4g + 3) and step j takes nibble half j % 2 of sub-block 4g + j / 2, i.e.
// values 128 g + 16 j .. +16 -- activation chunk 8g + j instead of the other types' 2j + g.
struct wiq4xs {
  static constexpr int kBytes = 136;
  static constexpr int kPlanes = 2;
  static constexpr int kShift = 8;  // split256
  static constexpr bool kMin = false;
  static constexpr bool kDma = true;
  static constexpr int kLoads = 5;  // one 8-byte header load and four 16-byte loads (none adjacent to another)
#ifndef QMM_IQ4XS_LW_TM
#define QMM_IQ4XS_LW_TM 4
#endif
  static constexpr bool kLdsWeights = QMM_IQ4XS_LW_TM != 0;
  static constexpr int kLwTM = QMM_IQ4XS_LW_TM;
  static __device__ __forceinline__ int chunk(int j, int g) { return 8 * g + j; }
  struct Raw {
    u32x2 h;  // d | scales_h << 16, scales_l
    u32x4 q[4];
  };
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t row, uint32_t sb, int g, Raw &r) {
    const uint32_t o = row + sb * kBytes;
    r.h = __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 8 + 64 * g + 16 * c, 0, 0);
  }
  // The same bytes from LDS, where the superblock (4-byte aligned: it starts its window) lies as 16-byte pieces PS
  // bytes apart; a 16-byte chunk at byte 8 + 16 k is the back half of piece k and the front half of piece k + 1
  template <int PS>
  static __device__ __forceinline__ void load_lds(const uint8_t *p, uint32_t, int g, Raw &r) {
    r.h = *(const u32x2 *)p;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int k = 4 * g + c;
      const u32x2 lo = *(const u32x2 *)(p + PS * k + 8), hi = *(const u32x2 *)(p + PS * (k + 1));
      r.q[c] = (u32x4){lo.x, lo.y, hi.x, hi.y};
    }
  }
  struct Prep {
    int sc[4];  // ls - 32 of sub-blocks 4g .. 4g + 3
    float d, dmin;
    v8h bmin;
  };
  static __device__ __forceinline__ void prepare(const Raw &r, int g, Prep &p) {
#pragma unroll
    for (int i = 0; i < 4; i++) {  // iq4_xs_sub_scale (cpu_dot.rs:416-420)
      const int ib = 4 * g + i;
      p.sc[i] = (int)(((r.h.y >> (4 * ib)) & 15u) | (((r.h.x >> (16 + 2 * ib)) & 3u) << 4)) - 32;
    }
    p.d = f16_bits_to_f32(r.h.x & 0xffff);
    p.dmin = 0.0f;
    p.bmin = (v8h){};
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int j, v4i &b1, v4i &b2) {
    const u32x4 q = r.q[j >> 1];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const s2 sc2 = {(short)p.sc[j >> 1], (short)p.sc[j >> 1]};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t nib = (j & 1) ? ((w[i] >> 4) & 0x0f0f0f0fu) : (w[i] & 0x0f0f0f0fu);
      const uint32_t v = unit_iq4xs::lookup(nib);  // four int8 table values
      // bytes 0,2 and 1,3 sign-extended into 16-bit lanes, times the scale, plus 128
      const s2 lo = (__builtin_bit_cast(s2, v << 8) >> (s2){8, 8}) * sc2 + (s2){128, 128};
      const s2 hi = (__builtin_bit_cast(s2, v) >> (s2){8, 8}) * sc2 + (s2){128, 128};
      split256(lo, hi, b1, b2, i);
    }
  }
};

// ------------------------------------------------------------------------------------------ 16x16x64 policies

// Operands of v_mfma_i32_16x16x64_i8 for 16 weight rows x 16 activation rows.  Lane l = 16 kg + r holds weight row
// r (B column) and activation row r (A row); per 256-value superblock four MFMA steps t = 0..3 of 64 values, where
// lane group kg supplies 16 values.  The value order is chosen per weight type so that every 16-byte load a lane
// makes is used whole and every lane's 16 values share one sub-block scale; the activation side takes the same
// values, 16 contiguous bytes at act_offset(t, kg) of the activation superblock.
__device__ __forceinline__ v4i mfma16_i8(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4f mfma16_f16(v4h a, v4h b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Q4_K: step t = 2p + h takes nibble h of bytes qs[64p + 16kg .. +16], i.e. values 128p + 64(kg/2) + 32h +
// 16(kg%2) + (0..15) of sub-block 4p + 2(kg/2) + h.  Per lane per superblock: the 16-byte header and two 16-byte
// chunks of nibbles.
struct wq4k16 {
  static constexpr int kBytes = 144;
  static constexpr int kShift = 3;
  static constexpr bool kMin = true;
  struct Raw {
    u32x4 hdr, q[2];
  };
  static __device__ __forceinline__ uint32_t act_offset(int t, int kg) {
    return 128 * (t >> 1) + 64 * (kg >> 1) + 32 * (t & 1) + 16 * (kg & 1);
  }
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t row, uint32_t sb, int kg, Raw &r) {
    const uint32_t o = row + sb * kBytes;
    r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
#pragma unroll
    for (int p = 0; p < 2; p++) r.q[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 16 + 64 * p + 16 * kg, 0, 0);
  }
  struct Prep {
    uint32_t sh[4], sl[4];
    float d, dmin;
    v4h bmin;
  };
  static __device__ __forceinline__ void prepare(const Raw &r, int kg, Prep &p) {
    const uint32_t s[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
    auto byte = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    uint32_t sc[8], m[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {  // get_scale_min_k4 (quantized/utils.rs:119-129)
      sc[j] = j < 4 ? byte(j) & 63 : (byte(j + 4) & 0xf) | ((byte(j - 4) >> 6) << 4);
      m[j] = j < 4 ? byte(j + 4) & 63 : (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
    const bool hi = kg >= 2;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int j = 4 * (t >> 1) + (t & 1);  // sub-block for kg < 2; kg >= 2 adds 2
      const uint32_t v = hi ? sc[j + 2] : sc[j];
      p.sh[t] = v >> 3;
      p.sl[t] = v & 7;
    }
    p.d = f16_bits_to_f32(r.hdr.x & 0xffff);
    p.dmin = f16_bits_to_f32(r.hdr.x >> 16);
    // min-term B of sub-blocks 2kg, 2kg + 1: (64 m0, 64 m1, m0, m1), min_frag's order
    uint32_t m0 = m[0], m1 = m[1];
#pragma unroll
    for (int q = 1; q < 4; q++)
      if (kg == q) {
        m0 = m[2 * q];
        m1 = m[2 * q + 1];
      }
    p.bmin = (v4h){(_Float16)(float)(64 * m0), (_Float16)(float)(64 * m1), (_Float16)(float)m0, (_Float16)(float)m1};
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int t, v4i &b1, v4i &b2, int) {
    const u32x4 q = r.q[t >> 1];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t nib = (t & 1) ? ((w[i] >> 4) & 0x0f0f0f0fu) : (w[i] & 0x0f0f0f0fu);
      b1[i] = (int)mul_bytes(nib, p.sh[t]);
      b2[i] = (int)mul_bytes(nib, p.sl[t]);
    }
  }
};

// Q6_K: step t takes values 64t + 16kg + (0..15): low (t even) or high (t odd) nibbles of ql[64(t/2) + 16kg ..],
// the 2-bit fields 2q, q = 2(t%2) + kg/2, of qh[32(t/2) + 16(kg%2) ..], scale sc[4t + kg].
struct wq6k16 {
  static constexpr int kBytes = 210;
  static constexpr int kShift = 8;  // split256
  static constexpr bool kMin = false;
  // chunks kept unaligned until prepare(), as in wq6k
  typedef wq6k::Chunk Chunk;
  struct Raw {
    Chunk ql[2], qh[2], sc;
    uint32_t off;
    uint32_t d;
  };
  static __device__ __forceinline__ uint32_t act_offset(int t, int kg) { return 64 * t + 16 * kg; }
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t row, uint32_t sb, int kg, Raw &r) {
    const uint32_t o = row + sb * kBytes, off = o & 3, a4 = o - off;
#pragma unroll
    for (int x = 0; x < 2; x++) {
      wq6k::ld16(rs, a4, 64 * x + 16 * kg, r.ql[x]);
      wq6k::ld16(rs, a4, 128 + 32 * x + 16 * (kg & 1), r.qh[x]);
    }
    wq6k::ld16(rs, a4, 192, r.sc);  // the fifth dword may end past the last row: it then reads as 0, unused
    r.off = off;
    r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, o + 208, 0, 0);
  }
  struct Prep {
    int sc[4];
    float d, dmin;
    v4h bmin;
    uint32_t ql[2][4], qh[2][4];  // realigned
  };
  static __device__ __forceinline__ void prepare(const Raw &r, int kg, Prep &p) {
    uint32_t sc[4];
    wq6k::words(r.sc, r.off, sc);
#pragma unroll
    for (int t = 0; t < 4; t++)  // byte 4t + kg of the 16 scales = byte kg of dword t
      p.sc[t] = (int)(int8_t)((sc[t] >> (8 * kg)) & 0xff);
#pragma unroll
    for (int x = 0; x < 2; x++) {
      wq6k::words(r.ql[x], r.off, p.ql[x]);
      wq6k::words(r.qh[x], r.off, p.qh[x]);
    }
    p.d = f16_bits_to_f32(r.d);
    p.dmin = 0.0f;
    p.bmin = (v4h){};
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int t, v4i &b1, v4i &b2, int kg) {
    (void)r;
    const uint32_t *ql = p.ql[t >> 1], *qh = p.qh[t >> 1];
    const int nsh = 4 * (t & 1), hsh = 4 * (t & 1) + 2 * (kg >> 1);
    const s2 sc2 = {(short)p.sc[t], (short)p.sc[t]};
    const s2 c2 = (s2){128, 128} - (s2){32, 32} * sc2;  // (q6 - 32) sc + 128 = q6 sc + c2
#pragma unroll
    for (int i = 0; i < 4; i++) {
      s2 lo, hi;
      q6_lanes(ql[i] >> nsh, qh[i], hsh, lo, hi);
      split256(lo * sc2 + c2, hi * sc2 + c2, b1, b2, i);  // w + 128
    }
  }
};
