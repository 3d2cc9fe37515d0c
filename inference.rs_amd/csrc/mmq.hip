// Prefill matmul for GGUF Q4_K / Q6_K / Q8_0 weights against activations quantized to Q8_K / Q8_0 blocks,
// on CDNA4 int8 MFMA (v_mfma_i32_32x32x32_i8), plus its expert-grouped MoE form.
//
// Replaces the llama.cpp-derived MMQ of crates/inference-quant/kernels/cuda/mmq_gguf (mmq_instance.cuh:8-268,
// mmq_gguf.cuh:3533-3875, 4020-4061).  Exactness: the reference CPU QMatMul sums integer block dots and scales
// each by f32 factors per 256 values (Q4_K, Q6_K) or per 32 (Q8_0).  The int8 MFMA reproduces the integer
// dots exactly; the per-32 / per-16 integer scales of the K-quants are folded into the weight operand, which
// then needs more than 8 bits, so it is split into two int8 planes:
//   Q4_K  sc (6 bit) = 8 sh + sl:   sc*q4 = 8 (sh*q4) + (sl*q4), both planes <= 105
//         min term  sum_j m_j * bsum32_j  through one f16 MFMA (bsums per 16 and 6-bit mins are exact in f16)
//   Q6_K  w = sc * (q6 - 32) in [-4096, 4064] = 64 wh + wl, wl in [0, 63], wh in [-64, 63]
//   Q8_0  one plane; the f32 scales apply per 32-value block (so this one is VALU-bound by design)
// Each superblock's integer result is exact in int32; the f32 epilogue per superblock mirrors the
// reference's d * dy * integer (k_quants.rs:1848-1928, 2518-2575).
//
// Tiling: a 256-thread workgroup owns BM = 128 activation rows x BN = 128 weight rows; wave w takes weight
// rows [32w, 32w+32) against all 128 activation rows (4 MFMA tiles of 32x32).  Per 256-value K step the
// workgroup stages the activation tile (int8 qs, f32 d, f16 bsums) in LDS; each wave streams its weight
// rows straight from HBM into registers and builds the B operands there.  A and B fragments use the same
// lane/byte -> k assignment, so the hardware's k order inside an MFMA does not matter.
#include "common.h"
#include "inferencequant.h"
#include "units.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef short s2 __attribute__((ext_vector_type(2)));

// waves per SIMD the K-quant prefill kernels are register-limited to
#ifndef QMM_MMQ_WAVES
#define QMM_MMQ_WAVES 2
#endif

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int TM = BM / 32;
constexpr int QS_STRIDE = 272;  // LDS row stride of the activation tile: 256 + 16 (bank spread)

struct ActTile {
  // global views of one channel of the prefill activation layout (include/inferencequant.h)
  const uint8_t *qs;     // [nsb][rows][256]
  const float *d;        // [nsb][rows]             (Q8_K)
  const int16_t *bsums;  // [nsb][rows][16]         (Q8_K)
  const uint16_t *d8;    // [nsb][rows][8] f16      (Q8_0)
  int64_t rows;
};

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }
__device__ __forceinline__ v16f mfma_f16(v8h a, v8h b, v16f c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }

__device__ __forceinline__ uint32_t mul_bytes(uint32_t v, uint32_t s) {
  // four byte lanes times a small factor; every product < 256 so no lane carries into the next
  const us2 r = __builtin_bit_cast(us2, v) * (us2){(unsigned short)s, (unsigned short)s};
  return __builtin_bit_cast(uint32_t, r);
}

// Row of 32x32 output register r of lane group g (v_mfma 32x32 D layout): 8 (r / 4) + 4 g + r % 4
__device__ __forceinline__ int out_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// ------------------------------------------------------------------------------------------ weight policies

// Q4_K: per lane (weight row n, lane group g), per superblock: 16 B header + 4 x 16 B of nibbles
// (qs[32c + 16g .. +16], c = 0..3) -> sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles).
struct wq4k {
  static constexpr int kBytes = 144;
  static constexpr int kShift = 3;  // I1 = 8 * plane1 + plane2
  static constexpr bool kMin = true;
  struct Raw {
    u32x4 hdr, q[4];
  };
  static __device__ __forceinline__ void load(const uint8_t *blk, int g, Raw &r) {
    r.hdr = ld_a16(blk);
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = ld_a16(blk + 16 + 32 * c + 16 * g);
  }
  struct Prep {
    uint32_t sh[8], sl[8];
    float d, dmin;
    v8h bmin;
  };
  static __device__ __forceinline__ void prepare(const Raw &r, int g, Prep &p) {
    const uint32_t s[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
    auto byte = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    uint32_t m[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {  // get_scale_min_k4 (quantized/utils.rs:119-129)
      uint32_t sc;
      if (j < 4) {
        sc = byte(j) & 63;
        m[j] = byte(j + 4) & 63;
      } else {
        sc = (byte(j + 4) & 0xf) | ((byte(j - 4) >> 6) << 4);
        m[j] = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
      }
      p.sh[j] = sc >> 3;
      p.sl[j] = sc & 7;
    }
    p.d = f16_bits_to_f32(r.hdr.x & 0xffff);
    p.dmin = f16_bits_to_f32(r.hdr.x >> 16);
    // B operand of the min-term MFMA: k = 8g + b <-> bsum16 index 8g + b <-> sub-block (8g + b) / 2
#pragma unroll
    for (int b = 0; b < 8; b++) p.bmin[b] = (_Float16)(float)m[4 * g + (b >> 1)];
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int j, v4i &b1, v4i &b2) {
    const u32x4 q = r.q[j >> 1];
    const uint32_t sh = p.sh[j], sl = p.sl[j];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t nib = (j & 1) ? ((w[i] >> 4) & 0x0f0f0f0fu) : (w[i] & 0x0f0f0f0fu);
      b1[i] = (int)mul_bytes(nib, sh);
      b2[i] = (int)mul_bytes(nib, sl);
    }
  }
};

// Q6_K: per lane, per superblock: ql[64h + 32p + 16g ..+16], qh[32h + 16g ..+16] (h, p in {0,1}), the 8 scales
// sc[2j + g] and d.  Chunk j (32 values 32j..32j+31) covers h = j / 4, q = j % 4, l = 16g + (0..15).
struct wq6k {
  static constexpr int kBytes = 210;
  static constexpr int kShift = 6;  // I = 64 * wh + wl
  static constexpr bool kMin = false;
  struct Raw {
    uint32_t ql[2][2][4], qh[2][4];
    uint32_t sc[4];
    uint32_t d;
  };
  static __device__ __forceinline__ void load(const uint8_t *blk, int g, Raw &r) {
    const uint32_t off = (uint32_t)((uintptr_t)blk & 3);
    const uint8_t *a4 = blk - off;
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int p = 0; p < 2; p++) unit_q6k::ld16_off(a4 + 64 * h + 32 * p + 16 * g, off, r.ql[h][p]);
      unit_q6k::ld16_off(a4 + 128 + 32 * h + 16 * g, off, r.qh[h]);
    }
    unit_q6k::ld16_off(a4 + 192, off, r.sc);
    r.d = ld16(blk + 208);
  }
  struct Prep {
    int sc[8];
    float d;
    float dmin;  // unused: Q6_K has no min term
    v8h bmin;
  };
  static __device__ __forceinline__ void prepare(const Raw &r, int g, Prep &p) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int idx = 2 * j + g;  // scale of values 16 (2j + g) .. +16
      p.sc[j] = (int)(int8_t)((r.sc[idx >> 2] >> (8 * (idx & 3))) & 0xff);
    }
    p.d = f16_bits_to_f32(r.d);
    p.dmin = 0.0f;
    p.bmin = (v8h){};
  }
  static __device__ __forceinline__ void planes(const Raw &r, const Prep &p, int j, v4i &b1, v4i &b2) {
    const int h = j >> 2, q = j & 3;
    const uint32_t *ql = r.ql[h][q & 1];
    const int nsh = (q >> 1) * 4;
    const s2 sc2 = {(short)p.sc[j], (short)p.sc[j]};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t v6 = ((ql[i] >> nsh) & 0x0f0f0f0fu) | (((r.qh[h][i] >> (2 * q)) & 0x03030303u) << 4);
      // bytes 0,2 and 1,3 in 16-bit lanes, minus 32, times the scale: w in [-4096, 4064]
      const s2 lo = (__builtin_bit_cast(s2, v6 & 0x00ff00ffu) - (s2){32, 32}) * sc2;
      const s2 hi = (__builtin_bit_cast(s2, (v6 >> 8) & 0x00ff00ffu) - (s2){32, 32}) * sc2;
      const uint32_t lo_u = __builtin_bit_cast(uint32_t, lo), hi_u = __builtin_bit_cast(uint32_t, hi);
      b2[i] = (int)((lo_u & 0x003f003fu) | ((hi_u & 0x003f003fu) << 8));
      const uint32_t lh = __builtin_bit_cast(uint32_t, lo >> (s2){6, 6}), hh = __builtin_bit_cast(uint32_t, hi >> (s2){6, 6});
      b1[i] = (int)((lh & 0x00ff00ffu) | ((hh & 0x00ff00ffu) << 8));
    }
  }
};

// ------------------------------------------------------------------------------------------ K-quant kernel

// One superblock of the activation tile (BMt rows x 256 values: int8 qs, f32 d, bsums as f16) moves
// global -> registers -> LDS; the caller double-buffers the LDS copy so the next superblock's loads are in
// flight during this one's MFMAs.  Rows past `mrows` stage as zeros.
template <int BMt>
struct StageQ8K {
  static constexpr int QCH = BMt * 16 / 256;  // 16-byte qs chunks per thread
  u32x4 qs[QCH];
  u32x4 bs;  // threads < 2 BMt: 8 bsums (half a row)
  float dy;  // threads < BMt

  __device__ __forceinline__ void load(const ActTile &a, int64_t sb, int64_t m0, int64_t mrows,
                                       const int32_t *__restrict__ row_map) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < QCH; it++) {
      const int i = it * 256 + tid;
      const int64_t m = m0 + (i >> 4);
      qs[it] = (u32x4){0, 0, 0, 0};
      if (m < mrows) {
        const int64_t src = row_map ? row_map[m] : m;
        qs[it] = ld_a16(a.qs + (sb * a.rows + src) * 256 + 16 * (i & 15));
      }
    }
    bs = (u32x4){0, 0, 0, 0};
    dy = 0.0f;
    if (tid < 2 * BMt) {
      const int64_t m = m0 + (tid >> 1);
      if (m < mrows) {
        const int64_t src = row_map ? row_map[m] : m;
        bs = ld_a16((const uint8_t *)(a.bsums + (sb * a.rows + src) * 16) + 16 * (tid & 1));
      }
    }
    if (tid < BMt) {
      const int64_t m = m0 + tid;
      dy = 0.0f;
      if (m < mrows) dy = a.d[sb * a.rows + (row_map ? row_map[m] : m)];
    }
  }

  __device__ __forceinline__ void store(uint8_t *s_qs, float *s_dy, _Float16 *s_bs) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < QCH; it++) {
      const int i = it * 256 + tid;
      *(u32x4 *)(s_qs + (i >> 4) * QS_STRIDE + 16 * (i & 15)) = qs[it];
    }
    if (tid < 2 * BMt) {
      // |bsum16| <= 16 * 127 = 2032: exact in f16
      const uint32_t w[4] = {bs.x, bs.y, bs.z, bs.w};
      v8h h;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        h[2 * i] = (_Float16)(float)(int16_t)(w[i] & 0xffff);
        h[2 * i + 1] = (_Float16)(float)(int16_t)(w[i] >> 16);
      }
      *(v8h *)(s_bs + (tid >> 1) * 16 + 8 * (tid & 1)) = h;
    }
    if (tid < BMt) s_dy[tid] = dy;
  }
};

// One workgroup: 4 waves x 32 weight rows (BN = 128) against BMt = 32 TM activation rows; wave w's lanes hold
// weight row n0 + 32w + (lane % 32) as the MFMA B column and TM 32x32 output tiles.
template <class WT, class Out, int TM>
__device__ __forceinline__ void mmq_kq_tile(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                            const ActTile &a, const int32_t *__restrict__ row_map, int64_t m0,
                                            int64_t mrows, int64_t n0, int64_t sb0, int64_t sb1,
                                            typename Out::T *__restrict__ dst, int64_t ldd,
                                            const int32_t *__restrict__ dst_rows, bool accumulate) {
  constexpr int BMt = 32 * TM;
  __shared__ __attribute__((aligned(16))) uint8_t s_qs[2][BMt * QS_STRIDE];
  __shared__ __attribute__((aligned(16))) float s_dy[2][BMt];
  __shared__ __attribute__((aligned(16))) _Float16 s_bs[2][BMt * 16];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int64_t n = n0 + 32 * wave + li;
  const int64_t n_ld = n < nrows_w ? n : nrows_w - 1;
  const uint8_t *wrow = W + n_ld * w_row_bytes;

  v16f fa[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) fa[t] = (v16f){};

  StageQ8K<BMt> st;
  typename WT::Raw raw, raw_next;
  WT::load(wrow + sb0 * WT::kBytes, g, raw);
  st.load(a, sb0, m0, mrows, row_map);
  st.store(s_qs[0], s_dy[0], s_bs[0]);
  __syncthreads();

  for (int64_t sb = sb0; sb < sb1; sb++) {
    const int buf = (int)((sb - sb0) & 1);
    const bool more = sb + 1 < sb1;
    if (more) {  // next superblock's weights and activations, in flight during this one's MFMAs
      WT::load(wrow + (sb + 1) * WT::kBytes, g, raw_next);
      st.load(a, sb + 1, m0, mrows, row_map);
    }
    typename WT::Prep p;
    WT::prepare(raw, g, p);
    v16i acc1[TM], acc2[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc1[t] = acc2[t] = (v16i){};
#pragma unroll
    for (int j = 0; j < 8; j++) {
      v4i b1, b2;
      WT::planes(raw, p, j, b1, b2);
#pragma unroll
      for (int t = 0; t < TM; t++) {
        const v4i av = *(const v4i *)(s_qs[buf] + (32 * t + li) * QS_STRIDE + 32 * j + 16 * g);
        acc1[t] = mfma_i8(av, b1, acc1[t]);
        acc2[t] = mfma_i8(av, b2, acc2[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < TM; t++) {
      v16f fmin = (v16f){};
      if (WT::kMin) {
        const v8h abs_ = *(const v8h *)(s_bs[buf] + (32 * t + li) * 16 + 8 * g);
        fmin = mfma_f16(abs_, p.bmin, fmin);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const v4f dy4 = *(const v4f *)(s_dy[buf] + 32 * t + 8 * q + 4 * g);  // rows 8q + 4g + 0..3
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int r = 4 * q + i;
          const int iv = (acc1[t][r] << WT::kShift) + acc2[t][r];
          float v = p.d * (float)iv;
          if (WT::kMin) v -= p.dmin * fmin[r];
          fa[t][r] += dy4[i] * v;
        }
      }
    }
    if (more) {
      st.store(s_qs[buf ^ 1], s_dy[buf ^ 1], s_bs[buf ^ 1]);
      raw = raw_next;
    }
    __syncthreads();
  }
  if (n >= nrows_w) return;
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int64_t m = m0 + 32 * t + out_row(r, g);
      if (m < mrows) {
        const int64_t drow = dst_rows ? dst_rows[m] : m;
        if (accumulate)  // split K: f32 partial sums meet in dst (zeroed first)
          __hip_atomic_fetch_add((float *)dst + drow * ldd + n, fa[t][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          Out::store(dst, drow * ldd + n, fa[t][r]);
      }
    }
}

// Zero rows of an f32 matrix before split-K partial sums land in it (a kernel, not a memset node, so the
// launch sequence can sit in a HIP graph).  rows_map != nullptr: zero rows rows_map[0..rows).
__global__ __launch_bounds__(256) void k_zero_rows(float *__restrict__ dst, int64_t rows, int64_t cols, int64_t ldd,
                                                   const int32_t *__restrict__ rows_map) {
  const int64_t r = blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows || c >= cols) return;
  const int64_t dr = rows_map ? rows_map[r] : r;
  dst[dr * ldd + c] = 0.0f;
}

// ------------------------------------------------------------------------------------------ Q8_0 kernel

// Q8_0 weights against Q8_0 activations: one MFMA per 32-value block, scaled in f32 per block as
// k_quants.rs:982-999 does ((sum as f32 * d_w) * d_a, summed over blocks).
template <class Out>
__device__ __forceinline__ void mmq_q8_0_tile(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                              int64_t nblk_w, const ActTile &a, int64_t m0, int64_t mrows, int64_t n0,
                                              int64_t nsb, typename Out::T *__restrict__ dst, int64_t ldd,
                                              const int32_t *__restrict__ dst_rows) {
  __shared__ __attribute__((aligned(16))) uint8_t s_qs[BM * QS_STRIDE];
  __shared__ float s_da[BM * 9];  // 8 block scales per row (stride 9 against bank conflicts)

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int64_t n = n0 + 32 * wave + li;
  const int64_t n_ld = n < nrows_w ? n : nrows_w - 1;
  const uint8_t *wrow = W + n_ld * w_row_bytes;

  v16f fa[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) fa[t] = (v16f){};

  for (int64_t sb = 0; sb < nsb; sb++) {
    uint32_t wq[8][4];
    float dw[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int64_t blk = sb * 8 + j;
      if (blk < nblk_w) {
        const uint8_t *p = wrow + blk * 34;
        dw[j] = f16_bits_to_f32(ld16(p));
        const uint8_t *q = p + 2 + 16 * g;
        const uint32_t off = (uint32_t)((uintptr_t)q & 3);
        unit_q6k::ld16_off(q - off, off, wq[j]);
      } else {
        dw[j] = 0.0f;
        wq[j][0] = wq[j][1] = wq[j][2] = wq[j][3] = 0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < BM * 16 / 256; it++) {
      const int i = it * 256 + tid;
      const int row = i >> 4, c = i & 15;
      const int64_t m = m0 + row;
      u32x4 v = {0, 0, 0, 0};
      if (m < mrows) v = ld_a16(a.qs + (sb * a.rows + m) * 256 + 16 * c);
      *(u32x4 *)(s_qs + row * QS_STRIDE + 16 * c) = v;
    }
#pragma unroll
    for (int it = 0; it < BM * 8 / 256; it++) {
      const int i = it * 256 + tid;
      const int row = i >> 3, j = i & 7;
      const int64_t m = m0 + row;
      s_da[row * 9 + j] = m < mrows ? f16_bits_to_f32(a.d8[(sb * a.rows + m) * 8 + j]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const v4i b = {(int)wq[j][0], (int)wq[j][1], (int)wq[j][2], (int)wq[j][3]};
#pragma unroll
      for (int t = 0; t < TM; t++) {
        const v4i av = *(const v4i *)(s_qs + (32 * t + li) * QS_STRIDE + 32 * j + 16 * g);
        const v16i acc = mfma_i8(av, b, (v16i){});
#pragma unroll
        for (int r = 0; r < 16; r++) fa[t][r] += ((float)acc[r] * dw[j]) * s_da[(32 * t + out_row(r, g)) * 9 + j];
      }
    }
  }
  if (n >= nrows_w) return;
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int64_t m = m0 + 32 * t + out_row(r, g);
      if (m < mrows) {
        const int64_t drow = dst_rows ? dst_rows[m] : m;
        Out::store(dst, drow * ldd + n, fa[t][r]);
      }
    }
}

// ------------------------------------------------------------------------------------------ kernels

// Workgroups are numbered so that the BM-row tiles sharing one weight tile are consecutive, then spread over
// the 8 XCDs (dispatch assigns workgroup i to XCD i % 8): each XCD's L2 sees whole weight tiles.
__device__ __forceinline__ void tile_of(int64_t mtiles, int64_t ntiles, int64_t splits, int64_t &mt, int64_t &nt,
                                        int64_t &split) {
  const int64_t total = mtiles * ntiles * splits;
  const int64_t b = blockIdx.x;
  int64_t id = b;
  if (total % 8 == 0) id = (b % 8) * (total / 8) + b / 8;
  split = id % splits;
  const int64_t tile = id / splits;
  mt = tile % mtiles;
  nt = tile / mtiles;
}

ActTile act_tile(int wtype, const void *y, int64_t rows, int64_t nsb) {
  ActTile a;
  a.qs = (const uint8_t *)y;
  a.rows = rows;
  const uint8_t *tail = (const uint8_t *)y + nsb * rows * 256;
  a.d = (const float *)tail;
  a.bsums = (const int16_t *)(tail + nsb * rows * 4);
  a.d8 = (const uint16_t *)tail;
  (void)wtype;
  return a;
}

// grid: tiles x splits; split s of a tile sums superblocks [s * per, min((s + 1) * per, nsb)) into dst
template <class WT, class Out, int TMv>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(QMM_MMQ_WAVES))) void k_mmq_kq(
    const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes, ActTile a, int64_t mrows, int64_t nsb,
    int64_t splits, typename Out::T *__restrict__ dst, int64_t ldd) {
  constexpr int BMt = 32 * TMv;
  int64_t mt, nt, split;
  tile_of((mrows + BMt - 1) / BMt, (nrows_w + BN - 1) / BN, splits, mt, nt, split);
  const int64_t per = (nsb + splits - 1) / splits;
  const int64_t sb0 = split * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  if (sb0 >= sb1) return;
  mmq_kq_tile<WT, Out, TMv>(W, nrows_w, w_row_bytes, a, nullptr, mt * BMt, mrows, nt * BN, sb0, sb1, dst, ldd,
                            nullptr, splits > 1);
}

template <class Out>
__global__ __launch_bounds__(256) void k_mmq_q8_0(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                                  int64_t nblk_w, ActTile a, int64_t mrows, int64_t nsb,
                                                  typename Out::T *__restrict__ dst, int64_t ldd) {
  int64_t mt, nt, split;
  tile_of((mrows + BM - 1) / BM, (nrows_w + BN - 1) / BN, 1, mt, nt, split);
  mmq_q8_0_tile<Out>(W, nrows_w, w_row_bytes, nblk_w, a, mt * BM, mrows, nt * BN, nsb, dst, ldd, nullptr);
}

// Expert-grouped: grid (n tiles, m tiles of the largest expert, experts).  Expert e's rows of `a` are
// [bounds[e], bounds[e+1]); its weights start at W + e * expert_bytes; row m is written to dst row ids_dst[m].
template <class WT, int TMv>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(QMM_MMQ_WAVES))) void k_mmq_kq_moe(const uint8_t *__restrict__ W, int64_t expert_bytes,
                                                    int64_t nrows_w, int64_t w_row_bytes, ActTile a,
                                                    const int32_t *__restrict__ bounds,
                                                    const int32_t *__restrict__ ids_dst, int64_t nsb, int64_t splits,
                                                    float *__restrict__ dst, int64_t ldd) {
  const int64_t e = blockIdx.z;
  const int64_t m0 = bounds[e] + (int64_t)blockIdx.y * (32 * TMv), m1 = bounds[e + 1];
  if (m0 >= m1) return;  // uniform over the workgroup
  const int64_t split = blockIdx.x % splits, per = (nsb + splits - 1) / splits;
  const int64_t sb0 = split * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  if (sb0 >= sb1) return;
  mmq_kq_tile<WT, out_f32, TMv>(W + e * expert_bytes, nrows_w, w_row_bytes, a, nullptr, m0, m1,
                                (int64_t)(blockIdx.x / splits) * BN, sb0, sb1, dst, ldd, ids_dst, splits > 1);
}

__global__ __launch_bounds__(256) void k_mmq_q8_0_moe(const uint8_t *__restrict__ W, int64_t expert_bytes,
                                                      int64_t nrows_w, int64_t w_row_bytes, int64_t nblk_w, ActTile a,
                                                      const int32_t *__restrict__ bounds,
                                                      const int32_t *__restrict__ ids_dst, int64_t nsb,
                                                      float *__restrict__ dst, int64_t ldd) {
  const int64_t e = blockIdx.z;
  const int64_t m0 = bounds[e] + (int64_t)blockIdx.y * BM, m1 = bounds[e + 1];
  if (m0 >= m1) return;
  mmq_q8_0_tile<out_f32>(W + e * expert_bytes, nrows_w, w_row_bytes, nblk_w, a, m0, m1, (int64_t)blockIdx.x * BN, nsb,
                         dst, ldd, ids_dst);
}

bool check_mmq(const char *who, int type, const void *x, int64_t ncols_x, int64_t nrows_x, int64_t stride_row_x) {
  const int64_t bs = (int64_t)qmm_block_size(type);
  if (ncols_x <= 0 || nrows_x <= 0 || ncols_x % bs != 0 || stride_row_x < ncols_x / bs) {
    qmm_set_error("%s: ncols_x=%lld nrows_x=%lld stride_row_x=%lld", who, (long long)ncols_x, (long long)nrows_x,
                  (long long)stride_row_x);
    return false;
  }
  if (type == QMM_TYPE_Q4K && ((uintptr_t)x % 16 != 0)) {
    qmm_set_error("%s: Q4_K weights must be 16-byte aligned", who);
    return false;
  }
  if ((uintptr_t)x % 2 != 0) {
    qmm_set_error("%s: weights must be 2-byte aligned", who);
    return false;
  }
  return true;
}

// K splits so that tiles x splits fills every CU twice over, each split keeping at least 4 superblocks;
// only for f32 outputs (the partial sums meet through f32 atomics).
int64_t k_splits(int64_t tiles, int64_t nsb, bool f32_out) {
  if (!f32_out) return 1;
  const int64_t want = 2 * qmm_device_cus();
  int64_t s = 1;
  while (tiles * s < want && nsb / (s * 2) >= 4) s *= 2;
  return s;
}

template <class WT, class Out>
void launch_kq(const uint8_t *w, int64_t nrows_x, int64_t w_row_bytes, const ActTile &a, int64_t ncols_y, int64_t nsb,
               typename Out::T *d, int64_t ldd, hipStream_t s) {
  const int64_t ntiles = (nrows_x + BN - 1) / BN;
  const int tm = ncols_y <= 32 ? 1 : 2;  // 32 activation rows per wave when that covers the batch, else 64
  const int64_t tiles = ((ncols_y + 32 * tm - 1) / (32 * tm)) * ntiles;
  const int64_t splits = k_splits(tiles, nsb, sizeof(typename Out::T) == 4);
  if (splits > 1)
    k_zero_rows<<<dim3((unsigned)((nrows_x + 255) / 256), (unsigned)ncols_y), 256, 0, s>>>((float *)d, ncols_y, nrows_x,
                                                                                          ldd, nullptr);
  const dim3 grid((unsigned)(tiles * splits));
  if (tm == 1) k_mmq_kq<WT, Out, 1><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd);
  else k_mmq_kq<WT, Out, 2><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd);
}

template <class Out>
void mmq_plain(int type, const void *x, const void *y, void *dst, int64_t ncols_x, int64_t nrows_x, int64_t ncols_y,
               int64_t stride_row_x, int64_t ldd, hipStream_t s) {
  const int64_t nsb = (ncols_x + 255) / 256;
  const int64_t w_row_bytes = stride_row_x * (int64_t)qmm_type_size(type);
  const ActTile a = act_tile(type, y, ncols_y, nsb);
  typename Out::T *d = (typename Out::T *)dst;
  const uint8_t *w = (const uint8_t *)x;
  switch (type) {
    case QMM_TYPE_Q4K: launch_kq<wq4k, Out>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, s); break;
    case QMM_TYPE_Q6K: launch_kq<wq6k, Out>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, s); break;
    default: {
      const dim3 grid((unsigned)(((ncols_y + BM - 1) / BM) * ((nrows_x + BN - 1) / BN)));
      k_mmq_q8_0<Out><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, ncols_x / 32, a, ncols_y, nsb, d, ldd);
    }
  }
}

void mmq(int type, void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x, int64_t nrows_x,
         int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int type_dst, void *stream, const char *who) {
  (void)tmp_fixup;
  if (!check_mmq(who, type, x, ncols_x, nrows_x, stride_row_x)) return;
  if (ncols_y < 0 || stride_col_dst < nrows_x) {
    qmm_set_error("%s: ncols_y=%lld stride_col_dst=%lld", who, (long long)ncols_y, (long long)stride_col_dst);
    return;
  }
  if (ncols_y == 0) return;
  hipStream_t s = (hipStream_t)stream;
  switch (type_dst) {
    case QMM_TYPE_F32: mmq_plain<out_f32>(type, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, s); break;
    case QMM_TYPE_F16: mmq_plain<out_f16>(type, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, s); break;
    case QMM_TYPE_BF16: mmq_plain<out_bf16>(type, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, s); break;
    default: qmm_set_error("%s: type_dst=%d (0 f32, 1 f16, 30 bf16)", who, type_dst);
  }
}

void mmq_moe(int type, const void *x, const void *y, const int32_t *ids_dst, const int32_t *bounds, void *dst,
             int64_t ncols_x, int64_t nrows_x, int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst,
             int64_t num_experts, int64_t ncols_max, void *stream, const char *who) {
  if (!check_mmq(who, type, x, ncols_x, nrows_x, stride_row_x)) return;
  if (num_experts <= 0 || ncols_max < 0 || ncols_dst < 0 || stride_col_dst < nrows_x || num_experts > 65535) {
    qmm_set_error("%s: num_experts=%lld ncols_max=%lld ncols_dst=%lld stride_col_dst=%lld", who,
                  (long long)num_experts, (long long)ncols_max, (long long)ncols_dst, (long long)stride_col_dst);
    return;
  }
  if (ncols_max == 0 || ncols_dst == 0) return;
  const int64_t nsb = (ncols_x + 255) / 256;
  const int64_t w_row_bytes = stride_row_x * (int64_t)qmm_type_size(type);
  const int64_t expert_bytes = nrows_x * w_row_bytes;
  const ActTile a = act_tile(type, y, ncols_dst, nsb);
  const dim3 grid((unsigned)((nrows_x + BN - 1) / BN), (unsigned)((ncols_max + BM - 1) / BM), (unsigned)num_experts);
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *w = (const uint8_t *)x;
  float *d = (float *)dst;
  const bool small = ncols_max <= 32;
  const int64_t ntiles = (nrows_x + BN - 1) / BN;
  const int64_t mt = small ? (ncols_max + 31) / 32 : (ncols_max + 63) / 64;
  // expected work: about ncols_dst / (32 tm) row tiles per n tile over all experts
  const int64_t busy = ntiles * (small ? (ncols_dst + 31) / 32 : (ncols_dst + 63) / 64);
  const int64_t splits = type == QMM_TYPE_Q8_0 ? 1 : k_splits(busy, nsb, true);
  if (splits > 1)
    k_zero_rows<<<dim3((unsigned)((nrows_x + 255) / 256), (unsigned)ncols_dst), 256, 0, s>>>(d, ncols_dst, nrows_x,
                                                                                            stride_col_dst, ids_dst);
  const dim3 gridk((unsigned)(ntiles * splits), (unsigned)mt, (unsigned)num_experts);
  switch (type) {
    case QMM_TYPE_Q4K:
      if (small)
        k_mmq_kq_moe<wq4k, 1><<<gridk, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                                    splits, d, stride_col_dst);
      else
        k_mmq_kq_moe<wq4k, 2><<<gridk, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                                    splits, d, stride_col_dst);
      break;
    case QMM_TYPE_Q6K:
      if (small)
        k_mmq_kq_moe<wq6k, 1><<<gridk, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                                    splits, d, stride_col_dst);
      else
        k_mmq_kq_moe<wq6k, 2><<<gridk, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                                    splits, d, stride_col_dst);
      break;
    default:
      k_mmq_q8_0_moe<<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, ncols_x / 32, a, bounds, ids_dst, nsb,
                                          d, stride_col_dst);
  }
}

}  // namespace

#define QMM_DEFINE_MMQ(t, TYPE)                                                                                    \
  void launch_mmq_gguf_##t(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,             \
                           int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int cc, \
                           int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream) {                    \
    (void)cc, (void)nsm, (void)smpbo, (void)warp_size;                                                             \
    mmq(TYPE, tmp_fixup, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, type_dst, stream,     \
        "mmq_" #t);                                                                                                \
  }                                                                                                                \
  void launch_mmq_gguf_##t##_moe(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,           \
                                 const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,        \
                                 int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst,                  \
                                 int64_t num_experts, int64_t ncols_max, int cc, int nsm, int64_t smpbo,           \
                                 int warp_size, void *stream) {                                                    \
    (void)tmp_fixup, (void)cc, (void)nsm, (void)smpbo, (void)warp_size;                                            \
    mmq_moe(TYPE, x, y, ids_dst, expert_bounds, dst, ncols_x, nrows_x, ncols_dst, stride_row_x, stride_col_dst,    \
            num_experts, ncols_max, stream, "mmq_" #t "_moe");                                                     \
  }

extern "C" {
QMM_DEFINE_MMQ(q8_0, QMM_TYPE_Q8_0)
QMM_DEFINE_MMQ(q4_k, QMM_TYPE_Q4K)
QMM_DEFINE_MMQ(q6_k, QMM_TYPE_Q6K)
}
