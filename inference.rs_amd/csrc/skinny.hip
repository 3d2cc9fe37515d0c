// Few-row matmul for Q4_K / Q6_K weights on int8 MFMA: up to 32 activation rows against a weight matrix
// streamed once from HBM.  Serves the decode matvec at b >= 2 (the reference's tensor-core matvec,
// mmvq_tc_k.cuh, fast_mmvq.rs:1897-2126, and its plain launcher at b <= 8) and any matmul whose activation side
// is at most 32 rows (the expert-grouped prefill at a handful of tokens per expert).
//
// Two forms.  32x32x32: a workgroup owns 32 (or 16) weight rows and all activation rows; its 4 or 8 waves split
// the superblocks of K, so every weight byte is loaded by exactly one wave, straight into registers, two
// superblocks ahead.  16x16x64 (narrower weights, at most 16 activation rows): 16 weight rows per workgroup and a
// quarter of the registers, so 4 waves fit per SIMD and K is split up to 16 ways.
// Each wave's lane (g, li) builds the two int8 weight planes of row n0 + li (planes.h) as the MFMA B column and
// loads activation row li's int8 values as the A row; one 32x32x32 MFMA per plane per 32 values, the Q4_K min
// term through one f16 MFMA per superblock, and the per-superblock f32 scaling of the reference
// (k_quants.rs:1848-1928, 2518-2575).  The four waves' partial tiles are summed through LDS at the end.
#include "common.h"
#include "inferencequant.h"
#include "planes.h"
#include "skinny.h"
#include "units.h"

namespace {

// Q4_K weight superblocks in flight per wave (a register ring; a multiple of 2)
#ifndef QMM_SKINNY_WDEPTH
#define QMM_SKINNY_WDEPTH 2
#endif
// 1: the 16x16x64 form serves every weight at b <= 16; 0 (measured faster on MI355X): only weights with fewer
// 32-row tiles than QMM_SKINNY_WIDE_TILES, wide weights keep the 32x32x32 form
#ifndef QMM_SKINNY16_WIDE
#define QMM_SKINNY16_WIDE 0
#endif
// from this many activation rows on, short weights split K over 8 waves as long rows do (MI355X, b = 24 / 32:
// Q6_K 1024x4096 10.8 / 11.4 -> 10.1 / 10.9 us, Q4_K 4096x4096 10.0 / 11.0 -> 10.0 / 10.8 us)
#ifndef QMM_SKINNY_K8_B
#define QMM_SKINNY_K8_B 17
#endif
// weights with fewer 32-row tiles than this go in 16-row tiles (twice the workgroups)
#ifndef QMM_SKINNY_WIDE_TILES
#define QMM_SKINNY_WIDE_TILES 384
#endif

// A-side fragments of one superblock for activation row li: 8 x 16 int8 (k = 32j + 16g + 0..15), the min-term
// operand of sub-blocks 4g .. 4g + 3 (planes.h min_frag: their 32-value sums split as 64 h + l, in f16), and the
// row's scale d.
struct ActFrag {
  v4i q[8];
  v8h bs;
  float d;
};

// Q8_1-slot layout (units.h): row m = 288-byte slots {f32 d; int8 qs[256]; int16 s32[8]; pad}, row_bytes apart.
struct act_slot {
  const uint8_t *base;
  int64_t bytes;
  uint32_t row_bytes;
  __device__ __forceinline__ rsrc_t rsrc() const { return make_rsrc(base, bytes); }
  // per-lane handle of row m; a row that is not valid reads as zero (its offset lies beyond every buffer's end)
  __device__ __forceinline__ uint32_t handle(int64_t m, bool valid) const {
    return valid ? (uint32_t)m * row_bytes : 0x80000000u;
  }
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row_off, int64_t sb, int g, bool min, ActFrag &f) const {
    const uint32_t o = row_off + (uint32_t)sb * kSlotBytes;
#pragma unroll
    for (int j = 0; j < 8; j++)
      f.q[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, o + 4 + 32 * j + 16 * g, 0, 0));
    if (min) {
      const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(r, o + 260 + 8 * g, 0, 0);  // sums of 4g .. 4g + 3
      f.bs = min_frag(b.x, b.y);
    }
    f.d = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0));
  }
};

// Tensor-core entry layout (units.h): row m = K / 256 blocks of 260 bytes {f32 d; int8 qs[256]}, no sums.  Lane
// (li, g) sums its own fragments -- q[j] is values 32 j + 16 g .. +16 -- and adds its partner lane's sum of the
// other half of the same 32 values, so both lanes hold S_j; lane half g keeps sub-blocks 4g .. 4g + 3.
struct act_tc {
  const uint8_t *base;
  int64_t bytes;
  uint32_t row_bytes;
  __device__ __forceinline__ rsrc_t rsrc() const { return make_rsrc(base, bytes); }
  __device__ __forceinline__ uint32_t handle(int64_t m, bool valid) const {
    return valid ? (uint32_t)m * row_bytes : 0x80000000u;
  }
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row_off, int64_t sb, int g, bool min, ActFrag &f) const {
    const uint32_t o = row_off + (uint32_t)sb * 260;
#pragma unroll
    for (int j = 0; j < 8; j++)
      f.q[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, o + 4 + 32 * j + 16 * g, 0, 0));
    if (min) {
      int s[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) acc = sdot4(f.q[j][i], 0x01010101, acc);
        s[j] = acc;
      }
      // s[j]: this lane's 16 values of sub-block j.  After the swap lane half 0 holds both lanes' sums of sub-block i
      // and lane half 1 both lanes' sums of sub-block i + 4, so w[i] is the whole sum of sub-block 4g + i.
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t pa = (uint32_t)s[i], pb = (uint32_t)s[i + 4];
        swap_lane_halves(pa, pb);
        w[i] = (uint32_t)((int)pa + (int)pb);
      }
      f.bs = min_frag((w[0] & 0xffffu) | (w[1] << 16), (w[2] & 0xffffu) | (w[3] << 16));
    }
    f.d = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0));
  }
};

// Prefill layout of one channel (include/inferencequant.h): qs[nsb][rows][256] int8, then d[nsb][rows] f32, then
// s32[nsb][rows][8] int16 sums of 32.  The handle is the lane's offset 256 m of row m inside one superblock's qs slab,
// with bit 31 set for a row that reads as zero; the superblock's part of every offset is uniform and goes in the
// scalar offset, outside the range check, which the vector part alone fails for such a row.
struct act_tiles {
  const uint8_t *base;
  int64_t bytes;
  uint32_t rows, nsb;
  __device__ __forceinline__ rsrc_t rsrc() const { return make_rsrc(base, bytes); }
  __device__ __forceinline__ uint32_t handle(int64_t m, bool valid) const {
    return valid ? 256 * (uint32_t)m : 0x80000000u;
  }
  __device__ __forceinline__ void load(rsrc_t r, uint32_t h, int64_t sb, int g, bool min, ActFrag &f) const {
    const uint32_t srow = (uint32_t)sb * rows, zero = h & 0x80000000u;
#pragma unroll
    for (int j = 0; j < 8; j++)
      f.q[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, h + 32 * j + 16 * g, 256 * srow, 0));
    if (min) {
      const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(r, ((h >> 4) + 8 * g) | zero, nsb * rows * 260 + 16 * srow, 0);
      f.bs = min_frag(b.x, b.y);
    }
    f.d = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (h >> 6) | zero,
                                                                          nsb * rows * 256 + 4 * srow, 0));
  }
};

// Expert-grouped row space: expert e = blockIdx.z owns activation rows [bounds[e], bounds[e + 1]) and weights
// W + e * expert_bytes; row m is stored to destination row ids_dst[m].  Workgroup (x, y) takes the 32-row chunks
// y, y + gridDim.y, ... of its expert, so every row is covered whatever the grid's height.
struct moe_route {
  const int32_t *bounds;
  const int32_t *ids_dst;
  int64_t expert_bytes;
};

// The NW waves' partial 32x32 tiles, summed through LDS.  Plain: lane (g, li) of wave w stores output registers
// (16 / NW) w ...; GLU (waves [0, NW/2) hold gate partials, [NW/2, NW) up partials): the first NW/2 waves store
// act(gate) * up.
// Activation rows m0 + 0..31 below m1 are stored, to destination row ids[m] when ids is given, else m.
template <class Out, int NW, bool GLU>
__device__ __forceinline__ void reduce_store(const v16f &fa, int wave, int lane, int g, int li, int64_t n0,
                                             int64_t n1, int64_t m0, int64_t m1, const int32_t *__restrict__ ids,
                                             typename Out::T *__restrict__ dst, int64_t ldd, int activation) {
  __shared__ float red[NW][16][64];
#pragma unroll
  for (int r = 0; r < 16; r++) red[wave][r][lane] = fa[r];
  __syncthreads();
  const int64_t n = n0 + li;
  constexpr int KW = GLU ? NW / 2 : NW;  // waves per K split
  constexpr int RPW = 16 / KW;
  if (GLU && wave >= KW) return;
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const int r = RPW * wave + i;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < KW; w++) v += red[w][r][lane];
    if (GLU) {
      float u = 0.0f;
#pragma unroll
      for (int w = KW; w < NW; w++) u += red[w][r][lane];
      v = glu_act(activation, v) * u;
    }
    const int64_t m = m0 + out_row(r, g);
    if (m < m1 && n < n1) Out::store(dst, (ids ? (int64_t)ids[m] : m) * ldd + n, v);
  }
}

// TR: weight rows per workgroup, 32 (every MFMA column used) or 16 (twice the workgroups for short weights; lanes
// 16..31 load nothing and their columns come out zero)
// GLU: W2 holds the up weights; waves [0, NW/2) take the gate rows and [NW/2, NW) the up rows.
// MOE: the activation rows and weights of expert blockIdx.z (moe_route); otherwise rows [0, mrows).
template <class WT, class AP, class Out, int NW, int TR, bool GLU, bool MOE = false>
__global__ __launch_bounds__(64 * NW) void k_skinny(const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2,
                                                    int64_t nrows_w, int64_t w_row_bytes, AP ap, int mrows,
                                                    int64_t nsb, typename Out::T *__restrict__ dst, int64_t ldd,
                                                    int activation, moe_route route) {
  __shared__ float dys[NW][32];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  constexpr int KW = GLU ? NW / 2 : NW;  // waves splitting K
  const int kw = wave % KW;
  int64_t m_first = 0, m_end = mrows, m_step = 32;
  const int32_t *ids = nullptr;
  if (MOE) {
    const int64_t e = blockIdx.z;
    m_first = route.bounds[e] + 32 * (int64_t)blockIdx.y;
    m_end = route.bounds[e + 1];
    if (m_first >= m_end) return;  // uniform over the workgroup
    m_step = 32 * (int64_t)gridDim.y;
    ids = route.ids_dst;
    W += e * route.expert_bytes;
    if (GLU) W2 += e * route.expert_bytes;
  }
  const int64_t n0 = (int64_t)blockIdx.x * TR;
  const int64_t rows_here = nrows_w - n0 < TR ? nrows_w - n0 : TR;
  const rsrc_t rw = make_rsrc((GLU && wave >= KW ? W2 : W) + n0 * w_row_bytes, rows_here * w_row_bytes);
  const uint32_t wrow = li < rows_here ? (uint32_t)(li * w_row_bytes) : 0x80000000u;
  const rsrc_t ra = ap.rsrc();

  const int64_t per = (nsb + KW - 1) / KW;
  const int64_t s0 = kw * per, s1 = s0 + per < nsb ? s0 + per : nsb;

  // weights WD superblocks ahead (a register ring), activations two ahead
  constexpr int WD = WT::kMin ? QMM_SKINNY_WDEPTH : 2;
  for (int64_t m0 = m_first; m0 < m_end; m0 += m_step) {
    // rows past the batch (or the expert) read as zero
    const uint32_t arow = ap.handle(m0 + li, m0 + li < m_end);
    v16f fa = (v16f){};
    typename WT::Raw raw[WD];
    ActFrag af[2];
    auto compute = [&](const typename WT::Raw &rr, const ActFrag &a) {
      typename WT::Prep p;
      WT::prepare(rr, g, p);
      v16i acc1 = (v16i){}, acc2 = (v16i){};
#pragma unroll
      for (int j = 0; j < 8; j++) {
        v4i b1, b2;
        WT::planes(rr, p, j, b1, b2);
        acc1 = mfma_i8(a.q[j], b1, acc1);
        acc2 = mfma_i8(a.q[j], b2, acc2);
      }
      v16f fmin = (v16f){};
      if (WT::kMin) fmin = mfma_f16(a.bs, p.bmin, fmin);
      // the scales of output rows 8q + 4g + i, from the lanes that loaded them
      if (g == 0) dys[wave][li] = a.d;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const v4f dy4 = *(const v4f *)&dys[wave][8 * q + 4 * g];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int r = 4 * q + i;
          const int iv = (acc1[r] << WT::kShift) + acc2[r];
          float v = p.d * (float)iv;
          if (WT::kMin) v -= p.dmin * fmin[r];
          fa[r] += dy4[i] * v;
        }
      }
    };

#pragma unroll
    for (int u = 0; u < WD; u++)
      if (s0 + u < s1) WT::load(rw, wrow, (uint32_t)(s0 + u), g, raw[u]);
#pragma unroll
    for (int u = 0; u < 2; u++)
      if (s0 + u < s1) ap.load(ra, arow, s0 + u, g, WT::kMin, af[u]);
    for (int64_t sb = s0; sb < s1; sb += WD) {
#pragma unroll
      for (int u = 0; u < WD; u++) {
        const int64_t s = sb + u;
        if (s < s1) {
          compute(raw[u], af[u & 1]);
          if (s + 2 < s1) ap.load(ra, arow, s + 2, g, WT::kMin, af[u & 1]);
          if (s + WD < s1) WT::load(rw, wrow, (uint32_t)(s + WD), g, raw[u]);
        }
      }
    }
    reduce_store<Out, NW, GLU>(fa, wave, lane, g, li, n0, n0 + rows_here, m0, m_end, ids, dst, ldd, activation);
    if (!MOE) break;
    __syncthreads();  // the next chunk rewrites the reduction buffer
  }
}

// ------------------------------------------------------------------------------------------ 16-row form

template <class WT>
struct Wt16;
template <>
struct Wt16<wq4k> {
  typedef wq4k16 T;
};
template <>
struct Wt16<wq6k> {
  typedef wq6k16 T;
};

// A-side fragments of one superblock for the 16x16x64 form: lane (kg, r) holds activation row r's values
// act_offset(t, kg) .. +16 for the four steps, the min-term operand of sub-blocks 2kg, 2kg + 1 of row r, and the
// scales of output rows 4kg + i.
struct ActFrag16 {
  v4i q[4];
  v4h bs;
  v4f dy;
};

// Up to 16 activation rows: NW waves split K, 16 weight rows per workgroup; output register i of lane (kg, r) is
// D[activation row 4kg + i][weight row r] (v_mfma 16x16 D layout).
template <class WT, class Out, int NW>
__global__ __launch_bounds__(64 * NW) void k_skinny16(const uint8_t *__restrict__ W, int64_t nrows_w,
                                                      int64_t w_row_bytes, act_slot ap, int mrows, int64_t nsb,
                                                      typename Out::T *__restrict__ dst, int64_t ldd) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kg = lane >> 4, r = lane & 15;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t rows_here = nrows_w - n0 < 16 ? nrows_w - n0 : 16;
  const rsrc_t rw = make_rsrc(W + n0 * w_row_bytes, rows_here * w_row_bytes);
  const uint32_t wrow = r < rows_here ? (uint32_t)(r * w_row_bytes) : 0x80000000u;
  const rsrc_t ra = ap.rsrc();
  // rows past the batch read as zero: their offset lies beyond every buffer's end
  const uint32_t arow = r < mrows ? (uint32_t)r * ap.row_bytes : 0x80000000u;
  uint32_t dyrow[4];
#pragma unroll
  for (int i = 0; i < 4; i++) dyrow[i] = 4 * kg + i < mrows ? (uint32_t)(4 * kg + i) * ap.row_bytes : 0x80000000u;

  const int64_t per = (nsb + NW - 1) / NW;
  const int64_t s0 = wave * per, s1 = s0 + per < nsb ? s0 + per : nsb;

  v4f fa = (v4f){};
  typename WT::Raw raw[2];
  ActFrag16 af[2];
  auto issue = [&](int64_t sb, int u) {
    WT::load(rw, wrow, (uint32_t)sb, kg, raw[u]);
    const uint32_t o = arow + (uint32_t)sb * kSlotBytes;
#pragma unroll
    for (int t = 0; t < 4; t++)
      af[u].q[t] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, o + 4 + WT::act_offset(t, kg), 0, 0));
    if (WT::kMin) {  // sums of sub-blocks 2kg, 2kg + 1, split as planes.h min_frag does
      uint32_t hp, lp;
      s32_split(__builtin_amdgcn_raw_buffer_load_b32(ra, o + 260 + 4 * kg, 0, 0), hp, lp);
      af[u].bs = __builtin_bit_cast(v4h, (u32x2){hp, lp});
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
      af[u].dy[i] =
          __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ra, dyrow[i] + (uint32_t)sb * kSlotBytes, 0, 0));
  };
  auto compute = [&](int u) {
    typename WT::Prep p;
    WT::prepare(raw[u], kg, p);
    v4i acc1 = (v4i){}, acc2 = (v4i){};
#pragma unroll
    for (int t = 0; t < 4; t++) {
      v4i b1, b2;
      WT::planes(raw[u], p, t, b1, b2, kg);
      acc1 = mfma16_i8(af[u].q[t], b1, acc1);
      acc2 = mfma16_i8(af[u].q[t], b2, acc2);
    }
    v4f fmin = (v4f){};
    if (WT::kMin) fmin = mfma16_f16(af[u].bs, p.bmin, fmin);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int iv = (acc1[i] << WT::kShift) + acc2[i];
      float v = p.d * (float)iv;
      if (WT::kMin) v -= p.dmin * fmin[i];
      fa[i] += af[u].dy[i] * v;
    }
  };

  if (s0 < s1) issue(s0, 0);
  if (s0 + 1 < s1) issue(s0 + 1, 1);
  for (int64_t sb = s0; sb < s1; sb += 2) {
    compute(0);
    if (sb + 2 < s1) issue(sb + 2, 0);
    if (sb + 1 < s1) {
      compute(1);
      if (sb + 3 < s1) issue(sb + 3, 1);
    }
  }

  __shared__ float red[NW][4][64];
#pragma unroll
  for (int i = 0; i < 4; i++) red[wave][i][lane] = fa[i];
  __syncthreads();
  if (wave >= 4) return;
  float v = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; w++) v += red[w][wave][lane];
  const int m = 4 * kg + wave;
  if (m < mrows && r < rows_here) Out::store(dst, (int64_t)m * ldd + n0 + r, v);
}

template <class WT, class Out>
void launch_decode(const void *vx, const void *vx2, const void *vy, void *dst, int ncols_x, int nrows_x,
                   int stride_col_y, int stride_col_dst, int b, int activation, hipStream_t s) {
  const int64_t nsb = ncols_x / 256;
  act_slot ap;
  ap.row_bytes = (uint32_t)stride_col_y * 36;
  ap.base = (const uint8_t *)vy;
  ap.bytes = (int64_t)b * ap.row_bytes;
  const uint8_t *w = (const uint8_t *)vx, *w2 = (const uint8_t *)vx2;
  typename Out::T *d = (typename Out::T *)dst;
  const int64_t wrb = nsb * WT::kBytes;
  if (w2) {  // gate and up in one workgroup: QMM_SKINNY_GLU_NW / 2 waves each
    if (qmm_ceil_div(nrows_x, 32) >= QMM_SKINNY_WIDE_TILES)
      k_skinny<WT, act_slot, Out, QMM_SKINNY_GLU_NW, 32, true><<<dim3((unsigned)qmm_ceil_div(nrows_x, 32)),
                                                                  64 * QMM_SKINNY_GLU_NW, 0, s>>>(
          w, w2, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, activation, moe_route{});
    else
      k_skinny<WT, act_slot, Out, 8, 16, true><<<dim3((unsigned)qmm_ceil_div(nrows_x, 16)), 512, 0, s>>>(
          w, w2, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, activation, moe_route{});
    return;
  }
  const unsigned g16 = (unsigned)qmm_ceil_div(nrows_x, 16);
  if (b <= 16 && (QMM_SKINNY16_WIDE || qmm_ceil_div(nrows_x, 32) < QMM_SKINNY_WIDE_TILES)) {
    // 16x16x64 form: a quarter of the registers, 4 waves per SIMD; the widest K split whose waves are all resident
    // at once (16 x CUs of them)
    const int64_t slots = 16 * (int64_t)qmm_device_cus();
    if (WT::kMin && nsb >= 16 && (int64_t)g16 * 16 <= slots)  // Q4_K fits 128 VGPRs at 16 waves; Q6_K does not
      k_skinny16<typename Wt16<WT>::T, Out, 16><<<g16, 1024, 0, s>>>(w, nrows_x, wrb, ap, b, nsb, d, stride_col_dst);
    else if (nsb >= 8 && (int64_t)g16 * 8 <= slots)
      k_skinny16<typename Wt16<WT>::T, Out, 8><<<g16, 512, 0, s>>>(w, nrows_x, wrb, ap, b, nsb, d, stride_col_dst);
    else
      k_skinny16<typename Wt16<WT>::T, Out, 4><<<g16, 256, 0, s>>>(w, nrows_x, wrb, ap, b, nsb, d, stride_col_dst);
    return;
  }
  if (qmm_ceil_div(nrows_x, 32) >= QMM_SKINNY_WIDE_TILES)
    k_skinny<WT, act_slot, Out, 4, 32, false><<<dim3((unsigned)qmm_ceil_div(nrows_x, 32)), 256, 0, s>>>(
        w, nullptr, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, 0, moe_route{});
  else if (nsb >= 32 || b >= QMM_SKINNY_K8_B)  // long rows: 8 waves split K, so each wave's chain of superblocks stays short
    k_skinny<WT, act_slot, Out, 8, 16, false><<<dim3((unsigned)qmm_ceil_div(nrows_x, 16)), 512, 0, s>>>(
        w, nullptr, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, 0, moe_route{});
  else
    k_skinny<WT, act_slot, Out, 4, 16, false><<<dim3((unsigned)qmm_ceil_div(nrows_x, 16)), 256, 0, s>>>(
        w, nullptr, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, 0, moe_route{});
}

// The tensor-core entries: the 32x32 form over act_tc, 4 waves splitting K (8 for long rows).
template <class WT, class Out>
void launch_tc(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int stride_col_dst, int b,
               hipStream_t s) {
  const int64_t nsb = ncols_x / 256;
  act_tc ap;
  ap.row_bytes = (uint32_t)(nsb * 260);
  ap.base = (const uint8_t *)vy;
  ap.bytes = (int64_t)b * ap.row_bytes;
  const uint8_t *w = (const uint8_t *)vx;
  typename Out::T *d = (typename Out::T *)dst;
  const int64_t wrb = nsb * WT::kBytes;
  if (qmm_ceil_div(nrows_x, 32) >= QMM_SKINNY_WIDE_TILES)
    k_skinny<WT, act_tc, Out, 4, 32, false><<<dim3((unsigned)qmm_ceil_div(nrows_x, 32)), 256, 0, s>>>(
        w, nullptr, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, 0, moe_route{});
  else if (nsb >= 32)
    k_skinny<WT, act_tc, Out, 8, 16, false><<<dim3((unsigned)qmm_ceil_div(nrows_x, 16)), 512, 0, s>>>(
        w, nullptr, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, 0, moe_route{});
  else
    k_skinny<WT, act_tc, Out, 4, 16, false><<<dim3((unsigned)qmm_ceil_div(nrows_x, 16)), 256, 0, s>>>(
        w, nullptr, nrows_x, wrb, ap, b, nsb, d, stride_col_dst, 0, moe_route{});
}

template <class WT>
void launch_moe(const void *x, const void *y, const int32_t *ids_dst, const int32_t *bounds, float *dst,
                int64_t nrows_x, int64_t w_row_bytes, int64_t nsb, int64_t ncols_dst, int64_t ldd, int64_t num_experts,
                int64_t chunks, hipStream_t s) {
  act_tiles ap;
  ap.base = (const uint8_t *)y;
  ap.rows = (uint32_t)ncols_dst;
  ap.nsb = (uint32_t)nsb;
  ap.bytes = nsb * ncols_dst * 276;
  const moe_route rt{bounds, ids_dst, nrows_x * w_row_bytes};
  const dim3 grid((unsigned)qmm_ceil_div(nrows_x, 32), (unsigned)chunks, (unsigned)num_experts);
  const uint8_t *w = (const uint8_t *)x;
  if (nsb >= 32)  // long rows: 8 waves split K
    k_skinny<WT, act_tiles, out_f32, 8, 32, false, true><<<grid, 512, 0, s>>>(w, nullptr, nrows_x, w_row_bytes, ap, 0,
                                                                              nsb, dst, ldd, 0, rt);
  else
    k_skinny<WT, act_tiles, out_f32, 4, 32, false, true><<<grid, 256, 0, s>>>(w, nullptr, nrows_x, w_row_bytes, ap, 0,
                                                                              nsb, dst, ldd, 0, rt);
}

bool dispatch(int type, int out_type, const void *vx, const void *vx2, const void *vy, void *dst, int ncols_x,
              int nrows_x, int stride_col_y, int stride_col_dst, int b, int activation, hipStream_t s) {
  if (b < 1 || b > 32 || ncols_x % 256 != 0 || stride_col_y % 8 != 0 || (int64_t)b * stride_col_y * 36 > 0x7ffffff0)
    return false;
  if (type != QMM_TYPE_Q4K && type != QMM_TYPE_Q6K) return false;
#define QMM_SK(WT)                                                                                              \
  switch (out_type) {                                                                                           \
    case QMM_TYPE_F16:                                                                                          \
      launch_decode<WT, out_f16>(vx, vx2, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b, activation, s); \
      break;                                                                                                    \
    case QMM_TYPE_BF16:                                                                                         \
      launch_decode<WT, out_bf16>(vx, vx2, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b, activation, s); \
      break;                                                                                                    \
    default:                                                                                                    \
      launch_decode<WT, out_f32>(vx, vx2, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b, activation, s); \
  }
  if (type == QMM_TYPE_Q4K) {
    QMM_SK(wq4k)
  } else {
    QMM_SK(wq6k)
  }
#undef QMM_SK
  return true;
}

}  // namespace

bool qmm_skinny_decode(int type, int out_type, const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,
                       int stride_col_y, int stride_col_dst, int b, hipStream_t s) {
  return dispatch(type, out_type, vx, nullptr, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b, 0, s);
}

bool qmm_skinny_glu(int type, int out_type, const void *vx_gate, const void *vx_up, const void *vy, void *dst,
                    int ncols_x, int nrows_x, int stride_col_y, int stride_col_dst, int b, int activation,
                    hipStream_t s) {
  return dispatch(type, out_type, vx_gate, vx_up, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b,
                  activation, s);
}

bool qmm_skinny_tc(int type, int out_type, const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,
                   int stride_col_dst, int b, hipStream_t s) {
  if (b < 1 || b > 32 || ncols_x % 256 != 0 || (int64_t)b * (ncols_x / 256) * 260 > 0x7ffffff0) return false;
  if (type != QMM_TYPE_Q4K && type != QMM_TYPE_Q6K) return false;
#define QMM_TC(WT)                                                                                   \
  switch (out_type) {                                                                                \
    case QMM_TYPE_F16: launch_tc<WT, out_f16>(vx, vy, dst, ncols_x, nrows_x, stride_col_dst, b, s); break;   \
    case QMM_TYPE_BF16: launch_tc<WT, out_bf16>(vx, vy, dst, ncols_x, nrows_x, stride_col_dst, b, s); break; \
    default: launch_tc<WT, out_f32>(vx, vy, dst, ncols_x, nrows_x, stride_col_dst, b, s);            \
  }
  if (type == QMM_TYPE_Q4K) {
    QMM_TC(wq4k)
  } else {
    QMM_TC(wq6k)
  }
#undef QMM_TC
  return true;
}

bool qmm_skinny_moe(int type, const void *x, const void *y, const int32_t *ids_dst, const int32_t *bounds, float *dst,
                    int64_t ncols_x, int64_t nrows_x, int64_t w_row_bytes, int64_t ncols_dst, int64_t ldd,
                    int64_t num_experts, hipStream_t s) {
  if (ncols_x % 256 != 0 || ncols_dst <= 0 || num_experts <= 0 || num_experts > 65535) return false;
  if (ncols_dst > QMM_SKINNY_MOE_ROWS * num_experts) return false;
  const int64_t nsb = ncols_x / 256;
  if (nsb * ncols_dst * 276 > 0x7ffffff0 || 32 * w_row_bytes > 0x7ffffff0) return false;
  // enough 32-row chunks for an expert of average size; larger experts loop over theirs
  const int64_t chunks = qmm_ceil_div(qmm_ceil_div(ncols_dst, num_experts), 32);
  if (type == QMM_TYPE_Q4K)
    launch_moe<wq4k>(x, y, ids_dst, bounds, dst, nrows_x, w_row_bytes, nsb, ncols_dst, ldd, num_experts, chunks, s);
  else if (type == QMM_TYPE_Q6K)
    launch_moe<wq6k>(x, y, ids_dst, bounds, dst, nrows_x, w_row_bytes, nsb, ncols_dst, ldd, num_experts, chunks, s);
  else
    return false;
  return true;
}
