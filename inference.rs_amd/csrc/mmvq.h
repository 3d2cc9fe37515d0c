// Decode matvec kernels shared by the per-type translation units mmvq_<t>.hip: GGUF Q8_0 / Q4_K / Q6_K (and Q4_0 /
// Q5_0 / Q5_K / IQ4_XS) weights against quantized activations (b = 1..16 rows; 32 for Q4_K / Q6_K), plus the
// expert-indexed MoE matvec (optionally fused gate/up with the GLU activation).  Each translation unit instantiates
// the kernels of its weight types only, so the library builds in parallel.
//
// Replaces mmvq_gguf.cuh:650-759 (mmvq_core_impl) and its launchers (1542-1553, 1647-1702, 1762-1834),
// mmvq_gguf.cuh:961-1038 / 1600-1643 (MoE) and indexed_moe.cu:664-1000, all in
// crates/inference-quant/kernels/cuda/.  HBM-bound: each wave owns R consecutive weight rows; its 64 lanes
// stride over the rows' units (units.h), issue every 16-byte weight load of the R rows before using any,
// dot them with v_dot4 against activation units read once per column, and reduce each row with a wave
// butterfly.  Activations are tiny and hit L2.
//
// Two activation layouts (units.h): the Q8_1 slots of the reference-named entries (every weight type, 288 bytes per
// 256 values, stride_col_y in 36-byte Q8_1 blocks as the reference passes it) and, for the 32-value weight types, the
// Q8_0 blocks of their CPU dot product (the _q8_0 entries, 34 bytes per 32 values, stride_col_y in blocks).
#pragma once

#include <type_traits>

#include "common.h"
#include "inferencequant.h"
#include "q8.h"
#include "skinny.h"
#include "units.h"

namespace {

constexpr int kWaves = 4;  // waves per workgroup
// rows of up to this many 64-value units per lane go through the persistent kernel, longer ones through k_mmvq
#ifndef QMM_PERSISTENT_MAX_S
#define QMM_PERSISTENT_MAX_S 4
#endif
// the persistent kernels hold at most 4 units per lane (k_mmvq_p's widest instantiation; k_mmvq_p2's two waves of two)
static_assert(QMM_PERSISTENT_MAX_S >= 1 && QMM_PERSISTENT_MAX_S <= 4, "persistent rows hold at most 4 units per lane");


template <class U, class Out, int NC, int R>
__global__ __launch_bounds__(256) void k_mmvq(const uint8_t *__restrict__ vx, const uint8_t *__restrict__ vy,
                                              typename Out::T *__restrict__ dst, int nrows, int64_t row_bytes,
                                              int nunits, int64_t act_row_bytes, int stride_col_dst) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= nrows) return;  // whole wave
  float acc[R][NC];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int j = 0; j < NC; j++) acc[r][j] = 0.0f;

  for (int u = lane; u < nunits; u += QMM_WAVE) {
    typename U::W w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = min(row0 + r, nrows - 1);  // a short last group re-reads its last row; never stored
      U::load_w(vx + (int64_t)row * row_bytes, u, w[r]);
    }
#pragma unroll
    for (int j = 0; j < NC; j++) {
      typename U::A a;
      U::load_a(vy + (int64_t)j * act_row_bytes, u, a);
#pragma unroll
      for (int r = 0; r < R; r++) acc[r][j] += U::dot(w[r], a, u);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int j = 0; j < NC; j++) {
      const float v = wave_sum_to_lane63(acc[r][j]);
      if (lane == 63 && row0 + r < nrows) Out::store(dst, (int64_t)j * stride_col_dst + row0 + r, v);
    }
}

// ------------------------------------------------------------------------------------------------ persistent form

// Pieces of the one-launch kernel's row loop.  A wave holds two rows' weights, in two buffers that are loaded and
// used in place: the loop is unrolled by two so that no buffer is ever copied, because a copy of a register that a
// load is still filling waits for that load, and the wait the compiler places at a loop-carried copy covers every
// load in flight, the next row's included.  Loads are unconditional, so each wait covers exactly the row about to be
// used: a row past the end is read through an empty buffer resource (zeros, no memory traffic), and lanes past the
// last unit re-read the row's last unit.
template <class U, int S, bool FULL>
__device__ __forceinline__ void load_row(const uint8_t *vx, int64_t row_bytes, int nunits, int nrows, int r, int lane,
                                         typename U::W (&w)[S]) {
  r = __builtin_amdgcn_readfirstlane(r);  // one row per wave: a scalar buffer resource
  const bool live = r < nrows;
  const row_buf src = make_row_buf(vx + (int64_t)(live ? r : 0) * row_bytes, live ? row_bytes : 0);
#pragma unroll
  for (int s = 0; s < S; s++) {
    const int u = (FULL || lane + 64 * s < nunits) ? lane + 64 * s : nunits - 1;
    U::load_w(src, u, w[s]);
  }
}

// One row's dot products against NC activation rows (held in registers when kRegs, else read from act), per lane.
template <class U, int NC, int S, bool FULL, bool kRegs>
__device__ __forceinline__ void row_dots(const typename U::W (&w)[S], const typename U::A *areg, const uint8_t *act,
                                         int64_t act_row_bytes, int nunits, int lane, float (&acc)[NC]) {
#pragma unroll
  for (int j = 0; j < NC; j++) acc[j] = 0.0f;
#pragma unroll
  for (int s = 0; s < S; s++) {
    if (!(FULL || lane + 64 * s < nunits)) continue;
    const int u = lane + 64 * s;
#pragma unroll
    for (int j = 0; j < NC; j++) {
      if (kRegs) {
        acc[j] += U::dot(w[s], areg[s * NC + j], u);
      } else {
        typename U::A a;
        U::load_a(act + j * act_row_bytes, u, a);
        acc[j] += U::dot(w[s], a, u);
      }
    }
  }
}

// The wave sums of acc.  Every lane stores the same value to the same address (one write): a store under
// `lane == 63` would sit behind a branch, and the compiler's wait counts after a conditional store assume the
// worst of both paths, which makes the next row's math wait for loads that are still in flight.
template <class Out, int NC>
__device__ __forceinline__ void row_store(const float (&acc)[NC], int lane, typename Out::T *dst, int stride_col_dst,
                                          int row) {
  (void)lane;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const float v = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_to_lane63(acc[j])), 63));
    Out::store(dst, (int64_t)j * stride_col_dst + row, v);
  }
}

// Rows row, row + tw, ... (row < nrows) of one wave with two rows in flight: buffer a holds row r and buffer b row
// r + tw, both requested before this is called.  Each buffer is reloaded between its row's dot products and the
// row's store, so no stored value shares a register with a load in flight.
template <class U, class Out, int NC, int S, bool FULL, bool kRegs>
__device__ __forceinline__ void row_pairs(const uint8_t *vx, int64_t row_bytes, int nunits, int nrows, int row, int tw,
                                          int lane, typename U::W (&wa)[S], typename U::W (&wb)[S],
                                          const typename U::A *areg, const uint8_t *act, int64_t act_row_bytes,
                                          typename Out::T *dst, int stride_col_dst) {
  float acc[NC];
  for (;;) {
    row_dots<U, NC, S, FULL, kRegs>(wa, areg, act, act_row_bytes, nunits, lane, acc);
    load_row<U, S, FULL>(vx, row_bytes, nunits, nrows, row + 2 * tw, lane, wa);
    row_store<Out, NC>(acc, lane, dst, stride_col_dst, row);
    if (row + tw >= nrows) break;
    row_dots<U, NC, S, FULL, kRegs>(wb, areg, act, act_row_bytes, nunits, lane, acc);
    load_row<U, S, FULL>(vx, row_bytes, nunits, nrows, row + 3 * tw, lane, wb);
    row_store<Out, NC>(acc, lane, dst, stride_col_dst, row + tw);
    row += 2 * tw;
    if (row >= nrows) break;
  }
}

// Persistent decode matvec: wave w of the grid takes rows w, w + T, w + 2T, ... (T waves in the grid), so a few
// thousand resident waves keep the HBM queues full, and each wave requests its next row's weights before it
// does the current row's math.  Lane l owns units l + 64 s (s < S) of every row, so with NC * S <= 2 its
// activation units stay in registers for the whole launch.  FULL: every lane has all S units (no guards).
template <class U, class Out, int NC, int S, bool FULL>
__global__ __launch_bounds__(256) void k_mmvq_p(const uint8_t *__restrict__ vx, const uint8_t *__restrict__ act,
                                                typename Out::T *__restrict__ dst, int nrows, int64_t row_bytes,
                                                int nunits, int64_t act_row_bytes, int stride_col_dst) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tw = gridDim.x * kWaves;
  int row = blockIdx.x * kWaves + wave;
  if (row >= nrows) return;  // whole wave
  auto has = [&](int s) { return FULL || lane + 64 * s < nunits; };
  constexpr bool kRegs = NC * S <= 2;
  typename U::A areg[kRegs ? NC * S : 1];
  if (kRegs) {
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
      for (int j = 0; j < NC; j++)
        if (has(s)) U::load_a(act + j * act_row_bytes, lane + 64 * s, areg[kRegs ? s * NC + j : 0]);
  }
  typename U::W w[S];
#pragma unroll
  for (int s = 0; s < S; s++)
    if (has(s)) U::load_w(vx + (int64_t)row * row_bytes, lane + 64 * s, w[s]);
  // the next row's weights are requested before this row's math when they fit in 64 more registers; longer rows
  // keep enough bytes in flight within one row
  constexpr bool kNext = S * sizeof(typename U::W) <= 64 * 4;
  for (; row < nrows; row += tw) {
    typename U::W wn[kNext ? S : 1];
    if (kNext && row + tw < nrows) {
#pragma unroll
      for (int s = 0; s < S; s++)
        if (has(s)) U::load_w(vx + (int64_t)(row + tw) * row_bytes, lane + 64 * s, wn[kNext ? s : 0]);
    }
    float acc[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) acc[j] = 0.0f;
#pragma unroll
    for (int s = 0; s < S; s++) {
      if (!has(s)) continue;
      const int u = lane + 64 * s;
#pragma unroll
      for (int j = 0; j < NC; j++) {
        if (kRegs) {
          acc[j] += U::dot(w[s], areg[s * NC + j], u);
        } else {
          typename U::A a;
          U::load_a(act + j * act_row_bytes, u, a);
          acc[j] += U::dot(w[s], a, u);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NC; j++) {
      const float v = wave_sum_to_lane63(acc[j]);
      if (lane == 63) Out::store(dst, (int64_t)j * stride_col_dst + row, v);
    }
    if (kNext) {
#pragma unroll
      for (int s = 0; s < S; s++) w[s] = wn[kNext ? s : 0];
    } else if (row + tw < nrows) {
#pragma unroll
      for (int s = 0; s < S; s++)
        if (has(s)) U::load_w(vx + (int64_t)(row + tw) * row_bytes, lane + 64 * s, w[s]);
    }
  }
}

// Wide rows at one column (more than two units per lane): the two waves of a pair split each row's units, wave 2p
// taking units [0, 128) and wave 2p + 1 units [128, 256), so each wave holds two units per lane (its activation units
// in registers for the whole launch, and the next row's weights requested before this row's math) and more waves fit
// on a CU.  A workgroup's two pairs take rows 2b and 2b + 1, then 2b + 2G and 2b + 2G + 1 (G workgroups), every wave
// running the same number of iterations, so every wave reaches every barrier.  The second half's sum reaches the
// first through one of two LDS slots (alternating, so a slot is rewritten only after the barrier that follows its
// read) and is added to the first half's sum: a fixed order.
template <class U, class Out, int NC, bool FULL>
__global__ __launch_bounds__(256) void k_mmvq_p2(const uint8_t *__restrict__ vx, const uint8_t *__restrict__ act,
                                                 typename Out::T *__restrict__ dst, int nrows, int64_t row_bytes,
                                                 int nunits, int64_t act_row_bytes, int stride_col_dst) {
  constexpr int S = 2;
  __shared__ float part[2][2][NC];  // [slot][pair][column]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pair = wave >> 1, half = wave & 1;
  const int ubase = half * 64 * S;
  auto has = [&](int s) { return FULL || ubase + lane + 64 * s < nunits; };
  typename U::A areg[S * NC];
#pragma unroll
  for (int s = 0; s < S; s++)
#pragma unroll
    for (int j = 0; j < NC; j++)
      if (has(s)) U::load_a(act + j * act_row_bytes, ubase + lane + 64 * s, areg[s * NC + j]);
  const int step = gridDim.x * 2;
  const int iters = (nrows + step - 1) / step;  // the same for every wave of the grid
  int row = blockIdx.x * 2 + pair;
  typename U::W w[S];
  if (row < nrows) {
#pragma unroll
    for (int s = 0; s < S; s++)
      if (has(s)) U::load_w(vx + (int64_t)row * row_bytes, ubase + lane + 64 * s, w[s]);
  }
  for (int it = 0; it < iters; it++, row += step) {
    typename U::W wn[S];
    if (row + step < nrows) {
#pragma unroll
      for (int s = 0; s < S; s++)
        if (has(s)) U::load_w(vx + (int64_t)(row + step) * row_bytes, ubase + lane + 64 * s, wn[s]);
    }
    float acc[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) acc[j] = 0.0f;
    if (row < nrows) {
#pragma unroll
      for (int s = 0; s < S; s++)
#pragma unroll
        for (int j = 0; j < NC; j++)
          if (has(s)) acc[j] += U::dot(w[s], areg[s * NC + j], ubase + lane + 64 * s);
    }
    float v[NC];
#pragma unroll
    for (int j = 0; j < NC; j++)
      v[j] = __builtin_bit_cast(float,
                                __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_to_lane63(acc[j])), 63));
    if (half == 1 && lane == 0) {
#pragma unroll
      for (int j = 0; j < NC; j++) part[it & 1][pair][j] = v[j];
    }
    __syncthreads();
    if (half == 0 && row < nrows && lane == 0) {
#pragma unroll
      for (int j = 0; j < NC; j++) Out::store(dst, (int64_t)j * stride_col_dst + row, v[j] + part[it & 1][pair][j]);
    }
#pragma unroll
    for (int s = 0; s < S; s++) w[s] = wn[s];
  }
}

// Wide rows at one column, four waves to a row: wave p of a workgroup takes units [64 p, 64 p + 64) of every row it
// walks (one per lane; a lane past the row's units reads through an offset past the row's buffer, zeros with no
// traffic), holds that activation unit in registers for the whole launch, and walks the workgroup's rows
// b, b + G, ... (G workgroups, at most kP4Rows of them) with two in flight in place, as row_pairs does.  Each wave leaves
// its partial sum of a row in LDS; after one barrier the workgroup adds the four in wave order and stores the rows.
// Measured on MI355X at 4096 x 14336, b = 1, against k_mmvq_p / k_mmvq_p2: Q6_K 14.3 -> 13.5 us, Q5_K 12.0 -> 10.4,
// Q4_K 9.8 -> 8.6, Q8_0 13.6 -> 12.4, Q4_0 9.6 -> 8.2, Q5_0 11.2 -> 10.1; 4 and 16 rows per workgroup measured slower
// than 8 (Q6_K 15.1 and 14.9 us).
//
// QX: act is the f32 activation row, which every lane quantizes for its own unit (U::quantize_a) after requesting the
// first two rows' weights, so the launch needs no quantizer before it.  Every workgroup quantizes the whole row again
// (56 KB of f32 at K = 14336, from L2).
constexpr int kP4Rows = 8;
template <class U, class Out, bool QX = false>
__global__ __launch_bounds__(256) void k_mmvq_p4(const uint8_t *__restrict__ vx, const void *__restrict__ act,
                                                 typename Out::T *__restrict__ dst, int nrows, int64_t row_bytes,
                                                 int nunits) {
  __shared__ float part[4][kP4Rows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int u = 64 * wave + lane;
  const bool has = u < nunits;
  const int ul = has ? u : nunits + 64;  // (past the row: the buffer range check reads zeros)
  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  const int n = (nrows - b + G - 1) / G;  // this workgroup's rows, at most kP4Rows (the launcher's grid)
  auto load = [&](int i, typename U::W &w) {
    const bool live = i < n;
    const row_buf src = make_row_buf(vx + (int64_t)(b + (live ? i : 0) * G) * row_bytes, live ? row_bytes : 0);
    U::load_w(src, ul, w);
  };
  auto sum = [&](float acc) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_to_lane63(acc)), 63));
  };
  typename U::A a;
  typename U::W wa, wb;
  if constexpr (QX) {
    load(0, wa);
    load(1, wb);
    U::quantize_a((const float *)act, has ? u : 0, a);  // (a lane past the units quantizes the first, unused)
  } else {
    U::load_a((const uint8_t *)act, has ? u : 0, a);
    load(0, wa);
    load(1, wb);
  }
  for (int i = 0; i < n; i += 2) {
    float acc = has ? U::dot(wa, a, u) : 0.0f;
    load(i + 2, wa);
    part[wave][i] = sum(acc);  // (every lane writes the same value: no store behind a branch)
    if (i + 1 >= n) break;
    acc = has ? U::dot(wb, a, u) : 0.0f;
    load(i + 3, wb);
    part[wave][i + 1] = sum(acc);
  }
  __syncthreads();
  const int t = (int)threadIdx.x;
  if (t < n) Out::store(dst, (int64_t)b + (int64_t)t * G, ((part[0][t] + part[1][t]) + part[2][t]) + part[3][t]);
}

// The four-wave form where the rows give every CU two workgroups of kP4Rows rows (fewer rows measured slower than
// k_mmvq_p / k_mmvq_p2: Q6_K 1024 x 14336 5.1 -> 7.1 us)
template <class U>
bool use_p4(int units, int nc, int nrows) {
  return nc == 1 && units > 128 && units <= 256 && qmm_ceil_div(nrows, kP4Rows) >= 2 * (int64_t)qmm_device_cus();
}

template <class U, class Out, bool QX = false>
void launch_p4(const uint8_t *vx, const void *act, typename Out::T *dst, int k, int nrows, hipStream_t s) {
  k_mmvq_p4<U, Out, QX><<<dim3((unsigned)qmm_ceil_div(nrows, kP4Rows)), 256, 0, s>>>(vx, act, dst, nrows,
                                                                                     U::row_bytes(k), U::units(k));
}

// Which types take k_mmvq_p2 for wide rows at one column.  On MI355X at 4096 x 14336, b = 1: Q4_K 10.7 -> 10.0 us,
// IQ4_XS 10.65 -> 10.17, Q5_0 11.75 -> 11.22, Q4_0 9.8 -> 9.57, Q8_0 13.76 -> 13.54; slower for Q6_K (14.3 -> 14.9,
// whose 84-byte units held twice over leave three waves per SIMD) and Q5_K (12.1 -> 12.5), which keep k_mmvq_p.
// At two columns (b = 2): Q4_K 14.9 -> 13.5 us, Q4_0 14.1 -> 12.5, Q8_0 18.3 -> 16.0; IQ4_XS (14.1 -> 16.1) and Q5_0
// (15.5 -> 16.0) keep k_mmvq_p there.
template <class U>
constexpr bool split_wide_rows(int nc) {
  if (nc == 1) return U::kType != QMM_TYPE_Q6K && U::kType != QMM_TYPE_Q5K;
  return nc == 2 && (U::kType == QMM_TYPE_Q4K || U::kType == QMM_TYPE_Q4_0 || U::kType == QMM_TYPE_Q8_0);
}

// The form of the decode kernel a row of `units` units takes at nc columns: k_mmvq_p (kFormP) holds s = 1, 2 or 4 units
// per lane, k_mmvq_p2 (kFormP2) two waves of two per row (256 units), k_mmvq (kFormPasses) any row, its units in
// passes.  `full` (no per-unit guard) only where the row fills every lane's units exactly: three units per lane run
// the four-unit kernel, so 192 units are not full.  Exported as qmm_decode_form for the tests.
enum { kFormP = 0, kFormP2 = 1, kFormPasses = 2 };
struct DecodeForm {
  int kernel, s;
  bool full;
};
template <class U>
constexpr DecodeForm decode_form(int units, int nc) {
  const int S = (units + 63) / 64;
  if (S > QMM_PERSISTENT_MAX_S) return {kFormPasses, S, false};
  if (S > 2 && split_wide_rows<U>(nc)) return {kFormP2, 4, units == 256};
  const int s = S <= 2 ? S : 4;
  return {kFormP, s, units == 64 * s};
}

// Grid of k_mmvq_p2: row pairs spread evenly over as many rounds of the workgroups a CU holds as they need.
template <class U, class Out>
void launch_p2(int nc, const uint8_t *vx, const uint8_t *act, typename Out::T *dst, int k, int nrows,
               int64_t act_row_bytes, int stride_col_dst, hipStream_t s) {
  const int64_t rb = U::row_bytes(k);
  const int nu = U::units(k);
  const int64_t pairs = qmm_ceil_div(nrows, 2);
  auto grid = [&](int per_cu) {
    const int64_t cap = (int64_t)(per_cu < 8 ? per_cu : 8) * qmm_device_cus();
    const int64_t rounds = qmm_ceil_div(pairs, cap);
    return dim3((unsigned)qmm_ceil_div(pairs, rounds));
  };
#define QMM_P2_F(NC, FF)                                                                                  \
  k_mmvq_p2<U, Out, NC, FF><<<grid(qmm_resident_per_cu<k_mmvq_p2<U, Out, NC, FF>>(256, 0)), 256, 0, s>>>( \
      vx, act, dst, nrows, rb, nu, act_row_bytes, stride_col_dst)
  const bool full = decode_form<U>(nu, nc).full;
  if (nc == 1) {
    if (full)
      QMM_P2_F(1, true);
    else
      QMM_P2_F(1, false);
  } else {
    if (full)
      QMM_P2_F(2, true);
    else
      QMM_P2_F(2, false);
  }
#undef QMM_P2_F
}

// ------------------------------------------------------------------------------------------------ fused quantization

// The persistent matvec against NC f32 activation rows that it quantizes itself.  Every workgroup quantizes the rows
// into LDS, in the decode activation layout, with the standalone quantizers' device code (q8.h), so the blocks are
// bit-identical to launch_mmvq_gguf_quantize_{q8k,q8_0}_f32's.  The f32 loads go out first and the first two rows'
// weights right after them, so the quantization runs while the weights are in flight.  A wave step quantizes one
// Q8_K block (4 values per lane) or eight Q8_0 blocks (8 lanes each); wave w takes steps w, w + NW, ... (at most
// G of them).
template <class U, class Out, int NC, int S, bool FULL, int NW, int G>
__global__ __launch_bounds__(64 * NW) void k_mmvq_pq(const uint8_t *__restrict__ vx, const float *__restrict__ x,
                                                     int64_t stride_x, typename Out::T *__restrict__ dst, int nrows,
                                                     int64_t row_bytes, int nunits, int stride_col_dst) {
  extern __shared__ __align__(16) uint8_t s_act[];
  constexpr bool kQ8K = U::kActBlockValues == 256;
  constexpr int kBlocksPerStep = kQ8K ? 1 : 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = nunits * U::kValuesPerUnit / U::kActBlockValues;  // activation blocks per row
  const int total = NC * nblk;
  const int64_t act_row_bytes = (int64_t)nblk * U::kActBlockBytes;

  // 1. this wave's f32 values: rows hold whole blocks, so every load is in range (a lane past the last block
  // reloads block 0 and stores nothing)
  float v[G][4];
  int blk[G];
#pragma unroll
  for (int t = 0; t < G; t++) {
    blk[t] = (wave + NW * t) * kBlocksPerStep + (kQ8K ? 0 : lane >> 3);
    const int b = blk[t] < total ? blk[t] : 0;
    const int j = NC > 1 && b >= nblk ? 1 : 0;
    const int k0 = (b - j * nblk) * U::kActBlockValues + 4 * (kQ8K ? lane : lane & 7);
    // (a float vector: this compiler's __builtin_bit_cast of a u32 vector element reads element 0)
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 f;
    __builtin_memcpy(&f, __builtin_assume_aligned(x + j * stride_x + k0, 4), 16);
    v[t][0] = f.x, v[t][1] = f.y, v[t][2] = f.z, v[t][3] = f.w;
  }
  // 2. the first two rows' weights, so the quantization below waits for the f32 loads only
  auto has = [&](int s) { return FULL || lane + 64 * s < nunits; };
  const int tw = gridDim.x * NW;
  int row = blockIdx.x * NW + wave;
  typename U::W wa[S], wb[S];
  load_row<U, S, FULL>(vx, row_bytes, nunits, nrows, row, lane, wa);  // a wave with no row reads zeros
  load_row<U, S, FULL>(vx, row_bytes, nunits, nrows, row + tw, lane, wb);
  __builtin_amdgcn_sched_barrier(0);
  // 3. quantize into LDS
  if constexpr (kQ8K) {
    qmm_q8::q8k_dst d[G];
    bool st[G];
#pragma unroll
    for (int t = 0; t < G; t++) {
      st[t] = blk[t] < total;
      d[t] = qmm_q8::q8k_decode_dst(s_act, st[t] ? blk[t] : 0);
    }
    qmm_q8::q8k_waves<G>(v, lane, d, st);
  }
#pragma unroll
  for (int t = 0; t < G; t++) {
    if constexpr (!kQ8K) {
      uint8_t *b = s_act + (int64_t)(blk[t] < total ? blk[t] : 0) * 34;
      qmm_q8::q8_0_group(v[t], lane & 7, (int8_t *)(b + 2), (uint16_t *)b, blk[t] < total);
    }
  }
  __syncthreads();
  if (row >= nrows) return;  // whole wave
  constexpr bool kRegs = NC * S <= 2;
  typename U::A areg[kRegs ? NC * S : 1];
  if (kRegs) {
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
      for (int j = 0; j < NC; j++)
        if (has(s)) U::load_a(s_act + j * act_row_bytes, lane + 64 * s, areg[kRegs ? s * NC + j : 0]);
  }
  // 4. rows row, row + tw, ... with two in flight
  row_pairs<U, Out, NC, S, FULL, kRegs>(vx, row_bytes, nunits, nrows, row, tw, lane, wa, wb, areg, s_act,
                                        act_row_bytes, dst, stride_col_dst);
}

// ------------------------------------------------------------------------------------------------ several weights

// One-launch decode over up to three weights that share one f32 activation (q / k / v, or gate and up): the
// workgroups are split between the segments in proportion to their bytes, and each workgroup quantizes the
// activation into LDS, as k_mmvq_pq does, then walks its segment's rows with two in flight.  So the activation is
// quantized in the launch that reads it, once per workgroup, and the segments share the chip in one launch.
struct PqSeg {
  const uint8_t *w;   // weight rows (GLU: the gate rows)
  const uint8_t *w2;  // GLU: the up rows
  void *dst;          // output, stride_col_dst elements per activation row
  int nrows, stride_col_dst, wg0;  // wg0: the segment's first workgroup
};
struct PqSegs {
  PqSeg s[3];
};

// pq_quantize: the f32 loads of this wave's activation blocks (step 1 of k_mmvq_pq), then, once the caller has
// issued its first weight loads, their quantization into LDS (step 3).
template <class U, int NC, int NW, int G>
struct PqAct {
  static constexpr bool kQ8K = U::kActBlockValues == 256;
  static constexpr int kBlocksPerStep = kQ8K ? 1 : 8;
  float v[G][4];
  int blk[G];
  int total;
  __device__ __forceinline__ void load(const float *__restrict__ x, int64_t stride_x, int nblk, int lane, int wave) {
    total = NC * nblk;
#pragma unroll
    for (int t = 0; t < G; t++) {
      blk[t] = (wave + NW * t) * kBlocksPerStep + (kQ8K ? 0 : lane >> 3);
      const int b = blk[t] < total ? blk[t] : 0;
      const int j = NC > 1 && b >= nblk ? 1 : 0;
      const int k0 = (b - j * nblk) * U::kActBlockValues + 4 * (kQ8K ? lane : lane & 7);
      typedef float f32x4 __attribute__((ext_vector_type(4)));
      f32x4 f;
      __builtin_memcpy(&f, __builtin_assume_aligned(x + j * stride_x + k0, 4), 16);
      v[t][0] = f.x, v[t][1] = f.y, v[t][2] = f.z, v[t][3] = f.w;
    }
  }
  __device__ __forceinline__ void quantize(uint8_t *s_act, int lane) {
    if constexpr (kQ8K) {
      qmm_q8::q8k_dst d[G];
      bool st[G];
#pragma unroll
      for (int t = 0; t < G; t++) {
        st[t] = blk[t] < total;
        d[t] = qmm_q8::q8k_decode_dst(s_act, st[t] ? blk[t] : 0);
      }
      qmm_q8::q8k_waves<G>(v, lane, d, st);
    } else {
#pragma unroll
      for (int t = 0; t < G; t++) {
        uint8_t *b = s_act + (int64_t)(blk[t] < total ? blk[t] : 0) * 34;
        qmm_q8::q8_0_group(v[t], lane & 7, (int8_t *)(b + 2), (uint16_t *)b, blk[t] < total);
      }
    }
  }
};

// The GLU form of row_pairs: buffers (ga, ua) hold row r's gate and up weights and (gb, ub) row r + tw's; each row
// stores act(W_gate . y) * (W_up . y).
template <class U, class Out, int NC, int S, bool FULL, bool kRegs>
__device__ __forceinline__ void row_pairs_glu(const uint8_t *vg, const uint8_t *vu, int64_t row_bytes, int nunits,
                                              int nrows, int row, int tw, int lane, typename U::W (&ga)[S],
                                              typename U::W (&ua)[S], typename U::W (&gb)[S], typename U::W (&ub)[S],
                                              const typename U::A *areg, const uint8_t *act, int64_t act_row_bytes,
                                              typename Out::T *dst, int stride_col_dst, int activation) {
  float g[NC], u[NC];
  auto store = [&](int r) {
#pragma unroll
    for (int j = 0; j < NC; j++) {
      const float gs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_to_lane63(g[j])), 63));
      const float us = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_to_lane63(u[j])), 63));
      Out::store(dst, (int64_t)j * stride_col_dst + r, glu_act(activation, gs) * us);
    }
  };
  for (;;) {
    row_dots<U, NC, S, FULL, kRegs>(ga, areg, act, act_row_bytes, nunits, lane, g);
    row_dots<U, NC, S, FULL, kRegs>(ua, areg, act, act_row_bytes, nunits, lane, u);
    load_row<U, S, FULL>(vg, row_bytes, nunits, nrows, row + 2 * tw, lane, ga);
    load_row<U, S, FULL>(vu, row_bytes, nunits, nrows, row + 2 * tw, lane, ua);
    store(row);
    if (row + tw >= nrows) break;
    row_dots<U, NC, S, FULL, kRegs>(gb, areg, act, act_row_bytes, nunits, lane, g);
    row_dots<U, NC, S, FULL, kRegs>(ub, areg, act, act_row_bytes, nunits, lane, u);
    load_row<U, S, FULL>(vg, row_bytes, nunits, nrows, row + 3 * tw, lane, gb);
    load_row<U, S, FULL>(vu, row_bytes, nunits, nrows, row + 3 * tw, lane, ub);
    store(row + tw);
    row += 2 * tw;
    if (row >= nrows) break;
  }
}

// One segment's part of k_mmvq_pqs: the workgroup's rows are local_block * kPqsWaves + wave + t * local_grid *
// kPqsWaves.  S units per lane (FULL: all of them in every lane).
constexpr int kPqsWaves = 8;
template <class U, class Out, int NC, int S, bool FULL, int G, bool GLU>
__device__ __forceinline__ void pqs_segment(const PqSeg &sg, int local_block, int local_grid,
                                            const float *__restrict__ x, int64_t stride_x, int nunits,
                                            uint8_t *s_act, int activation) {
  constexpr int NW = kPqsWaves;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = nunits * U::kValuesPerUnit / U::kActBlockValues;
  const int64_t act_row_bytes = (int64_t)nblk * U::kActBlockBytes;
  const int64_t row_bytes = U::row_bytes((int64_t)nunits * U::kValuesPerUnit);
  PqAct<U, NC, NW, G> qa;
  qa.load(x, stride_x, nblk, lane, wave);
  const int tw = local_grid * NW;
  int row = local_block * NW + wave;
  typename U::W ga[S], gb[S], ua[GLU ? S : 1], ub[GLU ? S : 1];
  load_row<U, S, FULL>(sg.w, row_bytes, nunits, sg.nrows, row, lane, ga);
  load_row<U, S, FULL>(sg.w, row_bytes, nunits, sg.nrows, row + tw, lane, gb);
  if constexpr (GLU) {
    load_row<U, S, FULL>(sg.w2, row_bytes, nunits, sg.nrows, row, lane, ua);
    load_row<U, S, FULL>(sg.w2, row_bytes, nunits, sg.nrows, row + tw, lane, ub);
  }
  __builtin_amdgcn_sched_barrier(0);
  qa.quantize(s_act, lane);
  __syncthreads();
  if (row >= sg.nrows) return;  // whole wave
  constexpr bool kRegs = NC * S <= 2;
  typename U::A areg[kRegs ? NC * S : 1];
  if (kRegs) {
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
      for (int j = 0; j < NC; j++)
        if (FULL || lane + 64 * s < nunits) U::load_a(s_act + j * act_row_bytes, lane + 64 * s, areg[kRegs ? s * NC + j : 0]);
  }
  typename Out::T *dst = (typename Out::T *)sg.dst;
  if constexpr (GLU)
    row_pairs_glu<U, Out, NC, S, FULL, kRegs>(sg.w, sg.w2, row_bytes, nunits, sg.nrows, row, tw, lane, ga, ua, gb, ub,
                                              areg, s_act, act_row_bytes, dst, sg.stride_col_dst, activation);
  else
    row_pairs<U, Out, NC, S, FULL, kRegs>(sg.w, row_bytes, nunits, sg.nrows, row, tw, lane, ga, gb, areg, s_act,
                                          act_row_bytes, dst, sg.stride_col_dst);
}

// Segments [0, NA) take unit UA, the rest UB (which share UA's activation format); NS segments in all.
template <class UA, class UB, int NA, int NS, class Out, int NC, int S, bool FULL, int G, bool GLU>
__global__ __launch_bounds__(64 * kPqsWaves) void k_mmvq_pqs(PqSegs segs, const float *__restrict__ x,
                                                             int64_t stride_x, int nunits, int activation) {
  static_assert(UA::kActBlockValues == UB::kActBlockValues && UA::kActBlockBytes == UB::kActBlockBytes,
                "segments share one quantized activation");
  extern __shared__ __align__(16) uint8_t s_act[];
  const int b = blockIdx.x;
  int si = 0;
#pragma unroll
  for (int i = 1; i < NS; i++)
    if (b >= segs.s[i].wg0) si = i;
  const int end = si + 1 < NS ? segs.s[si + 1 < NS ? si + 1 : 0].wg0 : (int)gridDim.x;
  const int local = b - segs.s[si].wg0, grid = end - segs.s[si].wg0;
  // the segment is uniform over the workgroup
  if (si < NA)
    pqs_segment<UA, Out, NC, S, FULL, G, GLU>(segs.s[si], local, grid, x, stride_x, nunits, s_act, activation);
  else
    pqs_segment<UB, Out, NC, S, FULL, G, GLU>(segs.s[si], local, grid, x, stride_x, nunits, s_act, activation);
}

// MoE matvec: grid (pairs, row groups) -- pairs innermost so the pairs of one expert share the row group's
// weights through L2.  dst[p * nrows + row] = W_gate[ids[p]] . y[p / y_div]  (or act(gate) * up).
template <class U, int R, bool GLU>
__global__ __launch_bounds__(256) void k_mmvq_moe(const uint8_t *__restrict__ vx_gate, const uint8_t *__restrict__ vx_up,
                                                  int64_t expert_stride, const uint8_t *__restrict__ vy,
                                                  const uint32_t *__restrict__ ids, float *__restrict__ dst, int nrows,
                                                  int64_t row_bytes, int nunits, int64_t act_row_bytes, int y_div,
                                                  int activation) {
  const int lane = threadIdx.x & 63;
  const int pair = blockIdx.x;
  const int row0 = (blockIdx.y * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= nrows) return;
  const int64_t e = ids[pair];
  const uint8_t *wg = vx_gate + e * expert_stride;
  const uint8_t *wu = GLU ? vx_up + e * expert_stride : nullptr;
  const uint8_t *act = vy + (int64_t)(pair / y_div) * act_row_bytes;
  float ag[R], au[R];
#pragma unroll
  for (int r = 0; r < R; r++) ag[r] = au[r] = 0.0f;
  for (int u = lane; u < nunits; u += QMM_WAVE) {
    typename U::W w[R], w2[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = min(row0 + r, nrows - 1);
      U::load_w(wg + (int64_t)row * row_bytes, u, w[r]);
      if (GLU) U::load_w(wu + (int64_t)row * row_bytes, u, w2[r]);
    }
    typename U::A a;
    U::load_a(act, u, a);
#pragma unroll
    for (int r = 0; r < R; r++) {
      ag[r] += U::dot(w[r], a, u);
      if (GLU) au[r] += U::dot(w2[r], a, u);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float g = wave_sum_to_lane63(ag[r]);
    float v = g;
    if (GLU) v = glu_act(activation, g) * wave_sum_to_lane63(au[r]);
    if (lane == 63 && row0 + r < nrows) dst[(int64_t)pair * nrows + row0 + r] = v;
  }
}

// The MoE down projection with the weighted sum over a token's routes folded in: grid (tokens, row groups);
// dst[t * nrows + row] = sum over s < topk, in order, of w[t, s] * (W[ids[t, s]] . y[t * topk + s]).  Each route's
// dot is the same per-lane sum and wave reduction as k_mmvq_moe's, and the sum over routes is the same expression,
// in the same order, as the standalone weighted reduce, so the result equals the two-kernel sequence's.  A route of
// weight zero is skipped, as the reduce skips reading it.
// ACC: added to what dst holds (the reference's fused down projection accumulates into a zeroed buffer)
template <class U, int R, bool ACC = false>
__global__ __launch_bounds__(256) void k_mmvq_moe_wsum(const uint8_t *__restrict__ vx, int64_t expert_stride,
                                                       const uint8_t *__restrict__ vy, const uint32_t *__restrict__ ids,
                                                       const float *__restrict__ weights, float *__restrict__ dst,
                                                       int nrows, int64_t row_bytes, int nunits, int64_t act_row_bytes,
                                                       int topk) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  const int row0 = (blockIdx.y * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= nrows) return;
  float out[R];
#pragma unroll
  for (int r = 0; r < R; r++) out[r] = 0.0f;
  for (int sl = 0; sl < topk; sl++) {
    const int64_t pair = (int64_t)t * topk + sl;
    const float ws = weights[pair];
    if (ws == 0.0f) continue;  // uniform over the workgroup
    const uint8_t *w = vx + (int64_t)ids[pair] * expert_stride;
    const uint8_t *act = vy + pair * act_row_bytes;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int u = lane; u < nunits; u += QMM_WAVE) {
      typename U::W wr[R];
#pragma unroll
      for (int r = 0; r < R; r++) U::load_w(w + (int64_t)min(row0 + r, nrows - 1) * row_bytes, u, wr[r]);
      typename U::A a;
      U::load_a(act, u, a);
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] += U::dot(wr[r], a, u);
    }
#pragma unroll
    for (int r = 0; r < R; r++) out[r] += wave_sum_to_lane63(acc[r]) * ws;
  }
#pragma unroll
  for (int r = 0; r < R; r++)
    if (lane == 63 && row0 + r < nrows) {
      float *o = dst + (int64_t)t * nrows + row0 + r;
      *o = ACC ? *o + out[r] : out[r];
    }
}

template <class U, class Out, int NC>
void launch_nc(const uint8_t *vx, const uint8_t *vy, typename Out::T *dst, int k, int nrows, int64_t act_row_bytes,
               int stride_col_dst, hipStream_t s) {
  constexpr int R = NC <= 2 ? 4 : 2;
  const dim3 grid((unsigned)qmm_ceil_div(nrows, kWaves * R));
  k_mmvq<U, Out, NC, R><<<grid, 256, 0, s>>>(vx, vy, dst, nrows, U::row_bytes(k), U::units(k), act_row_bytes,
                                             stride_col_dst);
}

// Persistent launch of NC columns with S units per lane: grid capped at 8 workgroups per CU.  When the rows would
// last at most two rounds of the workgroups the kernel's registers let a CU hold, the grid is capped at one round
// instead, so each wave takes both of its rows with the second one's weights requested before the first one's
// math (a second round of one-row workgroups requests nothing early).  On MI355X at b = 1 that measured: Q6_K
// 4096 x 14336 (2 waves per SIMD) 14.7 -> 14.2 us, IQ4_XS 11.7 -> 10.5 us, Q5_0 12.8 -> 11.8 us.  Longer runs keep
// the 8-per-CU grid, whose queued workgroups the hardware hands out as CUs free up: capped at one round, Q5_K
// 14336 x 4096 (3 waves per SIMD, 4.7 rows per wave) measured 9.9 -> 10.2 us.
template <class U, class Out>
void launch_p(int nc, int S, const uint8_t *vx, const uint8_t *act, typename Out::T *dst, int k, int nrows,
              int64_t act_row_bytes, int stride_col_dst, hipStream_t s) {
  const int64_t wgs = qmm_ceil_div(nrows, kWaves);
  auto grid = [&](int per_cu) {
    const int64_t round = (int64_t)(per_cu < 8 ? per_cu : 8) * qmm_device_cus();
    const int64_t cap = wgs <= 2 * round ? round : 8 * (int64_t)qmm_device_cus();
    return dim3((unsigned)(wgs < cap ? wgs : cap));
  };
  const int64_t rb = U::row_bytes(k);
  const int nu = U::units(k);
  const bool full = decode_form<U>(nu, nc).full;
#define QMM_P_F(NC, SS, FF)                                                                                    \
  k_mmvq_p<U, Out, NC, SS, FF><<<grid(qmm_resident_per_cu<k_mmvq_p<U, Out, NC, SS, FF>>(256, 0)), 256, 0, s>>>( \
      vx, act, dst, nrows, rb, nu, act_row_bytes, stride_col_dst)
#define QMM_P(NC, SS)         \
  do {                        \
    if (full)                 \
      QMM_P_F(NC, SS, true);  \
    else                      \
      QMM_P_F(NC, SS, false); \
  } while (0)
#define QMM_P_S(NC)                \
  switch (S) {                     \
    case 1: QMM_P(NC, 1); break;   \
    case 2: QMM_P(NC, 2); break;   \
    default: QMM_P(NC, 4); break;  \
  }
  switch (nc) {
    case 1: QMM_P_S(1) break;
    case 2: QMM_P_S(2) break;
    case 3: QMM_P_S(3) break;
    case 4: QMM_P_S(4) break;
    case 5: QMM_P_S(5) break;
    case 6: QMM_P_S(6) break;
    case 7: QMM_P_S(7) break;
    default: QMM_P_S(8) break;
  }
#undef QMM_P_S
#undef QMM_P
#undef QMM_P_F
}

inline int out_type_of(const out_f32 *) { return QMM_TYPE_F32; }
inline int out_type_of(const out_f16 *) { return QMM_TYPE_F16; }
inline int out_type_of(const out_bf16 *) { return QMM_TYPE_BF16; }

template <class U, class Out>
void launch_cols(const uint8_t *vx, const uint8_t *vy, typename Out::T *dst, int k, int nrows, int64_t act_row_bytes,
                 int stride_col_dst, int b, hipStream_t s) {
  if (decode_form<U>(U::units(k), 1).kernel != kFormPasses) {
    for (int j0 = 0; j0 < b; j0 += 8) {
      const int nc = b - j0 < 8 ? b - j0 : 8;
      const DecodeForm f = decode_form<U>(U::units(k), nc);
      if (use_p4<U>(U::units(k), nc, nrows))
        launch_p4<U, Out>(vx, vy + (int64_t)j0 * act_row_bytes, dst + (int64_t)j0 * stride_col_dst, k, nrows, s);
      else if (f.kernel == kFormP2)
        launch_p2<U, Out>(nc, vx, vy + (int64_t)j0 * act_row_bytes, dst + (int64_t)j0 * stride_col_dst, k, nrows,
                          act_row_bytes, stride_col_dst, s);
      else
        launch_p<U, Out>(nc, f.s, vx, vy + (int64_t)j0 * act_row_bytes, dst + (int64_t)j0 * stride_col_dst, k, nrows,
                         act_row_bytes, stride_col_dst, s);
    }
    return;
  }
  // up to 8 columns per pass; weights are re-streamed once per further pass
  for (int j0 = 0; j0 < b; j0 += 8) {
    const int nc = b - j0 < 8 ? b - j0 : 8;
    const uint8_t *y = vy + (int64_t)j0 * act_row_bytes;
    typename Out::T *d = dst + (int64_t)j0 * stride_col_dst;
    switch (nc) {
      case 1: launch_nc<U, Out, 1>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 2: launch_nc<U, Out, 2>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 3: launch_nc<U, Out, 3>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 4: launch_nc<U, Out, 4>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 5: launch_nc<U, Out, 5>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 6: launch_nc<U, Out, 6>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 7: launch_nc<U, Out, 7>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      default: launch_nc<U, Out, 8>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
    }
  }
}

// Fused quantization: two workgroups per CU, of 8 waves for tall weights (at least 8192 rows: more rows per wave)
// and of 16 below (each activation row quantized by half as many workgroups), as measured fastest on MI355X;
// one unit per lane (rows of at most 4096 values, which keeps the kernel within 64 VGPRs).
template <class U, class Out, int NC, int NW>
void launch_pq_nw(const uint8_t *vx, const float *x, int64_t stride_x, typename Out::T *dst, int k, int nrows,
                  int stride_col_dst, hipStream_t s) {
  const int nu = U::units(k);
  const bool full = nu % 64 == 0;
  const int nblk = nu * U::kValuesPerUnit / U::kActBlockValues;
  const int steps = (int)qmm_ceil_div((int64_t)NC * nblk, U::kActBlockValues == 256 ? 1 : 8);  // <= 32
  const int64_t wgs = qmm_ceil_div(nrows, NW);
  const size_t lds = (size_t)NC * nblk * U::kActBlockBytes;
  const int64_t rb = U::row_bytes(k);
  // Resident workgroups per CU: one for the 8-wave form (tall weights: 7 rows per wave at 14336 rows, so the two-row
  // pipeline of each wave runs long; two measured 3% slower on MI355X), two for the 16-wave form (short weights),
  // fewer when the kernel's registers allow only one.
  const int kCap = NW == 8 ? 1 : 2;
  auto grid = [&](int per_cu) {
    const int64_t cap = (int64_t)(per_cu < kCap ? per_cu : kCap) * qmm_device_cus();
    return dim3((unsigned)(wgs < cap ? wgs : cap));
  };
#define QMM_PQ_F(FF, GG)                                                                                            \
  k_mmvq_pq<U, Out, NC, 1, FF, NW, GG><<<grid(qmm_resident_per_cu<k_mmvq_pq<U, Out, NC, 1, FF, NW, GG>>(64 * NW, lds)), \
                                         64 * NW, lds, s>>>(vx, x, stride_x, dst, nrows, rb, nu, stride_col_dst)
#define QMM_PQ(GG)          \
  do {                      \
    if (full)               \
      QMM_PQ_F(true, GG);   \
    else                    \
      QMM_PQ_F(false, GG);  \
  } while (0)
  if (steps <= NW)
    QMM_PQ(1);
  else if (steps <= 2 * NW)
    QMM_PQ(2);
  else
    QMM_PQ(4);
#undef QMM_PQ
#undef QMM_PQ_F
}

template <class U, class Out, int NC>
void launch_pq(const uint8_t *vx, const float *x, int64_t stride_x, typename Out::T *dst, int k, int nrows,
               int stride_col_dst, hipStream_t s) {
  if (nrows >= 8192)
    launch_pq_nw<U, Out, NC, 8>(vx, x, stride_x, dst, k, nrows, stride_col_dst, s);
  else
    launch_pq_nw<U, Out, NC, 16>(vx, x, stride_x, dst, k, nrows, stride_col_dst, s);
}


// Grid of k_mmvq_pqs: 8-wave workgroups, two per CU (one for the GLU form, whose waves hold two rows' weights per
// step; measured on MI355X at the Llama-3 shapes: q/k/v 8.5 us at two per CU against 10.3 us for one 16-wave
// workgroup per CU, gate/up 15.2 against 16.1 us at two), split between the segments in proportion to their weight
// bytes (each at least one workgroup, and none more workgroups than its rows fill).  rows[i], w[i], w2[i], dst[i] per
// segment.  One unit per lane (k <= 4096).
template <class UA, class UB, int NA, int NS, class Out, int NC, bool GLU>
void launch_pqs(const uint8_t *const *w, const uint8_t *const *w2, typename Out::T *const *dst, const int *rows,
                const float *x, int64_t stride_x, int k, const int *stride_col_dst, int activation, hipStream_t s) {
  constexpr int NW = kPqsWaves;
  const int nu = UA::units(k);
  const int nblk = nu * UA::kValuesPerUnit / UA::kActBlockValues;
  const int steps = (int)qmm_ceil_div((int64_t)NC * nblk, UA::kActBlockValues == 256 ? 1 : 8);
  const size_t lds = (size_t)NC * nblk * UA::kActBlockBytes;
  double bytes[3] = {0, 0, 0}, all = 0;
  for (int i = 0; i < NS; i++) {
    bytes[i] = (double)rows[i] * (double)(i < NA ? UA::row_bytes(k) : UB::row_bytes(k)) * (GLU ? 2 : 1);
    all += bytes[i];
  }
  auto go = [&](auto s_tag, auto g_tag, auto full_tag) {
    constexpr int S = decltype(s_tag)::value, G = decltype(g_tag)::value;
    constexpr bool FF = decltype(full_tag)::value;
    const int per_cu = qmm_resident_per_cu<k_mmvq_pqs<UA, UB, NA, NS, Out, NC, S, FF, G, GLU>>(64 * NW, lds);
    const int cap = GLU ? 1 : 2;
    const int wgs = (per_cu < cap ? per_cu : cap) * qmm_device_cus();
    PqSegs segs = {};
    int next = 0;
    for (int i = 0; i < NS; i++) {
      int n = (int)(wgs * bytes[i] / all + 0.5);
      const int most = (int)qmm_ceil_div(rows[i], NW);
      n = n < 1 ? 1 : (n > most ? most : n);
      segs.s[i] = PqSeg{w[i], GLU ? w2[i] : nullptr, (void *)dst[i], rows[i], stride_col_dst[i], next};
      next += n;
    }
    k_mmvq_pqs<UA, UB, NA, NS, Out, NC, S, FF, G, GLU><<<dim3((unsigned)next), 64 * NW, lds, s>>>(segs, x, stride_x,
                                                                                                 nu, activation);
  };
  typedef std::integral_constant<int, 1> i1;
  typedef std::integral_constant<int, 2> i2;
  typedef std::integral_constant<int, 4> i4;
  auto pick_full = [&](auto s_tag, auto g_tag) {
    if (nu == 64 * decltype(s_tag)::value)
      go(s_tag, g_tag, std::true_type());
    else
      go(s_tag, g_tag, std::false_type());
  };
  if (steps <= NW)
    pick_full(i1(), i1());
  else if (steps <= 2 * NW)
    pick_full(i1(), i2());
  else
    pick_full(i1(), i4());
}

template <class U>
void moe_launch(const void *vx_gate, const void *vx_up, int64_t expert_stride, const void *vy, const void *ids,
                float *dst, int ncols_x, int nrows_x, int64_t act_row_bytes, int y_div, int n_pairs, int activation,
                hipStream_t s) {
  constexpr int R = 2;
  const dim3 grid((unsigned)n_pairs, (unsigned)qmm_ceil_div(nrows_x, kWaves * R));
  if (vx_up)
    k_mmvq_moe<U, R, true><<<grid, 256, 0, s>>>((const uint8_t *)vx_gate, (const uint8_t *)vx_up, expert_stride,
                                                (const uint8_t *)vy, (const uint32_t *)ids, dst, nrows_x,
                                                U::row_bytes(ncols_x), U::units(ncols_x), act_row_bytes, y_div,
                                                activation);
  else
    k_mmvq_moe<U, R, false><<<grid, 256, 0, s>>>((const uint8_t *)vx_gate, nullptr, expert_stride,
                                                 (const uint8_t *)vy, (const uint32_t *)ids, dst, nrows_x,
                                                 U::row_bytes(ncols_x), U::units(ncols_x), act_row_bytes, y_div,
                                                 activation);
}


template <class U, bool ACC = false>
void moe_wsum_launch(const void *vx, int64_t expert_stride, const void *vy, const void *ids, const float *weights,
                     float *dst, int ncols_x, int nrows_x, int64_t act_row_bytes, int n_tokens, int topk,
                     hipStream_t s) {
  constexpr int R = 2;  // as moe_launch, so each route's dot is the same sum
  const dim3 grid((unsigned)n_tokens, (unsigned)qmm_ceil_div(nrows_x, kWaves * R));
  k_mmvq_moe_wsum<U, R, ACC><<<grid, 256, 0, s>>>((const uint8_t *)vx, expert_stride, (const uint8_t *)vy,
                                             (const uint32_t *)ids, weights, dst, nrows_x, U::row_bytes(ncols_x),
                                             U::units(ncols_x), act_row_bytes, topk);
}


// ------------------------------------------------------------------------------------------------ per-type dispatch

// Shape checks shared by the decode launchers. Returns false (and records why) when the arguments cannot be served.
// Slots: stride_col_y counts 36-byte Q8_1 blocks of 32 values, a whole number of 288-byte slots (a multiple of 8);
// Q8_0 blocks: stride_col_y counts 34-byte blocks.
template <int T, int F>
bool check_mmvq(const char *who, const void *vx, int ncols_x, int nrows_x, int stride_col_y, int b) {
  const int bs = (int)qmm_block_size(T);
  if (ncols_x <= 0 || nrows_x <= 0 || ncols_x % bs != 0) {
    qmm_set_error("%s: ncols_x=%d nrows_x=%d (ncols_x must be a positive multiple of %d)", who, ncols_x, nrows_x, bs);
    return false;
  }
  if ((int64_t)stride_col_y * 32 < ncols_x || (F == kActSlots && stride_col_y % 8 != 0)) {
    qmm_set_error("%s: stride_col_y=%d blocks of 32 values hold fewer than ncols_x=%d values%s", who, stride_col_y,
                  ncols_x, F == kActSlots ? " or are not whole 256-value slots" : "");
    return false;
  }
  // Q4_K / Q6_K take up to 32 rows (the few-row MFMA kernel holds 32 activation rows in one tile); the rest 16
  const int bmax = T == QMM_TYPE_Q4K || T == QMM_TYPE_Q6K ? 32 : 16;
  if (b < 0 || b > bmax) {
    qmm_set_error("%s: b_size=%d outside 1..%d", who, b, bmax);
    return false;
  }
  if ((uintptr_t)vx % weight_align(T) != 0) {
    qmm_set_error("%s: weight pointer not %zu-byte aligned", who, (size_t)weight_align(T));
    return false;
  }
  return true;
}

// Rows the non-persistent kernel serves: the 32-value types' odd-block rows (a rare shape) take only k_mmvq, so their
// units add few kernels to the build.
template <class U, class Out>
void launch_nc_cols(const uint8_t *vx, const uint8_t *vy, typename Out::T *dst, int k, int nrows, int64_t act_row_bytes,
                    int stride_col_dst, int b, hipStream_t s) {
  for (int j0 = 0; j0 < b; j0 += 8) {
    const int nc = b - j0 < 8 ? b - j0 : 8;
    const uint8_t *y = vy + (int64_t)j0 * act_row_bytes;
    typename Out::T *d = dst + (int64_t)j0 * stride_col_dst;
    switch (nc) {
      case 1: launch_nc<U, Out, 1>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 2: launch_nc<U, Out, 2>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 3: launch_nc<U, Out, 3>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 4: launch_nc<U, Out, 4>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 5: launch_nc<U, Out, 5>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 6: launch_nc<U, Out, 6>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      case 7: launch_nc<U, Out, 7>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
      default: launch_nc<U, Out, 8>(vx, y, d, k, nrows, act_row_bytes, stride_col_dst, s); break;
    }
  }
}

// launch_mmvq_gguf_<t>_<dt>_plain (slots) and its _plain_q8_0 twin
template <int T, int F, class Out>
void plain_t(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int stride_col_y, int stride_col_dst,
             int b, void *stream, const char *who) {
  if (!check_mmvq<T, F>(who, vx, ncols_x, nrows_x, stride_col_y, b)) return;
  if (b == 0) return;
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
  typename Out::T *d = (typename Out::T *)dst;
  if constexpr (T == QMM_TYPE_Q4K || T == QMM_TYPE_Q6K) {
    if (b >= qmm_skinny_min_rows(T) &&
        qmm_skinny_decode(T, out_type_of((const Out *)nullptr), vx, vy, dst, ncols_x, nrows_x, stride_col_y,
                          stride_col_dst, b, s))
      return;
  }
  typedef decode_units<T, F> DU;
  const int64_t ay = act_row_bytes<F>(stride_col_y);
  if (reads_pairs<T, F>(ncols_x, stride_col_y, vy, {vx}))
    launch_cols<typename DU::pairs, Out>(x, y, d, ncols_x, nrows_x, ay, stride_col_dst, b, s);
  else
    launch_nc_cols<typename DU::odd, Out>(x, y, d, ncols_x, nrows_x, ay, stride_col_dst, b, s);
}

// launch_mmvq_gguf_<t>_<dt>_quantize_plain: the one-launch decode of Q8_0 / Q4_K / Q6_K (b 1 or 2, K <= 4096)
template <int T, class Out>
void quantize_plain_t(const void *vx, const float *x, void *dst, int ncols_x, int nrows_x, int stride_col_x,
                      int stride_col_dst, int b, void *stream, const char *who) {
  const int bs = (int)qmm_block_size(T);
  if (ncols_x <= 0 || nrows_x <= 0 || ncols_x % bs != 0 || (T == QMM_TYPE_Q8_0 && ncols_x % 64 != 0)) {
    qmm_set_error("%s: ncols_x=%d nrows_x=%d (ncols_x must be a positive multiple of %d)", who, ncols_x, nrows_x,
                  T == QMM_TYPE_Q8_0 ? 64 : bs);
    return;
  }
  if (b < 0 || b > 2 || (b > 1 && stride_col_x < ncols_x)) {
    qmm_set_error("%s: b_size=%d (1 or 2) stride_col_x=%d ncols_x=%d", who, b, stride_col_x, ncols_x);
    return;
  }
  // Up to 4096 values: one unit per lane, every activation block of the b rows within a few wave steps of one
  // workgroup, quantized into LDS.  (Rows of four units per lane, K = 14336, quantized into LDS the same way measured
  // slower on MI355X than the two launches: Q6_K 4096 x 14336 26.3 against 17.2 us.)  Above, at one column: the
  // four-wave form, each lane quantizing its own unit in registers.
  const bool wide = ncols_x > 64 * 64;
  if (wide && (b > 1 || ncols_x > 256 * 64)) {
    qmm_set_error("%s: ncols_x=%d b_size=%d (at most 4096, or 16384 at b_size 1)", who, ncols_x, b);
    return;
  }
  const uintptr_t align = T == QMM_TYPE_Q6K ? 2 : (T == QMM_TYPE_Q8_0 ? 4 : 16);
  const uintptr_t xalign = wide ? 16 : 4;
  if ((uintptr_t)vx % align != 0 || (uintptr_t)x % xalign != 0) {
    qmm_set_error("%s: weights must be %zu-byte and x %zu-byte aligned", who, (size_t)align, (size_t)xalign);
    return;
  }
  if (b == 0) return;
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *w = (const uint8_t *)vx;
  typename Out::T *d = (typename Out::T *)dst;
  typedef typename std::conditional<T == QMM_TYPE_Q4K, unit_q4k,
                                    typename std::conditional<T == QMM_TYPE_Q6K, unit_q6k, unit_q8_0>::type>::type U;
  if (wide)
    launch_p4<U, Out, true>(w, x, d, ncols_x, nrows_x, s);
  else if (b == 1)
    launch_pq<U, Out, 1>(w, x, stride_col_x, d, ncols_x, nrows_x, stride_col_dst, s);
  else
    launch_pq<U, Out, 2>(w, x, stride_col_x, d, ncols_x, nrows_x, stride_col_dst, s);
}

// The reference's tensor-core matvec entries (launch_mmvq_tc_gguf_<t>_<dt>_plain, crates/inference-quant/src/gguf/
// ffi.rs:966-998; routed by fast_mmvq.rs:505-513 for 1..16 rows) over the tensor-core entries' activation layout
// (launch_mmvq_tc_quantize_*: rows of ncols_x / 256 blocks {f32 d; int8 qs[256]}, units.h): the persistent matvec
// below the few-row threshold, the few-row MFMA kernel from it, with the same integer dots as the plain entries.
// cfg names one of the reference's CUDA tile shapes (fast_mmvq.rs:1845-1881); it is accepted and has no meaning here.
// b_size 1..32 (the reference passes at most 16).
// the unit of the one-launch forms (their activation is quantized into LDS in the 292- / 34-byte block layouts)
template <int T>
using pq_unit = typename std::conditional<T == QMM_TYPE_Q4K, unit_q4k,
                                          typename std::conditional<T == QMM_TYPE_Q6K, unit_q6k, unit_q8_0>::type>::type;

// the argument checks of the one-launch forms: b 1 or 2, ncols_x <= 4096 (one unit per lane), aligned weights
// (a null weight among ws is skipped: the caller's empty projection)
inline bool check_pq(const char *who, int type, std::initializer_list<const void *> ws, const float *x, int ncols_x,
                     int stride_col_x, int b, bool null_ok = false) {
  const int bs = (int)qmm_block_size(type);
  if (ncols_x <= 0 || ncols_x % bs != 0 || (type == QMM_TYPE_Q8_0 && ncols_x % 64 != 0) || ncols_x > 64 * 64) {
    qmm_set_error("%s: ncols_x=%d (a positive multiple of %d, at most 4096)", who, ncols_x,
                  type == QMM_TYPE_Q8_0 ? 64 : bs);
    return false;
  }
  if (b < 0 || b > 2 || (b > 1 && stride_col_x < ncols_x)) {
    qmm_set_error("%s: b_size=%d (1 or 2) stride_col_x=%d ncols_x=%d", who, b, stride_col_x, ncols_x);
    return false;
  }
  const uintptr_t align = type == QMM_TYPE_Q6K ? 2 : (type == QMM_TYPE_Q8_0 ? 4 : 16);
  for (const void *w : ws)
    if ((!w && !null_ok) || (uintptr_t)w % align != 0) {
      qmm_set_error("%s: weights must be non-null and %zu-byte aligned", who, (size_t)align);
      return false;
    }
  if (!x || (uintptr_t)x % 4 != 0) {
    qmm_set_error("%s: x must be non-null and 4-byte aligned", who);
    return false;
  }
  return true;
}

// launch_mmvq_gguf_<t>_<dt>_fused_glu_quantize: dst = act(W_gate . Q(x)) * (W_up . Q(x)), x quantized in the launch
template <int T, class Out>
void fused_glu_quantize_t(const void *vx_gate, const void *vx_up, const float *x, void *dst, int ncols_x,
                          int nrows_x, int stride_col_x, int stride_col_dst, int b, int activation, void *stream,
                          const char *who) {
  if (!check_pq(who, T, {vx_gate, vx_up}, x, ncols_x, stride_col_x, b)) return;
  if (nrows_x < 0 || stride_col_dst < nrows_x || activation < 0 || activation >= kGluActivations) {
    qmm_set_error("%s: nrows_x=%d stride_col_dst=%d activation=%d", who, nrows_x, stride_col_dst, activation);
    return;
  }
  if (b == 0 || nrows_x == 0) return;
  typedef pq_unit<T> U;
  const uint8_t *w[1] = {(const uint8_t *)vx_gate}, *w2[1] = {(const uint8_t *)vx_up};
  typename Out::T *d[1] = {(typename Out::T *)dst};
  const int rows[1] = {nrows_x}, ldd[1] = {stride_col_dst};
  if (b == 1)
    launch_pqs<U, U, 1, 1, Out, 1, true>(w, w2, d, rows, x, stride_col_x, ncols_x, ldd, activation, (hipStream_t)stream);
  else
    launch_pqs<U, U, 1, 1, Out, 2, true>(w, w2, d, rows, x, stride_col_x, ncols_x, ldd, activation, (hipStream_t)stream);
}

// launch_mmvq_gguf_<t>_<dt>_fused_qkv_quantize (TV = T) and the mixed form with Q6_K v weights (T = Q4_K):
// q / k / v = W_q / W_k / W_v . Q(x), x quantized in the launch; each output row holds nrows_* values
template <int T, int TV, class Out>
void fused_qkv_quantize_t(const void *vx_q, const void *vx_k, const void *vx_v, const float *x, void *q_dst,
                          void *k_dst, void *v_dst, int ncols_x, int nrows_q, int nrows_k, int nrows_v,
                          int stride_col_x, int b, void *stream, const char *who) {
  // the weights and outputs of an empty projection are not read and may be null
  const void *none = nullptr;
  if (!check_pq(who, T, {nrows_q ? vx_q : none, nrows_k ? vx_k : none}, x, ncols_x, stride_col_x, b, true)) return;
  if (!check_pq(who, TV, {nrows_v ? vx_v : none}, x, ncols_x, stride_col_x, b, true)) return;
  if ((nrows_q && !vx_q) || (nrows_k && !vx_k) || (nrows_v && !vx_v)) {
    qmm_set_error("%s: weights of non-empty projections must be non-null", who);
    return;
  }
  if (nrows_q < 0 || nrows_k < 0 || nrows_v < 0 || (nrows_q && !q_dst) || (nrows_k && !k_dst) ||
      (nrows_v && !v_dst)) {
    qmm_set_error("%s: nrows_q=%d nrows_k=%d nrows_v=%d (outputs of non-empty projections non-null)", who, nrows_q,
                  nrows_k, nrows_v);
    return;
  }
  if (b == 0) return;
  typedef pq_unit<T> UA;
  typedef pq_unit<TV> UB;
  // empty segments are left out
  const uint8_t *w[3];
  typename Out::T *d[3];
  int rows[3], ldd[3], n = 0, na = 0;
  const void *ws[3] = {vx_q, vx_k, vx_v};
  void *ds[3] = {q_dst, k_dst, v_dst};
  const int rs[3] = {nrows_q, nrows_k, nrows_v};
  for (int i = 0; i < 3; i++) {
    if (rs[i] == 0) continue;
    w[n] = (const uint8_t *)ws[i];
    d[n] = (typename Out::T *)ds[i];
    rows[n] = ldd[n] = rs[i];
    n++;
    if (i < 2) na = n;
  }
  if (n == 0) return;
  hipStream_t s = (hipStream_t)stream;
#define QMM_PQS(NA, NS)                                                                                          \
  (b == 1 ? launch_pqs<UA, UB, NA, NS, Out, 1, false>(w, nullptr, d, rows, x, stride_col_x, ncols_x, ldd, 0, s)  \
          : launch_pqs<UA, UB, NA, NS, Out, 2, false>(w, nullptr, d, rows, x, stride_col_x, ncols_x, ldd, 0, s))
  if (n == 3)
    QMM_PQS(2, 3);
  else if (n == 2 && na == 2)
    QMM_PQS(2, 2);
  else if (n == 2)
    QMM_PQS(1, 2);
  else if (na == 1)
    QMM_PQS(1, 1);
  else
    QMM_PQS(0, 1);
#undef QMM_PQS
}

template <int T, class Out>
void tc_plain_t(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int stride_col_dst, int b,
                int cfg, void *stream, const char *who) {
  (void)cfg;
  if (!check_mmvq<T, kActSlots>(who, vx, ncols_x, nrows_x, ncols_x / 32, b)) return;
  if (b == 0) return;
  hipStream_t s = (hipStream_t)stream;
  if (b >= qmm_skinny_min_rows(T) &&
      qmm_skinny_tc(T, out_type_of((const Out *)nullptr), vx, vy, dst, ncols_x, nrows_x, stride_col_dst, b, s))
    return;
  typedef typename std::conditional<T == QMM_TYPE_Q4K, unit_q4k_tc, unit_q6k_tc>::type U;
  launch_cols<U, Out>((const uint8_t *)vx, (const uint8_t *)vy, (typename Out::T *)dst, ncols_x, nrows_x,
                      (int64_t)(ncols_x / 256) * 260, stride_col_dst, b, s);
}

// launch_mmvq_gguf_<t>_moe (slots) and its _moe_q8_0 twin
template <int T, int F>
void moe_t(const void *vx_gate, const void *vx_up, int64_t expert_stride, const void *vy, const void *ids, float *dst,
           int ncols_x, int nrows_x, int stride_col_y, int y_div, int n_pairs, int activation, void *stream,
           const char *who) {
  if (!check_mmvq<T, F>(who, vx_gate, ncols_x, nrows_x, stride_col_y, 1)) return;
  if (n_pairs < 0 || y_div <= 0 || activation < 0 || activation >= kGluActivations || expert_stride < 0) {
    qmm_set_error("%s: n_pairs=%d y_div=%d activation=%d expert_stride=%lld", who, n_pairs, y_div, activation,
                  (long long)expert_stride);
    return;
  }
  if (n_pairs == 0) return;
  if (n_pairs > 65535 * 1024) {
    qmm_set_error("%s: n_pairs=%d too large", who, n_pairs);
    return;
  }
  if (expert_stride % (int64_t)weight_align(T) != 0 || (vx_up && (uintptr_t)vx_up % weight_align(T) != 0)) {
    qmm_set_error("%s: expert_stride / vx_up not %zu-byte aligned", who, (size_t)weight_align(T));
    return;
  }
  hipStream_t s = (hipStream_t)stream;
  typedef decode_units<T, F> DU;
  const int64_t ay = act_row_bytes<F>(stride_col_y);
  if (reads_pairs<T, F>(ncols_x, stride_col_y, vy, {vx_gate, vx_up}, expert_stride))
    moe_launch<typename DU::pairs>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x, ay, y_div, n_pairs,
                                   activation, s);
  else
    moe_launch<typename DU::odd>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x, ay, y_div, n_pairs,
                                 activation, s);
}

// launch_mmvq_gguf_<t>_moe_wsum (slots) and its _moe_wsum_q8_0 twin (ACC: added to dst)
template <int T, int F, bool ACC = false>
void moe_wsum_t(const void *vx, int64_t expert_stride, const void *vy, const void *ids, const float *weights,
                float *dst, int ncols_x, int nrows_x, int stride_col_y, int n_tokens, int topk, void *stream,
                const char *who) {
  if (!check_mmvq<T, F>(who, vx, ncols_x, nrows_x, stride_col_y, 1)) return;
  if (n_tokens < 0 || n_tokens > 65535 * 1024 || topk <= 0 || expert_stride < 0 || !weights) {
    qmm_set_error("%s: n_tokens=%d topk=%d expert_stride=%lld weights=%p", who, n_tokens, topk,
                  (long long)expert_stride, (const void *)weights);
    return;
  }
  if (n_tokens == 0) return;
  if (expert_stride % (int64_t)weight_align(T) != 0) {
    qmm_set_error("%s: expert_stride not %zu-byte aligned", who, (size_t)weight_align(T));
    return;
  }
  hipStream_t s = (hipStream_t)stream;
  typedef decode_units<T, F> DU;
  const int64_t ay = act_row_bytes<F>(stride_col_y);
  if (reads_pairs<T, F>(ncols_x, stride_col_y, vy, {vx}, expert_stride))
    moe_wsum_launch<typename DU::pairs, ACC>(vx, expert_stride, vy, ids, weights, dst, ncols_x, nrows_x, ay,
                                             n_tokens, topk, s);
  else
    moe_wsum_launch<typename DU::odd, ACC>(vx, expert_stride, vy, ids, weights, dst, ncols_x, nrows_x, ay, n_tokens,
                                           topk, s);
}

// launch_indexed_moe_forward_<t>_q8_1 (slots; k_padded / 32 Q8_1 blocks per input row) and the _q8_0 forms of the
// 32-value types (k_padded / 32 Q8_0 blocks per input row): all_outputs[(b * topk + s) * n + row] =
// W[indices[b * topk + s]][row] . x[b * input_dim1 + (input_dim1 == 1 ? 0 : s)]
template <int T, int F>
void indexed_t(const void *w, const void *x, const uint32_t *ids, float *out, int n, int k, int batch, int topk,
               int k_padded, int input_dim1, void *stream, const char *who) {
  if (batch < 0 || topk <= 0 || (input_dim1 != 1 && input_dim1 != topk) || k_padded < k || k <= 0 ||
      k % (int)qmm_block_size(T) != 0) {
    qmm_set_error("%s: batch=%d topk=%d input_dim1=%d k=%d k_padded=%d", who, batch, topk, input_dim1, k, k_padded);
    return;
  }
  if (k_padded % (F == kActSlots ? 256 : 32) != 0) {
    qmm_set_error("%s: k_padded=%d not a multiple of %d", who, k_padded, F == kActSlots ? 256 : 32);
    return;
  }
  const int64_t expert_stride = (int64_t)n * (k / (int)qmm_block_size(T)) * (int64_t)qmm_type_size(T);
  moe_t<T, F>(w, nullptr, expert_stride, x, ids, out, k, n, k_padded / 32, input_dim1 == 1 ? topk : 1, batch * topk,
              0, stream, who);
}

// The reference's fused MoE decode launchers (gguf/ffi.rs:280-440; kernels indexed_moe.cu:1189-1330; host
// gguf/cuda.rs:1355-1520), over slot-layout inputs of k_padded values per row, f32 outputs:
//   launch_moe_gemv_fused_gate_up_<t>_q8_1: all_outputs[p * n + row] = act(W_gate[e] . x_b) * (W_up[e] . x_b) for
//       route p = b * topk + s, e = indices[p], x_b = input row b; act_type 0 is GELU (tanh form), any other SiLU,
//       as the reference's kernel reads it (indexed_moe.cu:1254-1256);
//   launch_moe_gemv_down_aggregate_<t>_q8_1: all_outputs[b * n + row] += sum over s < topk of topk_weights[p] *
//       (W[e] . x_p), x_p = input row p.  The reference adds each route with an atomic add into a buffer its caller
//       zeroes (gguf/cuda.rs:1475-1477); here one lane adds the routes' products in slot order and then adds that
//       to the buffer, so the result does not depend on scheduling.  A route of weight zero is not read.
// The experts' weight tensors hold n rows of k values each.
template <int T>
void moe_gemv_gate_up_t(const void *wg, const void *wu, const void *x, const uint32_t *ids, float *out, int n, int k,
                        int batch, int topk, int k_padded, int act_type, void *stream, const char *who) {
  if (!wg || !wu || n <= 0 || k <= 0 || k % (int)qmm_block_size(T) != 0 || k_padded < k || k_padded % 256 != 0 ||
      batch < 0 || topk <= 0) {
    qmm_set_error("%s: n=%d k=%d k_padded=%d batch=%d topk=%d", who, n, k, k_padded, batch, topk);
    return;
  }
  const int64_t expert_stride = (int64_t)n * (k / (int)qmm_block_size(T)) * (int64_t)qmm_type_size(T);
  moe_t<T, kActSlots>(wg, wu, expert_stride, x, ids, out, k, n, k_padded / 32, topk, batch * topk,
                      act_type == 0 ? 1 : 0, stream, who);
}

template <int T>
void moe_gemv_down_aggregate_t(const void *w, const void *x, const uint32_t *ids, const float *weights, float *out,
                               int n, int k, int batch, int topk, int k_padded, void *stream, const char *who) {
  if (n <= 0 || k <= 0 || k % (int)qmm_block_size(T) != 0 || k_padded < k || k_padded % 256 != 0 || batch < 0 ||
      topk <= 0) {
    qmm_set_error("%s: n=%d k=%d k_padded=%d batch=%d topk=%d", who, n, k, k_padded, batch, topk);
    return;
  }
  const int64_t expert_stride = (int64_t)n * (k / (int)qmm_block_size(T)) * (int64_t)qmm_type_size(T);
  moe_wsum_t<T, kActSlots, true>(w, expert_stride, x, ids, weights, out, k, n, k_padded / 32, batch, topk, stream,
                                 who);
}

}  // namespace

// ------------------------------------------------------------------------------------------------ entry points

#define QMM_MMVQ_PLAIN_DT(t, T, F, sfx, dt, Out)                                                                 \
  void launch_mmvq_gguf_##t##_##dt##_plain##sfx(const void *vx, const void *vy, void *dst, int ncols_x,          \
                                                int nrows_x, int stride_col_y, int stride_col_dst, int b_size,   \
                                                void *stream) {                                                  \
    plain_t<T, F, Out>(vx, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b_size, stream,              \
                       "mmvq_" #t "_" #dt "_plain" #sfx);                                                        \
  }
// launch_mmvq_gguf_<t>_{f32,f16,bf16}_plain<sfx>
#define QMM_MMVQ_PLAIN(t, T, F, sfx)                   \
  QMM_MMVQ_PLAIN_DT(t, T, F, sfx, f32, out_f32)        \
  QMM_MMVQ_PLAIN_DT(t, T, F, sfx, f16, out_f16)        \
  QMM_MMVQ_PLAIN_DT(t, T, F, sfx, bf16, out_bf16)

#define QMM_MMVQ_QUANTIZE_PLAIN_DT(t, T, dt, Out)                                                                \
  void launch_mmvq_gguf_##t##_##dt##_quantize_plain(const void *vx, const float *x, void *dst, int ncols_x,      \
                                                    int nrows_x, int stride_col_x, int stride_col_dst,          \
                                                    int b_size, void *stream) {                                 \
    quantize_plain_t<T, Out>(vx, x, dst, ncols_x, nrows_x, stride_col_x, stride_col_dst, b_size, stream,         \
                             "mmvq_" #t "_" #dt "_quantize");                                                    \
  }
#define QMM_MMVQ_QUANTIZE_PLAIN(t, T)               \
  QMM_MMVQ_QUANTIZE_PLAIN_DT(t, T, f32, out_f32)    \
  QMM_MMVQ_QUANTIZE_PLAIN_DT(t, T, f16, out_f16)    \
  QMM_MMVQ_QUANTIZE_PLAIN_DT(t, T, bf16, out_bf16)

#define QMM_MMVQ_FUSED_QUANTIZE_DT(t, T, dt, Out)                                                                  \
  void launch_mmvq_gguf_##t##_##dt##_fused_glu_quantize(const void *vx_gate, const void *vx_up, const float *x,      \
                                                        void *dst, int ncols_x, int nrows_x, int stride_col_x,       \
                                                        int stride_col_dst, int b_size, int activation,              \
                                                        void *stream) {                                              \
    fused_glu_quantize_t<T, Out>(vx_gate, vx_up, x, dst, ncols_x, nrows_x, stride_col_x, stride_col_dst, b_size,     \
                                 activation, stream, "mmvq_" #t "_" #dt "_fused_glu_quantize");                      \
  }                                                                                                                  \
  void launch_mmvq_gguf_##t##_##dt##_fused_qkv_quantize(const void *vx_q, const void *vx_k, const void *vx_v,        \
                                                        const float *x, void *q_dst, void *k_dst, void *v_dst,       \
                                                        int ncols_x, int nrows_q, int nrows_k, int nrows_v,          \
                                                        int stride_col_x, int b_size, void *stream) {                \
    fused_qkv_quantize_t<T, T, Out>(vx_q, vx_k, vx_v, x, q_dst, k_dst, v_dst, ncols_x, nrows_q, nrows_k, nrows_v,    \
                                    stride_col_x, b_size, stream, "mmvq_" #t "_" #dt "_fused_qkv_quantize");         \
  }
// launch_mmvq_gguf_<t>_{f32,f16,bf16}_fused_{glu,qkv}_quantize
#define QMM_MMVQ_FUSED_QUANTIZE(t, T)               \
  QMM_MMVQ_FUSED_QUANTIZE_DT(t, T, f32, out_f32)    \
  QMM_MMVQ_FUSED_QUANTIZE_DT(t, T, f16, out_f16)    \
  QMM_MMVQ_FUSED_QUANTIZE_DT(t, T, bf16, out_bf16)

// launch_mmvq_gguf_<t>_moe<sfx> and launch_mmvq_gguf_<t>_moe_wsum<sfx>
#define QMM_MMVQ_MOE(t, T, F, sfx)                                                                                 \
  void launch_mmvq_gguf_##t##_moe##sfx(const void *vx_gate, const void *vx_up, int64_t expert_stride,             \
                                       const void *vy, const void *ids, float *dst, int ncols_x, int nrows_x,     \
                                       int stride_col_y, int y_div, int n_pairs, int activation, int grouped,     \
                                       void *stream) {                                                            \
    (void)grouped;                                                                                                \
    moe_t<T, F>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x, stride_col_y, y_div, n_pairs,      \
                activation, stream, "mmvq_" #t "_moe" #sfx);                                                      \
  }                                                                                                               \
  void launch_mmvq_gguf_##t##_moe_wsum##sfx(const void *vx, int64_t expert_stride, const void *vy,                \
                                            const void *ids, const float *weights, float *dst, int ncols_x,       \
                                            int nrows_x, int stride_col_y, int n_tokens, int topk, void *stream) { \
    moe_wsum_t<T, F>(vx, expert_stride, vy, ids, weights, dst, ncols_x, nrows_x, stride_col_y, n_tokens, topk,    \
                     stream, "mmvq_" #t "_moe_wsum" #sfx);                                                        \
  }

// launch_indexed_moe_forward_<rt>_<act> (rt: the reference's type name, q4k / q8_0 / ...)
#define QMM_MMVQ_INDEXED(rt, T, F, act)                                                                            \
  void launch_indexed_moe_forward_##rt##_##act(const void *all_weights, const void *all_inputs,                   \
                                               const uint32_t *indices, float *all_outputs, int n, int k,         \
                                               int batch, int topk, int k_padded, int input_dim1, void *stream) { \
    indexed_t<T, F>(all_weights, all_inputs, indices, all_outputs, n, k, batch, topk, k_padded, input_dim1,       \
                    stream, "indexed_moe_" #rt "_" #act);                                                         \
  }

// launch_moe_gemv_fused_gate_up_<rt>_q8_1 and launch_moe_gemv_down_aggregate_<rt>_q8_1
#define QMM_MOE_GEMV(rt, T)                                                                                        \
  void launch_moe_gemv_fused_gate_up_##rt##_q8_1(const void *gate_weights, const void *up_weights,                \
                                                 const void *all_inputs, const uint32_t *indices,                 \
                                                 float *all_outputs, int n, int k, int batch, int topk,           \
                                                 int k_padded, int act_type, void *stream) {                      \
    moe_gemv_gate_up_t<T>(gate_weights, up_weights, all_inputs, indices, all_outputs, n, k, batch, topk, k_padded, \
                          act_type, stream, "moe_gemv_fused_gate_up_" #rt);                                       \
  }                                                                                                               \
  void launch_moe_gemv_down_aggregate_##rt##_q8_1(const void *all_weights, const void *all_inputs,                \
                                                  const uint32_t *indices, const float *topk_weights,             \
                                                  float *all_outputs, int n, int k, int batch, int topk,          \
                                                  int k_padded, void *stream) {                                   \
    moe_gemv_down_aggregate_t<T>(all_weights, all_inputs, indices, topk_weights, all_outputs, n, k, batch, topk,  \
                                 k_padded, stream, "moe_gemv_down_aggregate_" #rt);                               \
  }

// launch_mmvq_tc_gguf_<t>_{f32,f16,bf16}_plain
#define QMM_MMVQ_TC_DT(t, T, dt, Out)                                                                              \
  void launch_mmvq_tc_gguf_##t##_##dt##_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, \
                                              int stride_col_dst, int b_size, int cfg, void *stream) {            \
    tc_plain_t<T, Out>(vx, vy, dst, ncols_x, nrows_x, stride_col_dst, b_size, cfg, stream, "mmvq_tc_" #t "_" #dt); \
  }
#define QMM_MMVQ_TC(t, T)               \
  QMM_MMVQ_TC_DT(t, T, f32, out_f32)    \
  QMM_MMVQ_TC_DT(t, T, f16, out_f16)    \
  QMM_MMVQ_TC_DT(t, T, bf16, out_bf16)
