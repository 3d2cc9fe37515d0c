// Decode matvec for GGUF Q8_0 / Q4_K / Q6_K weights against Q8_0 / Q8_K activations (b = 1..16 rows),
// plus the expert-indexed MoE matvec (optionally fused gate/up with the GLU activation).
//
// Replaces mmvq_gguf.cuh:650-759 (mmvq_core_impl) and its launchers (1542-1553, 1647-1702, 1762-1834),
// mmvq_gguf.cuh:961-1038 / 1600-1643 (MoE) and indexed_moe.cu:664-1000, all in
// crates/inference-quant/kernels/cuda/.  HBM-bound: each wave owns R consecutive weight rows; its 64 lanes
// stride over the rows' units (units.h), issue every 16-byte weight load of the R rows before using any,
// dot them with v_dot4 against activation units read once per column, and reduce each row with a wave
// butterfly.  Activations are tiny and hit L2.
#include "common.h"
#include "inferencequant.h"
#include "skinny.h"
#include "units.h"

namespace {

constexpr int kWaves = 4;  // waves per workgroup
// rows of up to this many 64-value units per lane go through the persistent kernel, longer ones through k_mmvq
#ifndef QMM_PERSISTENT_MAX_S
#define QMM_PERSISTENT_MAX_S 4
#endif


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
  for (; row < nrows; row += tw) {
    typename U::W wn[S];  // the next row's weights, in flight during this row's math
    if (row + tw < nrows) {
#pragma unroll
      for (int s = 0; s < S; s++)
        if (has(s)) U::load_w(vx + (int64_t)(row + tw) * row_bytes, lane + 64 * s, wn[s]);
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
#pragma unroll
    for (int s = 0; s < S; s++) w[s] = wn[s];
  }
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

template <class U, class Out, int NC>
void launch_nc(const uint8_t *vx, const uint8_t *vy, typename Out::T *dst, int k, int nrows, int64_t act_row_bytes,
               int stride_col_dst, hipStream_t s) {
  constexpr int R = NC <= 2 ? 4 : 2;
  const dim3 grid((unsigned)qmm_ceil_div(nrows, kWaves * R));
  k_mmvq<U, Out, NC, R><<<grid, 256, 0, s>>>(vx, vy, dst, nrows, U::row_bytes(k), U::units(k), act_row_bytes,
                                             stride_col_dst);
}

// Persistent launch of NC columns with S units per lane: grid capped at 8 workgroups per CU.
template <class U, class Out>
void launch_p(int nc, int S, const uint8_t *vx, const uint8_t *act, typename Out::T *dst, int k, int nrows,
              int64_t act_row_bytes, int stride_col_dst, hipStream_t s) {
  const int64_t wgs = qmm_ceil_div(nrows, kWaves);
  const dim3 grid((unsigned)(wgs < 8 * qmm_device_cus() ? wgs : 8 * qmm_device_cus()));
  const int64_t rb = U::row_bytes(k);
  const int nu = U::units(k);
  const bool full = nu % 64 == 0;
#define QMM_P(NC, SS)                                                                                             \
  do {                                                                                                            \
    if (full)                                                                                                     \
      k_mmvq_p<U, Out, NC, SS, true><<<grid, 256, 0, s>>>(vx, act, dst, nrows, rb, nu, act_row_bytes,             \
                                                          stride_col_dst);                                        \
    else                                                                                                          \
      k_mmvq_p<U, Out, NC, SS, false><<<grid, 256, 0, s>>>(vx, act, dst, nrows, rb, nu, act_row_bytes,            \
                                                           stride_col_dst);                                       \
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
}

int out_type_of(const out_f32 *) { return QMM_TYPE_F32; }
int out_type_of(const out_f16 *) { return QMM_TYPE_F16; }
int out_type_of(const out_bf16 *) { return QMM_TYPE_BF16; }

template <class U, class Out>
void launch_cols(const uint8_t *vx, const uint8_t *vy, typename Out::T *dst, int k, int nrows, int64_t act_row_bytes,
                 int stride_col_dst, int b, hipStream_t s) {
  const int S = (int)qmm_ceil_div(U::units(k), 64);
  if (S <= QMM_PERSISTENT_MAX_S) {
    for (int j0 = 0; j0 < b; j0 += 8) {
      const int nc = b - j0 < 8 ? b - j0 : 8;
      launch_p<U, Out>(nc, S, vx, vy + (int64_t)j0 * act_row_bytes, dst + (int64_t)j0 * stride_col_dst, k, nrows,
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

// Shape checks shared by the plain and MoE launchers. Returns false (and records why) when the
// arguments cannot be served.
bool check_mmvq(const char *who, int type, const void *vx, int ncols_x, int nrows_x, int stride_col_y, int b) {
  const int bs = (int)qmm_block_size(type);
  const int abs_ = type == QMM_TYPE_Q8_0 ? 32 : 256;
  if (ncols_x <= 0 || nrows_x <= 0 || ncols_x % bs != 0) {
    qmm_set_error("%s: ncols_x=%d nrows_x=%d (ncols_x must be a positive multiple of %d)", who, ncols_x, nrows_x, bs);
    return false;
  }
  if ((int64_t)stride_col_y * abs_ < ncols_x) {
    qmm_set_error("%s: stride_col_y=%d blocks holds fewer than ncols_x=%d values", who, stride_col_y, ncols_x);
    return false;
  }
  if (b < 0 || b > 16) {
    qmm_set_error("%s: b_size=%d outside 1..16", who, b);
    return false;
  }
  const uintptr_t align = type == QMM_TYPE_Q4K ? 16 : (type == QMM_TYPE_Q8_0 ? 2 : 2);
  if ((uintptr_t)vx % align != 0) {
    qmm_set_error("%s: weight pointer not %zu-byte aligned", who, (size_t)align);
    return false;
  }
  return true;
}

template <class Out>
void plain(int type, const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int stride_col_y,
           int stride_col_dst, int b, void *stream, const char *who) {
  if (!check_mmvq(who, type, vx, ncols_x, nrows_x, stride_col_y, b)) return;
  if (b == 0) return;
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
  typename Out::T *d = (typename Out::T *)dst;
  if (b >= qmm_skinny_min_rows(type) &&
      qmm_skinny_decode(type, out_type_of((const Out *)nullptr), vx, vy, dst, ncols_x, nrows_x, stride_col_y,
                        stride_col_dst, b, s))
    return;
  switch (type) {
    case QMM_TYPE_Q4K:
      launch_cols<unit_q4k, Out>(x, y, d, ncols_x, nrows_x, (int64_t)stride_col_y * 292, stride_col_dst, b, s);
      break;
    case QMM_TYPE_Q6K:
      launch_cols<unit_q6k, Out>(x, y, d, ncols_x, nrows_x, (int64_t)stride_col_y * 292, stride_col_dst, b, s);
      break;
    default:  // Q8_0
      if (ncols_x % 64 == 0 && stride_col_y % 2 == 0 && (uintptr_t)vx % 4 == 0 && (uintptr_t)vy % 4 == 0)
        launch_cols<unit_q8_0, Out>(x, y, d, ncols_x, nrows_x, (int64_t)stride_col_y * 34, stride_col_dst, b, s);
      else
        launch_cols<unit_q8_0_odd, Out>(x, y, d, ncols_x, nrows_x, (int64_t)stride_col_y * 34, stride_col_dst, b, s);
      break;
  }
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

void moe(int type, const void *vx_gate, const void *vx_up, int64_t expert_stride, const void *vy, const void *ids,
         float *dst, int ncols_x, int nrows_x, int stride_col_y, int y_div, int n_pairs, int activation,
         void *stream, const char *who) {
  if (!check_mmvq(who, type, vx_gate, ncols_x, nrows_x, stride_col_y, 1)) return;
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
  hipStream_t s = (hipStream_t)stream;
  switch (type) {
    case QMM_TYPE_Q4K:
      if (expert_stride % 16 != 0 || (vx_up && (uintptr_t)vx_up % 16 != 0)) {
        qmm_set_error("%s: Q4_K expert_stride / vx_up not 16-byte aligned", who);
        return;
      }
      moe_launch<unit_q4k>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x,
                           (int64_t)stride_col_y * 292, y_div, n_pairs, activation, s);
      break;
    case QMM_TYPE_Q6K:
      moe_launch<unit_q6k>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x,
                           (int64_t)stride_col_y * 292, y_div, n_pairs, activation, s);
      break;
    default: {
      const bool fast = ncols_x % 64 == 0 && stride_col_y % 2 == 0 && expert_stride % 4 == 0 &&
                        (uintptr_t)vx_gate % 4 == 0 && (!vx_up || (uintptr_t)vx_up % 4 == 0) && (uintptr_t)vy % 4 == 0;
      if (fast)
        moe_launch<unit_q8_0>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x,
                              (int64_t)stride_col_y * 34, y_div, n_pairs, activation, s);
      else
        moe_launch<unit_q8_0_odd>(vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x,
                                  (int64_t)stride_col_y * 34, y_div, n_pairs, activation, s);
    }
  }
}

void indexed(int type, const void *w, const void *x, const uint32_t *ids, float *out, int n, int k, int batch,
             int topk, int k_padded, int input_dim1, void *stream, const char *who) {
  if (batch < 0 || topk <= 0 || (input_dim1 != 1 && input_dim1 != topk) || k_padded < k) {
    qmm_set_error("%s: batch=%d topk=%d input_dim1=%d k=%d k_padded=%d", who, batch, topk, input_dim1, k, k_padded);
    return;
  }
  const int abs_ = type == QMM_TYPE_Q8_0 ? 32 : 256;
  if (k_padded % abs_ != 0) {
    qmm_set_error("%s: k_padded=%d not a multiple of %d", who, k_padded, abs_);
    return;
  }
  const int64_t expert_stride = (int64_t)n * (k / (int)qmm_block_size(type)) * (int64_t)qmm_type_size(type);
  moe(type, w, nullptr, expert_stride, x, ids, out, k, n, k_padded / abs_, input_dim1 == 1 ? topk : 1, batch * topk,
      0, stream, who);
}

}  // namespace

#define QMM_DEFINE_PLAIN(t, TYPE)                                                                                 \
  void launch_mmvq_gguf_##t##_f32_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,    \
                                        int stride_col_y, int stride_col_dst, int b_size, void *stream) {        \
    plain<out_f32>(TYPE, vx, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b_size, stream,           \
                   "mmvq_" #t "_f32");                                                                            \
  }                                                                                                               \
  void launch_mmvq_gguf_##t##_f16_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,    \
                                        int stride_col_y, int stride_col_dst, int b_size, void *stream) {        \
    plain<out_f16>(TYPE, vx, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b_size, stream,           \
                   "mmvq_" #t "_f16");                                                                            \
  }                                                                                                               \
  void launch_mmvq_gguf_##t##_bf16_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,   \
                                         int stride_col_y, int stride_col_dst, int b_size, void *stream) {       \
    plain<out_bf16>(TYPE, vx, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b_size, stream,          \
                    "mmvq_" #t "_bf16");                                                                          \
  }                                                                                                               \
  void launch_mmvq_gguf_##t##_moe(const void *vx_gate, const void *vx_up, int64_t expert_stride, const void *vy,  \
                                  const void *ids, float *dst, int ncols_x, int nrows_x, int stride_col_y,       \
                                  int y_div, int n_pairs, int activation, int grouped, void *stream) {            \
    (void)grouped;                                                                                                \
    moe(TYPE, vx_gate, vx_up, expert_stride, vy, ids, dst, ncols_x, nrows_x, stride_col_y, y_div, n_pairs,        \
        activation, stream, "mmvq_" #t "_moe");                                                                   \
  }

extern "C" {
QMM_DEFINE_PLAIN(q8_0, QMM_TYPE_Q8_0)
QMM_DEFINE_PLAIN(q4_k, QMM_TYPE_Q4K)
QMM_DEFINE_PLAIN(q6_k, QMM_TYPE_Q6K)

void launch_indexed_moe_forward_q8_0_q8_0(const void *all_weights, const void *all_inputs, const uint32_t *indices,
                                          float *all_outputs, int n, int k, int batch, int topk, int k_padded,
                                          int input_dim1, void *stream) {
  indexed(QMM_TYPE_Q8_0, all_weights, all_inputs, indices, all_outputs, n, k, batch, topk, k_padded, input_dim1,
          stream, "indexed_moe_q8_0");
}
void launch_indexed_moe_forward_q4k_q8k(const void *all_weights, const void *all_inputs, const uint32_t *indices,
                                        float *all_outputs, int n, int k, int batch, int topk, int k_padded,
                                        int input_dim1, void *stream) {
  indexed(QMM_TYPE_Q4K, all_weights, all_inputs, indices, all_outputs, n, k, batch, topk, k_padded, input_dim1,
          stream, "indexed_moe_q4k");
}
void launch_indexed_moe_forward_q6k_q8k(const void *all_weights, const void *all_inputs, const uint32_t *indices,
                                        float *all_outputs, int n, int k, int batch, int topk, int k_padded,
                                        int input_dim1, void *stream) {
  indexed(QMM_TYPE_Q6K, all_weights, all_inputs, indices, all_outputs, n, k, batch, topk, k_padded, input_dim1,
          stream, "indexed_moe_q6k");
}
}

