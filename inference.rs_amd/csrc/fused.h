// Fused decode forms: one launch over one quantized activation for several projections.  Shared by fused_kq.hip (the
// super-block types) and fused_b32.hip (the 32-value types), each instantiating its types only.
//   launch_mmvq_gguf_<t>_<dt>_fused_glu  dst = act(W_gate . y) * (W_up . y)          (gguf/ffi.rs:1032-1069)
//   launch_mmvq_gguf_<t>_<dt>_fused_qkv  q / k / v = W_q / W_k / W_v . y             (gguf/ffi.rs:1071-1118)
// Replace mmvq_gguf.cuh:761-959 and their launchers (1550-1600, 1860-1960) in
// crates/inference-quant/kernels/cuda/mmvq_gguf/.
//
// Few activation rows: a persistent wave-per-row kernel over the launch's whole row space (q rows, then k, then v;
// or gate/up row pairs), each wave requesting its next row's weights before its current row's math.  From the
// few-row MFMA crossover on, the K-quant forms run on the MFMA kernel (skinny.hip): one launch computes gate and up
// together; q, k and v are one launch each over the shared activation.
#pragma once

#include "common.h"
#include "inferencequant.h"
#include "skinny.h"
#include "units.h"

namespace {

constexpr int kWaves = 4;
enum { kQkv = 0, kGlu = 1 };

// The launch's rows: QKV numbers q rows [0, end[0]), k rows [end[0], end[1]), v rows [end[1], end[2]); GLU row r
// is the pair (gate row r, up row r) with end[0] = end[2] = rows.
struct RowSpace {
  const uint8_t *w[3];
  void *dst[3];
  int end[3];
  int ldd[3];
};

template <class U, class Out, int NC, int S, int MODE>
__global__ __launch_bounds__(256) void k_fused(RowSpace rs, const uint8_t *__restrict__ act, int ncols, int64_t row_bytes,
                                               int nunits, int64_t act_row_bytes, int activation) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tw = gridDim.x * kWaves;
  const int nrows = rs.end[2];
  int row = blockIdx.x * kWaves + wave;
  if (row >= nrows) return;  // whole wave
  auto has = [&](int s) { return lane + 64 * s < nunits; };
  // column j reads activation row min(j, ncols - 1); only j < ncols is stored
  auto arow = [&](int j) { return act + (int64_t)(j < ncols ? j : ncols - 1) * act_row_bytes; };
  constexpr int NW = MODE == kGlu ? 2 : 1;  // weight rows per item
  // weights of row `r`: segment and local row (QKV), or the gate / up rows (GLU)
  auto wrow = [&](int r, int i) -> const uint8_t * {
    if (MODE == kGlu) return rs.w[i] + (int64_t)r * row_bytes;
    const int seg = (r >= rs.end[0]) + (r >= rs.end[1]);
    const int local = r - (seg == 0 ? 0 : rs.end[seg - 1]);
    return rs.w[seg] + (int64_t)local * row_bytes;
  };
  typename U::W w[NW][S];
#pragma unroll
  for (int i = 0; i < NW; i++)
#pragma unroll
    for (int s = 0; s < S; s++)
      if (has(s)) U::load_w(wrow(row, i), lane + 64 * s, w[i][s]);
  for (; row < nrows; row += tw) {
    typename U::W wn[NW][S];
    if (row + tw < nrows) {
#pragma unroll
      for (int i = 0; i < NW; i++)
#pragma unroll
        for (int s = 0; s < S; s++)
          if (has(s)) U::load_w(wrow(row + tw, i), lane + 64 * s, wn[i][s]);
    }
    float acc[NW][NC];
#pragma unroll
    for (int i = 0; i < NW; i++)
#pragma unroll
      for (int j = 0; j < NC; j++) acc[i][j] = 0.0f;
#pragma unroll
    for (int s = 0; s < S; s++) {
      if (!has(s)) continue;
      const int u = lane + 64 * s;
#pragma unroll
      for (int j = 0; j < NC; j++) {
        typename U::A a;
        U::load_a(arow(j), u, a);
#pragma unroll
        for (int i = 0; i < NW; i++) acc[i][j] += U::dot(w[i][s], a, u);
      }
    }
    int seg = 0, local = row;
    if (MODE == kQkv) {
      seg = (row >= rs.end[0]) + (row >= rs.end[1]);
      local = row - (seg == 0 ? 0 : rs.end[seg - 1]);
    }
    typename Out::T *d = (typename Out::T *)rs.dst[seg];
#pragma unroll
    for (int j = 0; j < NC; j++) {
      float v = wave_sum_to_lane63(acc[0][j]);
      if (MODE == kGlu) v = glu_act(activation, v) * wave_sum_to_lane63(acc[NW - 1][j]);
      if (lane == 63 && j < ncols) Out::store(d, (int64_t)j * rs.ldd[seg] + local, v);
    }
#pragma unroll
    for (int i = 0; i < NW; i++)
#pragma unroll
      for (int s = 0; s < S; s++) w[i][s] = wn[i][s];
  }
}

// Rows of more than 4 units per lane (K > 16384 for the 64-value units): one wave per row at a time, the units walked
// in a loop with nothing held over to the next row.  The same per-lane sums and wave reduction as k_fused.
template <class U, class Out, int NC, int MODE>
__global__ __launch_bounds__(256) void k_fused_wide(RowSpace rs, const uint8_t *__restrict__ act, int ncols,
                                                    int64_t row_bytes, int nunits, int64_t act_row_bytes,
                                                    int activation) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tw = gridDim.x * kWaves;
  const int nrows = rs.end[2];
  constexpr int NW = MODE == kGlu ? 2 : 1;
  auto arow = [&](int j) { return act + (int64_t)(j < ncols ? j : ncols - 1) * act_row_bytes; };
  for (int row = blockIdx.x * kWaves + wave; row < nrows; row += tw) {
    int seg = 0, local = row;
    if (MODE == kQkv) {
      seg = (row >= rs.end[0]) + (row >= rs.end[1]);
      local = row - (seg == 0 ? 0 : rs.end[seg - 1]);
    }
    const uint8_t *wr[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) wr[i] = (MODE == kGlu ? rs.w[i] : rs.w[seg]) + (int64_t)local * row_bytes;
    float acc[NW][NC];
#pragma unroll
    for (int i = 0; i < NW; i++)
#pragma unroll
      for (int j = 0; j < NC; j++) acc[i][j] = 0.0f;
    for (int u = lane; u < nunits; u += 64) {
      typename U::W w[NW];
#pragma unroll
      for (int i = 0; i < NW; i++) U::load_w(wr[i], u, w[i]);
#pragma unroll
      for (int j = 0; j < NC; j++) {
        typename U::A a;
        U::load_a(arow(j), u, a);
#pragma unroll
        for (int i = 0; i < NW; i++) acc[i][j] += U::dot(w[i], a, u);
      }
    }
    typename Out::T *d = (typename Out::T *)rs.dst[seg];
#pragma unroll
    for (int j = 0; j < NC; j++) {
      float v = wave_sum_to_lane63(acc[0][j]);
      if (MODE == kGlu) v = glu_act(activation, v) * wave_sum_to_lane63(acc[NW - 1][j]);
      if (lane == 63 && j < ncols) Out::store(d, (int64_t)j * rs.ldd[seg] + local, v);
    }
  }
}

// The 32-value types' odd-block rows (a rare shape): the wide kernel only, so their units add few kernels to the build
template <class U, class Out, int MODE>
void launch_wide(const RowSpace &rs, const uint8_t *vy, int k, int64_t act_row_bytes, int b, int activation,
                 hipStream_t s) {
  const int64_t wgs = qmm_ceil_div(rs.end[2], kWaves);
  const dim3 grid((unsigned)(wgs < 8 * qmm_device_cus() ? wgs : 8 * qmm_device_cus()));
  for (int j0 = 0; j0 < b; j0 += 4) {
    const int nc = b - j0 < 4 ? b - j0 : 4;
    RowSpace r = rs;
    for (int i = 0; i < 3; i++)
      if (r.dst[i]) r.dst[i] = (typename Out::T *)r.dst[i] + (int64_t)j0 * r.ldd[i];
    const uint8_t *y = vy + (int64_t)j0 * act_row_bytes;
    const int64_t rb = U::row_bytes(k);
    const int nu = U::units(k);
    if (nc == 1)
      k_fused_wide<U, Out, 1, MODE><<<grid, 256, 0, s>>>(r, y, nc, rb, nu, act_row_bytes, activation);
    else if (nc == 2)
      k_fused_wide<U, Out, 2, MODE><<<grid, 256, 0, s>>>(r, y, nc, rb, nu, act_row_bytes, activation);
    else
      k_fused_wide<U, Out, 4, MODE><<<grid, 256, 0, s>>>(r, y, nc, rb, nu, act_row_bytes, activation);
  }
}

template <class U, class Out, int MODE>
void launch(const RowSpace &rs, const uint8_t *vy, int k, int64_t act_row_bytes, int b, int activation,
            hipStream_t s) {
  const int S = (int)qmm_ceil_div(U::units(k), 64);
  const int64_t wgs = qmm_ceil_div(rs.end[2], kWaves);
  const dim3 grid((unsigned)(wgs < 8 * qmm_device_cus() ? wgs : 8 * qmm_device_cus()));
  const int64_t rb = U::row_bytes(k);
  const int nu = U::units(k);
  for (int j0 = 0; j0 < b; j0 += 4) {
    const int nc = b - j0 < 4 ? b - j0 : 4;
    RowSpace r = rs;
    for (int i = 0; i < 3; i++)
      if (r.dst[i]) r.dst[i] = (typename Out::T *)r.dst[i] + (int64_t)j0 * r.ldd[i];
    const uint8_t *y = vy + (int64_t)j0 * act_row_bytes;
#define QMM_F(NC, SS) \
  k_fused<U, Out, NC, SS, MODE><<<grid, 256, 0, s>>>(r, y, nc, rb, nu, act_row_bytes, activation)
#define QMM_F_S(NC)                                                                                    \
  switch (S) {                                                                                         \
    case 1: QMM_F(NC, 1); break;                                                                       \
    case 2: QMM_F(NC, 2); break;                                                                       \
    case 3: case 4: QMM_F(NC, 4); break;                                                               \
    default:                                                                                           \
      k_fused_wide<U, Out, NC, MODE><<<grid, 256, 0, s>>>(r, y, nc, rb, nu, act_row_bytes, activation); \
  }
    if (nc == 1) {
      QMM_F_S(1)
    } else if (nc == 2) {
      QMM_F_S(2)
    } else {
      QMM_F_S(4)
    }
#undef QMM_F_S
#undef QMM_F
  }
}

// The launch for weight type T over activation layout F (units.h): the block-pair units where every row reads as
// pairs, else the odd units.
template <int T, int F, class Out, int MODE>
void launch_type(const RowSpace &rs, const void *vy, int k, int stride_col_y, int b, int activation, hipStream_t s) {
  typedef decode_units<T, F> DU;
  const uint8_t *y = (const uint8_t *)vy;
  const int64_t ay = act_row_bytes<F>(stride_col_y);
  if (reads_pairs<T, F>(k, stride_col_y, vy, {rs.w[0], rs.w[1], rs.w[2]}))
    launch<typename DU::pairs, Out, MODE>(rs, y, k, ay, b, activation, s);
  else
    launch_wide<typename DU::odd, Out, MODE>(rs, y, k, ay, b, activation, s);
}

inline int out_type_of(const out_f32 *) { return QMM_TYPE_F32; }
inline int out_type_of(const out_f16 *) { return QMM_TYPE_F16; }
inline int out_type_of(const out_bf16 *) { return QMM_TYPE_BF16; }

// Slots (F = kActSlots): stride_col_y counts 36-byte Q8_1 blocks, whole 288-byte slots; Q8_0 blocks: 34-byte blocks.
template <int T, int F>
bool check_weights(const char *who, int ncols_x, int stride_col_y, int b, std::initializer_list<const void *> ws,
                   std::initializer_list<int> rows) {
  const int bs = (int)qmm_block_size(T);
  const int bmax = T == QMM_TYPE_Q4K || T == QMM_TYPE_Q6K ? 32 : 16;  // as the plain launcher
  if (ncols_x <= 0 || ncols_x % bs != 0 || (int64_t)stride_col_y * 32 < ncols_x ||
      (F == kActSlots && stride_col_y % 8 != 0) || b < 0 || b > bmax) {
    qmm_set_error("%s: ncols_x=%d stride_col_y=%d b_size=%d", who, ncols_x, stride_col_y, b);
    return false;
  }
  for (int r : rows)
    if (r < 0) {
      qmm_set_error("%s: negative row count", who);
      return false;
    }
  for (const void *w : ws)
    if (w == nullptr || (uintptr_t)w % weight_align(T) != 0) {
      qmm_set_error("%s: weight pointer null or not %zu-byte aligned", who, (size_t)weight_align(T));
      return false;
    }
  return true;
}

template <int T, int F, class Out>
void fused_glu(const void *vx_gate, const void *vx_up, const void *vy, void *dst, int ncols_x, int nrows_x,
               int stride_col_y, int stride_col_dst, int b, int activation, void *stream, const char *who) {
  if (!check_weights<T, F>(who, ncols_x, stride_col_y, b, {vx_gate, vx_up}, {nrows_x})) return;
  if (activation < 0 || activation >= kGluActivations || stride_col_dst < nrows_x) {
    qmm_set_error("%s: activation=%d stride_col_dst=%d", who, activation, stride_col_dst);
    return;
  }
  if (b == 0 || nrows_x == 0) return;
  hipStream_t s = (hipStream_t)stream;
  if constexpr (T == QMM_TYPE_Q4K || T == QMM_TYPE_Q6K) {
    if (b >= qmm_skinny_min_rows(T) &&
        qmm_skinny_glu(T, out_type_of((const Out *)nullptr), vx_gate, vx_up, vy, dst, ncols_x, nrows_x, stride_col_y,
                       stride_col_dst, b, activation, s))
      return;
  }
  RowSpace rs = {};
  rs.w[0] = (const uint8_t *)vx_gate;
  rs.w[1] = (const uint8_t *)vx_up;
  rs.dst[0] = dst;
  rs.end[0] = rs.end[1] = rs.end[2] = nrows_x;
  rs.ldd[0] = stride_col_dst;
  launch_type<T, F, Out, kGlu>(rs, vy, ncols_x, stride_col_y, b, activation, s);
}

template <int T, int F, class Out>
void fused_qkv(const void *vx_q, const void *vx_k, const void *vx_v, const void *vy, void *q_dst, void *k_dst,
               void *v_dst, int ncols_x, int nrows_q, int nrows_k, int nrows_v, int stride_col_y, int b, void *stream,
               const char *who) {
  if (!check_weights<T, F>(who, ncols_x, stride_col_y, b, {vx_q, vx_k, vx_v}, {nrows_q, nrows_k, nrows_v})) return;
  if (b == 0 || nrows_q + nrows_k + nrows_v == 0) return;
  hipStream_t s = (hipStream_t)stream;
  if constexpr (T == QMM_TYPE_Q4K || T == QMM_TYPE_Q6K) {
    if (b >= qmm_skinny_min_rows(T)) {
      const int ot = out_type_of((const Out *)nullptr);
      const void *w[3] = {vx_q, vx_k, vx_v};
      void *d[3] = {q_dst, k_dst, v_dst};
      const int n[3] = {nrows_q, nrows_k, nrows_v};
      bool ok = true;
      for (int i = 0; i < 3 && ok; i++)
        if (n[i] > 0) ok = qmm_skinny_decode(T, ot, w[i], vy, d[i], ncols_x, n[i], stride_col_y, n[i], b, s);
      if (ok) return;
    }
  }
  RowSpace rs = {};
  rs.w[0] = (const uint8_t *)vx_q;
  rs.w[1] = (const uint8_t *)vx_k;
  rs.w[2] = (const uint8_t *)vx_v;
  rs.dst[0] = q_dst;
  rs.dst[1] = k_dst;
  rs.dst[2] = v_dst;
  rs.end[0] = nrows_q;
  rs.end[1] = nrows_q + nrows_k;
  rs.end[2] = nrows_q + nrows_k + nrows_v;
  rs.ldd[0] = nrows_q;
  rs.ldd[1] = nrows_k;
  rs.ldd[2] = nrows_v;
  launch_type<T, F, Out, kQkv>(rs, vy, ncols_x, stride_col_y, b, 0, s);
}

}  // namespace

// launch_mmvq_gguf_<t>_<dt>_fused_{glu,qkv}<sfx>
#define QMM_DEFINE_FUSED_DT(t, TYPE, F, sfx, dt, Out)                                                            \
  void launch_mmvq_gguf_##t##_##dt##_fused_glu##sfx(const void *vx_gate, const void *vx_up, const void *vy,      \
                                                    void *dst, int ncols_x, int nrows_x, int stride_col_y,      \
                                                    int stride_col_dst, int b_size, int activation,             \
                                                    void *stream) {                                             \
    fused_glu<TYPE, F, Out>(vx_gate, vx_up, vy, dst, ncols_x, nrows_x, stride_col_y, stride_col_dst, b_size,     \
                            activation, stream, "mmvq_" #t "_" #dt "_fused_glu" #sfx);                           \
  }                                                                                                              \
  void launch_mmvq_gguf_##t##_##dt##_fused_qkv##sfx(const void *vx_q, const void *vx_k, const void *vx_v,        \
                                                    const void *vy, void *q_dst, void *k_dst, void *v_dst,       \
                                                    int ncols_x, int nrows_q, int nrows_k, int nrows_v,          \
                                                    int stride_col_y, int b_size, void *stream) {                \
    fused_qkv<TYPE, F, Out>(vx_q, vx_k, vx_v, vy, q_dst, k_dst, v_dst, ncols_x, nrows_q, nrows_k, nrows_v,       \
                            stride_col_y, b_size, stream, "mmvq_" #t "_" #dt "_fused_qkv" #sfx);                 \
  }
#define QMM_DEFINE_FUSED(t, TYPE, F, sfx)                 \
  QMM_DEFINE_FUSED_DT(t, TYPE, F, sfx, f32, out_f32)      \
  QMM_DEFINE_FUSED_DT(t, TYPE, F, sfx, f16, out_f16)      \
  QMM_DEFINE_FUSED_DT(t, TYPE, F, sfx, bf16, out_bf16)
