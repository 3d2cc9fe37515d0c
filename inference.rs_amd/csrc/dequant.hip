// GGUF blocks decoded to floats on the GPU, and the Q8_0 matvec against unquantized activations.
//
//   launch_dequantize_<t>_{f32,f16,bf16}   QCudaStorage::dequantize / dequantize_f16 (quantized/cuda.rs:31-135,
//                                          283-334) over the kernels dequantize_block_<t>_{f32,f16}
//                                          (inference-tensor-kernels/src/quantized.cu:440-608, 647-660)
//   launch_get_rows_<t>                    the embedding gather get_rows_<t> (quantized.cu:900-975)
//   launch_mmvq_gguf_q8_0_{bf16,f32}_exact the Q8_0 matvec with activations left unquantized (gguf/ffi.rs:1001-1022,
//                                          fast_mmvq.rs:415-472, mmvq_instance_q8_0.cu:15-146)
//
// Every value is produced by the same f32 operations, in the same order, as the reference CPU to_float
// (k_quants.rs:905-921, 2096-2123, 2649-2680, 313-330, 720-743, 2433-2467; raw.rs:794-808): Q8_0 q * d;
// Q4_K (d * sc) * q - dmin * m; Q6_K (d * sc) * (q - 32); Q4_0 / Q5_0 (q - off) * d; Q5_K as Q4_K with the fifth
// bit; IQ4_XS (d * (ls - 32)) * table[q].
// This file is compiled with -ffp-contract=off, so the f32 results are bit-identical to the CPU's, and the f16 / bf16
// outputs are those f32 values rounded to nearest even.  HBM-bound: a thread decodes 8 consecutive values and writes
// them with one or two 16-byte stores.
#include "common.h"
#include "inferencequant.h"
#include "units.h"

namespace {

// ------------------------------------------------------------------------------------------ per-type chunk decoders
// chunk c of a block = values 8c .. 8c + 7.  Blocks are read a byte or a halfword at a time: Q8_0 and Q6_K blocks
// are only 2-byte aligned.

struct deq_q8_0 {
  static constexpr int kBytes = 34, kValues = 32;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const float d = f16_bits_to_f32(ld16(b));
    const uint8_t *q = b + 2 + 8 * c;
#pragma unroll
    for (int j = 0; j < 8; j++) out[j] = (float)(int8_t)q[j] * d;
  }
};

struct deq_q4k {
  static constexpr int kBytes = 144, kValues = 256;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const int g = c >> 3, v = 8 * (c & 7);  // 64-value group g, value v of it
    const int is = 2 * g + (v >= 32);        // sub-block
    const uint8_t *sc = b + 4;
    int s, m;  // get_scale_min_k4 (quantized/utils.rs:119-129)
    if (is < 4) {
      s = sc[is] & 63;
      m = sc[is + 4] & 63;
    } else {
      s = (sc[is + 4] & 0xf) | ((sc[is - 4] >> 6) << 4);
      m = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4);
    }
    const float d = f16_bits_to_f32(ld16(b)), dmin = f16_bits_to_f32(ld16(b + 2));
    const float d1 = d * (float)s, m1 = dmin * (float)m;
    const uint8_t *q = b + 16 + 32 * g + (v & 31);
    const int sh = v >= 32 ? 4 : 0;
#pragma unroll
    for (int j = 0; j < 8; j++) out[j] = d1 * (float)((q[j] >> sh) & 0xf) - m1;
  }
};

struct deq_q6k {
  static constexpr int kBytes = 210, kValues = 256;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const int n = 8 * c, half = n >> 7, k = (n & 127) >> 5, l0 = n & 31;
    const uint8_t *ql = b + 64 * half + (k & 1) * 32 + l0, *qh = b + 128 + 32 * half + l0;
    const int8_t sc = (int8_t)b[192 + 8 * half + (l0 >> 4) + 2 * k];
    const float d = f16_bits_to_f32(ld16(b + 208)), ds = d * (float)sc;
    const int lsh = (k >> 1) * 4, hsh = 2 * k;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int q = ((ql[j] >> lsh) & 0xf) | (((qh[j] >> hsh) & 3) << 4);
      out[j] = ds * (float)(q - 32);
    }
  }
};

struct deq_q4_0 {
  static constexpr int kBytes = 18, kValues = 32;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const float d = f16_bits_to_f32(ld16(b));
    const uint8_t *q = b + 2 + 8 * (c & 1);
    const int sh = c >= 2 ? 4 : 0;  // values 16..31 are the high nibbles
#pragma unroll
    for (int j = 0; j < 8; j++) out[j] = (float)((int)((q[j] >> sh) & 0xf) - 8) * d;
  }
};

struct deq_q5_0 {
  static constexpr int kBytes = 22, kValues = 32;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const float d = f16_bits_to_f32(ld16(b));
    const uint32_t qh = ld16(b + 2) | (ld16(b + 4) << 16);  // bit v = fifth bit of value v
    const uint8_t *q = b + 6 + 8 * (c & 1);
    const int sh = c >= 2 ? 4 : 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int v = ((q[j] >> sh) & 0xf) | (((qh >> (8 * c + j)) & 1) << 4);
      out[j] = (float)(v - 16) * d;
    }
  }
};

struct deq_q5k {
  static constexpr int kBytes = 176, kValues = 256;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const int g = c >> 3, v = 8 * (c & 7);
    const int is = 2 * g + (v >= 32);
    const uint8_t *sc = b + 4;
    int s, m;
    if (is < 4) {
      s = sc[is] & 63;
      m = sc[is + 4] & 63;
    } else {
      s = (sc[is + 4] & 0xf) | ((sc[is - 4] >> 6) << 4);
      m = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4);
    }
    const float d = f16_bits_to_f32(ld16(b)), dmin = f16_bits_to_f32(ld16(b + 2));
    const float d1 = d * (float)s, m1 = dmin * (float)m;
    const uint8_t *qh = b + 16 + (v & 31), *q = b + 48 + 32 * g + (v & 31);
    const int sh = v >= 32 ? 4 : 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      // (q & 0xf) + 16 * bit in f32 is exact, as the reference's (ql & 0xF) as f32 + to_add
      const int qv = ((q[j] >> sh) & 0xf) + 16 * ((qh[j] >> is) & 1);
      out[j] = d1 * (float)qv - m1;
    }
  }
};

// IQ4_XS (raw.rs:794-808 and the reference kernel dequantize_iq4_xs, mmvq_gguf.cuh:2128-2141): value =
// (d * (ls - 32)) * table[index]
struct deq_iq4xs {
  static constexpr int kBytes = 136, kValues = 256;
  static __device__ __forceinline__ void chunk(const uint8_t *b, int c, float out[8]) {
    const int ib = c >> 2, part = c & 3;
    const uint32_t sh = ld16(b + 2), sl = b[4 + ib / 2];
    const int ls = (int)(((sl >> (4 * (ib & 1))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
    const float scale = f16_bits_to_f32(ld16(b)) * (float)(ls - 32);
    const uint8_t *q = b + 8 + 16 * ib + 8 * (part & 1);
    const uint32_t lo = ld16(q) | (ld16(q + 2) << 16), hi = ld16(q + 4) | (ld16(q + 6) << 16);
    const int nsh = part >= 2 ? 4 : 0;
    const uint32_t v0 = unit_iq4xs::lookup((lo >> nsh) & 0x0f0f0f0fu), v1 = unit_iq4xs::lookup((hi >> nsh) & 0x0f0f0f0fu);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      out[j] = scale * (float)(int8_t)(v0 >> (8 * j));
      out[4 + j] = scale * (float)(int8_t)(v1 >> (8 * j));
    }
  }
};

template <class Out>
__device__ __forceinline__ void store8(typename Out::T *y, const float v[8]) {
  if constexpr (sizeof(typename Out::T) == 4) {
    *(v4f *)y = (v4f){v[0], v[1], v[2], v[3]};
    *(v4f *)(y + 4) = (v4f){v[4], v[5], v[6], v[7]};
  } else {
    u32x4 p;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // The f32 values are materialized first: without this the compiler folds "product, then round to f16" into
      // one v_fma_mixlo_f16 with a +0 addend, which rounds once instead of twice and turns -0 into +0.
      float a = v[2 * i], b = v[2 * i + 1];
      __asm__("" : "+v"(a), "+v"(b));
      typename Out::T lo, hi;
      Out::store(&lo, 0, a);
      Out::store(&hi, 0, b);
      w[i] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    p.x = w[0], p.y = w[1], p.z = w[2], p.w = w[3];
    *(u32x4 *)y = p;
  }
}

// values [0, n) of a contiguous block array; thread i of the grid-stride loop decodes chunk i
template <class D, class Out>
__global__ __launch_bounds__(256) void k_dequantize(const uint8_t *__restrict__ x, typename Out::T *__restrict__ y,
                                                    int64_t n) {
  constexpr int CPB = D::kValues / 8;
  const int64_t chunks = n / 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * 256) {
    float v[8];
    D::chunk(x + (i / CPB) * D::kBytes, (int)(i % CPB), v);
    store8<Out>(y + 8 * i, v);
  }
}

// dst row r = the ne00 values of row ids[r] of src (rows nb01 bytes apart), f32
template <class D>
__global__ __launch_bounds__(256) void k_get_rows(const uint8_t *__restrict__ src, const uint32_t *__restrict__ ids,
                                                  float *__restrict__ dst, int64_t ne00, int64_t nb01) {
  constexpr int CPB = D::kValues / 8;
  const int64_t r = blockIdx.y;
  const uint8_t *row = src + (int64_t)ids[r] * nb01;
  float *out = dst + r * ne00;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < ne00 / 8; i += (int64_t)gridDim.x * 256) {
    float v[8];
    D::chunk(row + (i / CPB) * D::kBytes, (int)(i % CPB), v);
    store8<out_f32>(out + 8 * i, v);
  }
}

int grid_for(int64_t work_items) {
  const int64_t g = qmm_ceil_div(work_items, 256), cap = 8 * (int64_t)qmm_device_cus();
  return (int)(g < 1 ? 1 : g > cap ? cap : g);
}

template <class D, class Out>
void dequantize(const void *x, void *y, int64_t n, void *stream, const char *who) {
  if (n < 0 || n % D::kValues != 0 || ((uintptr_t)y & 15) != 0 || ((uintptr_t)x & 1) != 0) {
    qmm_set_error("%s: n=%lld must be a multiple of %d, y 16-byte and x 2-byte aligned", who, (long long)n, D::kValues);
    return;
  }
  if (n == 0) return;
  k_dequantize<D, Out><<<grid_for(n / 8), 256, 0, (hipStream_t)stream>>>((const uint8_t *)x, (typename Out::T *)y, n);
}

template <class D>
void get_rows(const void *src, const uint32_t *ids, float *dst, int64_t ne00, int64_t nb01, int64_t n_ids,
              void *stream, const char *who) {
  if (ne00 <= 0 || ne00 % D::kValues != 0 || nb01 < ne00 / D::kValues * D::kBytes || n_ids < 0 || n_ids > 65535 ||
      ((uintptr_t)dst & 15) != 0 || ((uintptr_t)src & 1) != 0 || nb01 % 2 != 0) {
    qmm_set_error("%s: ne00=%lld nb01=%lld n_ids=%lld (ne00 a multiple of %d, n_ids <= 65535, dst 16-byte aligned)",
                  who, (long long)ne00, (long long)nb01, (long long)n_ids, D::kValues);
    return;
  }
  if (n_ids == 0) return;
  const int64_t gx = qmm_ceil_div(ne00 / 8, 256);
  k_get_rows<D><<<dim3((unsigned)(gx < 64 ? gx : 64), (unsigned)n_ids), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t *)src, ids, dst, ne00, nb01);
}

// ------------------------------------------------------------------------------------------ exact Q8_0 matvec

// Activation element types of the exact matvec.
struct act_f32 {
  typedef float T;
  static __device__ __forceinline__ void load8(const float *p, float v[8]) {
    const v4f a = *(const v4f *)p, b = *(const v4f *)(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
};
struct act_bf16 {
  typedef uint16_t T;
  static __device__ __forceinline__ void load8(const uint16_t *p, float v[8]) {
    const u32x4 a = *(const u32x4 *)p;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = __builtin_bit_cast(float, w[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
    }
  }
};

// dst[b][row] = sum_k (d_blk q_k) x[b][k] in f32 (the reference's sum_k d q_k x_k, its f32 sums in another order).
// A wave takes R consecutive rows; lane l takes the 32-value blocks l, l + 64, ... of all of them, so every
// activation value it loads serves R rows.  Per block: sum_k q_k x_k in f32, then one multiply-add by d.
template <class A, class Out, int B, int R>
__global__ __launch_bounds__(256) void k_q8_0_exact(const uint8_t *__restrict__ w, const typename A::T *__restrict__ x,
                                                    typename Out::T *__restrict__ dst, int ncols, int nrows) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (row0 >= nrows) return;  // whole wave
  const int nblk = ncols / 32;
  const int64_t row_bytes = (int64_t)nblk * 34;
  float acc[R][B];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int b = 0; b < B; b++) acc[r][b] = 0.0f;
  for (int k = lane; k < nblk; k += 64) {
    const uint8_t *p[R];
    float d[R], s[R][B];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r < nrows ? row0 + r : nrows - 1;  // a short last group re-reads its last row
      p[r] = w + row * row_bytes + (int64_t)k * 34;
      d[r] = f16_bits_to_f32(ld16(p[r]));
#pragma unroll
      for (int b = 0; b < B; b++) s[r][b] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {  // values 8c .. 8c + 7 of the block
      float qf[R][8];
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t h = ld16(p[r] + 2 + 8 * c + 2 * i);
          qf[r][2 * i] = (float)(int8_t)(h & 0xff);
          qf[r][2 * i + 1] = (float)(int8_t)(h >> 8);
        }
#pragma unroll
      for (int b = 0; b < B; b++) {
        float xv[8];
        A::load8(x + (int64_t)b * ncols + 32 * k + 8 * c, xv);
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
          for (int j = 0; j < 8; j++) s[r][b] += qf[r][j] * xv[j];
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int b = 0; b < B; b++) acc[r][b] += d[r] * s[r][b];
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int b = 0; b < B; b++) {
      const float v = wave_sum_to_lane63(acc[r][b]);
      if (lane == 63 && row0 + r < nrows) Out::store(dst, (int64_t)b * nrows + row0 + r, v);
    }
}

template <class A, class Out>
void q8_0_exact(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int b_size, void *stream,
                const char *who) {
  if (ncols_x <= 0 || ncols_x % 32 != 0 || nrows_x <= 0 || b_size < 1 || b_size > 8 || ((uintptr_t)vx & 1) != 0 ||
      ((uintptr_t)vy & 15) != 0) {
    qmm_set_error("%s: ncols_x=%d (a multiple of 32) nrows_x=%d b_size=%d (1..8); vx 2-byte, vy 16-byte aligned", who,
                  ncols_x, nrows_x, b_size);
    return;
  }
  constexpr int R = 4;
  const dim3 grid((unsigned)qmm_ceil_div(nrows_x, 4 * R));
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *w = (const uint8_t *)vx;
  const typename A::T *x = (const typename A::T *)vy;
  typename Out::T *d = (typename Out::T *)dst;
  switch (b_size) {
#define QMM_EXACT_B(B) \
  case B: k_q8_0_exact<A, Out, B, R><<<grid, 256, 0, s>>>(w, x, d, ncols_x, nrows_x); break;
    QMM_EXACT_B(1) QMM_EXACT_B(2) QMM_EXACT_B(3) QMM_EXACT_B(4) QMM_EXACT_B(5) QMM_EXACT_B(6) QMM_EXACT_B(7)
    QMM_EXACT_B(8)
#undef QMM_EXACT_B
  }
}


// ------------------------------------------------------------------------------------------------ raw row gather

// launch_gather_rows_u8: dst row r = src row ids[r] (rows of row_bytes bytes), zeros for an id past the last row.
// Workgroup (x, y) copies chunk x of rows y, y + gridDim.y, ...: 16-byte pieces when every row is, else bytes.
template <bool VEC>
__global__ __launch_bounds__(256) void k_gather_rows_u8(const uint8_t *__restrict__ src, const uint32_t *__restrict__ ids,
                                                        uint8_t *__restrict__ dst, int64_t row_bytes, int64_t rows,
                                                        int64_t n) {
  constexpr int W = VEC ? 16 : 1;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * W;
  if (i >= row_bytes) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) {
    const int64_t id = ids[r];
    uint8_t *o = dst + r * row_bytes + i;
    if (VEC) {
      u32x4 v = {0, 0, 0, 0};
      if (id < rows) v = *(const u32x4 *)(src + id * row_bytes + i);
      *(u32x4 *)o = v;
    } else {
      *o = id < rows ? src[id * row_bytes + i] : 0;
    }
  }
}

}  // namespace

extern "C" {

#define QMM_DEFINE_DEQ(t, D)                                                                                       \
  void launch_dequantize_##t##_f32(const void *x, void *y, int64_t n, void *stream) {                             \
    dequantize<D, out_f32>(x, y, n, stream, "dequantize_" #t "_f32");                                             \
  }                                                                                                                \
  void launch_dequantize_##t##_f16(const void *x, void *y, int64_t n, void *stream) {                             \
    dequantize<D, out_f16>(x, y, n, stream, "dequantize_" #t "_f16");                                             \
  }                                                                                                                \
  void launch_dequantize_##t##_bf16(const void *x, void *y, int64_t n, void *stream) {                            \
    dequantize<D, out_bf16>(x, y, n, stream, "dequantize_" #t "_bf16");                                           \
  }                                                                                                                \
  void launch_get_rows_##t(const void *src0, const uint32_t *ids, float *dst, int64_t ne00, int64_t nb01,         \
                           int64_t n_ids, void *stream) {                                                          \
    get_rows<D>(src0, ids, dst, ne00, nb01, n_ids, stream, "get_rows_" #t);                                       \
  }
QMM_DEFINE_DEQ(q8_0, deq_q8_0)
QMM_DEFINE_DEQ(q4_k, deq_q4k)
QMM_DEFINE_DEQ(q6_k, deq_q6k)
QMM_DEFINE_DEQ(q4_0, deq_q4_0)
QMM_DEFINE_DEQ(q5_0, deq_q5_0)
QMM_DEFINE_DEQ(q5_k, deq_q5k)
#undef QMM_DEFINE_DEQ

// IQ4_XS keeps the reference's (nrows, ncols) form of launch_dequantize_iq4_xs_<dt> (gguf/ffi.rs:1125-1150, 1265-1267;
// mmvq_gguf.cuh:2167-2174): nrows * ncols contiguous values
#define QMM_DEFINE_DEQ_IQ(t, D, dt, OUT)                                                                           \
  void launch_dequantize_##t##_##dt(const void *vx, void *dst, int64_t nrows, int64_t ncols, void *stream) {     \
    if (nrows < 0 || ncols < 0 || (nrows > 0 && ncols > INT64_MAX / nrows)) {                                    \
      qmm_set_error("dequantize_" #t "_" #dt ": nrows=%lld ncols=%lld", (long long)nrows, (long long)ncols);     \
      return;                                                                                                      \
    }                                                                                                              \
    dequantize<D, OUT>(vx, dst, nrows * ncols, stream, "dequantize_" #t "_" #dt);                                 \
  }
QMM_DEFINE_DEQ_IQ(iq4_xs, deq_iq4xs, f32, out_f32)
QMM_DEFINE_DEQ_IQ(iq4_xs, deq_iq4xs, f16, out_f16)
QMM_DEFINE_DEQ_IQ(iq4_xs, deq_iq4xs, bf16, out_bf16)
#undef QMM_DEFINE_DEQ_IQ

void launch_mmvq_gguf_q8_0_f32_exact(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int b_size,
                                     void *stream) {
  q8_0_exact<act_f32, out_f32>(vx, vy, dst, ncols_x, nrows_x, b_size, stream, "mmvq_q8_0_f32_exact");
}
void launch_mmvq_gguf_q8_0_bf16_exact(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, int b_size,
                                      void *stream) {
  q8_0_exact<act_bf16, out_bf16>(vx, vy, dst, ncols_x, nrows_x, b_size, stream, "mmvq_q8_0_bf16_exact");
}

}  // extern "C"

extern "C" void launch_gather_rows_u8(const void *src, const void *ids, void *dst, int64_t row_bytes, int64_t rows,
                                      int64_t n, void *stream) {
  if (!src || !ids || !dst || row_bytes <= 0 || rows < 0 || n < 0) {
    qmm_set_error("gather_rows_u8: row_bytes=%lld rows=%lld n=%lld", (long long)row_bytes, (long long)rows,
                  (long long)n);
    return;
  }
  if (n == 0) return;
  const bool vec = row_bytes % 16 == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0;
  const int64_t per = vec ? 16 : 1;
  const dim3 grid((unsigned)qmm_ceil_div(row_bytes, 256 * per), (unsigned)(n < 65535 ? n : 65535));
  if (vec)
    k_gather_rows_u8<true><<<grid, 256, 0, (hipStream_t)stream>>>((const uint8_t *)src, (const uint32_t *)ids,
                                                                  (uint8_t *)dst, row_bytes, rows, n);
  else
    k_gather_rows_u8<false><<<grid, 256, 0, (hipStream_t)stream>>>((const uint8_t *)src, (const uint32_t *)ids,
                                                                   (uint8_t *)dst, row_bytes, rows, n);
}
