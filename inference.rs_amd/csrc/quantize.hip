// Activation quantizers for the decode and prefill paths, bit-exact with the reference CPU quantizers:
//   Q8_K  BlockQ8K::from_float        crates/inference-tensor/src/quantized/k_quants.rs:2721-2760
//   Q8_0  quantize_block32 + f16 d    crates/inference-tensor/src/quantized/mod.rs:41-56, k_quants.rs:923-949
// Built with -ffp-contract=off; division and roundf are IEEE (no fast-math), so every step rounds as the
// CPU's does.  Q8_K: one wave per 256-value block, 4 values per lane; the signed value of largest magnitude
// is found with a (|x|, first index) wave reduction so ties resolve to the first occurrence as in the
// reference's sequential scan.
#include "common.h"
#include "inferencequant.h"
#include "q8.h"

namespace {

using namespace qmm_q8;

// ------------------------------------------------------------------ decode layout kernels

// the reference-named decode layout: rows of kx_padded / 256 qmm_block_q8ks (288 bytes: d, qs, int16 sums of 32)
template <class In>
__global__ __launch_bounds__(256) void k_quantize_q8ks_rows(const typename In::T *__restrict__ x,
                                                            uint8_t *__restrict__ vy, int kx, int kx_padded,
                                                            int num_rows) {
  const int lane = threadIdx.x & 63;
  // 32-bit index arithmetic: blocks = kx_padded / 256 * num_rows fits an int (the launcher checks)
  const unsigned nsb = (unsigned)kx_padded / 256;
  const unsigned blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nsb * (unsigned)num_rows) return;  // whole wave
  const unsigned row = blk / nsb, sb = blk - row * nsb;
  float v[4];
  load4<In>(x + (int64_t)row * kx, (int64_t)sb * 256 + lane * 4, kx, v);
  q8k_wave(v, lane, q8k_slot_dst(vy, blk));
}

// the tensor-core entries' layout: rows of kx / 256 blocks {f32 d; int8 qs[256]}
template <class In>
__global__ __launch_bounds__(256) void k_quantize_q8k_tc_rows(const typename In::T *__restrict__ x,
                                                              uint8_t *__restrict__ vy, int kx, int num_rows) {
  const int lane = threadIdx.x & 63;
  const unsigned nsb = (unsigned)kx / 256;
  const unsigned blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nsb * (unsigned)num_rows) return;  // whole wave
  const unsigned row = blk / nsb, sb = blk - row * nsb;
  float v[4];
  load4<In>(x + (int64_t)row * kx, (int64_t)sb * 256 + lane * 4, kx, v);
  q8k_wave(v, lane, q8k_tc_dst(vy, blk));
}

template <class In>
__global__ __launch_bounds__(256) void k_quantize_q8_0_rows(const typename In::T *__restrict__ x,
                                                            uint8_t *__restrict__ vy, int kx, int kx_padded,
                                                            int num_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = kx_padded / 32;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  const bool valid = blk < nb * num_rows;
  const int64_t b = valid ? blk : 0;
  const int64_t row = b / nb, ib = b % nb;
  float v[4];
  load4<In>(x + row * (int64_t)kx, ib * 32 + (lane & 7) * 4, valid ? kx : 0, v);
  uint8_t *blkp = vy + b * 34;
  q8_0_group(v, lane & 7, (int8_t *)(blkp + 2), (uint16_t *)blkp, valid);
}

// ------------------------------------------------------------------ prefill (tile) layout kernels

// Grid (row groups of 4, superblock columns, channels): one block per wave, its indices from the grid with no
// division (the 64-bit index divisions of a flat grid were a large share of each wave's few hundred instructions).
// S16: the `_q8k` tiles (f16 sums of 16, 292 bytes per 256 values), else the reference-named tiles (int16 sums of 32).
template <class In, bool S16>
__global__ __launch_bounds__(256) void k_quantize_q8k_tiles(const typename In::T *__restrict__ x,
                                                            const int32_t *__restrict__ ids, uint8_t *__restrict__ vy,
                                                            int64_t ne00, int64_t s01, int64_t s02, int64_t s03,
                                                            int64_t ne0, int64_t ne1, int ne2) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= ne1) return;  // whole wave
  const int64_t sb = blockIdx.y, nsb = ne0 / 256;
  const int ch = blockIdx.z, i2 = ch % ne2, i3 = ch / ne2;
  const int64_t src_row = ids ? ids[r] : r;
  float v[4];
  load4<In>(x + i3 * s03 + i2 * s02 + src_row * s01, sb * 256 + lane * 4, ne00, v);
  uint8_t *chan = vy + (int64_t)ch * nsb * ne1 * (S16 ? 292 : 276);
  q8k_wave(v, lane, S16 ? q8k_tile16_dst(chan, ne1, nsb, sb, r) : q8k_tile_dst(chan, ne1, nsb, sb, r));
}

template <class In>
__global__ __launch_bounds__(256) void k_quantize_q8_0_tiles(const typename In::T *__restrict__ x,
                                                             const int32_t *__restrict__ ids,
                                                             uint8_t *__restrict__ vy, int64_t ne00, int64_t s01,
                                                             int64_t s02, int64_t s03, int64_t ne0, int64_t ne1,
                                                             int64_t ne2, int64_t nblk32) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  const bool valid = blk < nblk32;
  const int64_t b = valid ? blk : 0;
  const int64_t nsb = ne0 / 256;
  const int64_t per_chan = nsb * ne1 * 8;  // 32-value blocks per channel
  const int64_t ch = b / per_chan, rem = b % per_chan;
  const int64_t sb = rem / (ne1 * 8), r = (rem / 8) % ne1, j = rem % 8;
  const int64_t i2 = ch % ne2, i3 = ch / ne2;
  const int64_t src_row = valid ? (ids ? ids[r] : r) : 0;
  float v[4];
  load4<In>(x + i3 * s03 + i2 * s02 + src_row * s01, sb * 256 + j * 32 + (lane & 7) * 4, valid ? ne00 : 0, v);
  uint8_t *chan = vy + ch * nsb * ne1 * 272;
  int8_t *qs = (int8_t *)(chan + (sb * ne1 + r) * 256 + j * 32);
  uint16_t *d = (uint16_t *)(chan + nsb * ne1 * 256) + (sb * ne1 + r) * 8 + j;
  q8_0_group(v, lane & 7, qs, d, valid);
}

// act(gate) * up of row ids[r] (or r), quantized into the prefill tile layout: the fused GLU requantization
// between the gate/up and down matmuls (mmq_gguf/mmq_quantize.cu:230-330).  f32 inputs: act(gate) * up in f32;
// f16 / bf16 inputs: act(gate) rounded to the input type, times up, rounded again, as the reference's
// mmq_glu_product<input_t> (mmq_quantize.cu:230-235).
template <class In>
__device__ __forceinline__ float glu_product(float g, float u, int activation);
template <>
__device__ __forceinline__ float glu_product<in_f32>(float g, float u, int activation) {
  return glu_act(activation, g) * u;
}
template <>
__device__ __forceinline__ float glu_product<in_f16>(float g, float u, int activation) {
  const float a = f16_bits_to_f32(f32_to_f16_bits(glu_act(activation, g)));
  return f16_bits_to_f32(f32_to_f16_bits(a * u));  // the product of two f16 is exact in f32: one rounding
}
template <>
__device__ __forceinline__ float glu_product<in_bf16>(float g, float u, int activation) {
  const float a = bf16_bits_to_f32(f32_to_bf16_bits(glu_act(activation, g)));
  return bf16_bits_to_f32(f32_to_bf16_bits(a * u));
}

template <class In, bool S16>
__global__ __launch_bounds__(256) void k_quantize_glu_q8k_tiles(const typename In::T *__restrict__ gate,
                                                                const typename In::T *__restrict__ up,
                                                                const int32_t *__restrict__ ids, uint8_t *__restrict__ vy,
                                                                int64_t ne00, int64_t s01, int64_t ne0, int64_t ne1,
                                                                int activation) {
  // grid (row groups of 4, superblock columns), as k_quantize_q8k_tiles
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= ne1) return;  // whole wave
  const int64_t nsb = ne0 / 256, sb = blockIdx.y;
  const int64_t src = (ids ? ids[r] : r) * s01;
  // one vector load per lane for each input where the four values are in the row and aligned (load4)
  float g[4], u[4], v[4];
  load4<In>(gate + src, sb * 256 + lane * 4, ne00, g);
  load4<In>(up + src, sb * 256 + lane * 4, ne00, u);
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = sb * 256 + lane * 4 + i < ne00 ? glu_product<In>(g[i], u[i], activation) : 0.0f;
  q8k_wave(v, lane, S16 ? q8k_tile16_dst(vy, ne1, nsb, sb, r) : q8k_tile_dst(vy, ne1, nsb, sb, r));
}

__global__ __launch_bounds__(256) void k_quantize_glu_q8_0_tiles(const float *__restrict__ gate,
                                                                 const float *__restrict__ up,
                                                                 const int32_t *__restrict__ ids,
                                                                 uint8_t *__restrict__ vy, int64_t ne00, int64_t s01,
                                                                 int64_t ne0, int64_t ne1, int activation,
                                                                 int64_t nblk32) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  const bool valid = blk < nblk32;
  const int64_t b = valid ? blk : 0;
  const int64_t nsb = ne0 / 256;
  const int64_t sb = b / (ne1 * 8), r = (b / 8) % ne1, j = b % 8;
  const int64_t src = valid ? (ids ? ids[r] : r) * s01 : 0;
  const int64_t k0 = sb * 256 + j * 32 + (lane & 7) * 4;
  float g[4], u[4], v[4];
  load4<in_f32>(gate + src, k0, valid ? ne00 : 0, g);
  load4<in_f32>(up + src, k0, valid ? ne00 : 0, u);
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = (valid && k0 + i < ne00) ? glu_act(activation, g[i]) * u[i] : 0.0f;
  int8_t *qs = (int8_t *)(vy + (sb * ne1 + r) * 256 + j * 32);
  uint16_t *d = (uint16_t *)(vy + nsb * ne1 * 256) + (sb * ne1 + r) * 8 + j;
  q8_0_group(v, lane & 7, qs, d, valid);
}

template <class In>
void decode_q8ks(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  if (kx < 0 || num_rows < 0 || kx_padded % 256 != 0 || kx_padded < kx) {
    qmm_set_error("quantize_q8_1: kx=%d kx_padded=%d num_rows=%d (kx_padded must be a multiple of 256, >= kx)", kx,
                  kx_padded, num_rows);
    return;
  }
  const int64_t blocks = (int64_t)kx_padded / 256 * num_rows;
  if (blocks == 0) return;
  if (blocks > INT32_MAX) {
    qmm_set_error("quantize_q8_1: %lld blocks (at most 2^31 - 1)", (long long)blocks);
    return;
  }
  k_quantize_q8ks_rows<In><<<dim3((unsigned)qmm_ceil_div(blocks, 4)), 256, 0, (hipStream_t)stream>>>(
      (const typename In::T *)x, (uint8_t *)vy, kx, kx_padded, num_rows);
}

template <class In>
void tc_q8k(const void *x, void *vy, int kx, int num_rows, void *stream) {
  if (kx <= 0 || num_rows < 0 || kx % 256 != 0) {
    qmm_set_error("mmvq_tc_quantize: kx=%d num_rows=%d (kx must be a positive multiple of 256)", kx, num_rows);
    return;
  }
  const int64_t blocks = (int64_t)kx / 256 * num_rows;
  if (blocks == 0) return;
  if (blocks > INT32_MAX) {
    qmm_set_error("mmvq_tc_quantize: %lld blocks (at most 2^31 - 1)", (long long)blocks);
    return;
  }
  k_quantize_q8k_tc_rows<In><<<dim3((unsigned)qmm_ceil_div(blocks, 4)), 256, 0, (hipStream_t)stream>>>(
      (const typename In::T *)x, (uint8_t *)vy, kx, num_rows);
}

template <class In>
void decode_q8_0(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  if (kx < 0 || num_rows < 0 || kx_padded % 32 != 0 || kx_padded < kx) {
    qmm_set_error("quantize_q8_0: kx=%d kx_padded=%d num_rows=%d (kx_padded must be a multiple of 32, >= kx)", kx,
                  kx_padded, num_rows);
    return;
  }
  const int64_t blocks = (int64_t)kx_padded / 32 * num_rows;
  if (blocks == 0) return;
  k_quantize_q8_0_rows<In><<<dim3((unsigned)qmm_ceil_div(blocks, 32)), 256, 0, (hipStream_t)stream>>>(
      (const typename In::T *)x, (uint8_t *)vy, kx, kx_padded, num_rows);
}

bool tile_args_ok(const char *who, int64_t ne00, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
  if (ne00 < 0 || ne0 % 256 != 0 || ne0 < ne00 || ne1 < 0 || ne2 < 1 || ne3 < 1) {
    qmm_set_error("%s: ne00=%lld ne0=%lld ne1=%lld ne2=%lld ne3=%lld (ne0 must be a multiple of 256, >= ne00)", who,
                  (long long)ne00, (long long)ne0, (long long)ne1, (long long)ne2, (long long)ne3);
    return false;
  }
  return true;
}

// The prefill tiles hold ceil(ne00 / 256) super-blocks per row, whatever ne0 (the caller's k_padded, a multiple of 256
// at least ne00): the matmuls are handed K, not k_padded, and read that many.  A reference caller pads K to 512
// (fast_mmq.rs) and sizes its scratch for that; the super-blocks past ceil(K / 256), all zeros there, are neither
// written nor read here.
int64_t tile_width(int64_t ne00) { return (ne00 + 255) / 256 * 256; }

}  // namespace

extern "C" {

void launch_mmvq_gguf_quantize_q8_1_f32(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  decode_q8ks<in_f32>(x, vy, kx, kx_padded, num_rows, stream);
}
void launch_mmvq_gguf_quantize_q8_1_f16(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  decode_q8ks<in_f16>(x, vy, kx, kx_padded, num_rows, stream);
}
void launch_mmvq_gguf_quantize_q8_1_bf16(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  decode_q8ks<in_bf16>(x, vy, kx, kx_padded, num_rows, stream);
}
void launch_mmvq_tc_quantize_f32(const void *x, void *vy, int kx, int num_rows, void *stream) {
  tc_q8k<in_f32>(x, vy, kx, num_rows, stream);
}
void launch_mmvq_tc_quantize_f16(const void *x, void *vy, int kx, int num_rows, void *stream) {
  tc_q8k<in_f16>(x, vy, kx, num_rows, stream);
}
void launch_mmvq_tc_quantize_bf16(const void *x, void *vy, int kx, int num_rows, void *stream) {
  tc_q8k<in_bf16>(x, vy, kx, num_rows, stream);
}
void launch_mmvq_gguf_quantize_q8_0_f32(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  decode_q8_0<in_f32>(x, vy, kx, kx_padded, num_rows, stream);
}
void launch_mmvq_gguf_quantize_q8_0_f16(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream) {
  decode_q8_0<in_f16>(x, vy, kx, kx_padded, num_rows, stream);
}
void launch_mmvq_gguf_quantize_q8_0_bf16(const void *x, void *vy, int kx, int kx_padded, int num_rows,
                                         void *stream) {
  decode_q8_0<in_bf16>(x, vy, kx, kx_padded, num_rows, stream);
}

}  // extern "C"

namespace {
template <bool S16>
void mmq_quantize_q8ks(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01, int64_t s02,
                       int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, void *stream) {
  if (!tile_args_ok(S16 ? "mmq_quantize_q8k" : "mmq_quantize_q8_1", ne00, ne0, ne1, ne2, ne3)) return;
  const int64_t kt = tile_width(ne00);
  if (kt == 0 || ne1 == 0) return;
  if (kt / 256 > 65535 || ne2 * ne3 > 65535 || qmm_ceil_div(ne1, 4) > INT32_MAX) {
    qmm_set_error("mmq_quantize_q8_1: ne0=%lld ne1=%lld ne2*ne3=%lld beyond the grid", (long long)ne0, (long long)ne1,
                  (long long)(ne2 * ne3));
    return;
  }
  const dim3 grid((unsigned)qmm_ceil_div(ne1, 4), (unsigned)(kt / 256), (unsigned)(ne2 * ne3));
  hipStream_t s = (hipStream_t)stream;
  uint8_t *y = (uint8_t *)vy;
  switch (type_x) {
    case QMM_TYPE_F32:
      k_quantize_q8k_tiles<in_f32, S16><<<grid, 256, 0, s>>>((const float *)x, ids, y, ne00, s01, s02, s03, kt, ne1, (int)ne2);
      break;
    case QMM_TYPE_F16:
      k_quantize_q8k_tiles<in_f16, S16><<<grid, 256, 0, s>>>((const uint16_t *)x, ids, y, ne00, s01, s02, s03, kt, ne1,
                                                        (int)ne2);
      break;
    case QMM_TYPE_BF16:
      k_quantize_q8k_tiles<in_bf16, S16><<<grid, 256, 0, s>>>((const uint16_t *)x, ids, y, ne00, s01, s02, s03, kt, ne1,
                                                         (int)ne2);
      break;
    default: qmm_set_error("mmq_quantize_q8_1: unsupported input type %d", type_x);
  }
}

template <bool S16>
void mmq_quantize_glu_q8ks(const void *gate, const void *up, const int32_t *ids, void *vy, int type_x, int64_t ne00,
                           int64_t s01, int64_t ne0, int64_t ne1, int activation, void *stream) {
  if (!tile_args_ok("mmq_quantize_glu_q8_1", ne00, ne0, ne1, 1, 1)) return;
  const int64_t kt = tile_width(ne00);
  if (activation < 0 || activation >= kGluActivations) {
    qmm_set_error("mmq_quantize_glu_q8_1: activation %d", activation);
    return;
  }
  if (kt == 0 || ne1 == 0) return;
  if (kt / 256 > 65535 || qmm_ceil_div(ne1, 4) > INT32_MAX) {
    qmm_set_error("mmq_quantize_glu_q8_1: ne0=%lld ne1=%lld beyond the grid", (long long)ne0, (long long)ne1);
    return;
  }
  const dim3 grid((unsigned)qmm_ceil_div(ne1, 4), (unsigned)(kt / 256));
  hipStream_t s = (hipStream_t)stream;
  uint8_t *y = (uint8_t *)vy;
  switch (type_x) {
    case QMM_TYPE_F32:
      k_quantize_glu_q8k_tiles<in_f32, S16><<<grid, 256, 0, s>>>((const float *)gate, (const float *)up, ids, y, ne00, s01,
                                                            kt, ne1, activation);
      break;
    case QMM_TYPE_F16:
      k_quantize_glu_q8k_tiles<in_f16, S16><<<grid, 256, 0, s>>>((const uint16_t *)gate, (const uint16_t *)up, ids, y, ne00,
                                                            s01, kt, ne1, activation);
      break;
    case QMM_TYPE_BF16:
      k_quantize_glu_q8k_tiles<in_bf16, S16><<<grid, 256, 0, s>>>((const uint16_t *)gate, (const uint16_t *)up, ids, y,
                                                             ne00, s01, kt, ne1, activation);
      break;
    default: qmm_set_error("mmq_quantize_glu_q8_1: unsupported input type %d", type_x);
  }
}
}  // namespace

extern "C" {

// The three scale layouts the reference's MMQ kernels distinguish (fast_mmq.rs:160-200) write one layout here:
// every prefill kernel of this library reads the same tile layout.
#define QMM_DEFINE_MMQ_Q8_1(L)                                                                                      \
  void launch_mmq_quantize_q8_1_##L(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00,         \
                                    int64_t s01, int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2,  \
                                    int64_t ne3, void *stream) {                                                   \
    mmq_quantize_q8ks<false>(x, ids, vy, type_x, ne00, s01, s02, s03, ne0, ne1, ne2, ne3, stream);                 \
  }                                                                                                                \
  void launch_mmq_quantize_glu_q8_1_##L##_f32(const float *gate, const float *up, const int32_t *ids, void *vy,    \
                                              int64_t ne00, int64_t s01, int64_t ne0, int64_t ne1, int activation, \
                                              void *stream) {                                                      \
    mmq_quantize_glu_q8ks<false>(gate, up, ids, vy, QMM_TYPE_F32, ne00, s01, ne0, ne1, activation, stream);        \
  }                                                                                                                \
  void launch_mmq_quantize_glu_q8_1_##L(const void *gate, const void *up, const int32_t *ids, void *vy, int type_x, \
                                        int64_t ne00, int64_t s01, int64_t ne0, int64_t ne1, int activation,       \
                                        void *stream) {                                                            \
    mmq_quantize_glu_q8ks<false>(gate, up, ids, vy, type_x, ne00, s01, ne0, ne1, activation, stream);              \
  }
QMM_DEFINE_MMQ_Q8_1(D4)
QMM_DEFINE_MMQ_Q8_1(DS4)
QMM_DEFINE_MMQ_Q8_1(D2S6)
#undef QMM_DEFINE_MMQ_Q8_1

void launch_mmq_quantize_q8k(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01,
                             int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                             void *stream) {
  mmq_quantize_q8ks<true>(x, ids, vy, type_x, ne00, s01, s02, s03, ne0, ne1, ne2, ne3, stream);
}

void launch_mmq_quantize_glu_q8k_f32(const float *gate, const float *up, const int32_t *ids, void *vy, int64_t ne00,
                                     int64_t s01, int64_t ne0, int64_t ne1, int activation, void *stream) {
  mmq_quantize_glu_q8ks<true>(gate, up, ids, vy, QMM_TYPE_F32, ne00, s01, ne0, ne1, activation, stream);
}

void launch_mmq_quantize_q8_0(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01,
                              int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                              void *stream) {
  if (!tile_args_ok("mmq_quantize_q8_0", ne00, ne0, ne1, ne2, ne3)) return;
  const int64_t kt = tile_width(ne00);
  const int64_t nblk = kt / 32 * ne1 * ne2 * ne3;
  if (nblk == 0) return;
  const dim3 grid((unsigned)qmm_ceil_div(nblk, 32));
  hipStream_t s = (hipStream_t)stream;
  uint8_t *y = (uint8_t *)vy;
  switch (type_x) {
    case QMM_TYPE_F32:
      k_quantize_q8_0_tiles<in_f32><<<grid, 256, 0, s>>>((const float *)x, ids, y, ne00, s01, s02, s03, kt, ne1, ne2,
                                                         nblk);
      break;
    case QMM_TYPE_F16:
      k_quantize_q8_0_tiles<in_f16><<<grid, 256, 0, s>>>((const uint16_t *)x, ids, y, ne00, s01, s02, s03, kt, ne1,
                                                         ne2, nblk);
      break;
    case QMM_TYPE_BF16:
      k_quantize_q8_0_tiles<in_bf16><<<grid, 256, 0, s>>>((const uint16_t *)x, ids, y, ne00, s01, s02, s03, kt, ne1,
                                                          ne2, nblk);
      break;
    default: qmm_set_error("mmq_quantize_q8_0: unsupported input type %d", type_x);
  }
}

void launch_mmq_quantize_glu_q8_0_f32(const float *gate, const float *up, const int32_t *ids, void *vy, int64_t ne00,
                                      int64_t s01, int64_t ne0, int64_t ne1, int activation, void *stream) {
  if (!tile_args_ok("mmq_quantize_glu_q8_0", ne00, ne0, ne1, 1, 1)) return;
  const int64_t kt = tile_width(ne00);
  if (activation < 0 || activation >= kGluActivations) {
    qmm_set_error("mmq_quantize_glu_q8_0: activation %d", activation);
    return;
  }
  const int64_t nblk = kt / 32 * ne1;
  if (nblk == 0) return;
  k_quantize_glu_q8_0_tiles<<<dim3((unsigned)qmm_ceil_div(nblk, 32)), 256, 0, (hipStream_t)stream>>>(
      gate, up, ids, (uint8_t *)vy, ne00, s01, kt, ne1, activation, nblk);
}

}  // extern "C"
