// Measurement probes for bench.py, built into lib/libqmmbench.so (not into the product library): no counterpart in
// the reference; they compute nothing but what keeps the compiler from dropping their loads or matrix operations.
//
// HBM read probes: the time one launch needs to stream a buffer of the decode weight's size, the floor the decode
// matvec is measured against (a per-lane XOR of what is read is written out).
//   pattern 0  grid stride: wave slot s of the persistent grid reads 16-byte chunks s * 64 + lane, s + S, ... with
//              `depth` loads in flight per lane
//   pattern 1  the decode matvec's walk over Q4_K rows (k_mmvq_p): row r of wave slot s = r mod S, each lane loading
//              the 16-byte header and two 16-byte nibble chunks of its quarter superblock, `depth` rows in flight
//   pattern 2  the same rows read as contiguous 16-byte chunks per lane (1 KB per wave instruction)
//   pattern 3  pattern 2 plus each lane's 16-byte superblock header
// Copy probe: a grid-stride 16-byte copy, the measured HBM copy rate (bytes read + bytes written per second).
// MFMA probe: the measured dense int8 matrix rate, every wave issuing independent v_mfma_i32_32x32x32_i8 chains.
#include "common.h"
#include "units.h"

namespace {

template <int D>
__global__ __launch_bounds__(256) void k_read_stride(const u32x4 *__restrict__ src, int64_t chunks,
                                                     uint32_t *__restrict__ out) {
  const int64_t S = (int64_t)gridDim.x * 4;  // wave slots
  const int lane = threadIdx.x & 63;
  const int64_t slot = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t x = 0;
  for (int64_t c = slot * 64 + lane; c < chunks; c += S * 64 * D) {
    u32x4 v[D];
#pragma unroll
    for (int i = 0; i < D; i++) v[i] = c + i * S * 64 < chunks ? src[c + i * S * 64] : (u32x4){};
#pragma unroll
    for (int i = 0; i < D; i++) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = x;
}

// rows of row_bytes (a multiple of 144), D rows in flight per wave.  Scattered (the decode units): lane l loads unit l
// of the row (the unit_q4k loads, units past the row skipped).  Contiguous: lane l loads 16-byte chunks l, l + 64, ...
// of the row (1 KB per wave instruction), plus, with HDR, the 16-byte header of its first chunk's superblock.
template <bool CONTIG, bool HDR, int D>
__global__ __launch_bounds__(256) void k_read_rows(const uint8_t *__restrict__ w, int64_t nrows, int64_t row_bytes,
                                                   uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t S = (int64_t)gridDim.x * 4;
  const int nunits = (int)(row_bytes / 144 * 4);
  const int nchunks = (int)(row_bytes / 16);
  uint32_t x = 0;
  int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  struct buf {
    u32x4 v[3];
  };
  auto load = [&](int64_t row, buf &u) {
    if (row >= nrows) return;
    const uint8_t *p = w + row * row_bytes;
    if (CONTIG) {
#pragma unroll
      for (int i = 0; i < 3; i++)
        if (64 * i + lane < nchunks) u.v[i] = ld_a16(p + 16 * (64 * i + lane));
      if (HDR) u.v[2].x ^= ld_a16(p + 144 * (lane / 9)).y;
    } else if (lane < nunits) {
      unit_q4k::W t;
      unit_q4k::load_w(p, lane, t);
      u.v[0] = t.hdr, u.v[1] = t.q0, u.v[2] = t.q1;
    }
  };
  buf b[D];
#pragma unroll
  for (int i = 0; i < D; i++) load(r + i * S, b[i]);
  for (; r < nrows; r += D * S) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      x ^= b[i].v[0].x ^ b[i].v[1].y ^ b[i].v[2].z;
      load(r + (D + i) * S, b[i]);
    }
  }
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = x;
}

// grid-stride copy of `chunks` 16-byte chunks, D chunks in flight per lane
template <int D>
__global__ __launch_bounds__(256) void k_copy(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, int64_t chunks) {
  const int64_t S = (int64_t)gridDim.x * 256;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += S * D) {
    u32x4 v[D];
#pragma unroll
    for (int i = 0; i < D; i++)
      if (c + i * S < chunks) v[i] = src[c + i * S];
#pragma unroll
    for (int i = 0; i < D; i++)
      if (c + i * S < chunks) dst[c + i * S] = v[i];
  }
}

// Four independent accumulator chains per wave hide the MFMA's dependency latency; operands differ per lane and
// iteration count comes from the host, so nothing folds.  2 * 32 * 32 * 32 int8 ops per instruction.
__global__ __launch_bounds__(256) void k_mfma_i8(int iters, int seed, int *__restrict__ out) {
  const int t = threadIdx.x + seed;
  const v4i a = {t, t * 3, t * 5, t * 7}, b = {t ^ 0x5a5a5a5a, t + 11, t * 13, ~t};
  v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; i++) {
    c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
  }
  int x = 0;
#pragma unroll
  for (int r = 0; r < 16; r++) x ^= c0[r] + c1[r] + c2[r] + c3[r];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = x;
}

}  // namespace

extern "C" int qmm_hbm_read_probe(const void *src, int64_t bytes, int pattern, int per_cu, int depth, uint32_t *out,
                                  void *stream) {
  if (!src || !out || bytes <= 0 || per_cu < 1 || per_cu > 16 || (uintptr_t)src % 16 != 0) {
    qmm_set_error("hbm_read_probe: src %p bytes %lld per_cu %d", src, (long long)bytes, per_cu);
    return -1;
  }
  const unsigned grid = (unsigned)(per_cu * qmm_device_cus());
  hipStream_t s = (hipStream_t)stream;
  if (pattern == 0) {
    const int64_t chunks = bytes / 16;
    switch (depth) {
      case 1: k_read_stride<1><<<grid, 256, 0, s>>>((const u32x4 *)src, chunks, out); break;
      case 2: k_read_stride<2><<<grid, 256, 0, s>>>((const u32x4 *)src, chunks, out); break;
      case 4: k_read_stride<4><<<grid, 256, 0, s>>>((const u32x4 *)src, chunks, out); break;
      default: k_read_stride<8><<<grid, 256, 0, s>>>((const u32x4 *)src, chunks, out); break;
    }
  } else {
    const int64_t row_bytes = 2304;  // Q4_K, K = 4096
    const int64_t nrows = bytes / row_bytes;
    const uint8_t *w = (const uint8_t *)src;
#define QMM_RR(C, H)                                                                               \
  do {                                                                                             \
    if (depth <= 1) k_read_rows<C, H, 1><<<grid, 256, 0, s>>>(w, nrows, row_bytes, out);           \
    else if (depth == 2) k_read_rows<C, H, 2><<<grid, 256, 0, s>>>(w, nrows, row_bytes, out);      \
    else k_read_rows<C, H, 3><<<grid, 256, 0, s>>>(w, nrows, row_bytes, out);                      \
  } while (0)
    if (pattern == 1) QMM_RR(false, false);
    else if (pattern == 2) QMM_RR(true, false);
    else QMM_RR(true, true);
#undef QMM_RR
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// One grid-stride copy of `bytes` (a multiple of 16; both pointers 16-byte aligned) from src to dst with per_cu
// workgroups of 256 threads per CU and `depth` (1, 2 or 4) chunks in flight per lane.  Returns 0, or -1 with
// qmm_last_error() set.
extern "C" int qmm_bench_copy(const void *src, void *dst, int64_t bytes, int per_cu, int depth, void *stream) {
  if (!src || !dst || bytes <= 0 || bytes % 16 != 0 || per_cu < 1 || per_cu > 16 || (uintptr_t)src % 16 != 0 ||
      (uintptr_t)dst % 16 != 0) {
    qmm_set_error("bench_copy: src %p dst %p bytes %lld per_cu %d", src, dst, (long long)bytes, per_cu);
    return -1;
  }
  const unsigned grid = (unsigned)(per_cu * qmm_device_cus());
  hipStream_t s = (hipStream_t)stream;
  const int64_t chunks = bytes / 16;
  if (depth <= 1) k_copy<1><<<grid, 256, 0, s>>>((const u32x4 *)src, (u32x4 *)dst, chunks);
  else if (depth == 2) k_copy<2><<<grid, 256, 0, s>>>((const u32x4 *)src, (u32x4 *)dst, chunks);
  else k_copy<4><<<grid, 256, 0, s>>>((const u32x4 *)src, (u32x4 *)dst, chunks);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// per_cu workgroups of 4 waves per CU, each wave issuing 4 * iters v_mfma_i32_32x32x32_i8 (65,536 int8 ops each);
// out holds per_cu * CUs * 256 ints.  Returns the int8 ops launched (> 0), or -1 with qmm_last_error() set.
extern "C" double qmm_bench_mfma_i8(int per_cu, int iters, int *out, void *stream) {
  if (!out || per_cu < 1 || per_cu > 8 || iters < 1) {
    qmm_set_error("bench_mfma_i8: per_cu %d iters %d", per_cu, iters);
    return -1.0;
  }
  const unsigned grid = (unsigned)(per_cu * qmm_device_cus());
  k_mfma_i8<<<grid, 256, 0, (hipStream_t)stream>>>(iters, per_cu, out);
  if (hipGetLastError() != hipSuccess) return -1.0;
  return (double)grid * 4 * 4 * (double)iters * 65536.0;
}
