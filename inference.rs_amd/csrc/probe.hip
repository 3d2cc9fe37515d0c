// HBM read probes: the time one launch needs to stream a buffer of the decode weight's size, the floor the decode
// matvec is measured against.  No counterpart in the reference; they compute nothing but a per-lane XOR of what they
// read (written out so the loads cannot be dropped).
//   pattern 0  grid stride: wave slot s of the persistent grid reads 16-byte chunks s * 64 + lane, s + S, ... with
//              `depth` loads in flight per lane
//   pattern 1  the decode matvec's walk over Q4_K rows (k_mmvq_p): row r of wave slot s = r mod S, each lane loading
//              the 16-byte header and two 16-byte nibble chunks of its quarter superblock, two rows in flight
#include "common.h"
#include "inferencequant.h"
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

// rows of row_bytes (a multiple of 144): lane l of a wave loads unit l of the row (the unit_q4k loads), units past
// the row skipped; two rows in flight
__global__ __launch_bounds__(256) void k_read_rows(const uint8_t *__restrict__ w, int64_t nrows, int64_t row_bytes,
                                                   uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t S = (int64_t)gridDim.x * 4;
  const int nunits = (int)(row_bytes / 144 * 4);
  uint32_t x = 0;
  int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  unit_q4k::W a, b;
  auto load = [&](int64_t row, unit_q4k::W &u) {
    if (row < nrows && lane < nunits) unit_q4k::load_w(w + row * row_bytes, lane, u);
  };
  load(r, a);
  load(r + S, b);
  for (; r < nrows; r += 2 * S) {
    x ^= a.hdr.x ^ a.q0.y ^ a.q1.z;
    load(r + 2 * S, a);
    x ^= b.hdr.x ^ b.q0.y ^ b.q1.z;
    load(r + 3 * S, b);
  }
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
    k_read_rows<<<grid, 256, 0, s>>>((const uint8_t *)src, bytes / row_bytes, row_bytes, out);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
