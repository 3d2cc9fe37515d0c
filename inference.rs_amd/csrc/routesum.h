// The weighted sum over each token's routes folded into the expert-grouped down projection
// (launch_mmq_gguf_<t>_moe_wsum): out[t, n] = sum_s w[t, s] * routes[t * topk + s, n], summed in slot order with the
// arithmetic of launch_moe_weighted_reduce_flat (moe.hip), so the result is the two launches' bit for bit and does
// not depend on which workgroup finished first.
//
// A token's routes go to different experts, so different workgroups write them.  Each workgroup stores its route
// rows of one column tile, then counts them: one counter per (token, column tile), incremented once per route row.
// The workgroup whose increment completes a token's count (topk) reads the token's topk route rows of that tile --
// its own and the ones other workgroups wrote -- and stores their weighted sum.  The stores are released at agent
// scope before the count and acquired after it, so rows written by workgroups on other XCDs (other L2s) are seen.
// The completing workgroup sets the counter back to zero: counters are zero between calls, which the caller
// establishes once when it allocates them.
#pragma once

#include "common.h"

struct RouteSum {
  float *out;              // [tokens, ldo] f32; nullptr: no fused sum (the kernel only stores the route rows)
  const float *weights;    // router weights [tokens * topk], route (pair) order
  int32_t *counters;       // [tokens * col_tiles], zero between calls
  int64_t ldo;
  int32_t topk, col_tiles;
};

// w * y accumulated as launch_moe_weighted_reduce_flat does; a zero-weight route is not read (the grouped kernels may
// never have written it)
__device__ __forceinline__ float route_acc(float acc, float y, float w) { return __builtin_fmaf(y, w, acc); }

// Every thread of the workgroup (NT threads) calls this after its stores of route rows m in [m0, min(m1, m0 + ROWS))
// (destination row ids_dst[m] of `routes`, ldr apart) at columns [n0, n0 + ncols) of column tile `tile`.
template <int NT, int ROWS>
__device__ __forceinline__ void route_sum_finish(const RouteSum &rs, const float *routes, int64_t ldr,
                                                 const int32_t *__restrict__ ids_dst, int64_t m0, int64_t m1,
                                                 int64_t n0, int ncols, int tile) {
  static_assert(ROWS <= NT, "one thread per chunk row");
  __shared__ int32_t done[ROWS];  // per chunk row: the token whose count this workgroup completed, or -1
  const int tid = threadIdx.x;
  const int rows = (int)(m1 - m0 < ROWS ? m1 - m0 : ROWS);
  __threadfence();  // release: this thread's route stores come before the counts below
  __syncthreads();
  if (tid < ROWS) {
    int32_t tok = -1;
    if (tid < rows) {
      const int32_t t = ids_dst[m0 + tid] / rs.topk;
      int32_t *c = rs.counters + (int64_t)t * rs.col_tiles + tile;
      if (atomicAdd(c, 1) == rs.topk - 1) {
        atomicExch(c, 0);  // the last route row of (t, tile) in this call: zero again for the next one
        tok = t;
      }
    }
    done[tid] = tok;
  }
  __syncthreads();
  __threadfence();  // acquire: the other workgroups' route rows of completed tokens are visible from here
  for (int i = tid; i < rows * ncols; i += NT) {
    const int r = i / ncols, col = i - r * ncols;
    const int32_t t = done[r];
    if (t < 0) continue;
    const int64_t n = n0 + col;
    float acc = 0.0f;
    for (int s = 0; s < rs.topk; s++) {
      const float w = rs.weights[(int64_t)t * rs.topk + s];
      if (w != 0.0f) acc = route_acc(acc, routes[((int64_t)t * rs.topk + s) * ldr + n], w);
    }
    rs.out[(int64_t)t * rs.ldo + n] = acc;
  }
}
