// MoE routing tables and the weighted top-k reduce around the expert-grouped matmul.
//   launch_moe_dispatch                crates/inference-quant/kernels/cuda/moe_dispatch/moe_dispatch.cu:78-104
//   launch_moe_weighted_reduce_flat*   moe_dispatch.cu:47-154
// The dispatch runs as one workgroup: counts in LDS, a scan, then the scatter through LDS cursors.  Route
// order inside an expert follows atomic arrival (as in the reference); only the grouping is contractual.
// No memset/memcpy nodes, so the sequence can be captured in a HIP graph.
#include "common.h"
#include "inferencequant.h"

namespace {

constexpr int kMaxExperts = 4096;

__global__ __launch_bounds__(1024) void k_moe_dispatch(const int32_t *__restrict__ topk_ids, int32_t *__restrict__ bounds,
                                                       int32_t *__restrict__ sorted_tok, int32_t *__restrict__ sorted_src,
                                                       int total, int n_experts, int topk, int32_t *__restrict__ counts,
                                                       int32_t *__restrict__ cursors) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int wsum[16];
  const int tid = threadIdx.x;
  for (int e = tid; e < n_experts; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < total; i += blockDim.x) {
    const int e = topk_ids[i];
    if (e >= 0 && e < n_experts) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scan of cnt over experts, in chunks of 1024 (one expert per thread per chunk)
  int carry = 0;
  for (int base = 0; base < n_experts; base += 1024) {
    const int e = base + tid;
    const int c = e < n_experts ? cnt[e] : 0;
    int incl = c;
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int wprefix = 0;
    for (int w = 0; w < wave; w++) wprefix += wsum[w];
    int chunk_total = 0;
    for (int w = 0; w < 16; w++) chunk_total += wsum[w];
    const int excl = carry + wprefix + incl - c;
    __syncthreads();
    if (e < n_experts) {
      bounds[e] = excl;
      counts[e] = c;
      cnt[e] = excl;  // becomes the scatter cursor
    }
    carry += chunk_total;
    __syncthreads();
  }
  if (tid == 0) bounds[n_experts] = carry;
  __syncthreads();
  for (int i = tid; i < total; i += blockDim.x) {
    const int e = topk_ids[i];
    if (e < 0 || e >= n_experts) continue;
    const int pos = atomicAdd(&cnt[e], 1);
    sorted_tok[pos] = i;  // flat route index: token = i / topk
    sorted_src[pos] = i / topk;
  }
  __syncthreads();
  for (int e = tid; e < n_experts; e += blockDim.x) cursors[e] = cnt[e];
}

template <class In, class Out>
__global__ __launch_bounds__(256) void k_weighted_reduce(const typename In::T *__restrict__ in,
                                                         const float *__restrict__ w, typename Out::T *__restrict__ out,
                                                         int tokens, int hidden, int topk) {
  const int t = blockIdx.x;
  const int h = blockIdx.y * blockDim.x + threadIdx.x;
  if (t >= tokens || h >= hidden) return;
  const int64_t base = (int64_t)t * topk * hidden + h;
  float acc = 0.0f;
  for (int s = 0; s < topk; s++) {
    const float ws = w[(int64_t)t * topk + s];
    // a zero-weight route may be one the grouped kernels parked and never wrote: it is not read
    if (ws != 0.0f) acc = __builtin_fmaf(In::load(in, base + (int64_t)s * hidden), ws, acc);
  }
  Out::store(out, (int64_t)t * hidden + h, acc);
}

template <class In, class Out>
int reduce(const void *inputs, const float *w, void *outputs, int tokens, int hidden, int topk, void *stream) {
  if (tokens < 0 || hidden < 0 || topk <= 0) {
    qmm_set_error("moe_weighted_reduce: tokens=%d hidden=%d topk=%d", tokens, hidden, topk);
    return (int)hipErrorInvalidValue;
  }
  if (tokens == 0 || hidden == 0) return 0;
  const dim3 grid((unsigned)tokens, (unsigned)qmm_ceil_div(hidden, 256));
  k_weighted_reduce<In, Out><<<grid, 256, 0, (hipStream_t)stream>>>((const typename In::T *)inputs, w,
                                                                     (typename Out::T *)outputs, tokens, hidden, topk);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

void launch_moe_dispatch(const int32_t *topk_ids, int32_t *expert_bounds, int32_t *sorted_token_ids,
                         int32_t *sorted_source_ids, int total_assignments, int num_experts, int topk,
                         int32_t *expert_counts, int32_t *expert_cursors, void *stream) {
  if (total_assignments < 0 || num_experts <= 0 || num_experts > kMaxExperts || topk <= 0) {
    qmm_set_error("moe_dispatch: total=%d num_experts=%d (max %d) topk=%d", total_assignments, num_experts,
                  kMaxExperts, topk);
    return;
  }
  k_moe_dispatch<<<1, 1024, 0, (hipStream_t)stream>>>(topk_ids, expert_bounds, sorted_token_ids, sorted_source_ids,
                                                      total_assignments, num_experts, topk, expert_counts,
                                                      expert_cursors);
}

int launch_moe_weighted_reduce_flat(const void *inputs, const float *topk_weights, void *outputs, int num_tokens,
                                    int hidden, int topk, void *stream) {
  return reduce<in_f32, out_f32>(inputs, topk_weights, outputs, num_tokens, hidden, topk, stream);
}
int launch_moe_weighted_reduce_flat_bf16(const void *inputs, const float *topk_weights, void *outputs,
                                         int num_tokens, int hidden, int topk, void *stream) {
  return reduce<in_f32, out_bf16>(inputs, topk_weights, outputs, num_tokens, hidden, topk, stream);
}
int launch_moe_weighted_reduce_flat_f16_input(const void *inputs, const float *topk_weights, void *outputs,
                                              int num_tokens, int hidden, int topk, void *stream) {
  return reduce<in_f16, out_f16>(inputs, topk_weights, outputs, num_tokens, hidden, topk, stream);
}
int launch_moe_weighted_reduce_flat_bf16_input(const void *inputs, const float *topk_weights, void *outputs,
                                               int num_tokens, int hidden, int topk, void *stream) {
  return reduce<in_bf16, out_bf16>(inputs, topk_weights, outputs, num_tokens, hidden, topk, stream);
}

}  // extern "C"
