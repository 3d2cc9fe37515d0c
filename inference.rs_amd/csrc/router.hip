// MoE router: per token, score the expert logits, pick the top k and produce the routing weights.
//
// Replaces moe_router_topk_{f32,bf16,f16} (crates/inference-nn/kernels/cuda/sort.cu:1374-1725; FFI
// crates/inference-nn/src/cuda/ffi.rs:1137-1190; op crates/inference-nn/src/ops/moe_router.rs:50-79) with the same
// arguments and results:
//   raw       = logit (clamped to [clamp_min, clamp_max] when clamp_logits; NaN -> -inf)
//   score     = raw, softmax(raw) over the experts, or sigmoid(raw)            (score_mode 0 / 1 / 2)
//   selection = score + selection_bias[e] (NaN -> -inf); the top_k largest, ties to the lower expert index
//   weight    = score, raw then a softmax over the k picks, or sigmoid(raw)      (weight_mode 0 / 1 / 2)
//   renormalize: weight /= max(sum of the k weights, norm_min); then weight *= output_scale * expert_scale[id]
// One wave per token; lane l holds experts l, l + 64, ...  Any expert count up to 1024 (the reference instantiates
// 1, 2, 4, ..., 512 and 576).
#include "common.h"
#include "inferencequant.h"

namespace {

constexpr int kMaxExperts = 1024;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

template <class In, int V>
__global__ __launch_bounds__(256) void k_router_topk(const typename In::T *__restrict__ logits,
                                                     float *__restrict__ weights, uint32_t *__restrict__ ids,
                                                     const float *__restrict__ bias, const float *__restrict__ escale,
                                                     int n_rows, int n_experts, int top_k, int score_mode,
                                                     int weight_mode, bool renormalize, bool clamp_logits,
                                                     float clamp_min, float clamp_max, float norm_min,
                                                     float output_scale) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // whole wave
  const typename In::T *lg = logits + (int64_t)row * n_experts;
  float raw[V], score[V], sel[V];
#pragma unroll
  for (int i = 0; i < V; i++) {
    const int e = lane + 64 * i;
    float v = -INFINITY;
    if (e < n_experts) {
      v = In::load(lg, e);
      if (clamp_logits) v = fminf(fmaxf(v, clamp_min), clamp_max);
      if (v != v) v = -INFINITY;
    }
    raw[i] = score[i] = v;
  }
  if (score_mode == 1) {  // softmax over the experts
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; i++) mx = fmaxf(mx, score[i]);
    mx = wave_max(mx);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++) {
      score[i] = lane + 64 * i < n_experts ? expf(score[i] - mx) : 0.0f;
      s += score[i];
    }
    const float inv = 1.0f / wave_sum(s);
#pragma unroll
    for (int i = 0; i < V; i++) score[i] *= inv;
  } else if (score_mode == 2) {
#pragma unroll
    for (int i = 0; i < V; i++) score[i] = lane + 64 * i < n_experts ? 1.0f / (1.0f + expf(-raw[i])) : -INFINITY;
  }
#pragma unroll
  for (int i = 0; i < V; i++) {
    const int e = lane + 64 * i;
    float s = score[i];
    if (bias && e < n_experts) s += bias[e];
    sel[i] = (s != s || e >= n_experts) ? -INFINITY : s;
  }

  // k rounds of a wave argmax over (selection desc, expert asc); pick k lands in lane k % 64, slot k / 64
  float outw[V];
  uint32_t outid[V];
#pragma unroll
  for (int i = 0; i < V; i++) outw[i] = 0.0f, outid[i] = 0;
  for (int k = 0; k < top_k; k++) {
    float bs = sel[0], bsc = score[0], br = raw[0];
    int be = lane;
#pragma unroll
    for (int i = 1; i < V; i++)
      if (lane + 64 * i < n_experts && sel[i] > bs) bs = sel[i], bsc = score[i], br = raw[i], be = lane + 64 * i;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
      const float os = __shfl_xor(bs, m), osc = __shfl_xor(bsc, m), orw = __shfl_xor(br, m);
      const int oe = __shfl_xor(be, m);
      if (os > bs || (os == bs && oe < be)) bs = os, bsc = osc, br = orw, be = oe;
    }
    const float w = weight_mode == 1 ? br : weight_mode == 2 ? 1.0f / (1.0f + expf(-br)) : bsc;
#pragma unroll
    for (int i = 0; i < V; i++) {
      if (k == lane + 64 * i) outw[i] = w, outid[i] = (uint32_t)be;
      if (be == lane + 64 * i) sel[i] = -INFINITY;
    }
  }
  if (weight_mode == 1) {  // softmax over the k picks
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; i++)
      if (lane + 64 * i < top_k) mx = fmaxf(mx, outw[i]);
    mx = wave_max(mx);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++) {
      outw[i] = lane + 64 * i < top_k ? expf(outw[i] - mx) : 0.0f;
      s += outw[i];
    }
    const float inv = 1.0f / wave_sum(s);
#pragma unroll
    for (int i = 0; i < V; i++) outw[i] *= inv;
  }
  if (renormalize) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++)
      if (lane + 64 * i < top_k) s += outw[i];
    const float inv = 1.0f / fmaxf(wave_sum(s), norm_min);
#pragma unroll
    for (int i = 0; i < V; i++) outw[i] *= inv;
  }
#pragma unroll
  for (int i = 0; i < V; i++) {
    const int k = lane + 64 * i;
    if (k < top_k) {
      float sc = output_scale;
      if (escale) sc *= escale[outid[i]];
      weights[(int64_t)row * top_k + k] = outw[i] * sc;
      ids[(int64_t)row * top_k + k] = outid[i];
    }
  }
}

struct ld_f32 {
  typedef float T;
  static __device__ __forceinline__ float load(const float *p, int i) { return p[i]; }
};
struct ld_bf16 {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const uint16_t *p, int i) { return bf16_bits_to_f32(p[i]); }
};
struct ld_f16 {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const uint16_t *p, int i) { return f16_bits_to_f32(p[i]); }
};

template <class In>
void router(const void *logits, float *weights, uint32_t *ids, const float *bias, const float *escale, int n_rows,
            int n_experts, int top_k, int score_mode, int weight_mode, bool renormalize, bool clamp_logits,
            float clamp_min, float clamp_max, float norm_min, float output_scale, int64_t stream, const char *who) {
  if (n_rows < 0 || n_experts < 1 || n_experts > kMaxExperts || top_k < 1 || top_k > n_experts || score_mode < 0 ||
      score_mode > 2 || weight_mode < 0 || weight_mode > 2) {
    qmm_set_error("%s: n_rows=%d n_experts=%d (1..%d) top_k=%d (1..n_experts) score_mode=%d weight_mode=%d (0..2)",
                  who, n_rows, n_experts, kMaxExperts, top_k, score_mode, weight_mode);
    return;
  }
  if (n_rows == 0) return;
  const dim3 grid((unsigned)qmm_ceil_div(n_rows, 4));
  hipStream_t s = (hipStream_t)stream;
  const typename In::T *lg = (const typename In::T *)logits;
#define QMM_ROUTER(V)                                                                                          \
  k_router_topk<In, V><<<grid, 256, 0, s>>>(lg, weights, ids, bias, escale, n_rows, n_experts, top_k,          \
                                            score_mode, weight_mode, renormalize, clamp_logits, clamp_min,     \
                                            clamp_max, norm_min, output_scale)
  const int v = (n_experts + 63) / 64;
  if (v <= 1) QMM_ROUTER(1);
  else if (v <= 2) QMM_ROUTER(2);
  else if (v <= 4) QMM_ROUTER(4);
  else if (v <= 8) QMM_ROUTER(8);
  else QMM_ROUTER(16);
#undef QMM_ROUTER
}

}  // namespace

extern "C" {

void moe_router_topk_f32(const float *logits, float *weights, uint32_t *ids, const float *selection_bias,
                         const float *expert_scale, int n_rows, int n_experts, int top_k, int score_mode,
                         int weight_mode, bool renormalize, bool clamp_logits, float clamp_min, float clamp_max,
                         float norm_min, float output_scale, int64_t stream) {
  router<ld_f32>(logits, weights, ids, selection_bias, expert_scale, n_rows, n_experts, top_k, score_mode,
                 weight_mode, renormalize, clamp_logits, clamp_min, clamp_max, norm_min, output_scale, stream,
                 "moe_router_topk_f32");
}
void moe_router_topk_bf16(const void *logits, float *weights, uint32_t *ids, const float *selection_bias,
                          const float *expert_scale, int n_rows, int n_experts, int top_k, int score_mode,
                          int weight_mode, bool renormalize, bool clamp_logits, float clamp_min, float clamp_max,
                          float norm_min, float output_scale, int64_t stream) {
  router<ld_bf16>(logits, weights, ids, selection_bias, expert_scale, n_rows, n_experts, top_k, score_mode,
                  weight_mode, renormalize, clamp_logits, clamp_min, clamp_max, norm_min, output_scale, stream,
                  "moe_router_topk_bf16");
}
void moe_router_topk_f16(const void *logits, float *weights, uint32_t *ids, const float *selection_bias,
                         const float *expert_scale, int n_rows, int n_experts, int top_k, int score_mode,
                         int weight_mode, bool renormalize, bool clamp_logits, float clamp_min, float clamp_max,
                         float norm_min, float output_scale, int64_t stream) {
  router<ld_f16>(logits, weights, ids, selection_bias, expert_scale, n_rows, n_experts, top_k, score_mode,
                 weight_mode, renormalize, clamp_logits, clamp_min, clamp_max, norm_min, output_scale, stream,
                 "moe_router_topk_f16");
}

}  // extern "C"
