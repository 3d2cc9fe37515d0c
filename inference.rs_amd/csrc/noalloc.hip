// QMatMul::forward for callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc): the same routes and kernels as the host layer's QMatMul::forward, with the
// quantized activations and the split-K planes in one file-scope device array instead of a per-thread workspace.
// Nothing here calls hipMalloc, hipFree or an allocating library routine.
//
// The array is `scratch`, kScratchBytes per device: kActBytes for the quantized activations, then kFixupBytes for
// the split-K planes (the reference's tmp_fixup size for 256 compute units, fast_mmq.rs:442-444).  Each device holds
// its own copy until the process ends; its device address is looked up once per device, on the first call made
// with that device current, and only that address is handed to kernels.  Every call on a device shares that
// device's array, so calls that overlap on one device (two host threads, two streams) race; every byte a call reads
// from the array it has written first, so nothing needs clearing between calls.
#include <mutex>

#include "common.h"
#include "inferencequant.h"

namespace {
constexpr size_t kActBytes = (size_t)16 << 20;
constexpr size_t kFixupBytes = (size_t)16 << 20;
constexpr size_t kScratchBytes = kActBytes + kFixupBytes;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::mutex g_mutex;
uint8_t *g_scratch[kMaxDevices];

// the current device's copy of `scratch`, looked up once per device with that device current; nullptr (error set)
// if the lookup fails
uint8_t *scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    qmm_set_error("qmatmul_forward_noalloc: no current HIP device (or ordinal >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      qmm_set_error("qmatmul_forward_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = (uint8_t *)p;
  }
  return g_scratch[dev];
}

typedef void (*quant_fn)(const void *, void *, int, int, int, void *);
typedef void (*mmvq_fn)(const void *, const void *, void *, int, int, int, int, int, void *);
typedef void (*mmvq_q_fn)(const void *, const float *, void *, int, int, int, int, int, void *);
typedef void (*mmq_fn)(void *, const void *, const void *, void *, int64_t, int64_t, int64_t, int64_t, int64_t, int,
                       int, int64_t, int, int, void *);

// activation geometry as the host layer's: Q8_0 blocks (34 bytes per 32 values) for the 32-value types, Q8_1 slots
// (288 bytes per 256) for the rest; stride_col_y in 32-value blocks either way; prefill tiles: Q8_0 (272 bytes per 256)
// for the 32-value types, `_q8k` (292) for Q4_K and Q5_K, Q8_K (276) for Q6_K
bool act_q8_0(int w) { return qmm_vec_dot_type(w) == QMM_TYPE_Q8_0; }
bool prefill_q8k(int w) { return w == QMM_TYPE_Q4K || w == QMM_TYPE_Q5K; }
int64_t act_block(int w) { return act_q8_0(w) ? 32 : 256; }
int64_t act_row_bytes(int w, int64_t kp) { return act_q8_0(w) ? kp / 32 * 34 : kp / 256 * 288; }
int64_t tile_bytes_per_256(int w) { return act_q8_0(w) ? 272 : prefill_q8k(w) ? 292 : 276; }
int64_t pad_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
bool has_all_routes(int t) { return t == QMM_TYPE_Q8_0 || t == QMM_TYPE_Q4K || t == QMM_TYPE_Q6K; }

quant_fn decode_quantizer(int w, int in) {
  const bool k = !act_q8_0(w);
  switch (in) {
    case QMM_TYPE_F32: return k ? launch_mmvq_gguf_quantize_q8_1_f32 : launch_mmvq_gguf_quantize_q8_0_f32;
    case QMM_TYPE_F16: return k ? launch_mmvq_gguf_quantize_q8_1_f16 : launch_mmvq_gguf_quantize_q8_0_f16;
    default: return k ? launch_mmvq_gguf_quantize_q8_1_bf16 : launch_mmvq_gguf_quantize_q8_0_bf16;
  }
}

mmvq_fn decode_matvec(int w, int out) {
#define QMM_PICK(t, sfx)                                                \
  return out == QMM_TYPE_F32   ? launch_mmvq_gguf_##t##_f32_plain##sfx \
         : out == QMM_TYPE_F16 ? launch_mmvq_gguf_##t##_f16_plain##sfx \
                               : launch_mmvq_gguf_##t##_bf16_plain##sfx;
  switch (w) {
    case QMM_TYPE_Q8_0: QMM_PICK(q8_0, _q8_0)
    case QMM_TYPE_Q4K: QMM_PICK(q4_k, )
    case QMM_TYPE_Q6K: QMM_PICK(q6_k, )
    case QMM_TYPE_Q4_0: QMM_PICK(q4_0, _q8_0)
    case QMM_TYPE_Q5_0: QMM_PICK(q5_0, _q8_0)
    default: QMM_PICK(q5_k, )
  }
#undef QMM_PICK
}

mmvq_q_fn decode_matvec_quantize(int w) {
  switch (w) {
    case QMM_TYPE_Q8_0: return launch_mmvq_gguf_q8_0_f32_quantize_plain;
    case QMM_TYPE_Q4K: return launch_mmvq_gguf_q4_k_f32_quantize_plain;
    default: return launch_mmvq_gguf_q6_k_f32_quantize_plain;
  }
}

mmq_fn prefill_matmul(int w) {
  switch (w) {
    case QMM_TYPE_Q8_0: return launch_mmq_gguf_q8_0_q8_0;
    case QMM_TYPE_Q4K: return launch_mmq_gguf_q4_k_q8k;
    case QMM_TYPE_Q6K: return launch_mmq_gguf_q6_k;
    case QMM_TYPE_Q4_0: return launch_mmq_gguf_q4_0_q8_0;
    case QMM_TYPE_Q5_0: return launch_mmq_gguf_q5_0_q8_0;
    default: return launch_mmq_gguf_q5_k_q8k;
  }
}

// the weight types the host QMatMul serves (IQ4_XS, which the reference's QTensor does not hold, is refused there
// and here)
bool supported(int t) {
  return has_all_routes(t) || t == QMM_TYPE_Q4_0 || t == QMM_TYPE_Q5_0 || t == QMM_TYPE_Q5K;
}

// returns 0, or -1 with the error recorded
int forward(const void *w, int wtype, int64_t n, int64_t k, const void *xs, int in_dtype, int64_t rows, void *ys,
            void *stream) {
  if (!supported(wtype)) {
    qmm_set_error("qmatmul_forward_noalloc: weight type %d has no kernels", wtype);
    return -1;
  }
  if (in_dtype != QMM_TYPE_F32 && in_dtype != QMM_TYPE_F16 && in_dtype != QMM_TYPE_BF16) {
    qmm_set_error("qmatmul_forward_noalloc: in_dtype %d (0 f32, 1 f16, 30 bf16)", in_dtype);
    return -1;
  }
  if (!w || !xs || !ys || n <= 0 || k <= 0 || rows < 0 || k % (int64_t)qmm_block_size(wtype) != 0 || n > INT32_MAX ||
      k > INT32_MAX) {
    qmm_set_error("qmatmul_forward_noalloc: n=%lld k=%lld rows=%lld (k a multiple of %d)", (long long)n, (long long)k,
                  (long long)rows, (int)qmm_block_size(wtype));
    return -1;
  }
  if (rows == 0) return 0;
  const mmq_fn mm = prefill_matmul(wtype);
  if (has_all_routes(wtype) && rows <= 2 && in_dtype == QMM_TYPE_F32 && k <= 4096 &&
      (wtype != QMM_TYPE_Q8_0 || k % 64 == 0) && (uintptr_t)xs % 4 == 0) {
    // the matvec quantizes its own activations: no scratch
    decode_matvec_quantize(wtype)(w, (const float *)xs, ys, (int)k, (int)n, (int)k, (int)n, (int)rows, stream);
    return 0;
  }
  uint8_t *ptr = scratch_ptr();
  if (!ptr) return -1;
  const int64_t per = qmm_max_decode_rows(wtype, k);
  if (rows <= per) {
    const int64_t kp = pad_to(k, act_block(wtype));
    const int64_t row_bytes = act_row_bytes(wtype, kp);
    if (rows * row_bytes > (int64_t)kActBytes) {
      qmm_set_error("qmatmul_forward_noalloc: %lld x %lld activations need %lld bytes of scratch, above the %zu held",
                    (long long)rows, (long long)k, (long long)(rows * row_bytes), kActBytes);
      return -1;
    }
    decode_quantizer(wtype, in_dtype)(xs, ptr, (int)k, (int)kp, (int)rows, stream);
    const int64_t out_elem = in_dtype == QMM_TYPE_F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < rows; r0 += per) {
      const int64_t b = rows - r0 < per ? rows - r0 : per;
      decode_matvec(wtype, in_dtype)(w, ptr + r0 * row_bytes, (uint8_t *)ys + r0 * n * out_elem, (int)k, (int)n,
                                     (int)(kp / 32), (int)n, (int)b, stream);
    }
    return 0;
  }
  const int64_t kp = pad_to(k, 256);
  const int64_t act = rows * (kp / 256) * tile_bytes_per_256(wtype);
  if (act > (int64_t)kActBytes) {
    qmm_set_error("qmatmul_forward_noalloc: %lld x %lld activations need %lld bytes of scratch, above the %zu held",
                  (long long)rows, (long long)k, (long long)act, kActBytes);
    return -1;
  }
  (act_q8_0(wtype)      ? launch_mmq_quantize_q8_0
   : prefill_q8k(wtype) ? launch_mmq_quantize_q8k
                        : launch_mmq_quantize_q8_1_DS4)(xs, nullptr, ptr, in_dtype, k, k, k * rows, k * rows, kp, rows, 1,
                                                        1, stream);
  // the fixup region holds nsm * 128 * 128 f32 for nsm up to 256 (MI355X has 256 compute units); a device with more
  // would split K less than the host layer does, and its output would then differ from QMatMul::forward's in the f32
  // summation order
  const int nsm = qmm_device_cus() < (int)(kFixupBytes / 65536) ? qmm_device_cus() : (int)(kFixupBytes / 65536);
  mm(ptr + kActBytes, w, ptr, ys, k, n, rows, k / (int64_t)qmm_block_size(wtype), n, 0, nsm, 160 * 1024, 64, in_dtype,
     stream);
  return 0;
}

}  // namespace

extern "C" int qmm_qmatmul_forward_noalloc(const void *w, uint32_t wtype, int64_t n, int64_t k, const void *xs,
                                           uint32_t in_dtype, int64_t rows, void *ys, void *stream) {
  const char *prev = qmm_last_error();
  if (prev && prev[0]) qmm_clear_error();
  if (forward(w, (int)wtype, n, k, xs, (int)in_dtype, rows, ys, stream) != 0) return -1;
  const char *msg = qmm_last_error();  // a launcher's own argument check
  if (msg && msg[0]) return -1;
  const hipError_t e = hipGetLastError();  // a launch the runtime refused
  if (e != hipSuccess) {
    qmm_set_error("qmatmul_forward_noalloc: launch failed: %s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}
