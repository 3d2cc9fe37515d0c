// QTensor / QMatMul / MoeExperts over the kernel C ABI.  Route choices follow
// crates/inference-quant/src/gguf/mod.rs:434-452 (decode vs prefill) and
// crates/inference-nn/src/moe/experts/backends.rs:1442-1454 (indexed decode vs grouped prefill); scratch for
// quantized activations is a per-(thread, device) growing workspace as in gguf/thread_workspace.rs.
#include "qtensor.h"

#include <cstring>
#include <map>
#include <string>

#include "inferencequant.h"

namespace inference_rs_amd {
namespace {

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

// A launcher's argument error (qmm_last_error), then a launch the runtime refused (hipGetLastError: an invalid
// configuration or a missing code object), which would otherwise leave the output unwritten without a word.
void abi_check(const char *what) {
  const char *msg = qmm_last_error();
  if (msg && msg[0]) {
    std::string m = std::string(what) + ": " + msg;
    qmm_clear_error();
    throw Error(m);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw Error(std::string(what) + ": launch failed: " + hipGetErrorString(e));
}

// Compute units of a device: the reference's `nsm` device hint (fast_mmq.rs:397-440)
int device_cus(int ordinal) {
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, ordinal) != hipSuccess || v <= 0) v = 256;
  return v;
}
// The split-K fixup workspace of one MMQ launch, nsm * 128 * 128 f32 (fast_mmq.rs:442-444)
size_t fixup_bytes(int nsm) { return (size_t)nsm * 128 * 128 * 4; }

int64_t pad_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Per-(thread, device) scratch: grows, never shrinks.  Growing waits for the stream, since earlier launches
// may still read the old buffer.
class Workspace {
 public:
  void *get(int ordinal, size_t bytes, hipStream_t stream) {
    Slot &s = slots_[ordinal];
    if (!s.buf || s.buf->size() < bytes) {
      if (s.buf) hip_check(hipStreamSynchronize(stream), "workspace: hipStreamSynchronize");
      s.buf.reset();
      s.buf = std::make_unique<DeviceBuffer>(ordinal, bytes + bytes / 4 + 4096);
    }
    return s.buf->ptr();
  }

 private:
  struct Slot {
    std::unique_ptr<DeviceBuffer> buf;
  };
  std::map<int, Slot> slots_;
};

Workspace &workspace() {
  thread_local Workspace ws;
  return ws;
}
// fused_ffn's intermediates (the gate and up outputs), kept apart from the scratch of the QMatMul calls it makes
Workspace &ffn_workspace() {
  thread_local Workspace ws;
  return ws;
}

// Carves consecutive 256-byte aligned slices out of one workspace allocation.
struct Carver {
  size_t total = 0;
  size_t add(size_t bytes) {
    const size_t off = total;
    total += (bytes + 255) / 256 * 256;
    return off;
  }
};

typedef void (*quant_fn)(const void *, void *, int, int, int, void *);
typedef void (*mmvq_fn)(const void *, const void *, void *, int, int, int, int, int, void *);
typedef void (*mmq_fn)(void *, const void *, const void *, void *, int64_t, int64_t, int64_t, int64_t, int64_t, int,
                       int, int64_t, int, int, void *);
typedef void (*mmq_moe_fn)(void *, const void *, const void *, const int32_t *, const int32_t *, void *, int64_t,
                           int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, int64_t, int, void *);
typedef void (*mmvq_moe_fn)(const void *, const void *, int64_t, const void *, const void *, float *, int, int, int,
                            int, int, int, int, void *);
typedef void (*indexed_fn)(const void *, const void *, const uint32_t *, float *, int, int, int, int, int, int,
                           void *);

quant_fn decode_quantizer(GgmlDType w, GgmlDType in) {
  const bool k = qmm_vec_dot_type((int)w) == QMM_TYPE_Q8K;
  switch (in) {
    case GgmlDType::F32: return k ? launch_mmvq_gguf_quantize_q8_1_f32 : launch_mmvq_gguf_quantize_q8_0_f32;
    case GgmlDType::F16: return k ? launch_mmvq_gguf_quantize_q8_1_f16 : launch_mmvq_gguf_quantize_q8_0_f16;
    case GgmlDType::BF16: return k ? launch_mmvq_gguf_quantize_q8_1_bf16 : launch_mmvq_gguf_quantize_q8_0_bf16;
    default: throw Error("QMatMul: activations must be F32, F16 or BF16");
  }
}

// The decode matvec that quantizes its own f32 activations (one launch; output f32).
using mmvq_q_fn = void (*)(const void *, const float *, void *, int, int, int, int, int, void *);
mmvq_q_fn decode_matvec_quantize(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_mmvq_gguf_q8_0_f32_quantize_plain;
    case GgmlDType::Q4K: return launch_mmvq_gguf_q4_k_f32_quantize_plain;
    case GgmlDType::Q6K: return launch_mmvq_gguf_q6_k_f32_quantize_plain;
    default: throw Error("QMatMul: unsupported weight type");
  }
}

// the weight types with kernels: every route (full), the prefill matmul besides the matvec, or the matvec route and
// dequantization only
bool has_all_routes(GgmlDType t) { return t == GgmlDType::Q8_0 || t == GgmlDType::Q4K || t == GgmlDType::Q6K; }
bool has_prefill(GgmlDType t) {
  return has_all_routes(t) || t == GgmlDType::Q4_0 || t == GgmlDType::Q5_0 || t == GgmlDType::Q5K;
}
bool has_matvec(GgmlDType t) {
  return has_all_routes(t) || t == GgmlDType::Q4_0 || t == GgmlDType::Q5_0 || t == GgmlDType::Q5K;
}

// The matvec over the quantizer's layout: Q8_1 slots for the super-block types (the reference-named entries), Q8_0
// blocks for the 32-value types (their _q8_0 entries), as each type's CPU dot product quantizes
mmvq_fn decode_matvec(GgmlDType w, GgmlDType out) {
#define QMM_PICK(t, sfx)                                                         \
  switch (out) {                                                                 \
    case GgmlDType::F32: return launch_mmvq_gguf_##t##_f32_plain##sfx;           \
    case GgmlDType::F16: return launch_mmvq_gguf_##t##_f16_plain##sfx;           \
    case GgmlDType::BF16: return launch_mmvq_gguf_##t##_bf16_plain##sfx;         \
    default: throw Error("QMatMul: output must be F32, F16 or BF16");            \
  }
  switch (w) {
    case GgmlDType::Q8_0: QMM_PICK(q8_0, _q8_0)
    case GgmlDType::Q4K: QMM_PICK(q4_k, )
    case GgmlDType::Q6K: QMM_PICK(q6_k, )
    case GgmlDType::Q4_0: QMM_PICK(q4_0, _q8_0)
    case GgmlDType::Q5_0: QMM_PICK(q5_0, _q8_0)
    case GgmlDType::Q5K: QMM_PICK(q5_k, )
    default: throw Error("QMatMul: unsupported weight type");
  }
#undef QMM_PICK
}

typedef void (*mmvq_glu_fn)(const void *, const void *, const void *, void *, int, int, int, int, int, int, void *);
mmvq_glu_fn decode_fused_glu(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_mmvq_gguf_q8_0_f32_fused_glu_q8_0;
    case GgmlDType::Q4K: return launch_mmvq_gguf_q4_k_f32_fused_glu;
    case GgmlDType::Q6K: return launch_mmvq_gguf_q6_k_f32_fused_glu;
    default: throw Error("fused_ffn: unsupported weight type");
  }
}

mmq_fn prefill_matmul(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_mmq_gguf_q8_0_q8_0;
    case GgmlDType::Q4_0: return launch_mmq_gguf_q4_0_q8_0;
    case GgmlDType::Q5_0: return launch_mmq_gguf_q5_0_q8_0;
    case GgmlDType::Q4K: return launch_mmq_gguf_q4_k_q8k;
    case GgmlDType::Q6K: return launch_mmq_gguf_q6_k;
    case GgmlDType::Q5K: return launch_mmq_gguf_q5_k_q8k;
    default: throw Error("QMatMul: unsupported weight type");
  }
}

mmq_moe_fn prefill_matmul_moe(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_mmq_gguf_q8_0_moe_q8_0;
    case GgmlDType::Q4_0: return launch_mmq_gguf_q4_0_moe_q8_0;
    case GgmlDType::Q5_0: return launch_mmq_gguf_q5_0_moe_q8_0;
    case GgmlDType::Q4K: return launch_mmq_gguf_q4_k_moe_q8k;
    case GgmlDType::Q6K: return launch_mmq_gguf_q6_k_moe;
    case GgmlDType::Q5K: return launch_mmq_gguf_q5_k_moe_q8k;
    default: throw Error("MoE: unsupported weight type");
  }
}

mmvq_moe_fn decode_matvec_moe(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_mmvq_gguf_q8_0_moe_q8_0;
    case GgmlDType::Q4K: return launch_mmvq_gguf_q4_k_moe;
    case GgmlDType::Q6K: return launch_mmvq_gguf_q6_k_moe;
    default: throw Error("MoE: unsupported weight type");
  }
}

typedef void (*mmvq_moe_wsum_fn)(const void *, int64_t, const void *, const void *, const float *, float *, int, int,
                                 int, int, int, void *);
mmvq_moe_wsum_fn decode_matvec_moe_wsum(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_mmvq_gguf_q8_0_moe_wsum_q8_0;
    case GgmlDType::Q4K: return launch_mmvq_gguf_q4_k_moe_wsum;
    case GgmlDType::Q6K: return launch_mmvq_gguf_q6_k_moe_wsum;
    default: throw Error("MoE: unsupported weight type");
  }
}

indexed_fn indexed_moe(GgmlDType w) {
  switch (w) {
    case GgmlDType::Q8_0: return launch_indexed_moe_forward_q8_0_q8_0;
    case GgmlDType::Q4K: return launch_indexed_moe_forward_q4k_q8_1;
    case GgmlDType::Q6K: return launch_indexed_moe_forward_q6k_q8_1;
    case GgmlDType::Q4_0: return launch_indexed_moe_forward_q4_0_q8_0;
    case GgmlDType::Q5_0: return launch_indexed_moe_forward_q5_0_q8_0;
    case GgmlDType::Q5K: return launch_indexed_moe_forward_q5k_q8_1;
    default: throw Error("gather_forward: unsupported weight type");
  }
}

// decode activation geometry of a weight type (GgmlType::VecDotType): Q8_0 blocks of 34 bytes per 32 values, or Q8_1
// slots of 288 bytes per 256 (qmm_block_q8ks); stride_col_y counts 32-value blocks either way
bool act_q8_0(GgmlDType w) { return qmm_vec_dot_type((int)w) == QMM_TYPE_Q8_0; }
int64_t act_block(GgmlDType w) { return act_q8_0(w) ? 32 : 256; }
int64_t act_row_bytes(GgmlDType w, int64_t kp) { return act_q8_0(w) ? kp / 32 * 34 : kp / 256 * 288; }

// prefill activations (prefill_matmul, prefill_matmul_moe and their quantizers): Q8_0 tiles for the 32-value types (272
// bytes per 256 values), the `_q8k` tiles (f16 sums of 16, which the min term reads as they are; 292) for Q4_K and
// Q5_K, the reference-named Q8_K tiles (276) for Q6_K
bool prefill_q8k(GgmlDType w) { return w == GgmlDType::Q4K || w == GgmlDType::Q5K; }
int64_t prefill_tile_bytes_per_256(GgmlDType w) { return act_q8_0(w) ? 272 : prefill_q8k(w) ? 292 : 276; }
typedef void (*tile_quant_fn)(const void *, const int32_t *, void *, int, int64_t, int64_t, int64_t, int64_t, int64_t,
                              int64_t, int64_t, int64_t, void *);
tile_quant_fn prefill_quantizer(GgmlDType w) {
  return act_q8_0(w) ? launch_mmq_quantize_q8_0 : prefill_q8k(w) ? launch_mmq_quantize_q8k : launch_mmq_quantize_q8_1_DS4;
}

// matvec_only: the route needs the decode matvec kernels alone (QMatMul::forward, gather_forward); else every route
void check_weight(const QTensor &w, const char *who, bool matvec_only = false) {
  if (!w.device().is_hip()) throw Error(std::string(who) + ": the weight is not on a HIP device");
  const GgmlDType t = w.dtype();
  if (!(matvec_only ? has_matvec(t) : has_all_routes(t)))
    throw Error(std::string(who) + ": weight type " + dtype_name(t) + " has no kernels here");
}

}  // namespace

// ------------------------------------------------------------------------------------------------ dtypes

GgmlDType dtype_from_u32(uint32_t u) {
  switch (u) {
    case 0: return GgmlDType::F32;
    case 1: return GgmlDType::F16;
    case 2: return GgmlDType::Q4_0;
    case 3: return GgmlDType::Q4_1;
    case 6: return GgmlDType::Q5_0;
    case 7: return GgmlDType::Q5_1;
    case 8: return GgmlDType::Q8_0;
    case 9: return GgmlDType::Q8_1;
    case 10: return GgmlDType::Q2K;
    case 11: return GgmlDType::Q3K;
    case 12: return GgmlDType::Q4K;
    case 13: return GgmlDType::Q5K;
    case 14: return GgmlDType::Q6K;
    case 15: return GgmlDType::Q8K;
    case 30: return GgmlDType::BF16;
    default: throw Error("unknown dtype for tensor " + std::to_string(u));
  }
}

size_t type_size(GgmlDType t) { return qmm_type_size((int)t); }
size_t block_size(GgmlDType t) { return qmm_block_size((int)t); }

const char *dtype_name(GgmlDType t) {
  switch (t) {
    case GgmlDType::F32: return "F32";
    case GgmlDType::F16: return "F16";
    case GgmlDType::Q4_0: return "Q4_0";
    case GgmlDType::Q4_1: return "Q4_1";
    case GgmlDType::Q5_0: return "Q5_0";
    case GgmlDType::Q5_1: return "Q5_1";
    case GgmlDType::Q8_0: return "Q8_0";
    case GgmlDType::Q8_1: return "Q8_1";
    case GgmlDType::Q2K: return "Q2K";
    case GgmlDType::Q3K: return "Q3K";
    case GgmlDType::Q4K: return "Q4K";
    case GgmlDType::Q5K: return "Q5K";
    case GgmlDType::Q6K: return "Q6K";
    case GgmlDType::Q8K: return "Q8K";
    case GgmlDType::BF16: return "BF16";
  }
  return "?";
}

// ------------------------------------------------------------------------------------------------ storage

DeviceBuffer::DeviceBuffer(int ordinal, size_t bytes) : size_(bytes), ordinal_(ordinal) {
  hip_check(hipSetDevice(ordinal), "hipSetDevice");
  hip_check(hipMalloc(&ptr_, bytes ? bytes : 1), "hipMalloc");
}

DeviceBuffer::~DeviceBuffer() {
  if (ptr_) (void)hipFree(ptr_);
}

int64_t QTensor::elem_count() const {
  int64_t n = 1;
  for (int64_t d : dims_) n *= d;
  return n;
}

std::shared_ptr<QTensor> QTensor::from_data(const void *bytes, size_t len, const std::vector<int64_t> &dims,
                                            GgmlDType dtype, Device device) {
  if (dims.size() < 2 || dims.size() > 3) throw Error("QTensor: dims must be [rows, cols] or [experts, rows, cols]");
  const size_t bs = block_size(dtype);
  if (bs == 0) throw Error(std::string("QTensor: ") + dtype_name(dtype) + " has no block size");
  for (int64_t d : dims)
    if (d <= 0) throw Error("QTensor: empty dimension");
  if (dims.back() % (int64_t)bs != 0)
    throw Error("QTensor: the last dimension " + std::to_string(dims.back()) + " is not a multiple of " +
                std::to_string(bs));
  std::shared_ptr<QTensor> t(new QTensor(dtype, dims, device));
  const size_t need = t->storage_size_in_bytes();
  if (len != need) throw Error("QTensor: " + std::to_string(len) + " bytes for a tensor of " + std::to_string(need));
  if (device.is_cpu()) {
    t->host_.assign((const uint8_t *)bytes, (const uint8_t *)bytes + len);
  } else {
    // MATRIX_ROW_PADDING (quantized/cuda.rs:25): 512 values of zero blocks past the end
    const size_t pad = 512 / bs * type_size(dtype);
    t->dev_ = std::make_unique<DeviceBuffer>(device.ordinal, len + pad);
    hip_check(hipMemcpy(t->dev_->ptr(), bytes, len, hipMemcpyHostToDevice), "QTensor upload");
    hip_check(hipMemset((uint8_t *)t->dev_->ptr() + len, 0, pad), "QTensor padding");
  }
  return t;
}

std::shared_ptr<QTensor> QTensor::quantize(const float *src, const std::vector<int64_t> &dims, GgmlDType dtype,
                                           Device device) {
  int64_t n = 1;
  for (int64_t d : dims) n *= d;
  const size_t bs = block_size(dtype);
  if (bs == 0 || dims.empty() || dims.back() % (int64_t)bs != 0)
    throw Error("QTensor::quantize: the last dimension is not a multiple of the block size");
  std::vector<uint8_t> bytes((size_t)(n / (int64_t)bs) * type_size(dtype));
  if (!cpu::quantize(dtype, src, n, bytes.data()))
    throw Error(std::string("QTensor::quantize: no quantizer for ") + dtype_name(dtype));
  return from_data(bytes.data(), bytes.size(), dims, dtype, device);
}

std::vector<uint8_t> QTensor::data() const {
  if (device_.is_cpu()) return host_;
  std::vector<uint8_t> out(storage_size_in_bytes());
  hip_check(hipMemcpy(out.data(), dev_->ptr(), out.size(), hipMemcpyDeviceToHost), "QTensor download");
  return out;
}

std::vector<float> QTensor::dequantize() const {
  const std::vector<uint8_t> bytes = data();
  std::vector<float> out((size_t)elem_count());
  if (!cpu::dequantize(dtype_, bytes.data(), elem_count(), out.data()))
    throw Error(std::string("QTensor::dequantize: no dequantizer for ") + dtype_name(dtype_));
  return out;
}

void QTensor::dequantize_on_device(void *out, GgmlDType out_dtype, hipStream_t stream) const {
  typedef void (*fn)(const void *, void *, int64_t, void *);
  static const fn table[6][3] = {
      {launch_dequantize_q8_0_f32, launch_dequantize_q8_0_f16, launch_dequantize_q8_0_bf16},
      {launch_dequantize_q4_k_f32, launch_dequantize_q4_k_f16, launch_dequantize_q4_k_bf16},
      {launch_dequantize_q6_k_f32, launch_dequantize_q6_k_f16, launch_dequantize_q6_k_bf16},
      {launch_dequantize_q4_0_f32, launch_dequantize_q4_0_f16, launch_dequantize_q4_0_bf16},
      {launch_dequantize_q5_0_f32, launch_dequantize_q5_0_f16, launch_dequantize_q5_0_bf16},
      {launch_dequantize_q5_k_f32, launch_dequantize_q5_k_f16, launch_dequantize_q5_k_bf16}};
  int ti = -1;
  switch (dtype_) {
    case GgmlDType::Q8_0: ti = 0; break;
    case GgmlDType::Q4K: ti = 1; break;
    case GgmlDType::Q6K: ti = 2; break;
    case GgmlDType::Q4_0: ti = 3; break;
    case GgmlDType::Q5_0: ti = 4; break;
    case GgmlDType::Q5K: ti = 5; break;
    default: break;
  }
  const int oi = out_dtype == GgmlDType::F32 ? 0 : out_dtype == GgmlDType::F16 ? 1 : out_dtype == GgmlDType::BF16 ? 2 : -1;
  if (ti < 0 || oi < 0)
    throw Error(std::string("QTensor::dequantize_on_device: ") + dtype_name(dtype_) + " -> " + dtype_name(out_dtype));
  hip_check(hipSetDevice(device().ordinal), "hipSetDevice");
  table[ti][oi](device_ptr(), out, elem_count(), stream);
  abi_check("QTensor::dequantize_on_device");
}

const void *QTensor::device_ptr() const {
  if (!dev_) throw Error("QTensor: not on a HIP device");
  return dev_->ptr();
}

// ------------------------------------------------------------------------------------------------ QMatMul

QMatMul::QMatMul(std::shared_ptr<QTensor> w) : w_(std::move(w)) {
  if (!w_) throw Error("QMatMul: null weight");
}

int64_t QMatMul::max_decode_rows(GgmlDType dtype, int64_t k) { return qmm_max_decode_rows((int)dtype, k); }

bool QMatMul::prefers_mmvq(GgmlDType dtype, int64_t rows, int64_t k) { return rows <= max_decode_rows(dtype, k); }

void QMatMul::forward(const void *xs, GgmlDType in_dtype, int64_t rows, void *ys, hipStream_t stream) const {
  const QTensor &w = *w_;
  check_weight(w, "QMatMul::forward", true);
  if (w.shape().size() != 2) throw Error("QMatMul::forward: the weight must be 2-D");
  if (in_dtype != GgmlDType::F32 && in_dtype != GgmlDType::F16 && in_dtype != GgmlDType::BF16)
    throw Error("QMatMul::forward: activations must be F32, F16 or BF16");
  if (rows < 0) throw Error("QMatMul::forward: negative row count");
  if (rows == 0) return;
  const int64_t k = w.cols(), n = w.rows();
  const GgmlDType t = w.dtype();
  hip_check(hipSetDevice(w.device().ordinal), "hipSetDevice");
  if (has_all_routes(t) && in_dtype == GgmlDType::F32 && rows <= 2 && k <= 4096 &&
      (t != GgmlDType::Q8_0 || k % 64 == 0) && (uintptr_t)xs % 4 == 0) {
    // one launch: the matvec quantizes its activations itself (the same bits as the two launches below)
    decode_matvec_quantize(t)(w.device_ptr(), (const float *)xs, ys, (int)k, (int)n, (int)k, (int)n, (int)rows, stream);
    abi_check("QMatMul::forward (matvec)");
  } else if (prefers_mmvq(t, rows, k) || !has_prefill(t)) {
    // the decode matvec; a type without a prefill kernel takes every batch this way, max_decode_rows rows a launch
    const int64_t per = max_decode_rows(t, k);
    const int64_t kp = pad_to(k, act_block(t));
    const int64_t row_bytes = act_row_bytes(t, kp);
    void *vy = workspace().get(w.device().ordinal, (size_t)(rows * row_bytes), stream);
    decode_quantizer(t, in_dtype)(xs, vy, (int)k, (int)kp, (int)rows, stream);
    abi_check("QMatMul::forward (quantize)");
    const size_t out_elem = in_dtype == GgmlDType::F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < rows; r0 += per) {
      const int64_t b = rows - r0 < per ? rows - r0 : per;
      decode_matvec(t, in_dtype)(w.device_ptr(), (const uint8_t *)vy + r0 * row_bytes, (uint8_t *)ys + r0 * n * out_elem,
                                 (int)k, (int)n, (int)(kp / 32), (int)n, (int)b, stream);
      abi_check("QMatMul::forward (matvec)");
    }
  } else {
    const int64_t kp = pad_to(k, 256);
    const int nsm = device_cus(w.device().ordinal);
    Carver c;
    const size_t o_y = c.add((size_t)(rows * kp / 256 * prefill_tile_bytes_per_256(t)));
    const size_t o_fix = c.add(fixup_bytes(nsm));
    uint8_t *ws = (uint8_t *)workspace().get(w.device().ordinal, c.total, stream);
    prefill_quantizer(t)(xs, nullptr, ws + o_y, (int)in_dtype, k, k, k * rows, k * rows, kp, rows, 1, 1, stream);
    abi_check("QMatMul::forward (quantize)");
    prefill_matmul(t)(ws + o_fix, w.device_ptr(), ws + o_y, ys, k, n, rows, k / (int64_t)block_size(t), n, 0, nsm,
                      160 * 1024, 64, (int)in_dtype, stream);
    abi_check("QMatMul::forward (matmul)");
  }
}

void QMatMul::down_from_glu(const float *gate, const float *up, int64_t rows, int activation, float *ys,
                            hipStream_t stream) const {
  const QTensor &w = *w_;
  check_weight(w, "QMatMul::down_from_glu", true);
  if (w.shape().size() != 2) throw Error("QMatMul::down_from_glu: the weight must be 2-D");
  if (!has_prefill(w.dtype())) throw Error("QMatMul::down_from_glu: weight type has no prefill matmul");
  if (activation < 0 || activation > 4) throw Error("QMatMul::down_from_glu: activation must be 0..4");
  if (rows < 0) throw Error("QMatMul::down_from_glu: negative row count");
  if (rows == 0) return;
  const int64_t k = w.cols(), n = w.rows();
  const GgmlDType t = w.dtype();
  if (k % (int64_t)block_size(t) != 0) throw Error("QMatMul::down_from_glu: K is not a multiple of the block size");
  hip_check(hipSetDevice(w.device().ordinal), "hipSetDevice");
  const int64_t kp = pad_to(k, 256);
  const int nsm = device_cus(w.device().ordinal);
  Carver c;
  const size_t o_y = c.add((size_t)(rows * kp / 256 * prefill_tile_bytes_per_256(t)));
  const size_t o_fix = c.add(fixup_bytes(nsm));
  uint8_t *ws = (uint8_t *)workspace().get(w.device().ordinal, c.total, stream);
  (act_q8_0(t)      ? launch_mmq_quantize_glu_q8_0_f32
   : prefill_q8k(t) ? launch_mmq_quantize_glu_q8k_f32
                    : launch_mmq_quantize_glu_q8_1_DS4_f32)(gate, up, nullptr, ws + o_y, k, k, kp, rows, activation,
                                                            stream);
  abi_check("QMatMul::down_from_glu (GLU + quantize)");
  prefill_matmul(t)(ws + o_fix, w.device_ptr(), ws + o_y, ys, k, n, rows, k / (int64_t)block_size(t), n, 0, nsm,
                    160 * 1024, 64, 0, stream);
  abi_check("QMatMul::down_from_glu (matmul)");
}

void fused_ffn(const QMatMul &gate, const QMatMul &up, const QMatMul &down, const float *xs, int64_t rows,
               int activation, float *ys, hipStream_t stream) {
  const QTensor &g = gate.weight(), &u = up.weight(), &d = down.weight();
  check_weight(g, "fused_ffn (gate)");
  check_weight(u, "fused_ffn (up)");
  check_weight(d, "fused_ffn (down)", true);
  if (g.shape().size() != 2 || g.shape() != u.shape() || g.dtype() != u.dtype())
    throw Error("fused_ffn: gate and up must be 2-D weights of one type and shape");
  if (d.shape().size() != 2 || d.cols() != g.rows() || d.rows() != g.cols())
    throw Error("fused_ffn: down must be [hidden, inter] for gate / up [inter, hidden]");
  if (g.device().ordinal != d.device().ordinal || u.device().ordinal != d.device().ordinal)
    throw Error("fused_ffn: the weights are on different devices");
  if (activation < 0 || activation > 4) throw Error("fused_ffn: activation must be 0..4");
  if (rows < 0) throw Error("fused_ffn: negative row count");
  if (rows == 0) return;
  const int64_t hidden = g.cols(), inter = g.rows();
  const GgmlDType t = g.dtype();
  const int ordinal = g.device().ordinal;
  hip_check(hipSetDevice(ordinal), "hipSetDevice");
  if (rows <= QMatMul::kMaxDecodeRows) {
    // decode: one activation quantization, the fused-GLU matvec, then down on act(gate) * up
    const int64_t kp = pad_to(hidden, act_block(t));
    Carver c;
    const size_t o_y = c.add((size_t)(rows * act_row_bytes(t, kp)));
    const size_t o_mid = c.add((size_t)(rows * inter * 4));
    uint8_t *ws = (uint8_t *)ffn_workspace().get(ordinal, c.total, stream);
    decode_quantizer(t, GgmlDType::F32)(xs, ws + o_y, (int)hidden, (int)kp, (int)rows, stream);
    abi_check("fused_ffn (quantize)");
    decode_fused_glu(t)(g.device_ptr(), u.device_ptr(), ws + o_y, ws + o_mid, (int)hidden, (int)inter,
                        (int)(kp / 32), (int)inter, (int)rows, activation, stream);
    abi_check("fused_ffn (gate/up)");
    down.forward(ws + o_mid, GgmlDType::F32, rows, ys, stream);
    return;
  }
  // prefill: one tile-layout quantization read by both matmuls, then down_from_glu on their f32 outputs
  const int64_t kp = pad_to(hidden, 256);
  const int nsm = device_cus(ordinal);
  Carver c;
  const size_t o_y = c.add((size_t)(rows * kp / 256 * prefill_tile_bytes_per_256(t)));
  const size_t o_fix = c.add(fixup_bytes(nsm));
  const size_t o_g = c.add((size_t)(rows * inter * 4));
  const size_t o_u = c.add((size_t)(rows * inter * 4));
  uint8_t *ws = (uint8_t *)ffn_workspace().get(ordinal, c.total, stream);
  prefill_quantizer(t)(xs, nullptr, ws + o_y, 0, hidden, hidden, hidden * rows, hidden * rows, kp, rows, 1, 1, stream);
  abi_check("fused_ffn (quantize)");
  for (int which = 0; which < 2; which++) {
    const QTensor &w = which == 0 ? g : u;
    prefill_matmul(t)(ws + o_fix, w.device_ptr(), ws + o_y, ws + (which == 0 ? o_g : o_u), hidden, inter, rows,
                      hidden / (int64_t)block_size(t), inter, 0, nsm, 160 * 1024, 64, 0, stream);
    abi_check("fused_ffn (gate/up)");
  }
  down.down_from_glu((const float *)(ws + o_g), (const float *)(ws + o_u), rows, activation, ys, stream);
}

void QMatMul::gather_forward(const float *xs, int64_t batch, int64_t xdim1, const uint32_t *ids, int64_t topk,
                             float *ys, hipStream_t stream) const {
  const QTensor &w = *w_;
  check_weight(w, "QMatMul::gather_forward", true);
  if (w.shape().size() != 3) throw Error("gather_forward: the weight must be [experts, rows, cols]");
  if (xdim1 != 1 && xdim1 != topk) throw Error("gather_forward: x's second dim must be 1 or topk");
  if (batch <= 0 || topk <= 0) return;
  const int64_t k = w.cols(), n = w.rows();
  const GgmlDType t = w.dtype();
  const int64_t kp = pad_to(k, act_block(t));
  hip_check(hipSetDevice(w.device().ordinal), "hipSetDevice");
  void *vy = workspace().get(w.device().ordinal, (size_t)(batch * xdim1 * act_row_bytes(t, kp)), stream);
  decode_quantizer(t, GgmlDType::F32)(xs, vy, (int)k, (int)kp, (int)(batch * xdim1), stream);
  abi_check("gather_forward (quantize)");
  indexed_moe(t)(w.device_ptr(), vy, ids, ys, (int)n, (int)k, (int)batch, (int)topk, (int)kp, (int)xdim1, stream);
  abi_check("gather_forward (matvec)");
}

// ------------------------------------------------------------------------------------------------ MoE experts

MoeExperts::MoeExperts(std::shared_ptr<QTensor> gate, std::shared_ptr<QTensor> up, std::shared_ptr<QTensor> down,
                       int activation)
    : gate_(std::move(gate)), up_(std::move(up)), down_(std::move(down)), activation_(activation) {
  if (!gate_ || !up_ || !down_) throw Error("MoeExperts: null weight");
  for (const QTensor *t : {gate_.get(), up_.get(), down_.get()}) {
    check_weight(*t, "MoeExperts");
    if (t->shape().size() != 3) throw Error("MoeExperts: weights must be [experts, rows, cols]");
  }
  if (gate_->shape() != up_->shape() || gate_->dtype() != up_->dtype())
    throw Error("MoeExperts: gate and up must match");
  if (down_->experts() != gate_->experts() || down_->cols() != gate_->rows() || down_->rows() != gate_->cols())
    throw Error("MoeExperts: down must be [experts, hidden, intermediate]");
  if (activation < 0 || activation > 4) throw Error("MoeExperts: activation must be 0..4 (SiLU, GELU, ReLU, GELU-erf, sigmoid)");
}

void MoeExperts::forward(const float *xs, int64_t tokens, const int32_t *ids, const float *weights, int64_t topk,
                         float *out, hipStream_t stream, bool force_grouped) const {
  if (tokens <= 0) return;
  if (topk <= 0) throw Error("MoeExperts::forward: topk must be positive");
  const int64_t E = gate_->experts(), hidden = gate_->cols(), inter = gate_->rows();
  const int64_t pairs = tokens * topk;
  const int ordinal = gate_->device().ordinal;
  hip_check(hipSetDevice(ordinal), "hipSetDevice");
  const GgmlDType tg = gate_->dtype(), td = down_->dtype();
  const bool grouped = force_grouped || tokens > kIndexedMaxTokens;
  if (!grouped) {
    // decode: fused gate/up matvec per routed pair, then down with the weighted sum over slots folded in
    const int64_t kp1 = pad_to(hidden, act_block(tg)), kp2 = pad_to(inter, act_block(td));
    Carver c;
    const size_t o_x = c.add((size_t)(tokens * act_row_bytes(tg, kp1)));
    const size_t o_mid = c.add((size_t)(pairs * inter * 4));
    const size_t o_midq = c.add((size_t)(pairs * act_row_bytes(td, kp2)));
    uint8_t *ws = (uint8_t *)workspace().get(ordinal, c.total, stream);
    decode_quantizer(tg, GgmlDType::F32)(xs, ws + o_x, (int)hidden, (int)kp1, (int)tokens, stream);
    abi_check("MoE decode (quantize x)");
    decode_matvec_moe(tg)(gate_->device_ptr(), up_->device_ptr(), (int64_t)(inter * gate_->row_bytes()), ws + o_x,
                          ids, (float *)(ws + o_mid), (int)hidden, (int)inter, (int)(kp1 / 32), (int)topk,
                          (int)pairs, activation_, 1, stream);
    abi_check("MoE decode (gate/up)");
    decode_quantizer(td, GgmlDType::F32)(ws + o_mid, ws + o_midq, (int)inter, (int)kp2, (int)pairs, stream);
    abi_check("MoE decode (quantize mid)");
    // down projection and the weighted sum over each token's routes in one launch
    decode_matvec_moe_wsum(td)(down_->device_ptr(), (int64_t)(hidden * down_->row_bytes()), ws + o_midq, ids, weights,
                               out, (int)inter, (int)hidden, (int)(kp2 / 32), (int)tokens, (int)topk,
                               stream);
    abi_check("MoE decode (down + weighted sum)");
    return;
  }
  // grouped prefill: dispatch tables, gate and up as expert-grouped matmuls over the gathered rows, the GLU
  // fused into the requantization of the intermediate, down, then the weighted sum over slots
  const int64_t kp1 = pad_to(hidden, 256), kp2 = pad_to(inter, 256);
  Carver c;
  const size_t o_bounds = c.add((size_t)(E + 1) * 4);
  const size_t o_tok = c.add((size_t)pairs * 4);
  const size_t o_src = c.add((size_t)pairs * 4);
  const size_t o_cnt = c.add((size_t)E * 4);
  const size_t o_cur = c.add((size_t)E * 4);
  const size_t o_x = c.add((size_t)(pairs * kp1 / 256 * prefill_tile_bytes_per_256(tg)));
  const size_t o_g = c.add((size_t)(pairs * inter * 4));
  const size_t o_u = c.add((size_t)(pairs * inter * 4));
  const size_t o_mq = c.add((size_t)(pairs * kp2 / 256 * prefill_tile_bytes_per_256(td)));
  const size_t o_y = c.add((size_t)(pairs * hidden * 4));
  const int nsm = device_cus(ordinal);
  const size_t o_fix = c.add(fixup_bytes(nsm));
  uint8_t *ws = (uint8_t *)workspace().get(ordinal, c.total, stream);
  int32_t *bounds = (int32_t *)(ws + o_bounds), *tok = (int32_t *)(ws + o_tok), *src = (int32_t *)(ws + o_src);
  launch_moe_dispatch(ids, bounds, tok, src, (int)pairs, (int)E, (int)topk, (int32_t *)(ws + o_cnt),
                      (int32_t *)(ws + o_cur), stream);
  abi_check("MoE grouped (dispatch)");
  prefill_quantizer(tg)(xs, src, ws + o_x, 0, hidden, hidden, hidden * tokens, hidden * tokens, kp1, pairs, 1, 1,
                        stream);
  abi_check("MoE grouped (quantize x)");
  for (int which = 0; which < 2; which++) {
    const QTensor &w = which == 0 ? *gate_ : *up_;
    prefill_matmul_moe(tg)(ws + o_fix, w.device_ptr(), ws + o_x, tok, bounds, ws + (which == 0 ? o_g : o_u), hidden,
                           inter, pairs, hidden / (int64_t)block_size(tg), inter, E, pairs, 0, nsm, 160 * 1024, 64,
                           stream);
    abi_check("MoE grouped (gate/up)");
  }
  (act_q8_0(td)      ? launch_mmq_quantize_glu_q8_0_f32
   : prefill_q8k(td) ? launch_mmq_quantize_glu_q8k_f32
                     : launch_mmq_quantize_glu_q8_1_DS4_f32)((const float *)(ws + o_g), (const float *)(ws + o_u), tok,
                                                             ws + o_mq, inter, inter, kp2, pairs, activation_, stream);
  abi_check("MoE grouped (GLU + quantize)");
  // down, then the weighted sum over each token's routes as its own launch: folded into the down projection (a
  // counter per token and column tile, the workgroup completing it summing the routes) it measured 381 us against
  // 94 us for the pair at 64 tokens top-2 over 8 Q4_K experts of 4096x14336 -- every workgroup's agent-scope release
  // and acquire write back and invalidate its XCD's L2
  prefill_matmul_moe(td)(ws + o_fix, down_->device_ptr(), ws + o_mq, tok, bounds, ws + o_y, inter, hidden, pairs,
                         inter / (int64_t)block_size(td), hidden, E, pairs, 0, nsm, 160 * 1024, 64, stream);
  abi_check("MoE grouped (down)");
  launch_moe_weighted_reduce_flat(ws + o_y, weights, out, (int)tokens, (int)hidden, (int)topk, stream);
  abi_check("MoE grouped (reduce)");
}

}  // namespace inference_rs_amd
