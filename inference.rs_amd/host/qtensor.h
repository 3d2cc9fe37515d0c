// C++ host layer over libinferencequant.so: the QTensor / QMatMul operator API and the Device enum of
// inference.rs (crates/inference-tensor/src/quantized/mod.rs:85-120, 277-479, 886-1187; device.rs:26-31)
// and the GGUF dispatch of crates/inference-quant/src/gguf/mod.rs:429-511 (try_fast_forward), with
// Device::Hip in place of Device::Cuda.  Errors throw qmm::Error where the reference returns
// candle's Result::Err (bail!).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "qmm_blocks.h"

namespace inference_rs_amd {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// GgmlDType (quantized/mod.rs:481-704).  Kernels serve Q8_0, Q4K, Q6K (every route) and Q4_0, Q5_0, Q5K (the
// matvec route and dequantization); Q4_1, Q5_1, Q8_1, Q2K and Q3K are held and saved but have no kernels here.
enum class GgmlDType : uint32_t {
  F32 = QMM_TYPE_F32,
  F16 = QMM_TYPE_F16,
  Q4_0 = QMM_TYPE_Q4_0,
  Q4_1 = QMM_TYPE_Q4_1,
  Q5_0 = QMM_TYPE_Q5_0,
  Q5_1 = QMM_TYPE_Q5_1,
  Q8_0 = QMM_TYPE_Q8_0,
  Q8_1 = QMM_TYPE_Q8_1,
  Q2K = QMM_TYPE_Q2K,
  Q3K = QMM_TYPE_Q3K,
  Q4K = QMM_TYPE_Q4K,
  Q5K = QMM_TYPE_Q5K,
  Q6K = QMM_TYPE_Q6K,
  Q8K = QMM_TYPE_Q8K,
  BF16 = QMM_TYPE_BF16,
};
GgmlDType dtype_from_u32(uint32_t u);  // GgmlDType::from_u32 (mod.rs:582-603); throws on an unknown id
size_t type_size(GgmlDType t);         // mod.rs:669-688
size_t block_size(GgmlDType t);        // mod.rs:691-703
const char *dtype_name(GgmlDType t);

// Device (device.rs:26-31): Cpu, or the ordinal-th HIP device (in place of Cuda)
struct Device {
  enum class Kind { Cpu, Hip } kind = Kind::Cpu;
  int ordinal = 0;
  static Device cpu() { return {}; }
  static Device hip(int ordinal) { return {Kind::Hip, ordinal}; }
  bool is_cpu() const { return kind == Kind::Cpu; }
  bool is_hip() const { return kind == Kind::Hip; }
};

// Device bytes of a QStorage::Hip, padded like QCudaStorage (quantized/cuda.rs:25, 245-258: a row padding of
// MATRIX_ROW_PADDING = 512 values, so kernels may read past the last block).
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  DeviceBuffer(int ordinal, size_t bytes);
  ~DeviceBuffer();
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  void *ptr() const { return ptr_; }
  size_t size() const { return size_; }
  int ordinal() const { return ordinal_; }

 private:
  void *ptr_ = nullptr;
  size_t size_ = 0;
  int ordinal_ = 0;
};

// QTensor: packed GGUF blocks of shape [..., rows, cols] (cols = the reduction dim K), on one device
class QTensor {
 public:
  // QTensor::quantize / quantize_onto (mod.rs:391-413): quantize f32 values on the host, then place them
  static std::shared_ptr<QTensor> quantize(const float *src, const std::vector<int64_t> &dims, GgmlDType dtype,
                                           Device device);
  // QTensor::new(QStorage::from_data(bytes, device, dtype), dims) (mod.rs:278-321)
  static std::shared_ptr<QTensor> from_data(const void *bytes, size_t len, const std::vector<int64_t> &dims,
                                            GgmlDType dtype, Device device);

  GgmlDType dtype() const { return dtype_; }
  const std::vector<int64_t> &shape() const { return dims_; }
  Device device() const { return device_; }
  int64_t cols() const { return dims_.back(); }            // K
  int64_t rows() const { return dims_[dims_.size() - 2]; }  // N (per expert for rank 3)
  int64_t experts() const { return dims_.size() == 3 ? dims_[0] : 1; }
  int64_t elem_count() const;
  size_t row_bytes() const { return (size_t)(cols() / (int64_t)block_size(dtype_)) * type_size(dtype_); }
  size_t storage_size_in_bytes() const { return (size_t)(elem_count() / (int64_t)block_size(dtype_)) * type_size(dtype_); }

  std::vector<uint8_t> data() const;      // the packed bytes (downloaded from a device)
  std::vector<float> dequantize() const;  // on the host, f32
  // QTensor::dequantize / dequantize_f16 on a HIP device (quantized/cuda.rs:283-334): the elem_count() values into
  // the device buffer `out` as F32, F16 or BF16, asynchronously on `stream`
  void dequantize_on_device(void *out, GgmlDType out_dtype, hipStream_t stream) const;
  const void *device_ptr() const;         // the device bytes (device_ptr_with_guard, mod.rs:474-480)

 private:
  QTensor(GgmlDType dtype, std::vector<int64_t> dims, Device device) : dtype_(dtype), dims_(std::move(dims)), device_(device) {}
  GgmlDType dtype_;
  std::vector<int64_t> dims_;
  Device device_;
  std::vector<uint8_t> host_;
  std::unique_ptr<DeviceBuffer> dev_;
};

// QMatMul (mod.rs:1117-1187, 1625-1648) over a quantized weight, with the GPU route choice of
// gguf/mod.rs:434-452: decode matvec (launch_mmvq_gguf_*) for a flat batch of at most max_decode_rows rows,
// the prefill matmul (launch_mmq_gguf_*) above it.
class QMatMul {
 public:
  static constexpr int64_t kMaxDecodeRows = 16;  // fast_mmvq.rs TENSOR_CORE_MAX_ROWS, re-derived for gfx950
  // Q4_K, and Q6_K with rows of at most kMaxFewRowK values, stay on the decode launcher up to 32 rows: its few-row
  // MFMA kernel streams the weight once for all of them and measured faster than the prefill tile there on MI355X
  // (Q4_K 4096x4096 at 32 rows 10.4 against 13.2 us; Q6_K 4096x14336 is the exception, 34.6 against 31.7 us, as
  // the reference keeps Q6_K's widest rows on MMQ, fast_mmvq.rs:1838-1881)
  static constexpr int64_t kMaxFewRows = 32;
  static constexpr int64_t kMaxFewRowK = 8192;

  explicit QMatMul(std::shared_ptr<QTensor> w);
  const QTensor &weight() const { return *w_; }

  static int64_t max_decode_rows(GgmlDType dtype, int64_t k);
  static bool prefers_mmvq(GgmlDType dtype, int64_t rows, int64_t k);

  // ys[rows, N] = xs[rows, K] . W^T on the weight's device; xs / ys device pointers of in_dtype
  // (F32, F16 or BF16), as QMatMul::forward keeps the activation dtype (gguf/mod.rs:656-661).
  void forward(const void *xs, GgmlDType in_dtype, int64_t rows, void *ys, hipStream_t stream) const;

  // QuantMethod::gather_forward (gguf/mod.rs:573-608): weight [E, N, K], xs [batch, xdim1, K] f32,
  // ids [batch, topk] u32 (device) -> ys [batch, topk, N] f32.  Expert ids must be < E.
  void gather_forward(const float *xs, int64_t batch, int64_t xdim1, const uint32_t *ids, int64_t topk, float *ys,
                      hipStream_t stream) const;

  // fast_mmq::down_from_glu (gguf/fast_mmq.rs:717-833): ys[rows, N] = (act(gate) * up)[rows, K] . W^T for this
  // [N, K] weight; gate, up f32 [rows, K] and ys f32 [rows, N] device pointers; activation 0 SiLU, 1 GELU (tanh
  // form), 2 ReLU, 3 GELU (erf form), 4 sigmoid.  The GLU is applied while the activations are quantized
  // (launch_mmq_quantize_glu_*, one launch), so act(gate) * up is never stored; every row count takes the prefill
  // matmul, as the reference's MMQ function does.
  void down_from_glu(const float *gate, const float *up, int64_t rows, int activation, float *ys,
                     hipStream_t stream) const;

 private:
  std::shared_ptr<QTensor> w_;
};

// fast_mmq::fused_ffn (gguf/fast_mmq.rs:883-899): ys[rows, hidden] = down(act(gate(xs)) * up(xs)) for f32 xs
// [rows, hidden], gate and up [inter, hidden] of one type, down [hidden, inter].  Gate and up read one activation
// quantization (shared_lhs, fast_mmq.rs:537-602).  Up to QMatMul::kMaxDecodeRows rows they run as the fused-GLU
// matvec (launch_mmvq_gguf_<t>_f32_fused_glu, which stores act(gate) * up) and down as QMatMul::forward; above, as
// two prefill matmuls whose f32 outputs go through down.down_from_glu.
void fused_ffn(const QMatMul &gate, const QMatMul &up, const QMatMul &down, const float *xs, int64_t rows,
               int activation, float *ys, hipStream_t stream);

// The MoE experts block of the reference's grouped prefill / indexed decode
// (crates/inference-nn/src/moe/experts/backends.rs:1382-1489, 1966-2402): gate/up/down expert stacks,
// routing tables built on the device, and the weighted top-k reduce.
class MoeExperts {
 public:
  static constexpr int64_t kIndexedMaxTokens = 8;      // backends.rs:25 INDEXED_MMVQ_MAX_TOKENS
  static constexpr int64_t kGroupedMinTokens = 32;     // backends.rs:22 GROUPED_PREFILL_MIN_TOKENS

  MoeExperts(std::shared_ptr<QTensor> gate, std::shared_ptr<QTensor> up, std::shared_ptr<QTensor> down,
             int activation);
  // out[tokens, hidden] = sum_s w[t, s] * down_e(act(gate_e(x_t)) * up_e(x_t)), e = ids[t, s].
  // xs f32 [tokens, hidden], ids int32 [tokens, topk], weights f32 [tokens, topk]; all device pointers.
  void forward(const float *xs, int64_t tokens, const int32_t *ids, const float *weights, int64_t topk, float *out,
               hipStream_t stream, bool force_grouped = false) const;

 private:
  std::shared_ptr<QTensor> gate_, up_, down_;
  int activation_;
};

namespace cpu {
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);
bool quantize(GgmlDType t, const float *x, int64_t n, void *out);
bool dequantize(GgmlDType t, const void *blocks, int64_t n, float *y);
}  // namespace cpu

}  // namespace inference_rs_amd
