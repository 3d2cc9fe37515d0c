/*
 * libinferencequant_host.so -- C entry points of the C++ host layer (inference.rs_amd/host/qtensor.h), the
 * QTensor / QMatMul / MoE-experts operator API of inference.rs restated over the kernel ABI
 * (include/inferencequant.h).  Handles are opaque; every function returns 0 on success or -1 with a message
 * in qmm_host_last_error().  Device pointers are HIP device memory; `stream` is a hipStream_t.
 */
#ifndef QMM_HOST_H
#define QMM_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qmm_qtensor qmm_qtensor;
typedef struct qmm_moe qmm_moe;

const char *qmm_host_last_error(void);

/* CPU block quantizers / dequantizer of QTensor::quantize and ::dequantize (quantized/mod.rs:391-479):
 * n values (a multiple of the block size) of GGUF type `dtype` (8 Q8_0, 12 Q4_K, 14 Q6_K, 15 Q8_K). */
int qmm_quantize_cpu(uint32_t dtype, const float *x, int64_t n, void *out);
int qmm_dequantize_cpu(uint32_t dtype, const void *blocks, int64_t n, float *y);

/* QTensor::new(QStorage::from_data(bytes, device, dtype), dims) for dims [rows, cols] or [experts, rows, cols];
 * device_ordinal < 0 keeps the tensor on the CPU.  QTensor::quantize_onto quantizes f32 values first. */
int qmm_qtensor_from_data(uint32_t dtype, const void *bytes, int64_t len, int64_t experts, int64_t rows, int64_t cols,
                          int device_ordinal, qmm_qtensor **out);
int qmm_qtensor_quantize(uint32_t dtype, const float *values, int64_t experts, int64_t rows, int64_t cols,
                         int device_ordinal, qmm_qtensor **out);
void qmm_qtensor_free(qmm_qtensor *t);
const void *qmm_qtensor_device_ptr(const qmm_qtensor *t);
int64_t qmm_qtensor_storage_bytes(const qmm_qtensor *t);
/* QTensor::dequantize on the tensor's HIP device (quantized/cuda.rs:283-334): all its values into the device
 * buffer `out` as out_dtype 0 f32, 1 f16 or 30 bf16, asynchronously on `stream`. */
int qmm_qtensor_dequantize_device(const qmm_qtensor *t, void *out, uint32_t out_dtype, void *stream);

/* QMatMul::forward: ys[rows, N] = xs[rows, K] . W^T; in_dtype 0 f32, 1 f16, 30 bf16 (xs and ys share it).
 * Decode matvec for rows <= 16, prefill matmul above (gguf/mod.rs:434-452). */
int qmm_qmatmul_forward(const qmm_qtensor *w, const void *xs, uint32_t in_dtype, int64_t rows, void *ys, void *stream);
/* QuantMethod::gather_forward: W [E, N, K]; xs [batch, xdim1, K] f32; ids [batch, topk] u32 -> ys [batch, topk, N]. */
int qmm_qmatmul_gather_forward(const qmm_qtensor *w, const float *xs, int64_t batch, int64_t xdim1,
                               const uint32_t *ids, int64_t topk, float *ys, void *stream);

/* fast_mmq::down_from_glu (gguf/fast_mmq.rs:717-833): ys[rows, N] = (act(gate) * up)[rows, K] . W^T, gate / up f32
 * [rows, K], ys f32 [rows, N]; the GLU is applied inside the activation quantization (prefill matmul at any rows).
 * activation 0 SiLU, 1 GELU (tanh form), 2 ReLU, 3 GELU (erf form), 4 sigmoid. */
int qmm_qmatmul_down_from_glu(const qmm_qtensor *w, const float *gate, const float *up, int64_t rows, int activation,
                              float *ys, void *stream);
/* fast_mmq::fused_ffn (gguf/fast_mmq.rs:883-899): ys[rows, hidden] = down(act(gate(xs)) * up(xs)), xs f32
 * [rows, hidden]; gate / up [inter, hidden] of one type (Q8_0, Q4_K or Q6_K), down [hidden, inter]. */
int qmm_fused_ffn(const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, const float *xs,
                  int64_t rows, int activation, float *ys, void *stream);

/* MoE experts block: gate/up [E, inter, hidden], down [E, hidden, inter]; activation 0 SiLU, 1 GELU, 2 ReLU, 3 GELU (erf), 4 sigmoid.
 * forward: out[t] = sum_s w[t,s] * down_e(act(gate_e(x_t)) * up_e(x_t)), e = ids[t,s]; f32 / int32 device
 * pointers.  force_grouped = 1 takes the grouped prefill path at any token count. */
int qmm_moe_new(const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, int activation,
                qmm_moe **out);
void qmm_moe_free(qmm_moe *m);
int qmm_moe_forward(const qmm_moe *m, const float *xs, int64_t tokens, const int32_t *ids, const float *weights,
                    int64_t topk, float *out, void *stream, int force_grouped);

/* ------------------------------------------------------------------ GGUF files
 * The reader and writer of crates/inference-tensor/src/quantized/gguf_file.rs.  qmm_gguf_open runs Content::read
 * (764-812), or Header::read_summary (603-608) when summary != 0, on the file at `path` and keeps it open for tensor
 * and large-array reads.  Tensors are listed in the file's table order; dims are outermost first. */
typedef struct qmm_gguf qmm_gguf;
int qmm_gguf_open(const char *path, int summary, qmm_gguf **out);
void qmm_gguf_close(qmm_gguf *g);
int qmm_gguf_version(const qmm_gguf *g);
uint64_t qmm_gguf_tensor_data_offset(const qmm_gguf *g);
int64_t qmm_gguf_tensor_count(const qmm_gguf *g);
int qmm_gguf_tensor_info(const qmm_gguf *g, int64_t idx, char *name, int64_t name_cap, uint32_t *ggml_dtype,
                         int64_t *dims, int *n_dims, uint64_t *offset);
/* metadata keys in sorted order; a value's type id 0..12 (gguf_file.rs:394-435), -1 absent, -2 a large array */
int64_t qmm_gguf_metadata_count(const qmm_gguf *g);
int qmm_gguf_metadata_key(const qmm_gguf *g, int64_t idx, char *key, int64_t cap);
int qmm_gguf_metadata_type(const qmm_gguf *g, const char *key);
/* Value::to_u64 (upcasts u8 / u16 / u32 / bool); signed integers; f32 or f64; strings (len = full length) */
int qmm_gguf_metadata_u64(const qmm_gguf *g, const char *key, uint64_t *v);
int qmm_gguf_metadata_i64(const qmm_gguf *g, const char *key, int64_t *v);
int qmm_gguf_metadata_f64(const qmm_gguf *g, const char *key, double *v);
int qmm_gguf_metadata_string(const qmm_gguf *g, const char *key, char *buf, int64_t cap, int64_t *len);
int qmm_gguf_metadata_array(const qmm_gguf *g, const char *key, int64_t *len, int *elem_type);
/* read_large_array (707-724): the raw bytes of elements [begin, end) of an array left in the file */
int qmm_gguf_large_array(const qmm_gguf *g, const char *key, uint64_t begin, uint64_t end, void *out, int64_t cap);
/* Content::tensor (800-811): the named tensor as a QTensor on the CPU (device_ordinal < 0) or a HIP device; a 1-D
 * tensor becomes one row */
int qmm_gguf_load_tensor(const qmm_gguf *g, const char *name, int device_ordinal, qmm_qtensor **out);
/* peek_architecture (553-572): general.architecture when it is the first key, else "" */
int qmm_gguf_peek_architecture(const char *path, char *buf, int64_t cap);
/* write_header + write_tensor_data (826-865): version 2, kv_count entries already serialized as kv_bytes
 * (metadata_bytes, 867-877), then the tensors in order, 32-byte aligned */
int qmm_gguf_write(const char *path, uint64_t kv_count, const void *kv_bytes, int64_t kv_len, int64_t n_tensors,
                   const char *const *names, const qmm_qtensor *const *tensors);

#ifdef __cplusplus
}
#endif
#endif
