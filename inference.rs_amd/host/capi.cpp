// C entry points of the host layer (include/qmm_host.h): thin handles over QTensor / QMatMul / MoeExperts,
// exceptions turned into -1 and a per-thread message.
#include <cstring>
#include <string>

#include "qmm_host.h"
#include "qtensor.h"

using namespace inference_rs_amd;

struct qmm_qtensor {
  std::shared_ptr<QTensor> t;
};
struct qmm_moe {
  MoeExperts m;
};

namespace {
thread_local std::string g_error;

template <class F>
int guarded(F &&f) {
  try {
    f();
    g_error.clear();
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}

std::vector<int64_t> dims_of(int64_t experts, int64_t rows, int64_t cols) {
  if (experts > 1) return {experts, rows, cols};
  return {rows, cols};
}

Device device_of(int ordinal) { return ordinal < 0 ? Device::cpu() : Device::hip(ordinal); }
}  // namespace

extern "C" {

const char *qmm_host_last_error(void) { return g_error.c_str(); }

int qmm_quantize_cpu(uint32_t dtype, const float *x, int64_t n, void *out) {
  return guarded([&] {
    if (!cpu::quantize(dtype_from_u32(dtype), x, n, out)) throw Error("quantize: unsupported type or length");
  });
}

int qmm_dequantize_cpu(uint32_t dtype, const void *blocks, int64_t n, float *y) {
  return guarded([&] {
    if (!cpu::dequantize(dtype_from_u32(dtype), blocks, n, y)) throw Error("dequantize: unsupported type");
  });
}

int qmm_qtensor_from_data(uint32_t dtype, const void *bytes, int64_t len, int64_t experts, int64_t rows, int64_t cols,
                          int device_ordinal, qmm_qtensor **out) {
  return guarded([&] {
    auto t = QTensor::from_data(bytes, (size_t)len, dims_of(experts, rows, cols), dtype_from_u32(dtype),
                                device_of(device_ordinal));
    *out = new qmm_qtensor{std::move(t)};
  });
}

int qmm_qtensor_quantize(uint32_t dtype, const float *values, int64_t experts, int64_t rows, int64_t cols,
                         int device_ordinal, qmm_qtensor **out) {
  return guarded([&] {
    auto t = QTensor::quantize(values, dims_of(experts, rows, cols), dtype_from_u32(dtype), device_of(device_ordinal));
    *out = new qmm_qtensor{std::move(t)};
  });
}

void qmm_qtensor_free(qmm_qtensor *t) { delete t; }

const void *qmm_qtensor_device_ptr(const qmm_qtensor *t) {
  const void *p = nullptr;
  guarded([&] { p = t->t->device_ptr(); });
  return p;
}

int64_t qmm_qtensor_storage_bytes(const qmm_qtensor *t) { return (int64_t)t->t->storage_size_in_bytes(); }

int qmm_qtensor_dequantize_device(const qmm_qtensor *t, void *out, uint32_t out_dtype, void *stream) {
  return guarded([&] { t->t->dequantize_on_device(out, dtype_from_u32(out_dtype), (hipStream_t)stream); });
}

int qmm_qmatmul_forward(const qmm_qtensor *w, const void *xs, uint32_t in_dtype, int64_t rows, void *ys, void *stream) {
  return guarded([&] { QMatMul(w->t).forward(xs, dtype_from_u32(in_dtype), rows, ys, (hipStream_t)stream); });
}

int qmm_qmatmul_gather_forward(const qmm_qtensor *w, const float *xs, int64_t batch, int64_t xdim1,
                               const uint32_t *ids, int64_t topk, float *ys, void *stream) {
  return guarded([&] { QMatMul(w->t).gather_forward(xs, batch, xdim1, ids, topk, ys, (hipStream_t)stream); });
}

int qmm_moe_new(const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, int activation,
                qmm_moe **out) {
  return guarded([&] { *out = new qmm_moe{MoeExperts(gate->t, up->t, down->t, activation)}; });
}

void qmm_moe_free(qmm_moe *m) { delete m; }

int qmm_moe_forward(const qmm_moe *m, const float *xs, int64_t tokens, const int32_t *ids, const float *weights,
                    int64_t topk, float *out, void *stream, int force_grouped) {
  return guarded([&] { m->m.forward(xs, tokens, ids, weights, topk, out, (hipStream_t)stream, force_grouped != 0); });
}

}  // extern "C"
