// C entry points of the host layer (include/qmm_host.h): thin handles over QTensor / QMatMul / MoeExperts,
// exceptions turned into -1 and a per-thread message.
#include <cstring>
#include <string>

#include "gguf.h"
#include "qmm_host.h"
#include "qtensor.h"

using namespace inference_rs_amd;

struct qmm_qtensor {
  std::shared_ptr<QTensor> t;
};
struct qmm_moe {
  MoeExperts m;
};
struct qmm_gguf {
  FILE *f = nullptr;
  gguf::Content c;
  ~qmm_gguf() {
    if (f) fclose(f);
  }
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

const gguf::Value &metadata(const qmm_gguf *g, const char *key) {
  auto it = g->c.header.metadata.find(key);
  if (it == g->c.header.metadata.end()) throw Error(std::string("gguf: no metadata key ") + key);
  return it->second;
}

void copy_out(const std::string &s, char *buf, int64_t cap) {
  if (!buf || cap <= 0) return;
  const size_t n = std::min((size_t)(cap - 1), s.size());
  memcpy(buf, s.data(), n);
  buf[n] = '\0';
}
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

int qmm_qmatmul_down_from_glu(const qmm_qtensor *w, const float *gate, const float *up, int64_t rows, int activation,
                              float *ys, void *stream) {
  return guarded([&] { QMatMul(w->t).down_from_glu(gate, up, rows, activation, ys, (hipStream_t)stream); });
}

int qmm_fused_ffn(const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, const float *xs,
                  int64_t rows, int activation, float *ys, void *stream) {
  return guarded([&] {
    fused_ffn(QMatMul(gate->t), QMatMul(up->t), QMatMul(down->t), xs, rows, activation, ys, (hipStream_t)stream);
  });
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


// ------------------------------------------------------------------------------------------------ GGUF files

int qmm_gguf_open(const char *path, int summary, qmm_gguf **out) {
  return guarded([&] {
    std::unique_ptr<qmm_gguf> g(new qmm_gguf);
    g->f = fopen(path, "rb");
    if (!g->f) throw Error(std::string("gguf: cannot open ") + path);
    if (summary) {
      g->c.header = gguf::Header::read(g->f, true);
      for (const auto &kv : g->c.header.tensor_infos)
        g->c.tensor_infos[kv.first] =
            gguf::TensorInfo{dtype_from_u32(kv.second.ggml_dtype), kv.second.shape, kv.second.offset};
    } else {
      g->c = gguf::Content::read(g->f);
    }
    *out = g.release();
  });
}

void qmm_gguf_close(qmm_gguf *g) { delete g; }

int qmm_gguf_version(const qmm_gguf *g) { return (int)g->c.header.version; }
uint64_t qmm_gguf_tensor_data_offset(const qmm_gguf *g) { return g->c.header.tensor_data_offset; }
int64_t qmm_gguf_tensor_count(const qmm_gguf *g) { return (int64_t)g->c.header.tensor_order.size(); }

int qmm_gguf_tensor_info(const qmm_gguf *g, int64_t idx, char *name, int64_t name_cap, uint32_t *ggml_dtype,
                         int64_t *dims, int *n_dims, uint64_t *offset) {
  return guarded([&] {
    const auto &order = g->c.header.tensor_order;
    if (idx < 0 || idx >= (int64_t)order.size()) throw Error("gguf: tensor index out of range");
    const gguf::RawTensorInfo &ti = g->c.header.tensor_infos.at(order[(size_t)idx]);
    copy_out(order[(size_t)idx], name, name_cap);
    *ggml_dtype = ti.ggml_dtype;
    *n_dims = (int)ti.shape.size();
    for (size_t d = 0; d < ti.shape.size(); d++) dims[d] = ti.shape[d];
    *offset = ti.offset;
  });
}

int64_t qmm_gguf_metadata_count(const qmm_gguf *g) { return (int64_t)g->c.header.metadata.size(); }

int qmm_gguf_metadata_key(const qmm_gguf *g, int64_t idx, char *key, int64_t cap) {
  return guarded([&] {
    if (idx < 0 || idx >= (int64_t)g->c.header.metadata.size()) throw Error("gguf: metadata index out of range");
    auto it = g->c.header.metadata.begin();
    std::advance(it, idx);
    copy_out(it->first, key, cap);
  });
}

int qmm_gguf_metadata_type(const qmm_gguf *g, const char *key) {
  auto it = g->c.header.metadata.find(key);
  if (it != g->c.header.metadata.end()) return (int)it->second.type;
  return g->c.header.large_arrays.count(key) ? -2 : -1;
}

int qmm_gguf_metadata_u64(const qmm_gguf *g, const char *key, uint64_t *v) {
  return guarded([&] { *v = metadata(g, key).to_u64(); });
}

int qmm_gguf_metadata_i64(const qmm_gguf *g, const char *key, int64_t *v) {
  return guarded([&] {
    const gguf::Value &x = metadata(g, key);
    switch (x.type) {
      case gguf::ValueType::I8: case gguf::ValueType::I16: case gguf::ValueType::I32: case gguf::ValueType::I64:
        *v = x.i;
        break;
      default: throw Error(std::string("gguf: ") + key + " is not a signed integer");
    }
  });
}

int qmm_gguf_metadata_f64(const qmm_gguf *g, const char *key, double *v) {
  return guarded([&] {
    const gguf::Value &x = metadata(g, key);
    *v = x.type == gguf::ValueType::F32 ? (double)x.to_f32() : x.to_f64();
  });
}

int qmm_gguf_metadata_string(const qmm_gguf *g, const char *key, char *buf, int64_t cap, int64_t *len) {
  return guarded([&] {
    const std::string &s = metadata(g, key).to_string();
    *len = (int64_t)s.size();
    copy_out(s, buf, cap);
  });
}

int qmm_gguf_metadata_array(const qmm_gguf *g, const char *key, int64_t *len, int *elem_type) {
  return guarded([&] {
    const std::vector<gguf::Value> &a = metadata(g, key).to_vec();
    *len = (int64_t)a.size();
    *elem_type = a.empty() ? -1 : (int)a[0].type;
  });
}

int qmm_gguf_large_array(const qmm_gguf *g, const char *key, uint64_t begin, uint64_t end, void *out, int64_t cap) {
  return guarded([&] {
    const std::vector<uint8_t> b = g->c.header.read_large_array(g->f, key, begin, end);
    if ((int64_t)b.size() > cap) throw Error("gguf: large array range does not fit the buffer");
    memcpy(out, b.data(), b.size());
  });
}

int qmm_gguf_load_tensor(const qmm_gguf *g, const char *name, int device_ordinal, qmm_qtensor **out) {
  return guarded([&] { *out = new qmm_qtensor{g->c.tensor(g->f, name, device_of(device_ordinal))}; });
}

int qmm_gguf_peek_architecture(const char *path, char *buf, int64_t cap) {
  return guarded([&] {
    FILE *f = fopen(path, "rb");
    if (!f) throw Error(std::string("gguf: cannot open ") + path);
    std::string a;
    try {
      a = gguf::peek_architecture(f);
    } catch (...) {
      fclose(f);
      throw;
    }
    fclose(f);
    copy_out(a, buf, cap);
  });
}

int qmm_gguf_write(const char *path, uint64_t kv_count, const void *kv_bytes, int64_t kv_len, int64_t n_tensors,
                   const char *const *names, const qmm_qtensor *const *tensors) {
  return guarded([&] {
    std::vector<std::pair<std::string, std::shared_ptr<QTensor>>> ts;
    for (int64_t i = 0; i < n_tensors; i++) ts.emplace_back(names[i], tensors[i]->t);
    const std::vector<uint8_t> kv((const uint8_t *)kv_bytes, (const uint8_t *)kv_bytes + kv_len);
    FILE *f = fopen(path, "wb");
    if (!f) throw Error(std::string("gguf: cannot create ") + path);
    try {
      gguf::write_raw(f, kv_count, kv, ts);
    } catch (...) {
      fclose(f);
      throw;
    }
    if (fclose(f) != 0) throw Error("gguf: close failed");
  });
}

}  // extern "C"
