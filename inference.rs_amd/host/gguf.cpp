// GGUF reader and writer; behaviour follows crates/inference-tensor/src/quantized/gguf_file.rs (cited per function).
#include "gguf.h"

#include <string.h>

#include <set>

namespace inference_rs_amd {
namespace gguf {
namespace {

[[noreturn]] void fail(const std::string &m) { throw Error("gguf: " + m); }

uint64_t tell(FILE *f) {
  const off_t p = ftello(f);
  if (p < 0) fail("ftell failed");
  return (uint64_t)p;
}
void seek(FILE *f, uint64_t pos) {
  if (fseeko(f, (off_t)pos, SEEK_SET) != 0) fail("seek failed");
}
uint64_t file_size(FILE *f) {
  const uint64_t here = tell(f);
  if (fseeko(f, 0, SEEK_END) != 0) fail("seek failed");
  const uint64_t n = tell(f);
  seek(f, here);
  return n;
}
void read_exact(FILE *f, void *dst, size_t n) {
  if (n && fread(dst, 1, n, f) != n) fail("unexpected end of file");
}
template <class T>
T rd(FILE *f) {
  T v;
  read_exact(f, &v, sizeof v);  // little-endian host (x86-64 / the GPU boxes)
  return v;
}

// the reader's state: the file, its size captured once, the length-prefix width of the version
struct Reader {
  FILE *f;
  uint64_t size;
  Version version;
  uint64_t remaining() { return size - std::min(size, tell(f)); }
  uint64_t length() { return version == Version::V1 ? rd<uint32_t>(f) : rd<uint64_t>(f); }  // read_length (34-39)
  uint64_t prefix() const { return version == Version::V1 ? 4 : 8; }
  // minimum on-disk size of one value (min_disk_size, 437-448)
  uint64_t min_size(ValueType t) const {
    switch (t) {
      case ValueType::U8: case ValueType::I8: case ValueType::Bool: return 1;
      case ValueType::U16: case ValueType::I16: return 2;
      case ValueType::U32: case ValueType::I32: case ValueType::F32: return 4;
      case ValueType::U64: case ValueType::I64: case ValueType::F64: return 8;
      case ValueType::String: return prefix();
      case ValueType::Array: return 4 + prefix();
    }
    return 1;
  }
  // read_string (145-166): length-checked, trailing NULs dropped
  std::string string() {
    const uint64_t len = length();
    if (len > kMaxStringLength) fail("string length " + std::to_string(len) + " exceeds max");
    if (len > remaining()) fail("string length " + std::to_string(len) + " exceeds remaining file bytes");
    std::string s(len, '\0');
    read_exact(f, &s[0], len);
    while (!s.empty() && s.back() == '\0') s.pop_back();
    return s;
  }
  // Value::read (330-392)
  Value value(ValueType t, int depth) {
    if (depth > kMaxValueDepth) fail("value nesting depth exceeds max");
    Value v;
    v.type = t;
    switch (t) {
      case ValueType::U8: v.u = rd<uint8_t>(f); break;
      case ValueType::I8: v.i = rd<int8_t>(f); break;
      case ValueType::U16: v.u = rd<uint16_t>(f); break;
      case ValueType::I16: v.i = rd<int16_t>(f); break;
      case ValueType::U32: v.u = rd<uint32_t>(f); break;
      case ValueType::I32: v.i = rd<int32_t>(f); break;
      case ValueType::U64: v.u = rd<uint64_t>(f); break;
      case ValueType::I64: v.i = rd<int64_t>(f); break;
      case ValueType::F32: v.f = rd<float>(f); break;
      case ValueType::F64: v.f = rd<double>(f); break;
      case ValueType::Bool: {
        const uint8_t b = rd<uint8_t>(f);
        if (b > 1) fail("unexpected bool value " + std::to_string(b));
        v.u = b;
        break;
      }
      case ValueType::String: v.s = string(); break;
      case ValueType::Array: {
        const ValueType et = value_type_from_u32(rd<uint32_t>(f));
        const uint64_t len = length();
        if (len > kMaxArrayElements) fail("array length " + std::to_string(len) + " exceeds max");
        const uint64_t need = len > UINT64_MAX / min_size(et) ? UINT64_MAX : len * min_size(et);
        if (need > remaining()) fail("array of " + std::to_string(len) + " elements needs more bytes than remain");
        v.array.reserve(len);
        for (uint64_t k = 0; k < len; k++) v.array.push_back(value(et, depth + 1));
        break;
      }
    }
    return v;
  }
  // skip_long_array (451-485): arrays over kSummaryArrayElements of fixed-size values or strings are skipped
  bool skip_long_array(ValueType t) {
    if (t != ValueType::Array) return false;
    const uint64_t start = tell(f);
    const ValueType et = value_type_from_u32(rd<uint32_t>(f));
    const uint64_t len = length();
    if (len <= kSummaryArrayElements || et == ValueType::Array) {
      seek(f, start);
      return false;
    }
    if (et == ValueType::String) {
      for (uint64_t k = 0; k < len; k++) {
        const uint64_t n = length();
        if (n > kMaxStringLength) fail("string length exceeds max");
        if (n > remaining()) fail("string past the end of the file");
        seek(f, tell(f) + n);
      }
      return true;
    }
    const uint64_t bytes = len > UINT64_MAX / min_size(et) ? UINT64_MAX : len * min_size(et);
    if (bytes > remaining()) fail("array past the end of the file");
    seek(f, tell(f) + bytes);
    return true;
  }
  // large_array (488-519): a top-level array of more than kInlineArrayElements fixed-size values is located
  bool large_array(ValueType t, LargeArray &out) {
    if (t != ValueType::Array) return false;
    const uint64_t start = tell(f);
    const ValueType et = value_type_from_u32(rd<uint32_t>(f));
    const uint64_t len = length();
    const bool fixed = et != ValueType::String && et != ValueType::Array;
    if (!fixed || len <= kInlineArrayElements) {
      seek(f, start);
      return false;
    }
    const uint64_t off = tell(f);
    const uint64_t bytes = len > UINT64_MAX / min_size(et) ? UINT64_MAX : len * min_size(et);
    if (bytes > size - std::min(size, off)) fail("array past the end of the file");
    seek(f, off + bytes);
    out = {et, len, off};
    return true;
  }
};

Version read_magic(FILE *f) {  // VersionedMagic::read (61-77)
  const uint32_t magic = rd<uint32_t>(f);
  if (magic != 0x46554747u && magic != 0x47475546u) {
    char b[64];
    snprintf(b, sizeof b, "unknown magic 0x%08x", magic);
    fail(b);
  }
  const uint32_t version = rd<uint32_t>(f);
  if (version < 1 || version > 3) fail("unsupported version " + std::to_string(version));
  return (Version)version;
}

[[noreturn]] void wrong(const Value &v, const char *want) {
  fail(std::string("not a ") + want + " (value type " + std::to_string((uint32_t)v.type) + ")");
}

void wr(std::vector<uint8_t> &o, const void *p, size_t n) {
  o.insert(o.end(), (const uint8_t *)p, (const uint8_t *)p + n);
}
template <class T>
void wr(std::vector<uint8_t> &o, T v) {
  wr(o, &v, sizeof v);
}
void write_string(std::vector<uint8_t> &o, const std::string &s) {  // write_string (814-819): u64 length
  wr<uint64_t>(o, s.size());
  wr(o, s.data(), s.size());
}
void write_value(std::vector<uint8_t> &o, const Value &v) {  // Value::write (394-392+)
  switch (v.type) {
    case ValueType::U8: wr<uint8_t>(o, (uint8_t)v.u); break;
    case ValueType::I8: wr<int8_t>(o, (int8_t)v.i); break;
    case ValueType::U16: wr<uint16_t>(o, (uint16_t)v.u); break;
    case ValueType::I16: wr<int16_t>(o, (int16_t)v.i); break;
    case ValueType::U32: wr<uint32_t>(o, (uint32_t)v.u); break;
    case ValueType::I32: wr<int32_t>(o, (int32_t)v.i); break;
    case ValueType::U64: wr<uint64_t>(o, v.u); break;
    case ValueType::I64: wr<int64_t>(o, v.i); break;
    case ValueType::F32: wr<float>(o, (float)v.f); break;
    case ValueType::F64: wr<double>(o, v.f); break;
    case ValueType::Bool: wr<uint8_t>(o, v.u ? 1 : 0); break;
    case ValueType::String: write_string(o, v.s); break;
    case ValueType::Array: {
      // every element must share one type; an empty array is written as u32
      std::set<uint32_t> types;
      for (const Value &e : v.array) types.insert((uint32_t)e.type);
      if (types.size() > 1) fail("multiple value-types in the same array");
      wr<uint32_t>(o, types.empty() ? (uint32_t)ValueType::U32 : *types.begin());
      wr<uint64_t>(o, v.array.size());
      for (const Value &e : v.array) write_value(o, e);
      break;
    }
  }
}
size_t padding(size_t len) { return 31 - (31 + len) % 32; }  // (821-823)
void put(FILE *f, const void *p, size_t n) {
  if (n && fwrite(p, 1, n, f) != n) fail("write failed");
}

}  // namespace

ValueType value_type_from_u32(uint32_t v) {
  if (v > 12) {
    char b[64];
    snprintf(b, sizeof b, "unrecognized value-type %#08x", v);
    fail(b);
  }
  return (ValueType)v;
}

#define QMM_MAKE(name, T, field, VT)     \
  Value Value::make_##name(T v) {        \
    Value r;                             \
    r.type = ValueType::VT;              \
    r.field = v;                         \
    return r;                            \
  }
QMM_MAKE(u8, uint8_t, u, U8)
QMM_MAKE(i8, int8_t, i, I8)
QMM_MAKE(u16, uint16_t, u, U16)
QMM_MAKE(i16, int16_t, i, I16)
QMM_MAKE(u32, uint32_t, u, U32)
QMM_MAKE(i32, int32_t, i, I32)
QMM_MAKE(u64, uint64_t, u, U64)
QMM_MAKE(i64, int64_t, i, I64)
QMM_MAKE(f32, float, f, F32)
QMM_MAKE(f64, double, f, F64)
QMM_MAKE(bool, bool, u, Bool)
#undef QMM_MAKE
Value Value::make_string(std::string v) {
  Value r;
  r.type = ValueType::String;
  r.s = std::move(v);
  return r;
}
Value Value::make_array(std::vector<Value> v) {
  Value r;
  r.type = ValueType::Array;
  r.array = std::move(v);
  return r;
}

uint8_t Value::to_u8() const { if (type != ValueType::U8) wrong(*this, "u8"); return (uint8_t)u; }
int8_t Value::to_i8() const { if (type != ValueType::I8) wrong(*this, "i8"); return (int8_t)i; }
uint16_t Value::to_u16() const { if (type != ValueType::U16) wrong(*this, "u16"); return (uint16_t)u; }
int16_t Value::to_i16() const { if (type != ValueType::I16) wrong(*this, "i16"); return (int16_t)i; }
uint32_t Value::to_u32() const { if (type != ValueType::U32) wrong(*this, "u32"); return (uint32_t)u; }
int32_t Value::to_i32() const { if (type != ValueType::I32) wrong(*this, "i32"); return (int32_t)i; }
uint64_t Value::to_u64() const {
  switch (type) {
    case ValueType::U64: case ValueType::U8: case ValueType::U16: case ValueType::U32: case ValueType::Bool: return u;
    default: wrong(*this, "u64 or upcastable to u64");
  }
}
int64_t Value::to_i64() const { if (type != ValueType::I64) wrong(*this, "i64"); return i; }
float Value::to_f32() const { if (type != ValueType::F32) wrong(*this, "f32"); return (float)f; }
double Value::to_f64() const { if (type != ValueType::F64) wrong(*this, "f64"); return f; }
bool Value::to_bool() const { if (type != ValueType::Bool) wrong(*this, "bool"); return u != 0; }
const std::string &Value::to_string() const { if (type != ValueType::String) wrong(*this, "string"); return s; }
const std::vector<Value> &Value::to_vec() const { if (type != ValueType::Array) wrong(*this, "vec"); return array; }

Header Header::read(FILE *f, bool summary) {
  Reader r{f, 0, Version::V3};
  const uint64_t start = tell(f);
  r.size = file_size(f);
  seek(f, start);
  Header h;
  h.version = r.version = read_magic(f);
  const uint64_t tensor_count = r.length(), kv_count = r.length();
  if (tensor_count > kMaxArrayElements) fail("tensor_count " + std::to_string(tensor_count) + " exceeds max");
  if (kv_count > kMaxArrayElements) fail("metadata_kv_count " + std::to_string(kv_count) + " exceeds max");
  // counts that cannot fit in the file at their minimum sizes are rejected before any allocation (629-645)
  const uint64_t need = kv_count * (r.prefix() + 4 + 1) + tensor_count * (r.prefix() + 4 + 4 + 8);
  if (need > r.remaining())
    fail("header declares " + std::to_string(tensor_count) + " tensors and " + std::to_string(kv_count) +
         " metadata entries, needs at least " + std::to_string(need) + " bytes");
  h.metadata_begin = tell(f);
  for (uint64_t k = 0; k < kv_count; k++) {
    std::string key = r.string();
    const ValueType t = value_type_from_u32(rd<uint32_t>(f));
    if (summary && r.skip_long_array(t)) continue;
    LargeArray la;
    if (r.large_array(t, la)) {
      h.large_arrays[key] = la;
      continue;
    }
    h.metadata[key] = r.value(t, 0);
  }
  h.metadata_end = tell(f);
  for (uint64_t k = 0; k < tensor_count; k++) {
    std::string name = r.string();
    const uint32_t nd = rd<uint32_t>(f);
    if (nd > kMaxTensorDims) fail("tensor '" + name + "' has " + std::to_string(nd) + " dimensions, max is 8");
    RawTensorInfo info;
    info.shape.resize(nd);
    for (uint32_t d = 0; d < nd; d++)
      info.shape[nd - 1 - d] = r.version == Version::V1 ? (int64_t)rd<uint32_t>(f) : (int64_t)rd<uint64_t>(f);
    info.ggml_dtype = rd<uint32_t>(f);
    info.offset = rd<uint64_t>(f);
    h.tensor_order.push_back(name);
    h.tensor_infos[name] = info;
  }
  // general.alignment: an unsigned or non-negative signed 8/16/32-bit value, else 32 (686-696)
  uint64_t alignment = kDefaultAlignment;
  auto it = h.metadata.find("general.alignment");
  if (it != h.metadata.end()) {
    const Value &v = it->second;
    if (v.type == ValueType::U8 || v.type == ValueType::U16 || v.type == ValueType::U32) alignment = v.u;
    else if ((v.type == ValueType::I8 || v.type == ValueType::I16 || v.type == ValueType::I32) && v.i >= 0)
      alignment = (uint64_t)v.i;
  }
  if (alignment == 0) fail("general.alignment is 0");
  const uint64_t pos = tell(f);
  h.tensor_data_offset = (pos + alignment - 1) / alignment * alignment;
  return h;
}

std::vector<uint8_t> Header::read_large_array(FILE *f, const std::string &name, uint64_t begin, uint64_t end) const {
  auto it = large_arrays.find(name);
  if (it == large_arrays.end()) fail("no large array " + name);
  const LargeArray &a = it->second;
  if (begin > end || end > a.len)
    fail("[" + std::to_string(begin) + ", " + std::to_string(end) + ") is outside " + name + "'s " +
         std::to_string(a.len) + " elements");
  Reader r{f, 0, version};
  const uint64_t sz = r.min_size(a.value_type);
  std::vector<uint8_t> out((size_t)((end - begin) * sz));
  seek(f, a.offset + begin * sz);
  read_exact(f, out.data(), out.size());
  return out;
}

Content Content::read(FILE *f) {
  Content c;
  c.header = Header::read(f, false);
  for (const auto &kv : c.header.tensor_infos)
    c.tensor_infos[kv.first] = TensorInfo{dtype_from_u32(kv.second.ggml_dtype), kv.second.shape, kv.second.offset};
  return c;
}

std::shared_ptr<QTensor> Content::tensor(FILE *f, const std::string &name, Device device) const {
  auto it = tensor_infos.find(name);
  if (it == tensor_infos.end()) fail("cannot find tensor info for " + name);
  const TensorInfo &ti = it->second;
  int64_t elems = 1;
  for (int64_t d : ti.shape) {
    if (d < 0 || (d > 0 && elems > INT64_MAX / d)) fail("tensor '" + name + "' has an impossible shape");
    elems *= d;
  }
  const int64_t bs = (int64_t)block_size(ti.dtype);
  if (elems % bs != 0)
    fail("the number of elements " + std::to_string(elems) + " is not divisible by the block size " +
         std::to_string(bs));
  const uint64_t bytes = (uint64_t)(elems / bs) * type_size(ti.dtype);
  const uint64_t start = header.tensor_data_offset + ti.offset, size = file_size(f);
  if (start < header.tensor_data_offset || bytes > size - std::min(size, start))
    fail("tensor needs " + std::to_string(bytes) + " bytes at offset " + std::to_string(start) + ", only " +
         std::to_string(size - std::min(size, start)) + " remaining in file");
  std::vector<uint8_t> raw((size_t)bytes);
  seek(f, start);
  read_exact(f, raw.data(), raw.size());
  // qtensor_from_ggml: QTensor dims are [..., rows, cols]; a 1-D tensor is one row
  std::vector<int64_t> dims = ti.shape;
  if (dims.empty()) dims = {1};
  if (dims.size() == 1) dims.insert(dims.begin(), 1);
  return QTensor::from_data(raw.data(), raw.size(), dims, ti.dtype, device);
}

std::string peek_architecture(FILE *f) {
  Reader r{f, 0, Version::V3};
  const uint64_t start = tell(f);
  r.size = file_size(f);
  seek(f, start);
  r.version = read_magic(f);
  (void)r.length();  // tensor count
  if (r.length() == 0 || r.string() != "general.architecture") return "";
  if (value_type_from_u32(rd<uint32_t>(f)) != ValueType::String) return "";
  return r.string();
}

std::vector<uint8_t> metadata_bytes(const std::vector<std::pair<std::string, Value>> &metadata) {
  std::vector<uint8_t> o;
  for (const auto &kv : metadata) {
    write_string(o, kv.first);
    wr<uint32_t>(o, (uint32_t)kv.second.type);
    write_value(o, kv.second);
  }
  return o;
}

void write_raw(FILE *f, uint64_t kv_count, const std::vector<uint8_t> &kv_bytes,
               const std::vector<std::pair<std::string, std::shared_ptr<QTensor>>> &tensors) {
  std::vector<uint8_t> h;
  wr<uint32_t>(h, 0x46554747u);
  wr<uint32_t>(h, 2);  // version 2, as the reference writes
  wr<uint64_t>(h, tensors.size());
  wr<uint64_t>(h, kv_count);
  wr(h, kv_bytes.data(), kv_bytes.size());
  uint64_t offset = 0;
  for (const auto &t : tensors) {
    write_string(h, t.first);
    const std::vector<int64_t> &dims = t.second->shape();
    wr<uint32_t>(h, (uint32_t)dims.size());
    for (size_t d = dims.size(); d-- > 0;) wr<uint64_t>(h, (uint64_t)dims[d]);  // innermost first
    wr<uint32_t>(h, (uint32_t)t.second->dtype());
    wr<uint64_t>(h, offset);
    const size_t n = t.second->storage_size_in_bytes();
    offset += n + padding(n);
  }
  h.resize(h.size() + padding(h.size()), 0);
  put(f, h.data(), h.size());
  static const uint8_t zeros[32] = {0};
  for (const auto &t : tensors) {
    const std::vector<uint8_t> data = t.second->data();
    put(f, data.data(), data.size());
    put(f, zeros, padding(data.size()));
  }
  if (fflush(f) != 0) fail("write failed");
}

void write(FILE *f, const std::vector<std::pair<std::string, Value>> &metadata,
           const std::vector<std::pair<std::string, std::shared_ptr<QTensor>>> &tensors) {
  write_raw(f, metadata.size(), metadata_bytes(metadata), tensors);
}

}  // namespace gguf
}  // namespace inference_rs_amd
