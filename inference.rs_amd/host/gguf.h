// GGUF container I/O for the QTensor host layer: the reader and writer of
// crates/inference-tensor/src/quantized/gguf_file.rs (Header::read / read_summary 598-705, Value::read 330-392,
// large arrays 506-546 and 707-735, Content::read / tensor 764-812, TensorInfo::read 92-126, write_header /
// write_tensor_data / metadata_bytes / write 814-895).  Tensors load into QTensor (QStorage::from_data) on the CPU or
// a HIP device.  Every malformed input throws Error; nothing is read past what the header's own checks allow.
#pragma once

#include <stdint.h>
#include <stdio.h>

#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "qtensor.h"

namespace inference_rs_amd {
namespace gguf {

// the reader's caps (gguf_file.rs:16-24)
constexpr uint64_t kMaxStringLength = 1ull << 30;
constexpr uint64_t kMaxArrayElements = 1ull << 30;
constexpr uint64_t kInlineArrayElements = 1ull << 20;  // longer arrays of fixed-size values are located, not parsed
constexpr uint64_t kSummaryArrayElements = 64;          // read_summary skips longer arrays
constexpr uint32_t kMaxTensorDims = 8;
constexpr int kMaxValueDepth = 64;
constexpr uint64_t kDefaultAlignment = 32;

// ValueType and its on-disk ids (gguf_file.rs:168-196, 394-435)
enum class ValueType : uint32_t {
  U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, Bool = 7, String = 8, Array = 9, U64 = 10, I64 = 11,
  F64 = 12,
};
ValueType value_type_from_u32(uint32_t v);  // throws on an unknown id

enum class Version { V1 = 1, V2 = 2, V3 = 3 };

// Value (gguf_file.rs:198-327): one typed metadata value; the accessors take exactly their own type, except to_u64,
// which also upcasts u8 / u16 / u32 / bool as the reference's does.
struct Value {
  ValueType type = ValueType::U32;
  uint64_t u = 0;  // U8 .. U64, Bool
  int64_t i = 0;   // I8 .. I64
  double f = 0;    // F32 (exactly representable), F64
  std::string s;
  std::vector<Value> array;

  static Value make_u8(uint8_t v);
  static Value make_i8(int8_t v);
  static Value make_u16(uint16_t v);
  static Value make_i16(int16_t v);
  static Value make_u32(uint32_t v);
  static Value make_i32(int32_t v);
  static Value make_u64(uint64_t v);
  static Value make_i64(int64_t v);
  static Value make_f32(float v);
  static Value make_f64(double v);
  static Value make_bool(bool v);
  static Value make_string(std::string v);
  static Value make_array(std::vector<Value> v);

  uint8_t to_u8() const;
  int8_t to_i8() const;
  uint16_t to_u16() const;
  int16_t to_i16() const;
  uint32_t to_u32() const;
  int32_t to_i32() const;
  uint64_t to_u64() const;
  int64_t to_i64() const;
  float to_f32() const;
  double to_f64() const;
  bool to_bool() const;
  const std::string &to_string() const;
  const std::vector<Value> &to_vec() const;
};

// A metadata array left in the file: len values of value_type from byte offset (gguf_file.rs:128-134)
struct LargeArray {
  ValueType value_type;
  uint64_t len, offset;
};

// A tensor's table entry with the raw GGML type id; shape outermost first (the file stores it innermost first)
struct RawTensorInfo {
  uint32_t ggml_dtype = 0;
  std::vector<int64_t> shape;
  uint64_t offset = 0;
};

// Everything before the tensor data (gguf_file.rs:585-705)
struct Header {
  Version version = Version::V3;
  std::map<std::string, Value> metadata;
  std::map<std::string, LargeArray> large_arrays;
  std::map<std::string, RawTensorInfo> tensor_infos;
  std::vector<std::string> tensor_order;  // the table's order
  uint64_t tensor_data_offset = 0;
  uint64_t metadata_begin = 0, metadata_end = 0;  // where the metadata entries lie in the file

  // Header::read / read_summary: from the stream's current position; summary skips metadata arrays longer than
  // kSummaryArrayElements
  static Header read(FILE *f, bool summary = false);
  // the raw little-endian bytes of elements [begin, end) of a large array (read_large_array, 707-724)
  std::vector<uint8_t> read_large_array(FILE *f, const std::string &name, uint64_t begin, uint64_t end) const;
};

// Content (gguf_file.rs:764-812): the header with every tensor's type resolved to a GgmlDType this library knows
struct TensorInfo {
  GgmlDType dtype;
  std::vector<int64_t> shape;
  uint64_t offset;
};
struct Content {
  Header header;
  std::map<std::string, TensorInfo> tensor_infos;

  static Content read(FILE *f);
  // TensorInfo::read + qtensor_from_ggml: the tensor's bytes into a QTensor on `device` (dims outermost first)
  std::shared_ptr<QTensor> tensor(FILE *f, const std::string &name, Device device) const;
};

// `general.architecture` when it is the first key (peek_architecture, 553-572); empty when it is not
std::string peek_architecture(FILE *f);

// metadata_bytes (867-877): the key/value entries as write_header takes them
std::vector<uint8_t> metadata_bytes(const std::vector<std::pair<std::string, Value>> &metadata);

// write (879-895): version 2, tensors 32-byte aligned, in the given order
void write(FILE *f, const std::vector<std::pair<std::string, Value>> &metadata,
           const std::vector<std::pair<std::string, std::shared_ptr<QTensor>>> &tensors);
// write_header + write_tensor_data with the metadata already serialized (826-865)
void write_raw(FILE *f, uint64_t kv_count, const std::vector<uint8_t> &kv_bytes,
               const std::vector<std::pair<std::string, std::shared_ptr<QTensor>>> &tensors);

}  // namespace gguf
}  // namespace inference_rs_amd
