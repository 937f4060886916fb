// C++ host API over the C ABI (include/mlxq.h), mirroring the reference
// crate's interface for the quantized-weight path so that a C++ caller, and
// the tests in tests/cpp/, read like the reference's own Rust:
//
//   mlxq::QuantSpec            <- primitives::projection::QuantSpec (src/primitives/projection.rs:15-31)
//   mlxq::QuantizedLinear      <- primitives::quant::QuantizedLinear (src/primitives/quant.rs:20-82)
//   mlxq::Projection           <- primitives::projection::Projection (src/primitives/projection.rs:36-104)
//   mlxq::gguf::GgmlType, block, tensor_byte_len, dequantize
//                              <- gguf::dequant (src/gguf/dequant.rs:31-211)
//   mlxq::gguf::requantize_projection
//                              <- the per-projection chain of gguf::convert (src/gguf/convert.rs:131-176)
//   mlxq::gguf::GgufFile, MetaValue, TensorInfo
//                              <- gguf::reader (src/gguf/reader.rs:39-298)
//   mlxq::gguf::convert, convert_file, remap_key
//                              <- gguf::convert (src/gguf/convert.rs:80-262, 264-360)
//   mlxq::snapshot::write_snapshot, save/load_safetensors, load_projection
//                              <- snapshot::write_snapshot (src/snapshot.rs:86-148) and the
//                                 pre-quantized loader branch (src/models/llama.rs:81-95)
//   mlxq::Error                <- error::Error (src/error.rs:10-45): Device for the
//                                 MLX-op failures, Unsupported, Msg
//
// mlxq::Array stands in for mlx_rs::Array: a reference-counted device buffer
// with a shape and a dtype.  Like MLX, the operations allocate their
// outputs; unlike MLX they run eagerly, in order, on the thread's current
// HIP stream (set_stream), and host reads synchronize that stream.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace mlxq {

class Error : public std::runtime_error {
 public:
  enum class Kind { Device, Unsupported, Msg };
  Error(Kind kind, const std::string& what) : std::runtime_error(what), kind_(kind) {}
  Kind kind() const { return kind_; }

 private:
  Kind kind_;
};

enum class DType { F32, F16, BF16, U32, U8 };
size_t dtype_size(DType t);

// Stream used by every operation of this thread (default: the null stream).
void set_stream(hipStream_t s);
hipStream_t stream();

class Array {
 public:
  Array() = default;
  Array(std::vector<int64_t> shape, DType dtype);  // uninitialised device storage

  // host data -> device.  from_f32 converts to `dtype` (F32 or BF16, round to
  // nearest even) on the host.
  static Array from_f32(const std::vector<float>& v, std::vector<int64_t> shape, DType dtype = DType::F32);
  static Array from_bytes(const void* data, size_t nbytes, std::vector<int64_t> shape, DType dtype);

  std::vector<float> to_f32() const;  // device -> host (F32 / F16 / BF16), synchronizes the stream
  std::vector<uint8_t> to_bytes() const;

  // The same storage under another shape of the same element count.
  Array reshape(std::vector<int64_t> shape) const;

  const std::vector<int64_t>& shape() const { return shape_; }
  int64_t dim(int i) const { return shape_.at(i < 0 ? shape_.size() + i : i); }
  DType dtype() const { return dtype_; }
  int64_t size() const;  // elements
  size_t nbytes() const { return static_cast<size_t>(size()) * dtype_size(dtype_); }
  void* data() const { return buf_.get(); }
  bool empty() const { return !buf_; }

 private:
  std::shared_ptr<void> buf_;
  std::vector<int64_t> shape_;
  DType dtype_ = DType::F32;
};

struct QuantSpec {
  int group_size;
  int bits;
  static QuantSpec q4() { return {64, 4}; }
  static QuantSpec q8() { return {64, 8}; }
  bool operator==(const QuantSpec& o) const { return group_size == o.group_size && bits == o.bits; }
};

struct QuantizedLinear {
  Array weight;   // packed codes, U32 [out, in*bits/32]
  Array scales;   // per-group scales [out, in/group_size], the weight's dtype
  Array biases;   // per-group biases (zero points), same
  int group_size = 64;
  int bits = 4;
  std::optional<Array> bias;  // optional additive [out] bias, BF16

  // Quantize a dense [out, in] weight (F32 or BF16).
  static QuantizedLinear quantize(const Array& weight, int group_size, int bits, std::optional<Array> bias = {});
  // x @ dequant(weight).T (+ bias); x BF16 [..., in] -> BF16 [..., out].
  Array forward(const Array& x) const;
  // The dense weight, in the scales' dtype.
  Array dequantize_weight() const;
};

class Projection {
 public:
  // A dense [out, in] weight, quantized if `quant` is set.
  static Projection load(Array weight, std::optional<QuantSpec> quant);
  static Projection load_with_bias(Array weight, std::optional<Array> bias, std::optional<QuantSpec> quant);
  // Already-quantized parts (a snapshot's weight / scales / biases), used as-is.
  static Projection from_quantized(Array weight, Array scales, Array biases, QuantSpec spec);
  // x @ weight.T (+ bias).  Dense projections stay on the caller's dense
  // GEMM: this library has none, and raises Unsupported for them.
  Array forward(const Array& x) const;
  bool is_quantized() const { return q_.has_value(); }
  const QuantizedLinear& quantized() const { return *q_; }

 private:
  std::optional<QuantizedLinear> q_;
  Array dense_weight_;
  std::optional<Array> dense_bias_;
};

namespace gguf {

enum class GgmlType : uint32_t {
  F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q2K = 10, Q3K = 11, Q4K = 12, Q5K = 13,
  Q6K = 14, Iq2Xxs = 16, Iq2Xs = 17, Iq3Xxs = 18, Iq1S = 19, Iq4Nl = 20, Iq3S = 21, Iq2S = 22, Iq4Xs = 23,
  Iq1M = 29, BF16 = 30
};

GgmlType from_tag(uint32_t tag);                    // Error::Unsupported for other tags
std::pair<size_t, size_t> block(GgmlType t);        // (elements per block, bytes per block)
size_t tensor_byte_len(uint32_t tag, size_t num_elements);
// The reference's host signature: raw block bytes in host memory -> f32
// values in host memory (through the device kernels).
std::vector<float> dequantize(uint32_t tag, const uint8_t* data, size_t data_len, size_t num_elements);
// Device form: block bytes already in device memory -> `out` (F32 or BF16).
Array dequantize(uint32_t tag, const Array& data, size_t num_elements, DType out = DType::F32);
// One projection tensor of a GGUF file straight to MLX affine parts:
// dequantize, undo llama's q/k row permutation (permute_heads > 0), round to
// bf16, quantize -- in one kernel, bit-identical with that chain.
QuantizedLinear requantize_projection(uint32_t tag, const Array& data, int64_t rows, int64_t cols,
                                      int permute_heads, QuantSpec spec);

// ---- GGUF container (src/gguf/reader.rs) ----

// A typed metadata value (reader.rs:39-134).  Integers keep their width and
// signedness in `type`; as_* follow the reference's conversions.
struct MetaValue {
  enum class Type { U8, I8, U16, I16, U32, I32, U64, I64, F32, F64, Bool, String, Array };
  Type type = Type::U8;
  uint64_t u = 0;  // unsigned and bool payloads
  int64_t i = 0;   // signed payloads
  double f = 0;    // float payloads (F32 widened exactly)
  std::string s;
  std::vector<MetaValue> arr;

  std::optional<uint64_t> as_u64() const;  // any integer >= 0, bool
  std::optional<int64_t> as_i64() const;   // any integer
  std::optional<double> as_f64() const;    // F32 / F64
  std::optional<std::string> as_str() const;
  std::optional<bool> as_bool() const;
  const std::vector<MetaValue>* as_array() const;
};

// One tensor of the header (reader.rs:137-156): shape in torch order (GGML
// `ne` reversed), GGML type tag, offset into the data section.
struct TensorInfo {
  std::string name;
  std::vector<int64_t> shape;
  uint32_t ggml_type = 0;
  uint64_t offset = 0;
  int64_t num_elements() const;
};

// A parsed GGUF file (reader.rs:158-298): v2/v3 only (v1 -> Unsupported),
// metadata, tensor table, data section at `general.alignment` (default 32).
// open() maps the file read-only instead of reading it whole.
class GgufFile {
 public:
  static GgufFile open(const std::string& path);
  static GgufFile parse(std::vector<uint8_t> bytes);

  const MetaValue* meta(const std::string& key) const;
  std::optional<std::string> meta_str(const std::string& key) const;
  std::optional<uint64_t> meta_u64(const std::string& key) const;
  std::optional<double> meta_f64(const std::string& key) const;
  // The tensor's raw block bytes (length from its type and element count);
  // Msg error when they run past the end of the file.
  std::pair<const uint8_t*, size_t> tensor_data(const TensorInfo& info) const;

  std::map<std::string, MetaValue> metadata;
  std::vector<TensorInfo> tensors;
  uint64_t alignment = 32;
  uint64_t data_start = 0;

 private:
  void parse_header();
  std::shared_ptr<const uint8_t> base_;  // the image (owned vector or mapping)
  size_t size_ = 0;
};

// ---- GGUF -> MLX snapshot (src/gguf/convert.rs) ----

// GGML tensor name -> transformer key (convert.rs:213-242); nullopt for
// names the engine does not load.
std::optional<std::string> remap_key(const std::string& name);
// Tensors the engine recomputes (rope frequencies; convert.rs:258-262).
bool is_ignorable(const std::string& name);

struct ConvertOptions {
  std::optional<QuantSpec> quantize;        // requantize the projections
  std::optional<std::string> tokenizer_json;  // written verbatim when given
};

struct ConvertReport {
  std::string architecture, model_type;
  size_t num_tensors = 0;
  std::optional<QuantSpec> quantized;
  std::string tokenizer;  // what happened to the tokenizer (not rebuilt from GGUF metadata here)
  std::string out_dir;
};

// convert.rs:89-186.  Each mapped tensor's blocks go to the device once:
// with `quantize`, projections run the fused requantize kernel (dequantize,
// llama q/k un-permute, bf16, MLX affine quantize); every other tensor is
// dequantized to bf16 (q/k of an unquantized llama conversion then have
// their rows un-permuted).  Errors as the reference: Unsupported for another
// architecture or an unmapped tensor, Msg for missing metadata.
ConvertReport convert(const GgufFile& g, const std::string& out_dir, const ConvertOptions& opts);
ConvertReport convert_file(const std::string& gguf_path, const std::string& out_dir, const ConvertOptions& opts);

}  // namespace gguf

// Quantized snapshot I/O (src/snapshot.rs): MLX's on-disk layout of a
// quantized projection -- `{base}.weight` U32 codes, `{base}.scales` and
// `{base}.biases` -- in a standard safetensors file, plus the `quantization`
// block of config.json that marks the snapshot pre-quantized.
namespace snapshot {

using Tensors = std::vector<std::pair<std::string, Array>>;

// snapshot.rs:41-54
bool is_projection(const std::string& key);

struct Report {  // snapshot.rs:68-77
  size_t num_tensors = 0;
  std::optional<QuantSpec> quantized;
  std::string out_dir;
};

// snapshot.rs:86-148: projections (by key) cast to bf16 and re-quantized when
// `quantize` is set, every other tensor written through; config_json must be
// a JSON object (the quantization block is added to it); tokenizer files are
// written verbatim when given.
Report write_snapshot(const std::string& out_dir, const Tensors& tensors, const std::string& config_json,
                      std::optional<QuantSpec> quantize, const std::optional<std::string>& tokenizer_json = {},
                      const std::optional<std::string>& tokenizer_config_json = {});

// The writing half of write_snapshot: `tensors` already in their stored form
// (projections as packed parts when `quantized` is set), which are written
// with config.json (plus the quantization block) and the tokenizer files.
Report write_parts(const std::string& out_dir, const Tensors& tensors, const std::string& config_json,
                   std::optional<QuantSpec> quantized, const std::optional<std::string>& tokenizer_json = {},
                   const std::optional<std::string>& tokenizer_config_json = {});

void save_safetensors(const std::string& path, const Tensors& tensors);
Tensors load_safetensors(const std::string& path);

// The pre-quantized loader branch (src/models/llama.rs:81-95): a projection
// from the snapshot's `{base}.weight/.scales/.biases`.
Projection load_projection(const Tensors& tensors, const std::string& base, QuantSpec spec);

}  // namespace snapshot
}  // namespace mlxq
