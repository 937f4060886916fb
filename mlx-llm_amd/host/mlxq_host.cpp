// C++ host API over the C ABI (declarations and reference mapping in
// mlxq.hpp).  Every device operation goes through the entry points of
// include/mlxq.h; this file only manages buffers, shapes and errors.
#include "mlxq.hpp"

#include <cstring>
#include <map>
#include <mutex>

#include "mlxq.h"

namespace mlxq {
namespace {

thread_local hipStream_t g_stream = nullptr;

[[noreturn]] void raise_status(int rc, const std::string& where) {
  const std::string msg = where + ": " + mlxq_last_error();
  if (rc == MLXQ_ERR_UNSUPPORTED) throw Error(Error::Kind::Unsupported, msg);
  if (rc == MLXQ_ERR_DEVICE) throw Error(Error::Kind::Device, msg);
  throw Error(Error::Kind::Msg, msg);
}

void check(int rc, const char* where) {
  if (rc != MLXQ_OK) raise_status(rc, where);
}

void check_hip(hipError_t e, const char* where) {
  if (e != hipSuccess) throw Error(Error::Kind::Device, std::string(where) + ": " + hipGetErrorString(e));
}

int abi_dtype(DType t) {
  switch (t) {
    case DType::F32: return MLXQ_F32;
    case DType::F16: return MLXQ_F16;
    case DType::BF16: return MLXQ_BF16;
    default: throw Error(Error::Kind::Unsupported, "dtype has no C ABI code");
  }
}

uint16_t f32_to_bf16(float f) {  // round to nearest even; NaN stays NaN
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float bf16_to_f32(uint16_t h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

float f16_to_f32(uint16_t h) {
  const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = s << 31;
    } else {  // subnormal: normalise
      int k = -1;
      uint32_t mm = m;
      do {
        k++;
        mm <<= 1;
      } while (!(mm & 0x400u));
      u = (s << 31) | ((127 - 15 - k) << 23) | ((mm & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    u = (s << 31) | 0x7F800000u | (m << 13);
  } else {
    u = (s << 31) | ((e + 127 - 15) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// x as BF16 (a host round trip for other dtypes: the slow path of callers
// that keep f32 activations; the kernels take bf16)
Array as_bf16(const Array& a) {
  if (a.dtype() == DType::BF16) return a;
  if (a.dtype() != DType::F32 && a.dtype() != DType::F16) throw Error(Error::Kind::Unsupported, "expected a float array");
  return Array::from_f32(a.to_f32(), a.shape(), DType::BF16);
}

// qmatmul workspace of the calling device, grown on demand and kept (work
// queued on the stream may still use an outgrown one until it completes,
// so the old buffer is retired only after a stream synchronization).
std::mutex g_ws_mutex;
std::map<int, Array> g_ws;

Array workspace(size_t bytes) {
  if (!bytes) return Array();
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Array& ws = g_ws[dev];
  if (ws.empty() || ws.nbytes() < bytes) {
    if (!ws.empty()) check_hip(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
    ws = Array({static_cast<int64_t>(bytes)}, DType::U8);
  }
  return ws;
}

}  // namespace

size_t dtype_size(DType t) {
  switch (t) {
    case DType::F32: case DType::U32: return 4;
    case DType::F16: case DType::BF16: return 2;
    case DType::U8: return 1;
  }
  return 1;
}

void set_stream(hipStream_t s) { g_stream = s; }
hipStream_t stream() { return g_stream; }

// ------------------------------------------------------------------ Array

Array::Array(std::vector<int64_t> shape, DType dtype) : shape_(std::move(shape)), dtype_(dtype) {
  for (int64_t d : shape_)
    if (d < 0) throw Error(Error::Kind::Msg, "Array: negative dimension");
  void* p = nullptr;
  check_hip(hipMalloc(&p, std::max<size_t>(nbytes(), 1)), "hipMalloc");
  buf_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
}

Array Array::reshape(std::vector<int64_t> shape) const {
  Array r = *this;
  r.shape_ = std::move(shape);
  if (r.size() != size()) throw Error(Error::Kind::Msg, "reshape: element count differs");
  return r;
}

int64_t Array::size() const {
  int64_t n = 1;
  for (int64_t d : shape_) n *= d;
  return n;
}

Array Array::from_bytes(const void* data, size_t nbytes, std::vector<int64_t> shape, DType dtype) {
  Array a(std::move(shape), dtype);
  if (nbytes != a.nbytes()) throw Error(Error::Kind::Msg, "Array::from_bytes: size does not match the shape");
  check_hip(hipMemcpyAsync(a.data(), data, nbytes, hipMemcpyHostToDevice, g_stream), "hipMemcpyAsync");
  check_hip(hipStreamSynchronize(g_stream), "hipStreamSynchronize");  // the host buffer may go away
  return a;
}

Array Array::from_f32(const std::vector<float>& v, std::vector<int64_t> shape, DType dtype) {
  if (dtype == DType::F32) return from_bytes(v.data(), v.size() * 4, std::move(shape), dtype);
  if (dtype != DType::BF16) throw Error(Error::Kind::Unsupported, "Array::from_f32: F32 or BF16 only");
  std::vector<uint16_t> h(v.size());
  for (size_t i = 0; i < v.size(); i++) h[i] = f32_to_bf16(v[i]);
  return from_bytes(h.data(), h.size() * 2, std::move(shape), dtype);
}

std::vector<uint8_t> Array::to_bytes() const {
  std::vector<uint8_t> out(nbytes());
  if (!out.empty()) {
    check_hip(hipMemcpyAsync(out.data(), data(), out.size(), hipMemcpyDeviceToHost, g_stream), "hipMemcpyAsync");
    check_hip(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
  }
  return out;
}

std::vector<float> Array::to_f32() const {
  const std::vector<uint8_t> b = to_bytes();
  std::vector<float> out(static_cast<size_t>(size()));
  if (dtype_ == DType::F32) {
    std::memcpy(out.data(), b.data(), b.size());
  } else if (dtype_ == DType::BF16 || dtype_ == DType::F16) {
    for (size_t i = 0; i < out.size(); i++) {
      uint16_t h;
      std::memcpy(&h, b.data() + 2 * i, 2);
      out[i] = dtype_ == DType::BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    }
  } else {
    throw Error(Error::Kind::Unsupported, "Array::to_f32: not a float array");
  }
  return out;
}

// ------------------------------------------------------------------ QuantizedLinear

QuantizedLinear QuantizedLinear::quantize(const Array& weight, int group_size, int bits, std::optional<Array> bias) {
  if (weight.shape().size() != 2) throw Error(Error::Kind::Msg, "quantize: weight must be [out, in]");
  const int64_t rows = weight.dim(0), cols = weight.dim(1);
  QuantizedLinear q;
  q.group_size = group_size;
  q.bits = bits;
  q.bias = std::move(bias);
  if (bits != 4 && bits != 8) throw Error(Error::Kind::Unsupported, "quantize: bits must be 4 or 8");
  if (group_size <= 0 || cols % group_size)
    throw Error(Error::Kind::Msg, "quantize: group_size must divide the input dimension");
  q.weight = Array({rows, cols * bits / 32}, DType::U32);
  q.scales = Array({rows, cols / group_size}, weight.dtype());
  q.biases = Array({rows, cols / group_size}, weight.dtype());
  check(mlxq_quantize(weight.data(), abi_dtype(weight.dtype()), rows, cols, group_size, bits,
                      static_cast<uint32_t*>(q.weight.data()), q.scales.data(), q.biases.data(), g_stream),
        "quantize");
  return q;
}

Array QuantizedLinear::forward(const Array& x) const {
  const int64_t n = scales.dim(0), k = scales.dim(1) * group_size;
  if (x.dim(-1) != k) throw Error(Error::Kind::Msg, "forward: x's last dimension is not the input dimension");
  const Array xb = as_bf16(x);
  const Array sb = as_bf16(scales), bb = as_bf16(biases);
  std::optional<Array> bias_b;
  if (bias) bias_b = as_bf16(*bias);
  const int64_t m = x.size() / k;
  std::vector<int64_t> yshape = x.shape();
  yshape.back() = n;
  Array y(yshape, DType::BF16);
  size_t wsb = 0;
  check(mlxq_qmatmul_workspace_size(m, n, k, group_size, bits, &wsb), "forward");
  const Array ws = workspace(wsb);
  check(mlxq_qmatmul(xb.data(), m, static_cast<const uint32_t*>(weight.data()), sb.data(), bb.data(),
                     bias_b ? bias_b->data() : nullptr, n, k, group_size, bits, y.data(), ws.empty() ? nullptr : ws.data(),
                     ws.empty() ? 0 : ws.nbytes(), g_stream),
        "forward");
  return y;
}

Array QuantizedLinear::dequantize_weight() const {
  const int64_t rows = scales.dim(0), cols = scales.dim(1) * group_size;
  Array out({rows, cols}, scales.dtype());
  check(mlxq_dequantize(static_cast<const uint32_t*>(weight.data()), scales.data(), biases.data(),
                        abi_dtype(scales.dtype()), rows, cols, group_size, bits, out.data(), g_stream),
        "dequantize_weight");
  return out;
}

// ------------------------------------------------------------------ Projection

Projection Projection::load(Array weight, std::optional<QuantSpec> quant) {
  return load_with_bias(std::move(weight), std::nullopt, quant);
}

Projection Projection::load_with_bias(Array weight, std::optional<Array> bias, std::optional<QuantSpec> quant) {
  Projection p;
  if (quant) {
    p.q_ = QuantizedLinear::quantize(weight, quant->group_size, quant->bits, std::move(bias));
  } else {
    p.dense_weight_ = std::move(weight);
    p.dense_bias_ = std::move(bias);
  }
  return p;
}

Projection Projection::from_quantized(Array weight, Array scales, Array biases, QuantSpec spec) {
  Projection p;
  QuantizedLinear q;
  q.weight = std::move(weight);
  q.scales = std::move(scales);
  q.biases = std::move(biases);
  q.group_size = spec.group_size;
  q.bits = spec.bits;
  p.q_ = std::move(q);
  return p;
}

Array Projection::forward(const Array& x) const {
  if (q_) return q_->forward(x);
  throw Error(Error::Kind::Unsupported, "Projection::forward: dense projections use the caller's dense GEMM");
}

// ------------------------------------------------------------------ gguf

namespace gguf {

GgmlType from_tag(uint32_t tag) {
  int64_t e = 0, b = 0;
  check(mlxq_gguf_block(tag, &e, &b), "gguf");
  return static_cast<GgmlType>(tag);
}

std::pair<size_t, size_t> block(GgmlType t) {
  int64_t e = 0, b = 0;
  check(mlxq_gguf_block(static_cast<uint32_t>(t), &e, &b), "gguf");
  return {static_cast<size_t>(e), static_cast<size_t>(b)};
}

size_t tensor_byte_len(uint32_t tag, size_t num_elements) {
  int64_t bytes = 0;
  check(mlxq_gguf_tensor_byte_len(tag, static_cast<int64_t>(num_elements), &bytes), "gguf");
  return static_cast<size_t>(bytes);
}

Array dequantize(uint32_t tag, const Array& data, size_t num_elements, DType out) {
  Array y({static_cast<int64_t>(num_elements)}, out);
  check(mlxq_gguf_dequantize(tag, data.data(), static_cast<int64_t>(data.nbytes()), static_cast<int64_t>(num_elements),
                             abi_dtype(out), y.data(), g_stream),
        "gguf");
  return y;
}

std::vector<float> dequantize(uint32_t tag, const uint8_t* data, size_t data_len, size_t num_elements) {
  from_tag(tag);  // the reference checks the tag first (Unsupported)
  const size_t need = tensor_byte_len(tag, num_elements);
  if (data_len < need)
    throw Error(Error::Kind::Msg, "gguf: needs " + std::to_string(need) + " bytes for " +
                                      std::to_string(num_elements) + " elements, got " + std::to_string(data_len));
  const Array d = Array::from_bytes(data, need, {static_cast<int64_t>(need)}, DType::U8);
  return dequantize(tag, d, num_elements, DType::F32).to_f32();
}

QuantizedLinear requantize_projection(uint32_t tag, const Array& data, int64_t rows, int64_t cols, int permute_heads,
                                      QuantSpec spec) {
  QuantizedLinear q;
  q.group_size = spec.group_size;
  q.bits = spec.bits;
  if (spec.group_size <= 0 || cols % spec.group_size)
    throw Error(Error::Kind::Msg, "requantize: group_size must divide the column count");
  q.weight = Array({rows, cols * spec.bits / 32}, DType::U32);
  q.scales = Array({rows, cols / spec.group_size}, DType::BF16);
  q.biases = Array({rows, cols / spec.group_size}, DType::BF16);
  check(mlxq_gguf_requantize(tag, data.data(), static_cast<int64_t>(data.nbytes()), rows, cols, permute_heads,
                             spec.group_size, spec.bits, static_cast<uint32_t*>(q.weight.data()), q.scales.data(),
                             q.biases.data(), g_stream),
        "requantize");
  return q;
}

}  // namespace gguf
}  // namespace mlxq
