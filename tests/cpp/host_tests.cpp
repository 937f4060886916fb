// The reference crate's own tests for the quantized-weight path, restated
// against the C++ host API (mlx-llm_amd/host/mlxq.hpp), which runs them on
// the GPU kernels.  Each case names the reference test it mirrors
// (file:line); the inputs and expected values are the reference's.
//
//   host_tests           run every case, print one line per case, exit 1 on any failure
//   host_tests --list    print the case names only (touches no GPU)
//   host_tests --cpu     run only the cases that touch no GPU (host parsing and checks)
//   host_tests --copy-safetensors IN OUT   load IN, save it as OUT
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>
#include <algorithm>
#include <functional>
#include <string>
#include <vector>

#include <unistd.h>

#include "mlxq.hpp"

using mlxq::Array;
using mlxq::DType;
using mlxq::Error;
using mlxq::Projection;
using mlxq::QuantizedLinear;
using mlxq::QuantSpec;
namespace gguf = mlxq::gguf;

namespace {

struct Failure {
  std::string msg;
};

#define EXPECT(cond)                                                                              \
  do {                                                                                            \
    if (!(cond)) throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond}; \
  } while (0)

template <typename F>
void expect_error(Error::Kind kind, F&& f) {
  try {
    f();
  } catch (const Error& e) {
    if (e.kind() != kind) throw Failure{std::string("wrong error kind: ") + e.what()};
    return;
  }
  throw Failure{"expected an error"};
}

// IEEE half of a small set of exactly representable values (the tests' d
// scales): sign, exponent, mantissa assembled from the float's bits.
uint16_t f16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  const uint32_t s = u >> 31, e = (u >> 23) & 0xFF, m = u & 0x7FFFFF;
  if (f == 0.0f) return static_cast<uint16_t>(s << 15);
  return static_cast<uint16_t>((s << 15) | ((e - 127 + 15) << 10) | (m >> 13));
}

uint16_t bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return static_cast<uint16_t>(u >> 16);  // exact for the tests' values
}

void push16(std::vector<uint8_t>& b, uint16_t v) {
  b.push_back(static_cast<uint8_t>(v & 0xFF));
  b.push_back(static_cast<uint8_t>(v >> 8));
}

// ---------------------------------------------------------------- quant.rs

// quant.rs:91-107 quantize_dequantize_roundtrip_q8
void quantize_dequantize_roundtrip_q8() {
  const int n = 2 * 64;
  std::vector<float> data(n);
  for (int i = 0; i < n; i++) data[i] = static_cast<float>(i) / n - 0.5f;
  const Array w = Array::from_f32(data, {2, 64});
  const QuantizedLinear q = QuantizedLinear::quantize(w, 64, 8);
  const std::vector<float> back = q.dequantize_weight().to_f32();
  float max_err = 0.f;
  for (int i = 0; i < n; i++) max_err = std::fmax(max_err, std::fabs(data[i] - back[i]));
  EXPECT(max_err < 0.01f);
}

// quant.rs:109-125 quantized_matmul_approximates_linear_q8
void quantized_matmul_approximates_linear_q8() {
  const int n = 4 * 64;
  std::vector<float> wd(n), xd(64);
  for (int i = 0; i < n; i++) wd[i] = static_cast<float>(i * 7 % 13) / 13.0f - 0.5f;
  for (int i = 0; i < 64; i++) xd[i] = static_cast<float>(i) / 64.0f - 0.5f;
  const Array w = Array::from_f32(wd, {4, 64});
  const Array x = Array::from_f32(xd, {1, 64});
  std::vector<double> dense(4, 0.0);  // linear(x, w) = x @ w.T
  for (int o = 0; o < 4; o++)
    for (int k = 0; k < 64; k++) dense[o] += static_cast<double>(xd[k]) * wd[o * 64 + k];
  const QuantizedLinear q = QuantizedLinear::quantize(w, 64, 8);
  const std::vector<float> quant = q.forward(x).to_f32();
  EXPECT(quant.size() == 4);
  for (int o = 0; o < 4; o++) EXPECT(std::fabs(dense[o] - quant[o]) < 0.05);
}

// ---------------------------------------------------------------- projection.rs

// projection.rs:24-31 (QuantSpec::q4 / q8), :50-71 (load / load_with_bias),
// :76-90 (from_quantized), :93-103 (forward / is_quantized)
void projection_load_and_dispatch() {
  EXPECT((QuantSpec::q4() == QuantSpec{64, 4}));
  EXPECT((QuantSpec::q8() == QuantSpec{64, 8}));
  std::vector<float> wd(128 * 256), xd(3 * 256);
  for (size_t i = 0; i < wd.size(); i++) wd[i] = static_cast<float>((i * 37) % 101) / 101.0f - 0.5f;
  for (size_t i = 0; i < xd.size(); i++) xd[i] = static_cast<float>((i * 13) % 29) / 29.0f - 0.5f;
  const Array w = Array::from_f32(wd, {128, 256}, DType::BF16);
  const Array x = Array::from_f32(xd, {3, 256}, DType::BF16);

  const Projection dense = Projection::load(w, std::nullopt);
  EXPECT(!dense.is_quantized());
  expect_error(Error::Kind::Unsupported, [&] { dense.forward(x); });

  const Projection p = Projection::load(w, QuantSpec::q4());
  EXPECT(p.is_quantized());
  const std::vector<float> y = p.forward(x).to_f32();
  EXPECT(y.size() == 3u * 128u);
  const QuantizedLinear& q = p.quantized();
  const Projection r = Projection::from_quantized(q.weight, q.scales, q.biases, QuantSpec::q4());
  EXPECT(r.is_quantized());
  EXPECT(r.forward(x).to_f32() == y);  // the same parts give the same bits

  // against the dense product of the dequantized weight (f64), the qmatmul bar
  const std::vector<float> wdq = q.dequantize_weight().to_f32();
  const std::vector<float> xb = x.to_f32();
  double max_ref = 0.0, max_err = 0.0;
  for (int m = 0; m < 3; m++)
    for (int o = 0; o < 128; o++) {
      double ref = 0.0;
      for (int k = 0; k < 256; k++) ref += static_cast<double>(xb[m * 256 + k]) * wdq[o * 256 + k];
      max_ref = std::fmax(max_ref, std::fabs(ref));
      max_err = std::fmax(max_err, std::fabs(ref - y[m * 128 + o]));
    }
  EXPECT(max_err / max_ref <= 1e-2);

  // with a bias: y_bias - y = bias (up to the bf16 output rounding)
  std::vector<float> bd(128);
  for (int o = 0; o < 128; o++) bd[o] = static_cast<float>(o % 7) - 3.0f;
  const Projection pb = Projection::load_with_bias(w, Array::from_f32(bd, {128}, DType::BF16), QuantSpec::q4());
  const std::vector<float> yb = pb.forward(x).to_f32();
  for (int m = 0; m < 3; m++)
    for (int o = 0; o < 128; o++) EXPECT(std::fabs(yb[m * 128 + o] - (y[m * 128 + o] + bd[o])) <= 0.05);
}

// ---------------------------------------------------------------- dequant.rs

// dequant.rs:725-747 type_geometry_matches_llama_cpp
void type_geometry_matches_llama_cpp() {
  using T = gguf::GgmlType;
  const std::pair<T, std::pair<size_t, size_t>> cases[] = {
      {T::Q4_0, {32, 18}},    {T::Q4_1, {32, 20}},    {T::Q5_0, {32, 22}},    {T::Q5_1, {32, 24}},
      {T::Q8_0, {32, 34}},    {T::Q2K, {256, 84}},    {T::Q3K, {256, 110}},   {T::Q4K, {256, 144}},
      {T::Q5K, {256, 176}},   {T::Q6K, {256, 210}},   {T::Iq4Nl, {32, 18}},   {T::Iq4Xs, {256, 136}},
      {T::Iq2Xxs, {256, 66}}, {T::Iq2Xs, {256, 74}},  {T::Iq2S, {256, 82}},   {T::Iq3Xxs, {256, 98}},
      {T::Iq3S, {256, 110}},  {T::Iq1S, {256, 50}},   {T::Iq1M, {256, 56}},
  };
  for (const auto& c : cases) EXPECT(gguf::block(c.first) == c.second);
}

// dequant.rs:749-767 supported_and_unsupported_types
void supported_and_unsupported_types() {
  using T = gguf::GgmlType;
  EXPECT(gguf::from_tag(20) == T::Iq4Nl);
  EXPECT(gguf::from_tag(23) == T::Iq4Xs);
  EXPECT(gguf::from_tag(16) == T::Iq2Xxs);
  EXPECT(gguf::from_tag(17) == T::Iq2Xs);
  EXPECT(gguf::from_tag(18) == T::Iq3Xxs);
  EXPECT(gguf::from_tag(19) == T::Iq1S);
  EXPECT(gguf::from_tag(21) == T::Iq3S);
  EXPECT(gguf::from_tag(22) == T::Iq2S);
  EXPECT(gguf::from_tag(29) == T::Iq1M);
  EXPECT(gguf::tensor_byte_len(16, 256) == 66);
  expect_error(Error::Kind::Unsupported, [] { gguf::from_tag(9); });   // Q8_1 (intermediate)
  expect_error(Error::Kind::Unsupported, [] { gguf::from_tag(15); });  // Q8_K (intermediate)
  expect_error(Error::Kind::Unsupported, [] { gguf::tensor_byte_len(9, 256); });
}

// dequant.rs:769-780 iq4_nl_codebook_decode
void iq4_nl_codebook_decode() {
  std::vector<uint8_t> b;
  push16(b, f16_bits(2.0f));
  b.push_back(0x80);
  b.resize(2 + 16, 0x00);
  const std::vector<float> out = gguf::dequantize(20, b.data(), b.size(), 32);
  EXPECT(out[0] == 2.0f * -127.0f);
  EXPECT(out[16] == 2.0f * 1.0f);
  EXPECT(out[1] == 2.0f * -127.0f);
}

// dequant.rs:782-802 f32_f16_bf16_passthrough
void f32_f16_bf16_passthrough() {
  const std::vector<float> vals = {1.0f, -2.5f, 3.25f, 0.0f};
  std::vector<uint8_t> f32b(16), f16b, bf16b;
  std::memcpy(f32b.data(), vals.data(), 16);
  EXPECT(gguf::dequantize(0, f32b.data(), f32b.size(), 4) == vals);
  for (float v : vals) push16(f16b, f16_bits(v));
  EXPECT(gguf::dequantize(1, f16b.data(), f16b.size(), 4) == vals);
  for (float v : vals) push16(bf16b, bf16_bits(v));
  EXPECT(gguf::dequantize(30, bf16b.data(), bf16b.size(), 4) == vals);
}

// dequant.rs:805-816 q8_0_block_dequant
void q8_0_block_dequant() {
  std::vector<uint8_t> b;
  push16(b, f16_bits(0.5f));
  for (int q = 0; q < 32; q++) b.push_back(static_cast<uint8_t>(static_cast<int8_t>(q - 16)));
  const std::vector<float> out = gguf::dequantize(8, b.data(), b.size(), 32);
  for (int i = 0; i < 32; i++) EXPECT(std::fabs(out[i] - (i - 16) * 0.5f) < 1e-3f);
}

// dequant.rs:820-836 q4_0_zero_centered
void q4_0_zero_centered() {
  std::vector<uint8_t> b;
  push16(b, f16_bits(1.0f));
  b.resize(2 + 16, 0x88);
  for (float v : gguf::dequantize(2, b.data(), b.size(), 32)) EXPECT(v == 0.0f);
  std::vector<uint8_t> b2;
  push16(b2, f16_bits(1.0f));
  b2.push_back(0x8F);
  b2.resize(2 + 16, 0x88);
  const std::vector<float> out2 = gguf::dequantize(2, b2.data(), b2.size(), 32);
  EXPECT(out2[0] == 7.0f);
  EXPECT(out2[16] == 0.0f);
}

// dequant.rs:838-850 q2_k_scale_and_unpack
void q2_k_scale_and_unpack() {
  std::vector<uint8_t> b(16, 0x01);
  b.resize(16 + 64, 0xFF);
  push16(b, f16_bits(1.0f));
  push16(b, f16_bits(1.0f));
  for (float v : gguf::dequantize(10, b.data(), b.size(), 256)) EXPECT(v == 3.0f);
}

// dequant.rs:854-875 q6_k_centered_is_zero
void q6_k_centered_is_zero() {
  std::vector<uint8_t> b(210, 0);
  for (int i = 128; i < 192; i++) b[i] = 0xAA;
  for (int i = 192; i < 208; i++) b[i] = 5;
  const uint16_t d = f16_bits(1.0f);
  b[208] = static_cast<uint8_t>(d & 0xFF);
  b[209] = static_cast<uint8_t>(d >> 8);
  for (float v : gguf::dequantize(14, b.data(), b.size(), 256)) EXPECT(v == 0.0f);
}

// dequant.rs:877-882 iq_block_d1: f16 d = 1, then a zero payload
std::vector<uint8_t> iq_block_d1(size_t total) {
  std::vector<uint8_t> b;
  push16(b, f16_bits(1.0f));
  b.resize(total, 0);
  return b;
}

bool all_equal(const std::vector<float>& v, size_t from, size_t to, float x) {
  for (size_t i = from; i < to; i++)
    if (v[i] != x) return false;
  return true;
}

// dequant.rs:889-900
void iq2_xxs_grid_scale_and_offset() {
  const std::vector<float> out = gguf::dequantize(16, iq_block_d1(66).data(), 66, 256);
  EXPECT(all_equal(out, 0, 256, 1.0f));
  std::vector<uint8_t> b2 = iq_block_d1(66);
  b2[9] = 0x30;
  const std::vector<float> out2 = gguf::dequantize(16, b2.data(), b2.size(), 256);
  EXPECT(all_equal(out2, 0, 32, 7.0f));
  EXPECT(out2[32] == 1.0f);
}

// dequant.rs:904-910
void iq2_xs_and_s_grid_zero_decode() {
  EXPECT(all_equal(gguf::dequantize(17, iq_block_d1(74).data(), 74, 256), 0, 256, 1.0f));
  EXPECT(all_equal(gguf::dequantize(22, iq_block_d1(82).data(), 82, 256), 0, 256, 1.0f));
}

// dequant.rs:914-920
void iq3_xxs_and_s_grid_zero_decode() {
  EXPECT(all_equal(gguf::dequantize(18, iq_block_d1(98).data(), 98, 256), 0, 256, 1.0f));
  EXPECT(all_equal(gguf::dequantize(21, iq_block_d1(110).data(), 110, 256), 0, 256, 1.0f));
}

// dequant.rs:925-937
void iq1_s_signed_grid_and_scale() {
  EXPECT(all_equal(gguf::dequantize(19, iq_block_d1(50).data(), 50, 256), 0, 256, -0.875f));
  std::vector<uint8_t> b = iq_block_d1(50);
  b[35] = 0x10;
  const std::vector<float> out2 = gguf::dequantize(19, b.data(), b.size(), 256);
  EXPECT(all_equal(out2, 0, 32, -2.625f));
  EXPECT(out2[32] == -0.875f);
}

// dequant.rs:941-955
void iq1_m_packed_f16_scale() {
  std::vector<uint8_t> b(56, 0);
  b[53] = 0xC0;
  b[55] = 0x30;
  EXPECT(all_equal(gguf::dequantize(29, b.data(), b.size(), 256), 0, 256, -0.875f));
  const std::vector<uint8_t> zero(56, 0);
  EXPECT(all_equal(gguf::dequantize(29, zero.data(), zero.size(), 256), 0, 256, 0.0f));
}

// dequant.rs:159-171: element count not a multiple of the block, short data
void dequantize_errors() {
  std::vector<uint8_t> b(18 * 2, 0x88);
  expect_error(Error::Kind::Msg, [&] { gguf::dequantize(2, b.data(), b.size(), 48); });
  expect_error(Error::Kind::Msg, [&] { gguf::dequantize(2, b.data(), b.size(), 96); });
  expect_error(Error::Kind::Msg, [&] { gguf::tensor_byte_len(12, 100); });
  expect_error(Error::Kind::Unsupported, [&] { gguf::dequantize(9, b.data(), b.size(), 32); });
}

// ---------------------------------------------------------------- convert.rs

// convert.rs:391-423 qk_permute_inverts_llama_cpp_forward, through the fused
// convert: GGUF rows in llama.cpp's q/k order come back in HF order.  A
// Q8_0 tensor whose row r holds the value r everywhere (d = 1): after the
// convert, HF row r must hold its source value in every column.
void requantize_projection_undoes_qk_permute() {
  const int n_head = 2, head_dim = 8, rows = n_head * head_dim, cols = 64;
  const int half = head_dim / 2;
  // GGUF row g of head h holds HF row k * half + j where g = 2 j + k
  std::vector<uint8_t> blocks;
  std::vector<int> hf_of_gguf(rows);
  for (int h = 0; h < n_head; h++)
    for (int k = 0; k < 2; k++)
      for (int j = 0; j < half; j++) hf_of_gguf[h * head_dim + 2 * j + k] = h * head_dim + k * half + j;
  for (int g = 0; g < rows; g++)
    for (int blk = 0; blk < cols / 32; blk++) {
      push16(blocks, f16_bits(1.0f));
      for (int i = 0; i < 32; i++) blocks.push_back(static_cast<uint8_t>(static_cast<int8_t>(hf_of_gguf[g] - 8)));
    }
  const Array data = Array::from_bytes(blocks.data(), blocks.size(), {static_cast<int64_t>(blocks.size())}, DType::U8);
  const QuantizedLinear q = gguf::requantize_projection(8, data, rows, cols, n_head, QuantSpec::q8());
  const std::vector<float> w = q.dequantize_weight().to_f32();
  for (int r = 0; r < rows; r++)
    for (int c = 0; c < cols; c++) EXPECT(std::fabs(w[r * cols + c] - static_cast<float>(r - 8)) < 1e-2f);
  // without the un-permute the rows keep the GGUF order
  const std::vector<float> w0 = gguf::requantize_projection(8, data, rows, cols, 0, QuantSpec::q8()).dequantize_weight().to_f32();
  bool differs = false;
  for (int r = 0; r < rows; r++) differs |= std::fabs(w0[r * cols] - static_cast<float>(hf_of_gguf[r] - 8)) < 1e-2f && hf_of_gguf[r] != r;
  EXPECT(differs);
}


// ---------------------------------------------------------------- snapshot.rs

namespace snapshot = mlxq::snapshot;

std::string tmp_dir(const char* label) {
  const char* t = std::getenv("TMPDIR");
  return std::string(t ? t : "/tmp") + "/mlxq-snapshot-" + label + "-" + std::to_string(getpid());
}

std::string read_text(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

// snapshot.rs:223-249 tiny_model: a two-layer tiny Llama tensor set (hidden
// 64, intermediate 128, q 64, kv 32, vocab 4), values uniform in [-0.2, 0.2)
// from a fixed xorshift stream.
snapshot::Tensors tiny_model() {
  const int64_t h = 64, v = 4, inter = 128, qd = 64, kvd = 32;
  uint64_t state = 0xABCDEFull;
  auto randn = [&](int64_t rows, int64_t cols) {
    std::vector<float> d(rows * cols);
    for (float& x : d) {
      state ^= state << 13;
      state ^= state >> 7;
      state ^= state << 17;
      x = (static_cast<float>(state >> 40) / 16777216.0f - 0.5f) * 0.4f;
    }
    return Array::from_f32(d, {rows, cols});
  };
  auto ones = [&](int64_t n) { return Array::from_f32(std::vector<float>(n, 1.0f), {n}); };
  snapshot::Tensors t;
  t.emplace_back("model.embed_tokens.weight", randn(v, h));
  t.emplace_back("model.norm.weight", ones(h));
  t.emplace_back("lm_head.weight", randn(v, h));
  for (int i = 0; i < 2; i++) {
    const std::string p = "model.layers." + std::to_string(i) + ".";
    t.emplace_back(p + "input_layernorm.weight", ones(h));
    t.emplace_back(p + "post_attention_layernorm.weight", ones(h));
    t.emplace_back(p + "self_attn.q_proj.weight", randn(qd, h));
    t.emplace_back(p + "self_attn.k_proj.weight", randn(kvd, h));
    t.emplace_back(p + "self_attn.v_proj.weight", randn(kvd, h));
    t.emplace_back(p + "self_attn.o_proj.weight", randn(h, qd));
    t.emplace_back(p + "mlp.gate_proj.weight", randn(inter, h));
    t.emplace_back(p + "mlp.up_proj.weight", randn(inter, h));
    t.emplace_back(p + "mlp.down_proj.weight", randn(h, inter));
  }
  return t;
}

const char* kTinyConfig =
    "{\"hidden_size\": 64, \"intermediate_size\": 128, \"num_hidden_layers\": 2, \"num_attention_heads\": 2, "
    "\"num_key_value_heads\": 1, \"vocab_size\": 4, \"rms_norm_eps\": 1e-5, \"rope_theta\": 10000.0, "
    "\"tie_word_embeddings\": false, \"eos_token_id\": 99}";

const Array* find(const snapshot::Tensors& t, const std::string& k) {
  for (const auto& e : t)
    if (e.first == k) return &e.second;
  return nullptr;
}

// snapshot.rs:251-270
void projection_predicate_selects_only_attn_mlp_projections() {
  for (const char* k : {"model.layers.0.self_attn.q_proj.weight", "model.layers.7.self_attn.o_proj.weight",
                        "model.layers.3.mlp.down_proj.weight"})
    EXPECT(snapshot::is_projection(k));
  for (const char* k : {"model.embed_tokens.weight", "lm_head.weight", "model.norm.weight",
                        "model.layers.0.input_layernorm.weight", "model.layers.0.self_attn.q_norm.weight"})
    EXPECT(!snapshot::is_projection(k));
}

// snapshot.rs:272-296: a dense write reloads every tensor bit-identical and
// adds no quantization block.
void dense_write_round_trips_bit_identical() {
  const std::string dir = tmp_dir("dense");
  const snapshot::Tensors tensors = tiny_model();
  const snapshot::Report r = snapshot::write_snapshot(dir, tensors, kTinyConfig, std::nullopt);
  EXPECT(!r.quantized.has_value());
  EXPECT(r.num_tensors == tensors.size());
  const snapshot::Tensors back = snapshot::load_safetensors(dir + "/model.safetensors");
  EXPECT(back.size() == tensors.size());
  for (const auto& [k, a] : tensors) {
    const Array* b = find(back, k);
    EXPECT(b != nullptr);
    EXPECT(b->dtype() == a.dtype() && b->shape() == a.shape());
    EXPECT(b->to_bytes() == a.to_bytes());
  }
  EXPECT(read_text(dir + "/config.json").find("quantization") == std::string::npos);
  std::filesystem::remove_all(dir);
}

// snapshot.rs:298-325: a quantized write stores each projection as packed
// weight / scales / biases, leaves embeddings dense, marks config.json, and
// the stored parts load as a quantized projection whose forward equals the
// in-memory quantization of the bf16 weight.
void quantized_write_loads_through_prequantized_branch() {
  const std::string dir = tmp_dir("q8");
  const snapshot::Tensors tensors = tiny_model();
  const QuantSpec spec = QuantSpec::q8();
  const snapshot::Report r =
      snapshot::write_snapshot(dir, tensors, kTinyConfig, spec, std::string("{\"model\": {}}"), std::nullopt);
  EXPECT(r.quantized.has_value() && *r.quantized == spec);
  EXPECT(r.num_tensors == 3 + 2 * 2 + 2 * 7 * 3);
  const snapshot::Tensors w = snapshot::load_safetensors(dir + "/model.safetensors");
  const std::string base = "model.layers.0.self_attn.q_proj";
  EXPECT(find(w, base + ".weight") && find(w, base + ".scales") && find(w, base + ".biases"));
  EXPECT(find(w, base + ".weight")->dtype() == DType::U32);
  EXPECT(find(w, base + ".scales")->dtype() == DType::BF16);
  EXPECT(!find(w, "model.embed_tokens.scales"));
  EXPECT(find(w, "model.embed_tokens.weight")->dtype() == DType::F32);
  const std::string cfg = read_text(dir + "/config.json");
  EXPECT(cfg.find("\"quantization\": {\"group_size\": 64, \"bits\": 8}") != std::string::npos);
  EXPECT(cfg.find("\"eos_token_id\": 99") != std::string::npos);
  EXPECT(read_text(dir + "/tokenizer.json") == "{\"model\": {}}");
  EXPECT(!std::filesystem::exists(dir + "/tokenizer_config.json"));

  const Projection p = snapshot::load_projection(w, base, spec);
  EXPECT(p.is_quantized());
  const Array* dense = find(tensors, base + ".weight");
  const Array wb = Array::from_f32(dense->to_f32(), dense->shape(), DType::BF16);
  const QuantizedLinear q = QuantizedLinear::quantize(wb, 64, 8);
  EXPECT(p.quantized().weight.to_bytes() == q.weight.to_bytes());
  EXPECT(p.quantized().scales.to_bytes() == q.scales.to_bytes());
  EXPECT(p.quantized().biases.to_bytes() == q.biases.to_bytes());
  std::vector<float> xv(3 * 64);
  for (size_t i = 0; i < xv.size(); i++) xv[i] = std::sin(0.37f * static_cast<float>(i));
  const Array x = Array::from_f32(xv, {3, 64}, DType::BF16);
  EXPECT(p.forward(x).to_bytes() == q.forward(x).to_bytes());
  expect_error(Error::Kind::Msg, [&] { snapshot::load_projection(w, "model.norm", spec); });
  expect_error(Error::Kind::Msg, [&] { snapshot::write_snapshot(dir, tensors, "[1, 2]", spec); });
  std::filesystem::remove_all(dir);
}


// ---------------------------------------------------------------- gguf/reader.rs

// A GGUF image builder (the reference's tests build their images the same
// way, reader.rs:397-430): little-endian header, metadata, tensor infos,
// padding to the data alignment, data.
struct GgufImage {
  std::vector<uint8_t> b;
  void u32(uint32_t v) {
    for (int i = 0; i < 4; i++) b.push_back(static_cast<uint8_t>(v >> (8 * i)));
  }
  void u64(uint64_t v) {
    for (int i = 0; i < 8; i++) b.push_back(static_cast<uint8_t>(v >> (8 * i)));
  }
  void str(const std::string& s) {
    u64(s.size());
    b.insert(b.end(), s.begin(), s.end());
  }
  void header(uint32_t version, uint64_t tensors, uint64_t meta) {
    u32(0x46554747u);
    u32(version);
    u64(tensors);
    u64(meta);
  }
  void pad(size_t align) {
    while (b.size() % align) b.push_back(0);
  }
};

// reader.rs:397-449 parse_minimal_gguf_roundtrip
void gguf_parse_minimal_roundtrip() {
  GgufImage g;
  g.header(3, 1, 2);
  g.str("general.architecture");
  g.u32(8);
  g.str("llama");
  g.str("llama.block_count");
  g.u32(4);
  g.u32(7);
  g.str("w");
  g.u32(2);
  g.u64(3);
  g.u64(2);
  g.u32(0);
  g.u64(0);
  g.pad(32);
  const float vals[6] = {1, 2, 3, 4, 5, 6};
  for (float v : vals) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    g.u32(u);
  }
  const gguf::GgufFile f = gguf::GgufFile::parse(g.b);
  EXPECT(f.meta_str("general.architecture") == std::string("llama"));
  EXPECT(f.meta_u64("llama.block_count") == uint64_t(7));
  EXPECT(f.tensors.size() == 1);
  const gguf::TensorInfo& t = f.tensors[0];
  EXPECT(t.name == "w");
  EXPECT((t.shape == std::vector<int64_t>{2, 3}));  // ne reversed
  EXPECT(t.num_elements() == 6);
  const auto [p, n] = f.tensor_data(t);
  EXPECT(n == 24);
  EXPECT(std::memcmp(p, vals, 24) == 0);
}

// reader.rs:451-459 rejects_bad_magic, :461-469 rejects_v1
void gguf_rejects_bad_magic_and_v1() {
  GgufImage bad;
  bad.u32(0xdeadbeefu);
  bad.u32(3);
  bad.u64(0);
  bad.u64(0);
  expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(bad.b); });
  GgufImage v1;
  v1.header(1, 0, 0);
  expect_error(Error::Kind::Unsupported, [&] { gguf::GgufFile::parse(v1.b); });
  GgufImage v4;
  v4.header(4, 0, 0);
  expect_error(Error::Kind::Unsupported, [&] { gguf::GgufFile::parse(v4.b); });
  GgufImage v2;  // v2 shares the u64 layout
  v2.header(2, 0, 0);
  EXPECT(gguf::GgufFile::parse(v2.b).tensors.empty());
}

// reader.rs:471-500 parses_int_and_float_and_array_metadata
void gguf_parses_int_float_array_metadata() {
  GgufImage g;
  g.header(3, 0, 3);
  g.str("a.f32");
  g.u32(6);
  const float f = 1.5f;
  uint32_t u;
  std::memcpy(&u, &f, 4);
  g.u32(u);
  g.str("a.i64");
  g.u32(11);
  g.u64(static_cast<uint64_t>(int64_t(-42)));
  g.str("a.arr");
  g.u32(9);
  g.u32(4);
  g.u64(2);
  g.u32(10);
  g.u32(20);
  const gguf::GgufFile h = gguf::GgufFile::parse(g.b);
  EXPECT(h.meta_f64("a.f32") == 1.5);
  EXPECT(h.meta("a.i64")->as_i64() == int64_t(-42));
  EXPECT(!h.meta("a.i64")->as_u64());  // a negative integer has no u64 reading
  const auto* arr = h.meta("a.arr")->as_array();
  EXPECT(arr && arr->size() == 2);
  EXPECT((*arr)[0].as_u64() == uint64_t(10) && (*arr)[1].as_u64() == uint64_t(20));
}

// The reader's error paths (reader.rs:206-211 dims, :240-244 data start,
// :282-298 tensor_data bounds, :321-329 truncation, :361-367 nested arrays,
// :375-377 unknown value types) and general.alignment (:231-236).
void gguf_reader_errors_and_alignment() {
  auto tensor_file = [](uint32_t n_dims, uint64_t offset, uint64_t align) {
    GgufImage g;
    g.header(3, 1, align ? 1 : 0);
    if (align) {
      g.str("general.alignment");
      g.u32(4);
      g.u32(static_cast<uint32_t>(align));
    }
    g.str("t");
    g.u32(n_dims);
    for (uint32_t d = 0; d < n_dims; d++) g.u64(4);
    g.u32(0);
    g.u64(offset);
    g.pad(align ? align : 32);
    for (int i = 0; i < 64; i++) g.u32(i);  // 256 bytes of data
    return g.b;
  };
  expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(tensor_file(0, 0, 0)); });
  expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(tensor_file(5, 0, 0)); });
  {  // 4x4 f32 = 64 bytes at offset 192 ends at 256: in range; at 200: not
    const gguf::GgufFile ok = gguf::GgufFile::parse(tensor_file(2, 192, 0));
    EXPECT(ok.tensor_data(ok.tensors[0]).second == 64);
    const gguf::GgufFile past = gguf::GgufFile::parse(tensor_file(2, 200, 0));
    expect_error(Error::Kind::Msg, [&] { past.tensor_data(past.tensors[0]); });
  }
  {  // general.alignment = 64 moves the data section to the next multiple of 64
    const gguf::GgufFile a = gguf::GgufFile::parse(tensor_file(1, 0, 64));
    EXPECT(a.alignment == 64 && a.data_start % 64 == 0);
    EXPECT(std::memcmp(a.tensor_data(a.tensors[0]).first, "\0\0\0\0\1\0\0\0", 8) == 0);
  }
  {  // truncated anywhere in the header
    const std::vector<uint8_t> full = tensor_file(2, 0, 0);
    for (size_t cut : {size_t(3), size_t(20), size_t(30), size_t(40)}) {
      std::vector<uint8_t> t(full.begin(), full.begin() + cut);
      expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(t); });
    }
  }
  {  // nested array: Unsupported; unknown value type: Msg; bad utf-8: Msg
    GgufImage g;
    g.header(3, 0, 1);
    g.str("n");
    g.u32(9);
    g.u32(9);
    g.u64(0);
    expect_error(Error::Kind::Unsupported, [&] { gguf::GgufFile::parse(g.b); });
    GgufImage h;
    h.header(3, 0, 1);
    h.str("x");
    h.u32(13);
    expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(h.b); });
    GgufImage k;
    k.header(3, 0, 1);
    k.str(std::string("\xC3\x28", 2));
    k.u32(0);
    k.b.push_back(1);
    expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(k.b); });
    GgufImage big;  // an array count far past the end of the image
    big.header(3, 0, 1);
    big.str("a");
    big.u32(9);
    big.u32(0);
    big.u64(uint64_t(1) << 60);
    expect_error(Error::Kind::Msg, [&] { gguf::GgufFile::parse(big.b); });
  }
  {  // a metadata-only file may end before the aligned boundary
    GgufImage g;
    g.header(3, 0, 1);
    g.str("k");
    g.u32(0);
    g.b.push_back(1);
    EXPECT(gguf::GgufFile::parse(g.b).meta_u64("k") == uint64_t(1));
  }
}

// ---------------------------------------------------------------- gguf/convert.rs

// convert.rs:366-371 remaps_non_layer_keys, :373-395 remaps_layer_keys,
// :425-432 unknown_keys_and_ignorables
void gguf_remap_keys_and_ignorables() {
  EXPECT(gguf::remap_key("token_embd.weight") == std::string("model.embed_tokens.weight"));
  EXPECT(gguf::remap_key("output_norm.weight") == std::string("model.norm.weight"));
  EXPECT(gguf::remap_key("output.weight") == std::string("lm_head.weight"));
  EXPECT(gguf::remap_key("blk.0.attn_q.weight") == std::string("model.layers.0.self_attn.q_proj.weight"));
  EXPECT(gguf::remap_key("blk.13.ffn_down.weight") == std::string("model.layers.13.mlp.down_proj.weight"));
  EXPECT(gguf::remap_key("blk.5.attn_norm.weight") == std::string("model.layers.5.input_layernorm.weight"));
  EXPECT(gguf::remap_key("blk.5.ffn_norm.weight") ==
         std::string("model.layers.5.post_attention_layernorm.weight"));
  EXPECT(gguf::remap_key("blk.2.attn_q_norm.weight") == std::string("model.layers.2.self_attn.q_norm.weight"));
  EXPECT(!gguf::remap_key("blk.0.some_future_tensor.weight"));
  EXPECT(!gguf::remap_key("rope_freqs.weight"));
  EXPECT(!gguf::remap_key("blk.x.attn_q.weight") && !gguf::remap_key("blk..attn_q.weight"));
  EXPECT(gguf::is_ignorable("rope_freqs.weight"));
  EXPECT(gguf::is_ignorable("blk.0.rope_freqs.weight"));
  EXPECT(!gguf::is_ignorable("blk.0.attn_q.weight"));
}

// convert.rs:96-147: unsupported architecture and unmapped tensors are
// refused before any tensor is decoded (host-only paths).
void gguf_convert_refuses_before_decoding() {
  GgufImage g;
  g.header(3, 0, 1);
  g.str("general.architecture");
  g.u32(8);
  g.str("gpt2");
  expect_error(Error::Kind::Unsupported, [&] { gguf::convert(gguf::GgufFile::parse(g.b), "/nonexistent", {}); });
  GgufImage h;
  h.header(3, 1, 2);
  h.str("general.architecture");
  h.u32(8);
  h.str("llama");
  h.str("llama.attention.head_count");
  h.u32(4);
  h.u32(2);
  h.str("blk.0.mystery.weight");
  h.u32(1);
  h.u64(4);
  h.u32(0);
  h.u64(0);
  h.pad(32);
  for (int i = 0; i < 4; i++) h.u32(0);
  expect_error(Error::Kind::Unsupported, [&] { gguf::convert(gguf::GgufFile::parse(h.b), "/nonexistent", {}); });
  GgufImage m;  // missing head count
  m.header(3, 0, 1);
  m.str("general.architecture");
  m.u32(8);
  m.str("llama");
  expect_error(Error::Kind::Msg, [&] { gguf::convert(gguf::GgufFile::parse(m.b), "/nonexistent", {}); });
}

// load_safetensors refuses malformed headers before sizing anything from
// them: negative dimensions, element counts that overflow, offsets outside
// the file or reversed.
void safetensors_rejects_malformed_headers() {
  const std::string dir = tmp_dir("st_bad");
  auto write = [&](const std::string& header, size_t data_bytes) {
    std::string h = header;
    while (h.size() % 8) h += ' ';
    std::ofstream f(dir + "/x.safetensors", std::ios::binary);
    const uint64_t n = h.size();
    for (int i = 0; i < 8; i++) f.put(static_cast<char>(n >> (8 * i)));
    f << h << std::string(data_bytes, '\0');
  };
  const std::pair<std::string, size_t> bad[] = {
      {R"({"t": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}})", 16},
      {R"({"t": {"dtype": "F32", "shape": [-2], "data_offsets": [8, 0]}})", 16},
      {R"({"t": {"dtype": "F32", "shape": [4611686018427387904, 4], "data_offsets": [0, 0]}})", 16},
      {R"({"t": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}})", 16},
      {R"({"t": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}})", 16},
      {R"({"t": {"dtype": "F32", "shape": [2], "data_offsets": [-8, 0]}})", 16},
  };
  for (const auto& [h, n] : bad) {
    write(h, n);
    expect_error(Error::Kind::Msg, [&] { mlxq::snapshot::load_safetensors(dir + "/x.safetensors"); });
  }
  std::filesystem::remove_all(dir);
}

}  // namespace

int main(int argc, char** argv) {
  const std::vector<std::pair<const char*, std::function<void()>>> cases = {
      {"quantize_dequantize_roundtrip_q8", quantize_dequantize_roundtrip_q8},
      {"quantized_matmul_approximates_linear_q8", quantized_matmul_approximates_linear_q8},
      {"projection_load_and_dispatch", projection_load_and_dispatch},
      {"type_geometry_matches_llama_cpp", type_geometry_matches_llama_cpp},
      {"supported_and_unsupported_types", supported_and_unsupported_types},
      {"iq4_nl_codebook_decode", iq4_nl_codebook_decode},
      {"f32_f16_bf16_passthrough", f32_f16_bf16_passthrough},
      {"q8_0_block_dequant", q8_0_block_dequant},
      {"q4_0_zero_centered", q4_0_zero_centered},
      {"q2_k_scale_and_unpack", q2_k_scale_and_unpack},
      {"q6_k_centered_is_zero", q6_k_centered_is_zero},
      {"dequantize_errors", dequantize_errors},
      {"iq2_xxs_grid_scale_and_offset", iq2_xxs_grid_scale_and_offset},
      {"iq2_xs_and_s_grid_zero_decode", iq2_xs_and_s_grid_zero_decode},
      {"iq3_xxs_and_s_grid_zero_decode", iq3_xxs_and_s_grid_zero_decode},
      {"iq1_s_signed_grid_and_scale", iq1_s_signed_grid_and_scale},
      {"iq1_m_packed_f16_scale", iq1_m_packed_f16_scale},
      {"requantize_projection_undoes_qk_permute", requantize_projection_undoes_qk_permute},
      {"projection_predicate_selects_only_attn_mlp_projections", projection_predicate_selects_only_attn_mlp_projections},
      {"dense_write_round_trips_bit_identical", dense_write_round_trips_bit_identical},
      {"quantized_write_loads_through_prequantized_branch", quantized_write_loads_through_prequantized_branch},
      {"gguf_parse_minimal_roundtrip", gguf_parse_minimal_roundtrip},
      {"gguf_rejects_bad_magic_and_v1", gguf_rejects_bad_magic_and_v1},
      {"gguf_parses_int_float_array_metadata", gguf_parses_int_float_array_metadata},
      {"gguf_reader_errors_and_alignment", gguf_reader_errors_and_alignment},
      {"gguf_remap_keys_and_ignorables", gguf_remap_keys_and_ignorables},
      {"gguf_convert_refuses_before_decoding", gguf_convert_refuses_before_decoding},
      {"safetensors_rejects_malformed_headers", safetensors_rejects_malformed_headers},
  };
  // cases that touch no GPU (run by the CPU test suite with --cpu)
  const std::vector<std::string> host_only = {
      "projection_predicate_selects_only_attn_mlp_projections", "gguf_parse_minimal_roundtrip",
      "gguf_rejects_bad_magic_and_v1", "gguf_parses_int_float_array_metadata", "gguf_reader_errors_and_alignment",
      "gguf_remap_keys_and_ignorables", "gguf_convert_refuses_before_decoding",
      "safetensors_rejects_malformed_headers"};
  const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
  if (argc == 4 && std::strcmp(argv[1], "--copy-safetensors") == 0) {
    // interop check driven from Python: read a file the safetensors package
    // wrote, write it back through this library
    mlxq::snapshot::save_safetensors(argv[3], mlxq::snapshot::load_safetensors(argv[2]));
    return 0;
  }
  if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
    for (const auto& c : cases) std::printf("%s\n", c.first);
    return 0;
  }
  int failed = 0;
  size_t ran = 0;
  for (const auto& c : cases) {
    if (cpu_only && std::find(host_only.begin(), host_only.end(), c.first) == host_only.end()) continue;
    ran++;
    try {
      c.second();
      std::printf("ok %s\n", c.first);
    } catch (const Failure& f) {
      failed++;
      std::printf("FAIL %s: %s\n", c.first, f.msg.c_str());
    } catch (const std::exception& e) {
      failed++;
      std::printf("FAIL %s: exception %s\n", c.first, e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%zu cases, %d failed\n", ran, failed);
  return failed ? 1 : 0;
}
