// GGUF container reader and the file-level GGUF -> MLX snapshot convert.
//
// Reader: src/gguf/reader.rs:180-298 (header, typed metadata, tensor table,
// aligned data section; v2/v3, ne reversed to torch order).  Convert:
// src/gguf/convert.rs:89-186 (remap keys, dequantize, q/k un-permute, bf16,
// requantize projections, rebuild config.json) over the device kernels of
// this library: each tensor's blocks are uploaded once and decoded on the
// GPU; projections take the fused requantize kernel when quantizing.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <set>
#include <sstream>

#include "mlxq.hpp"

namespace mlxq {
namespace gguf {
namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kDefaultAlignment = 32;

// GGUF metadata value-type tags (the on-disk format)
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kString = 8, kArray = 9,
  kU64 = 10, kI64 = 11, kF64 = 12
};

[[noreturn]] void msg(const std::string& m) { throw Error(Error::Kind::Msg, m); }
[[noreturn]] void unsupported(const std::string& m) { throw Error(Error::Kind::Unsupported, m); }

// Bounds-checked little-endian reads over the image (reader.rs:300-390).
struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;

  const uint8_t* take(uint64_t k) {
    if (k > n - pos) msg("gguf: unexpected end of file");
    const uint8_t* r = p + pos;
    pos += static_cast<size_t>(k);
    return r;
  }
  template <typename T>
  T le() {
    const uint8_t* b = take(sizeof(T));
    T v = 0;
    for (size_t i = 0; i < sizeof(T); i++) v |= static_cast<T>(static_cast<T>(b[i]) << (8 * i));
    return v;
  }
  std::string str() {
    const uint64_t len = le<uint64_t>();
    const uint8_t* b = take(len);
    std::string s(reinterpret_cast<const char*>(b), static_cast<size_t>(len));
    if (!valid_utf8(s)) msg("gguf: bad utf-8 string");
    return s;
  }
  static bool valid_utf8(const std::string& s) {
    size_t i = 0;
    while (i < s.size()) {
      const unsigned char c = static_cast<unsigned char>(s[i]);
      int extra;
      uint32_t cp;
      if (c < 0x80) { extra = 0; cp = c; }
      else if ((c & 0xE0) == 0xC0) { extra = 1; cp = c & 0x1F; }
      else if ((c & 0xF0) == 0xE0) { extra = 2; cp = c & 0x0F; }
      else if ((c & 0xF8) == 0xF0) { extra = 3; cp = c & 0x07; }
      else return false;
      for (int k = 1; k <= extra; k++) {
        if (i + k >= s.size()) return false;
        const unsigned char cc = static_cast<unsigned char>(s[i + k]);
        if ((cc & 0xC0) != 0x80) return false;
        cp = (cp << 6) | (cc & 0x3F);
      }
      // overlong forms, surrogates and values past U+10FFFF are not UTF-8
      static const uint32_t kMin[4] = {0, 0x80, 0x800, 0x10000};
      if (cp < kMin[extra] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
      i += extra + 1;
    }
    return true;
  }
  MetaValue value(uint32_t t) {
    MetaValue v;
    switch (t) {
      case kU8: v.type = MetaValue::Type::U8; v.u = le<uint8_t>(); break;
      case kI8: v.type = MetaValue::Type::I8; v.i = static_cast<int8_t>(le<uint8_t>()); break;
      case kU16: v.type = MetaValue::Type::U16; v.u = le<uint16_t>(); break;
      case kI16: v.type = MetaValue::Type::I16; v.i = static_cast<int16_t>(le<uint16_t>()); break;
      case kU32: v.type = MetaValue::Type::U32; v.u = le<uint32_t>(); break;
      case kI32: v.type = MetaValue::Type::I32; v.i = static_cast<int32_t>(le<uint32_t>()); break;
      case kF32: {
        const uint32_t b = le<uint32_t>();
        float f;
        std::memcpy(&f, &b, 4);
        v.type = MetaValue::Type::F32;
        v.f = f;
        break;
      }
      case kBool: v.type = MetaValue::Type::Bool; v.u = le<uint8_t>() != 0; break;
      case kString: v.type = MetaValue::Type::String; v.s = str(); break;
      case kU64: v.type = MetaValue::Type::U64; v.u = le<uint64_t>(); break;
      case kI64: v.type = MetaValue::Type::I64; v.i = static_cast<int64_t>(le<uint64_t>()); break;
      case kF64: {
        const uint64_t b = le<uint64_t>();
        std::memcpy(&v.f, &b, 8);
        v.type = MetaValue::Type::F64;
        break;
      }
      case kArray: {
        const uint32_t et = le<uint32_t>();
        if (et == kArray) unsupported("gguf: nested metadata arrays");
        const uint64_t len = le<uint64_t>();
        v.type = MetaValue::Type::Array;
        // every element takes at least one byte: a count past the end of
        // the image is a truncated file, not an allocation
        if (len > n - pos) msg("gguf: unexpected end of file");
        v.arr.reserve(static_cast<size_t>(len));
        for (uint64_t k = 0; k < len; k++) v.arr.push_back(value(et));
        break;
      }
      default: msg("gguf: unknown metadata value type " + std::to_string(t));
    }
    return v;
  }
};

// Shortest decimal that reads back as the same double (serde_json prints
// floats this way).
std::string json_number(double v) {
  if (!std::isfinite(v)) msg("gguf: non-finite metadata value in config");
  char buf[40];
  for (int prec = 1; prec <= 17; prec++) {
    std::snprintf(buf, sizeof buf, "%.*g", prec, v);
    if (std::strtod(buf, nullptr) == v) break;
  }
  std::string s = buf;
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";  // stays a float in JSON readers
  return s;
}

std::string json_string(const std::string& s) {
  std::string o = "\"";
  for (const char ch : s) {
    const unsigned char c = static_cast<unsigned char>(ch);
    if (c == '"' || c == '\\') {
      o += '\\';
      o += ch;
    } else if (c < 0x20) {
      char b[8];
      std::snprintf(b, sizeof b, "\\u%04x", c);
      o += b;
    } else {
      o += ch;
    }
  }
  return o + "\"";
}

// Rows of a [out, in] bf16 tensor gathered back from llama.cpp's q/k order
// (convert.rs:232-256): HF row r = k*(hd/2) + j of a head is GGUF row 2j + k.
std::vector<uint8_t> permute_inverse_qk_rows(const std::vector<uint8_t>& src, int64_t out, int64_t in, int n_head,
                                             size_t elem) {
  if (n_head <= 0 || out % n_head)
    msg("gguf: q/k permute: out " + std::to_string(out) + " not divisible by n_head " + std::to_string(n_head));
  const int64_t hd = out / n_head;
  if (hd % 2) msg("gguf: q/k permute: odd head_dim " + std::to_string(hd));
  const int64_t half = hd / 2;
  const size_t row = static_cast<size_t>(in) * elem;
  std::vector<uint8_t> res(src.size());
  for (int64_t h = 0; h < n_head; h++)
    for (int64_t r = 0; r < hd; r++) {
      const int64_t k = r / half, j = r % half;
      std::memcpy(res.data() + (h * hd + r) * row, src.data() + (h * hd + 2 * j + k) * row, row);
    }
  return res;
}

}  // namespace

// ---------------------------------------------------------------- values

std::optional<uint64_t> MetaValue::as_u64() const {
  switch (type) {
    case Type::U8: case Type::U16: case Type::U32: case Type::U64: case Type::Bool: return u;
    case Type::I8: case Type::I16: case Type::I32: case Type::I64:
      if (i >= 0) return static_cast<uint64_t>(i);
      return std::nullopt;
    default: return std::nullopt;
  }
}

std::optional<int64_t> MetaValue::as_i64() const {
  switch (type) {
    case Type::U8: case Type::U16: case Type::U32: case Type::U64: return static_cast<int64_t>(u);
    case Type::I8: case Type::I16: case Type::I32: case Type::I64: return i;
    default: return std::nullopt;
  }
}

std::optional<double> MetaValue::as_f64() const {
  if (type == Type::F32 || type == Type::F64) return f;
  return std::nullopt;
}

std::optional<std::string> MetaValue::as_str() const {
  if (type == Type::String) return s;
  return std::nullopt;
}

std::optional<bool> MetaValue::as_bool() const {
  if (type == Type::Bool) return u != 0;
  return std::nullopt;
}

const std::vector<MetaValue>* MetaValue::as_array() const { return type == Type::Array ? &arr : nullptr; }

int64_t TensorInfo::num_elements() const {
  // checked: the count sizes the tensor's data range and the dequantize call
  int64_t n = 1;
  for (int64_t d : shape) {
    if (d < 0 || (d > 0 && n > INT64_MAX / d)) msg("gguf: tensor too large: " + name);
    n *= d;
  }
  return n;
}

// ---------------------------------------------------------------- file

GgufFile GgufFile::parse(std::vector<uint8_t> bytes) {
  GgufFile g;
  auto owned = std::make_shared<std::vector<uint8_t>>(std::move(bytes));
  g.size_ = owned->size();
  g.base_ = std::shared_ptr<const uint8_t>(owned, owned->data());
  g.parse_header();
  return g;
}

GgufFile GgufFile::open(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) msg("gguf: read " + path + ": " + std::strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    msg("gguf: read " + path + ": " + std::strerror(errno));
  }
  const size_t n = static_cast<size_t>(st.st_size);
  GgufFile g;
  if (n == 0) {
    ::close(fd);
    return parse({});
  }
  void* p = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) msg("gguf: map " + path + ": " + std::strerror(errno));
  g.size_ = n;
  g.base_ = std::shared_ptr<const uint8_t>(static_cast<const uint8_t*>(p), [n](const uint8_t* q) {
    munmap(const_cast<uint8_t*>(q), n);
  });
  g.parse_header();
  return g;
}

void GgufFile::parse_header() {
  Reader c{base_.get(), size_};
  const uint32_t magic = c.le<uint32_t>();
  if (magic != kMagic) {
    char b[80];
    std::snprintf(b, sizeof b, "gguf: bad magic 0x%08x (expected 0x%08x)", magic, kMagic);
    msg(b);
  }
  const uint32_t version = c.le<uint32_t>();
  if (version < 2 || version > 3)
    unsupported("gguf version " + std::to_string(version) + " (only v2/v3 are supported)");
  const uint64_t tensor_count = c.le<uint64_t>();
  const uint64_t metadata_count = c.le<uint64_t>();
  for (uint64_t k = 0; k < metadata_count; k++) {
    std::string key = c.str();
    const uint32_t vt = c.le<uint32_t>();
    metadata[std::move(key)] = c.value(vt);  // a repeated key keeps the last value (a map insert)
  }
  // each tensor entry takes at least 28 bytes: a count beyond the image is
  // a truncated or corrupt header, not a reservation
  if (tensor_count > (size_ - c.pos) / 28 + 1) msg("gguf: unexpected end of file");
  tensors.reserve(static_cast<size_t>(tensor_count));
  for (uint64_t k = 0; k < tensor_count; k++) {
    TensorInfo t;
    t.name = c.str();
    const uint32_t n_dims = c.le<uint32_t>();
    if (n_dims == 0 || n_dims > 4)
      msg("gguf: tensor \"" + t.name + "\" has " + std::to_string(n_dims) + " dims (expected 1..=4)");
    std::vector<int64_t> ne(n_dims);
    for (uint32_t d = 0; d < n_dims; d++) {
      const uint64_t v = c.le<uint64_t>();
      if (v > (uint64_t(1) << 62)) msg("gguf: tensor \"" + t.name + "\" dimension too large");
      ne[d] = static_cast<int64_t>(v);
    }
    t.shape.assign(ne.rbegin(), ne.rend());  // GGML ne is fastest-axis-first: torch order is reversed
    t.ggml_type = c.le<uint32_t>();
    t.offset = c.le<uint64_t>();
    tensors.push_back(std::move(t));
  }
  alignment = kDefaultAlignment;
  if (const MetaValue* a = meta("general.alignment"))
    if (auto v = a->as_u64()) alignment = *v;
  if (alignment == 0) alignment = 1;
  const uint64_t header_end = c.pos;
  data_start = (header_end + alignment - 1) / alignment * alignment;
  // a metadata-only file may end before the aligned boundary
  if (!tensors.empty() && data_start > size_) msg("gguf: data section starts past end of file");
}

const MetaValue* GgufFile::meta(const std::string& key) const {
  auto it = metadata.find(key);
  return it == metadata.end() ? nullptr : &it->second;
}

std::optional<std::string> GgufFile::meta_str(const std::string& key) const {
  const MetaValue* v = meta(key);
  return v ? v->as_str() : std::nullopt;
}

std::optional<uint64_t> GgufFile::meta_u64(const std::string& key) const {
  const MetaValue* v = meta(key);
  return v ? v->as_u64() : std::nullopt;
}

std::optional<double> GgufFile::meta_f64(const std::string& key) const {
  const MetaValue* v = meta(key);
  return v ? v->as_f64() : std::nullopt;
}

std::pair<const uint8_t*, size_t> GgufFile::tensor_data(const TensorInfo& info) const {
  for (int64_t d : info.shape)
    if (d < 0) msg("gguf: tensor \"" + info.name + "\" has a negative dimension");
  const size_t nbytes = tensor_byte_len(info.ggml_type, static_cast<size_t>(info.num_elements()));
  if (info.offset > UINT64_MAX - data_start) msg("gguf: tensor offset overflow");
  const uint64_t start = data_start + info.offset;
  if (nbytes > UINT64_MAX - start) msg("gguf: tensor length overflow");
  const uint64_t end = start + nbytes;
  if (end > size_)
    msg("gguf: tensor \"" + info.name + "\" data [" + std::to_string(start) + ".." + std::to_string(end) +
        "] out of range (file " + std::to_string(size_) + " bytes)");
  return {base_.get() + start, nbytes};
}

// ---------------------------------------------------------------- convert

std::optional<std::string> remap_key(const std::string& name) {
  if (name == "token_embd.weight") return "model.embed_tokens.weight";
  if (name == "output_norm.weight") return "model.norm.weight";
  if (name == "output.weight") return "lm_head.weight";
  if (name.rfind("blk.", 0) != 0) return std::nullopt;
  const size_t dot = name.find('.', 4);
  if (dot == std::string::npos || dot == 4) return std::nullopt;
  const std::string idx = name.substr(4, dot - 4), suffix = name.substr(dot + 1);
  // the index must parse as a usize (Rust's parse: an optional '+', then
  // digits, no overflow); the key keeps the index text as written
  size_t d0 = idx[0] == '+' ? 1 : 0;
  if (d0 == idx.size()) return std::nullopt;
  uint64_t v = 0;
  for (size_t k = d0; k < idx.size(); k++) {
    const char ch = idx[k];
    if (ch < '0' || ch > '9') return std::nullopt;
    if (v > (UINT64_MAX - (ch - '0')) / 10) return std::nullopt;
    v = v * 10 + (ch - '0');
  }
  static const std::pair<const char*, const char*> kMap[] = {
      {"attn_q.weight", "self_attn.q_proj.weight"},
      {"attn_k.weight", "self_attn.k_proj.weight"},
      {"attn_v.weight", "self_attn.v_proj.weight"},
      {"attn_output.weight", "self_attn.o_proj.weight"},
      {"attn_norm.weight", "input_layernorm.weight"},
      {"ffn_norm.weight", "post_attention_layernorm.weight"},
      {"ffn_gate.weight", "mlp.gate_proj.weight"},
      {"ffn_up.weight", "mlp.up_proj.weight"},
      {"ffn_down.weight", "mlp.down_proj.weight"},
      {"attn_q_norm.weight", "self_attn.q_norm.weight"},
      {"attn_k_norm.weight", "self_attn.k_norm.weight"},
  };
  for (const auto& [g, h] : kMap)
    if (suffix == g) return "model.layers." + idx + "." + h;
  return std::nullopt;
}

bool is_ignorable(const std::string& name) {
  const std::string s = ".rope_freqs.weight";
  return name == "rope_freqs.weight" ||
         (name.size() >= s.size() && name.compare(name.size() - s.size(), s.size(), s) == 0);
}

namespace {

bool ends_with(const std::string& s, const std::string& t) {
  return s.size() >= t.size() && s.compare(s.size() - t.size(), t.size(), t) == 0;
}

// config.json from the metadata table (convert.rs:264-360)
std::string reconstruct_config(const GgufFile& g, const std::string& arch, const std::string& model_type,
                               const std::string& hf_arch, int64_t vocab, bool tied) {
  auto key = [&](const std::string& s) { return arch + "." + s; };
  auto req = [&](const std::string& s) -> int64_t {
    auto v = g.meta_u64(key(s));
    if (!v) msg("gguf: missing metadata " + key(s));
    return static_cast<int64_t>(*v);
  };
  const int64_t hidden = req("embedding_length"), blocks = req("block_count"), heads = req("attention.head_count");
  const int64_t kv_heads = static_cast<int64_t>(g.meta_u64(key("attention.head_count_kv")).value_or(heads));
  const int64_t ffn = req("feed_forward_length");
  if (heads == 0) msg("gguf: attention.head_count is 0");
  const int64_t head_dim = static_cast<int64_t>(g.meta_u64(key("attention.key_length")).value_or(hidden / heads));
  const double eps = g.meta_f64(key("attention.layer_norm_rms_epsilon")).value_or(1e-5);
  const double theta = g.meta_f64(key("rope.freq_base")).value_or(10000.0);
  const int64_t context = static_cast<int64_t>(g.meta_u64(key("context_length")).value_or(0));

  std::ostringstream o;
  o << "{\"architectures\": [" << json_string(hf_arch) << "], \"model_type\": " << json_string(model_type)
    << ", \"hidden_size\": " << hidden << ", \"intermediate_size\": " << ffn << ", \"num_hidden_layers\": " << blocks
    << ", \"num_attention_heads\": " << heads << ", \"num_key_value_heads\": " << kv_heads
    << ", \"head_dim\": " << head_dim << ", \"vocab_size\": " << vocab << ", \"rms_norm_eps\": " << json_number(eps)
    << ", \"rope_theta\": " << json_number(theta) << ", \"tie_word_embeddings\": " << (tied ? "true" : "false");
  if (context > 0) o << ", \"max_position_embeddings\": " << context;
  if (auto eos = g.meta_u64("tokenizer.ggml.eos_token_id")) o << ", \"eos_token_id\": " << static_cast<int64_t>(*eos);
  if (auto bos = g.meta_u64("tokenizer.ggml.bos_token_id")) o << ", \"bos_token_id\": " << static_cast<int64_t>(*bos);
  // llama3 RoPE scaling (convert.rs:339-360)
  const auto low = g.meta_f64(key("rope.scaling.low_freq_factor"));
  const auto high = g.meta_f64(key("rope.scaling.high_freq_factor"));
  const auto stype = g.meta_str(key("rope.scaling.type"));
  if ((stype && *stype == "llama3") || low || high) {
    const double factor = g.meta_f64(key("rope.scaling.factor")).value_or(8.0);
    const double orig = static_cast<double>(g.meta_u64(key("rope.scaling.original_context_length")).value_or(8192));
    o << ", \"rope_scaling\": {\"rope_type\": \"llama3\", \"factor\": " << json_number(factor)
      << ", \"low_freq_factor\": " << json_number(low.value_or(1.0))
      << ", \"high_freq_factor\": " << json_number(high.value_or(4.0))
      << ", \"original_max_position_embeddings\": " << json_number(orig) << "}";
  }
  o << "}";
  return o.str();
}

}  // namespace

ConvertReport convert(const GgufFile& g, const std::string& out_dir, const ConvertOptions& opts) {
  const auto arch_v = g.meta_str("general.architecture");
  if (!arch_v) msg("gguf: missing general.architecture");
  const std::string arch = *arch_v;
  std::string model_type, hf_arch;
  if (arch == "llama") {
    model_type = "llama";
    hf_arch = "LlamaForCausalLM";
  } else if (arch == "qwen3") {
    model_type = "qwen3";
    hf_arch = "Qwen3ForCausalLM";
  } else {
    unsupported("GGUF architecture \"" + arch +
                "\" (engine supports llama/mistral and qwen3; mistral GGUFs are labelled \"llama\")");
  }
  const auto heads_v = g.meta_u64(arch + ".attention.head_count");
  if (!heads_v) msg("gguf: missing metadata " + arch + ".attention.head_count");
  const int num_heads = static_cast<int>(*heads_v);
  const int num_kv_heads = static_cast<int>(g.meta_u64(arch + ".attention.head_count_kv").value_or(*heads_v));
  const bool permute_qk = arch == "llama";  // llama.cpp interleaves q/k rows for the NORM RoPE

  // every unmapped tensor is an error before any work (convert.rs:140-147)
  std::vector<std::string> unmapped;
  for (const TensorInfo& t : g.tensors)
    if (!remap_key(t.name) && !is_ignorable(t.name)) unmapped.push_back(t.name);
  if (!unmapped.empty()) {
    std::string list;
    for (size_t i = 0; i < unmapped.size(); i++) list += (i ? ", " : "") + unmapped[i];
    unsupported("gguf: " + std::to_string(unmapped.size()) +
                " tensor(s) with no transformer-key mapping (would be silently dropped): " + list);
  }

  snapshot::Tensors out;
  // a repeated tensor name replaces the earlier one (the reference collects
  // the converted tensors in a HashMap, convert.rs:121-137), so the
  // snapshot never holds a key twice
  auto put = [&out](const std::string& name, Array a) {
    for (auto& kv : out)
      if (kv.first == name) {
        kv.second = std::move(a);
        return;
      }
    out.emplace_back(name, std::move(a));
  };
  std::set<std::string> seen;
  int64_t vocab = -1;
  for (const TensorInfo& t : g.tensors) {
    const auto key = remap_key(t.name);
    if (!key) continue;
    const auto [ptr, nbytes] = g.tensor_data(t);
    const int64_t n = t.num_elements();
    const int heads = ends_with(*key, "self_attn.q_proj.weight") ? num_heads
                      : ends_with(*key, "self_attn.k_proj.weight") ? num_kv_heads
                                                                   : 0;
    const int perm = permute_qk ? heads : 0;
    if (*key == "model.embed_tokens.weight") vocab = t.shape.at(0);
    seen.insert(*key);
    const Array blocks = Array::from_bytes(ptr, nbytes, {static_cast<int64_t>(nbytes)}, DType::U8);
    if (opts.quantize && snapshot::is_projection(*key)) {
      // dequantize -> un-permute -> bf16 -> quantize, one kernel (the
      // snapshot writer's requant of the reference's dense bf16 tensor)
      if (t.shape.size() != 2) msg("gguf: projection " + t.name + " is not 2-D");
      const QuantizedLinear q =
          requantize_projection(t.ggml_type, blocks, t.shape[0], t.shape[1], perm, *opts.quantize);
      const std::string base = key->substr(0, key->size() - std::strlen(".weight"));
      put(base + ".weight", q.weight);
      put(base + ".scales", q.scales);
      put(base + ".biases", q.biases);
    } else {
      Array dense = dequantize(t.ggml_type, blocks, static_cast<size_t>(n), DType::BF16);
      if (perm) {
        const int64_t rows = t.shape.at(0), cols = n / std::max<int64_t>(rows, 1);
        const std::vector<uint8_t> host = permute_inverse_qk_rows(dense.to_bytes(), rows, cols, perm, 2);
        dense = Array::from_bytes(host.data(), host.size(), t.shape, DType::BF16);
      }
      put(*key, dense.reshape(t.shape));  // the snapshot stores the torch shape
    }
  }
  if (vocab < 0) msg("gguf: no token embedding tensor");
  const bool tied = !seen.count("lm_head.weight");
  const std::string config = reconstruct_config(g, arch, model_type, hf_arch, vocab, tied);
  const snapshot::Report r = snapshot::write_parts(out_dir, out, config, opts.quantize, opts.tokenizer_json);

  ConvertReport rep;
  rep.architecture = arch;
  rep.model_type = model_type;
  rep.num_tensors = r.num_tensors;
  rep.quantized = r.quantized;
  rep.out_dir = r.out_dir;
  rep.tokenizer = opts.tokenizer_json ? "written from the given tokenizer.json"
                                      : "not reconstructed from the GGUF metadata (pass a tokenizer.json)";
  return rep;
}

ConvertReport convert_file(const std::string& gguf_path, const std::string& out_dir, const ConvertOptions& opts) {
  return convert(GgufFile::open(gguf_path), out_dir, opts);
}

}  // namespace gguf
}  // namespace mlxq
