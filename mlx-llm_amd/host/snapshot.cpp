// Quantized snapshot I/O of the C++ host API (declarations and reference
// mapping in mlxq.hpp): a standard safetensors reader / writer and the
// snapshot writer's projection requant (src/snapshot.rs:86-148).
#include <cctype>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <sstream>

#include "mlxq.hpp"

namespace mlxq {
namespace snapshot {
namespace {

[[noreturn]] void msg(const std::string& m) { throw Error(Error::Kind::Msg, m); }

const char* dtype_name(DType t) {
  switch (t) {
    case DType::F32: return "F32";
    case DType::F16: return "F16";
    case DType::BF16: return "BF16";
    case DType::U32: return "U32";
    case DType::U8: return "U8";
  }
  return "U8";
}

DType dtype_of(const std::string& n) {
  if (n == "F32") return DType::F32;
  if (n == "F16") return DType::F16;
  if (n == "BF16") return DType::BF16;
  if (n == "U32") return DType::U32;
  if (n == "U8") return DType::U8;
  throw Error(Error::Kind::Unsupported, "safetensors: dtype " + n);
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o;
}

// A minimal reader for the safetensors header: an object of objects whose
// values are strings, integers or lists of integers.
struct Cursor {
  const std::string& s;
  size_t i = 0;
  void ws() {
    while (i < s.size() && std::isspace(static_cast<unsigned char>(s[i]))) i++;
  }
  void expect(char c) {
    ws();
    if (i >= s.size() || s[i] != c) msg(std::string("safetensors header: expected '") + c + "'");
    i++;
  }
  bool peek(char c) {
    ws();
    return i < s.size() && s[i] == c;
  }
  std::string str() {
    expect('"');
    std::string o;
    while (i < s.size() && s[i] != '"') {
      if (s[i] == '\\' && i + 1 < s.size()) i++;
      o += s[i++];
    }
    expect('"');
    return o;
  }
  int64_t integer() {
    ws();
    size_t j = i;
    if (j < s.size() && s[j] == '-') j++;
    while (j < s.size() && std::isdigit(static_cast<unsigned char>(s[j]))) j++;
    if (j == i || (j == i + 1 && s[i] == '-')) msg("safetensors header: expected an integer");
    int64_t v = 0;
    try {
      v = std::stoll(s.substr(i, j - i));
    } catch (const std::exception&) {
      msg("safetensors header: integer out of range");
    }
    i = j;
    return v;
  }
  std::vector<int64_t> ints() {
    std::vector<int64_t> v;
    expect('[');
    if (peek(']')) {
      i++;
      return v;
    }
    while (true) {
      v.push_back(integer());
      if (peek(',')) {
        i++;
        continue;
      }
      expect(']');
      return v;
    }
  }
  void skip_value() {  // string, number, list or object (the __metadata__ entry)
    ws();
    if (peek('"')) {
      str();
    } else if (peek('{') || peek('[')) {
      const char open = s[i], close = open == '{' ? '}' : ']';
      int depth = 0;
      do {
        if (s[i] == '"') {
          str();
          continue;
        }
        if (s[i] == open) depth++;
        if (s[i] == close) depth--;
        i++;
      } while (depth > 0 && i < s.size());
    } else {
      while (i < s.size() && s[i] != ',' && s[i] != '}') i++;
    }
  }
};

struct Entry {
  std::string name, dtype;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;
};

void write_file(const std::string& path, const std::string& text) {
  std::ofstream f(path, std::ios::binary);
  if (!f) msg("cannot write " + path);
  f << text;
  if (!f) msg("write failed: " + path);
}

}  // namespace

bool is_projection(const std::string& key) {
  static const char* kSuffixes[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                    "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                    "mlp.down_proj.weight"};
  for (const char* s : kSuffixes) {
    const size_t n = std::strlen(s);
    if (key.size() >= n && key.compare(key.size() - n, n, s) == 0) return true;
  }
  return false;
}

void save_safetensors(const std::string& path, const Tensors& tensors) {
  std::ostringstream h;
  h << "{\"__metadata__\":{\"format\":\"mlx\"}";
  int64_t off = 0;
  for (const auto& [name, a] : tensors) {
    h << ",\"" << json_escape(name) << "\":{\"dtype\":\"" << dtype_name(a.dtype()) << "\",\"shape\":[";
    for (size_t d = 0; d < a.shape().size(); d++) h << (d ? "," : "") << a.shape()[d];
    h << "],\"data_offsets\":[" << off << "," << off + static_cast<int64_t>(a.nbytes()) << "]}";
    off += static_cast<int64_t>(a.nbytes());
  }
  h << "}";
  std::string header = h.str();
  while (header.size() % 8) header += ' ';  // data starts 8-byte aligned
  std::ofstream f(path, std::ios::binary);
  if (!f) msg("cannot write " + path);
  const uint64_t n = header.size();
  unsigned char len[8];
  for (int b = 0; b < 8; b++) len[b] = static_cast<unsigned char>(n >> (8 * b));
  f.write(reinterpret_cast<const char*>(len), 8);
  f.write(header.data(), static_cast<std::streamsize>(header.size()));
  for (const auto& t : tensors) {
    const std::vector<uint8_t> bytes = t.second.to_bytes();
    f.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
  }
  if (!f) msg("write failed: " + path);
}

Tensors load_safetensors(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) msg("cannot read " + path);
  unsigned char len[8];
  if (!f.read(reinterpret_cast<char*>(len), 8)) msg("safetensors: short file " + path);
  uint64_t n = 0;
  for (int b = 0; b < 8; b++) n |= static_cast<uint64_t>(len[b]) << (8 * b);
  if (n > (uint64_t(1) << 30)) msg("safetensors: header too large");
  std::string header(n, '\0');
  if (!f.read(header.data(), static_cast<std::streamsize>(n))) msg("safetensors: short header");

  std::vector<Entry> entries;
  Cursor c{header};
  c.expect('{');
  while (!c.peek('}')) {
    const std::string key = c.str();
    c.expect(':');
    if (key == "__metadata__") {
      c.skip_value();
    } else {
      Entry e;
      e.name = key;
      c.expect('{');
      while (!c.peek('}')) {
        const std::string field = c.str();
        c.expect(':');
        if (field == "dtype") {
          e.dtype = c.str();
        } else if (field == "shape") {
          e.shape = c.ints();
        } else if (field == "data_offsets") {
          const std::vector<int64_t> o = c.ints();
          if (o.size() != 2) msg("safetensors: bad data_offsets for " + key);
          e.begin = o[0];
          e.end = o[1];
        } else {
          c.skip_value();
        }
        if (c.peek(',')) c.i++;
      }
      c.expect('}');
      entries.push_back(e);
    }
    if (c.peek(',')) c.i++;
  }
  const std::streamoff data0 = 8 + static_cast<std::streamoff>(n);
  f.seekg(0, std::ios::end);
  const int64_t data_len = static_cast<int64_t>(f.tellg()) - static_cast<int64_t>(data0);
  Tensors out;
  for (const Entry& e : entries) {
    const DType t = dtype_of(e.dtype);
    // every bound checked before anything is sized from it: dimensions >= 0,
    // no overflow of the element or byte count, 0 <= begin <= end <= data
    const int64_t esz = static_cast<int64_t>(dtype_size(t));
    int64_t count = 1;
    for (int64_t d : e.shape) {
      if (d < 0) msg("safetensors: negative dimension in the shape of " + e.name);
      if (d != 0 && count > INT64_MAX / esz / d) msg("safetensors: shape of " + e.name + " is too large");
      count *= d;
    }
    if (e.begin < 0 || e.end < e.begin || e.end > data_len)
      msg("safetensors: data_offsets of " + e.name + " lie outside the file");
    if (e.end - e.begin != count * esz) msg("safetensors: size of " + e.name + " does not match its shape");
    std::vector<uint8_t> bytes(static_cast<size_t>(e.end - e.begin));
    f.seekg(data0 + e.begin);
    if (!f.read(reinterpret_cast<char*>(bytes.data()), static_cast<std::streamsize>(bytes.size())))
      msg("safetensors: short data for " + e.name);
    out.emplace_back(e.name, Array::from_bytes(bytes.data(), bytes.size(), e.shape, t));
  }
  return out;
}

Report write_snapshot(const std::string& out_dir, const Tensors& tensors, const std::string& config_json,
                      std::optional<QuantSpec> quantize, const std::optional<std::string>& tokenizer_json,
                      const std::optional<std::string>& tokenizer_config_json) {
  Tensors out;
  for (const auto& [key, arr] : tensors) {
    if (quantize && is_projection(key)) {
      const Array w = arr.dtype() == DType::BF16 ? arr : Array::from_f32(arr.to_f32(), arr.shape(), DType::BF16);
      const QuantizedLinear q = QuantizedLinear::quantize(w, quantize->group_size, quantize->bits);
      const std::string base = key.substr(0, key.size() - std::strlen(".weight"));
      out.emplace_back(base + ".weight", q.weight);
      out.emplace_back(base + ".scales", q.scales);
      out.emplace_back(base + ".biases", q.biases);
    } else {
      out.emplace_back(key, arr);
    }
  }
  return write_parts(out_dir, out, config_json, quantize, tokenizer_json, tokenizer_config_json);
}

Report write_parts(const std::string& out_dir, const Tensors& out, const std::string& config_json,
                   std::optional<QuantSpec> quantized, const std::optional<std::string>& tokenizer_json,
                   const std::optional<std::string>& tokenizer_config_json) {
  std::string config = config_json;
  const size_t open = config.find_first_not_of(" \t\r\n"), close = config.find_last_not_of(" \t\r\n");
  if (open == std::string::npos || config[open] != '{' || config[close] != '}')
    throw Error(Error::Kind::Msg, "snapshot config.json is not a JSON object");
  std::filesystem::create_directories(out_dir);
  if (quantized) {
    const bool empty = config.find_first_not_of(" \t\r\n", open + 1) == close;
    config.insert(close, std::string(empty ? "" : ", ") + "\"quantization\": {\"group_size\": " +
                             std::to_string(quantized->group_size) + ", \"bits\": " + std::to_string(quantized->bits) +
                             "}");
  }
  write_file(out_dir + "/config.json", config);
  save_safetensors(out_dir + "/model.safetensors", out);
  if (tokenizer_json) write_file(out_dir + "/tokenizer.json", *tokenizer_json);
  if (tokenizer_config_json) write_file(out_dir + "/tokenizer_config.json", *tokenizer_config_json);
  Report r;
  r.num_tensors = out.size();
  r.quantized = quantized;
  r.out_dir = out_dir;
  return r;
}

Projection load_projection(const Tensors& tensors, const std::string& base, QuantSpec spec) {
  const Array* parts[3] = {nullptr, nullptr, nullptr};
  const std::string names[3] = {base + ".weight", base + ".scales", base + ".biases"};
  for (const auto& t : tensors)
    for (int i = 0; i < 3; i++)
      if (t.first == names[i]) parts[i] = &t.second;
  for (int i = 0; i < 3; i++)
    if (!parts[i]) throw Error(Error::Kind::Msg, "missing tensor: " + names[i]);
  return Projection::from_quantized(*parts[0], *parts[1], *parts[2], spec);
}

}  // namespace snapshot
}  // namespace mlxq
