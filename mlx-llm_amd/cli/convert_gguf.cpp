// Convert a llama.cpp *.gguf model into an MLX snapshot directory, the
// command-line front of mlxq::gguf::convert_file (the reference's
// examples/convert_gguf.rs:28-80):
//
//   convert_gguf <model.gguf> <out_dir> [--quant q4|q8] [--tokenizer tokenizer.json]
//   convert_gguf --inspect <model.gguf>     print the header as JSON (no GPU)
//
// The block decoding and the requantization run on the GPU.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>

#include "mlxq.hpp"

namespace {

std::string read_text(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw mlxq::Error(mlxq::Error::Kind::Msg, "cannot read " + path);
  std::ostringstream o;
  o << f.rdbuf();
  return o.str();
}

std::string quoted(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if (static_cast<unsigned char>(c) < 0x20) {
      char b[8];
      std::snprintf(b, sizeof b, "\\u%04x", c);
      o += b;
    } else {
      o += c;
    }
  }
  return o + "\"";
}

int inspect(const std::string& path) {
  const mlxq::gguf::GgufFile g = mlxq::gguf::GgufFile::open(path);
  std::printf("{\"alignment\": %llu, \"data_start\": %llu, \"metadata_keys\": [",
              static_cast<unsigned long long>(g.alignment), static_cast<unsigned long long>(g.data_start));
  bool first = true;
  for (const auto& kv : g.metadata) {
    std::printf("%s%s", first ? "" : ", ", quoted(kv.first).c_str());
    first = false;
  }
  std::printf("], \"tensors\": [");
  for (size_t i = 0; i < g.tensors.size(); i++) {
    const auto& t = g.tensors[i];
    std::printf("%s{\"name\": %s, \"shape\": [", i ? ", " : "", quoted(t.name).c_str());
    for (size_t d = 0; d < t.shape.size(); d++) std::printf("%s%lld", d ? ", " : "", static_cast<long long>(t.shape[d]));
    std::printf("], \"type\": %u, \"offset\": %llu}", t.ggml_type, static_cast<unsigned long long>(t.offset));
  }
  std::printf("]}\n");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc == 3 && std::strcmp(argv[1], "--inspect") == 0) return inspect(argv[2]);
    if (argc < 3) {
      std::fprintf(stderr, "usage: convert_gguf <model.gguf> <out_dir> [--quant q4|q8] [--tokenizer tokenizer.json]\n");
      return 1;
    }
    mlxq::gguf::ConvertOptions opts;
    for (int i = 3; i < argc; i++) {
      const std::string flag = argv[i];
      if (flag == "--quant" && i + 1 < argc) {
        const std::string v = argv[++i];
        if (v == "q4") opts.quantize = mlxq::QuantSpec::q4();
        else if (v == "q8") opts.quantize = mlxq::QuantSpec::q8();
        else throw mlxq::Error(mlxq::Error::Kind::Msg, "unknown --quant \"" + v + "\" (expected q4|q8)");
      } else if (flag == "--tokenizer" && i + 1 < argc) {
        opts.tokenizer_json = read_text(argv[++i]);
      } else {
        throw mlxq::Error(mlxq::Error::Kind::Msg, "unknown argument \"" + flag + "\"");
      }
    }
    const mlxq::gguf::ConvertReport r = mlxq::gguf::convert_file(argv[1], argv[2], opts);
    std::printf("tokenizer: %s\n", r.tokenizer.c_str());
    std::printf("converted %s (%s) -> %s: %zu tensors", argv[1], r.architecture.c_str(), r.out_dir.c_str(),
                r.num_tensors);
    if (r.quantized)
      std::printf(", projections quantized to %d-bit (group %d)\n", r.quantized->bits, r.quantized->group_size);
    else
      std::printf(", dense bf16\n");
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
}
