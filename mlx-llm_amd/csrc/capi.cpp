// Host-side C ABI pieces that launch nothing: error strings, version, GGUF
// block geometry.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <cxxabi.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <mutex>
#include <string>

#include "common.hpp"

namespace mlxq {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}
namespace {
thread_local std::string* g_route_log = nullptr;  // non-null while a route query runs on this thread
}
bool route_query_active() { return g_route_log != nullptr; }
void route_query_note(const char* what) {
  if (!g_route_log) return;
  if (!g_route_log->empty()) *g_route_log += " + ";
  *g_route_log += what;
}
void route_query_kernel(const void* kern) {
  if (!g_route_log) return;
  // the device function's name, demangled, without its argument list,
  // return type and the library's namespaces: e.g. "qmm_kernel<4, 64, 8, 2>"
  std::string name = "?";
  hipFunction_t f = nullptr;
  if (hipGetFuncBySymbol(&f, kern) == hipSuccess && f) {
    if (const char* raw = hipKernelNameRef(f)) {
      int st = 0;
      char* dm = abi::__cxa_demangle(raw, nullptr, nullptr, &st);
      name = st == 0 && dm ? dm : raw;
      free(dm);
    }
  }
  if (name.rfind("void ", 0) == 0) name = name.substr(5);
  int depth = 0;  // cut the argument list: the last top-level '(' ... ')'
  for (size_t i = name.size(); i-- > 0;) {
    if (name[i] == ')') depth++;
    if (name[i] == '(' && --depth == 0) {
      name = name.substr(0, i);
      break;
    }
  }
  for (const std::string pre : {std::string("(anonymous namespace)::"), std::string("mlxq::")}) {
    for (size_t at; (at = name.find(pre)) != std::string::npos;) name.erase(at, pre.size());
  }
  route_query_note(name.c_str());
}
int check_launch(const char* what) {
  if (g_route_log) return MLXQ_OK;  // nothing was launched (MLXQ_LAUNCH recorded it)
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(MLXQ_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
  return MLXQ_OK;
}

namespace {

const Overrides* read_overrides() {
  auto* o = new Overrides{};
  auto flag = [](const char* n) { return getenv(n) != nullptr; };
  auto pair = [](const char* n, int* a, int* b) {
    if (const char* e = getenv(n)) sscanf(e, "%d,%d", a, b);
  };
  auto num = [](const char* n) {
    const char* e = getenv(n);
    return e ? atoi(e) : 0;
  };
  o->qmv_row_all = flag("MLXQ_QMV_ROW_ALL");
  o->qmv_no_row = flag("MLXQ_QMV_NO_ROW");
  o->qmv_mfma = flag("MLXQ_QMV_MFMA");
  o->qmv_dot_all = flag("MLXQ_QMV_DOT_ALL");
  o->qmv_tile_all = flag("MLXQ_QMV_TILE_ALL");
  o->qmv_legacy = flag("MLXQ_QMV_LEGACY");
  o->qmv_narrow = flag("MLXQ_QMV_NARROW");
  o->tile_mb = flag("MLXQ_QMV_TILE_MB");
  o->qmv_no_tile_fused = flag("MLXQ_QMV_NO_TILE_FUSED");
  if (const char* e = getenv("MLXQ_QMV_TILE")) sscanf(e, "%d,%d,%d", &o->tile_wv, &o->tile_nch, &o->tile_kh);
  if (const char* e = getenv("MLXQ_QMV_TILE_FUSED_RG")) o->tile_fused_rg = atoi(e);
  o->stream64 = -1;
  if (const char* e = getenv("MLXQ_QMV_STREAM64")) o->stream64 = atoi(e);
  if (const char* e = getenv("MLXQ_QMV_TILE_STREAM")) {
    o->stream_set = true;
    sscanf(e, "%d,%d,%d,%d", &o->stream_wv, &o->stream_nch, &o->stream_kh, &o->stream_splits);
  }
  pair("MLXQ_QMV_DOT", &o->dot_sub, &o->dot_wv);
  pair("MLXQ_QMV_MFMA_CFG", &o->mfma_sub, &o->mfma_wv);
  o->qmv_sub = num("MLXQ_QMV_SUB");
  o->row_r = num("MLXQ_QMV_ROW_R");
  o->row_w = num("MLXQ_QMV_ROW_W");
  o->qmm_cfg = num("MLXQ_QMM_CFG");
  o->qmm_split = num("MLXQ_QMM_SPLIT");
  o->qmm_lib = flag("MLXQ_QMM_LIB");
  o->qmm_fused = flag("MLXQ_QMM_FUSED");
  o->qmm_lib_algo = num("MLXQ_QMM_LIB_ALGO");
  return o;
}

// Published once and replaced whole by a reload; a replaced table is never
// freed (a call on another thread may still be reading it).
std::atomic<const Overrides*> g_overrides{nullptr};
std::mutex g_overrides_mu;

}  // namespace

const Overrides& overrides() {
  const Overrides* o = g_overrides.load(std::memory_order_acquire);
  if (o) return *o;
  std::lock_guard<std::mutex> lk(g_overrides_mu);
  o = g_overrides.load(std::memory_order_relaxed);
  if (!o) {
    o = read_overrides();
    g_overrides.store(o, std::memory_order_release);
  }
  return *o;
}

}  // namespace mlxq

using namespace mlxq;

extern "C" int mlxq_reload_overrides(void) {
  std::lock_guard<std::mutex> lk(g_overrides_mu);
  g_overrides.store(read_overrides(), std::memory_order_release);
  return MLXQ_OK;
}

extern "C" const char* mlxq_last_error(void) { return g_last_error.c_str(); }

#ifndef MLXQ_SOURCE_HASH
#define MLXQ_SOURCE_HASH "unknown"
#endif
// The source hash is that of the kernel, host and header sources the
// library was built from (mlx-llm_amd/build.py), so that a caller can refuse
// a library built from other sources.
extern "C" const char* mlxq_version(void) { return "mlxq 0.2.0 (gfx950) src=" MLXQ_SOURCE_HASH; }

namespace mlxq {
// Run `call` as a route query: launches suppressed, families recorded.
int run_route_query(const std::function<int()>& call, char* buf, size_t len) {
  std::string log;
  g_route_log = &log;
  const int rc = call();
  g_route_log = nullptr;
  if (rc) return rc;
  if (!buf || len == 0) return fail(MLXQ_ERR_INVALID, "qmatmul_route: null buffer");
  const size_t n = std::min(log.size(), len - 1);
  memcpy(buf, log.data(), n);
  buf[n] = 0;
  return MLXQ_OK;
}
}  // namespace mlxq

// GgmlType::from_tag + block() (src/gguf/dequant.rs:85-141).  The table is
// the GGUF/ggml on-disk format, so it is necessarily identical.
extern "C" int mlxq_gguf_block(uint32_t tag, int64_t* elems, int64_t* bytes) {
  int64_t e, b;
  switch (tag) {
    case 0: e = 1; b = 4; break;            // F32
    case 1: case 30: e = 1; b = 2; break;   // F16, BF16
    case 2: e = 32; b = 18; break;          // Q4_0
    case 3: e = 32; b = 20; break;          // Q4_1
    case 6: e = 32; b = 22; break;          // Q5_0
    case 7: e = 32; b = 24; break;          // Q5_1
    case 8: e = 32; b = 34; break;          // Q8_0
    case 10: e = 256; b = 84; break;        // Q2_K
    case 11: e = 256; b = 110; break;       // Q3_K
    case 12: e = 256; b = 144; break;       // Q4_K
    case 13: e = 256; b = 176; break;       // Q5_K
    case 14: e = 256; b = 210; break;       // Q6_K
    case 16: e = 256; b = 66; break;        // IQ2_XXS
    case 17: e = 256; b = 74; break;        // IQ2_XS
    case 18: e = 256; b = 98; break;        // IQ3_XXS
    case 19: e = 256; b = 50; break;        // IQ1_S
    case 20: e = 32; b = 18; break;         // IQ4_NL
    case 21: e = 256; b = 110; break;       // IQ3_S
    case 22: e = 256; b = 82; break;        // IQ2_S
    case 23: e = 256; b = 136; break;       // IQ4_XS
    case 29: e = 256; b = 56; break;        // IQ1_M
    default:
      return fail(MLXQ_ERR_UNSUPPORTED, "unsupported: GGUF type tag " + std::to_string(tag));
  }
  if (elems) *elems = e;
  if (bytes) *bytes = b;
  return MLXQ_OK;
}

extern "C" int mlxq_gguf_tensor_byte_len(uint32_t tag, int64_t n, int64_t* bytes) {
  int64_t be = 0, bb = 0;
  int rc = mlxq_gguf_block(tag, &be, &bb);
  if (rc) return rc;
  if (!bytes) return fail(MLXQ_ERR_INVALID, "gguf: null output pointer");
  if (n < 0 || n % be)
    return fail(MLXQ_ERR_SHAPE, "gguf: " + std::to_string(n) + " elements not a multiple of " +
                                    std::to_string(be) + " for tag " + std::to_string(tag));
  *bytes = (n / be) * bb;
  return MLXQ_OK;
}
