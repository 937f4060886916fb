// Shared host/device helpers for the mlxq gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <functional>
#include <string>

#include "../../include/mlxq.h"

namespace mlxq {

// ---- error reporting (thread-local message behind mlxq_last_error) ----
void set_error(const std::string& msg);
void clear_error();
int fail(int status, const std::string& msg);
// Check the launch that was just enqueued.  During a route query (below)
// nothing was enqueued: it records `what` instead.
int check_launch(const char* what);

// ---- route queries (mlxq_qmatmul_route): the real dispatch runs on dummy
// pointers with every launch suppressed and recorded by kernel name, so the
// answer is by construction the route a call takes ----
bool route_query_active();
// record a kernel the dispatch would launch (its name from the runtime)
void route_query_kernel(const void* kern);
// record a launch that is not one of this library's kernels (library calls)
void route_query_note(const char* what);
// run `call` as a route query, the recorded families into buf
int run_route_query(const std::function<int()>& call, char* buf, size_t len);


// Kernel-choice overrides for tuning and tests, from MLXQ_* environment
// variables.  Read once, on first use (not on every call: the dispatch path
// does no environment lookups); mlxq_reload_overrides() reads them again.
struct Overrides {
  bool qmv_row_all, qmv_no_row, qmv_mfma, qmv_dot_all, qmv_tile_all, qmv_legacy, qmv_narrow;
  int tile_wv, tile_nch, tile_kh;  // MLXQ_QMV_TILE=waves,chunks[,K parts]
  int tile_fused_rg;               // MLXQ_QMV_TILE_FUSED_RG=1: 16-row whole-K tiles only
  int stream64;                    // MLXQ_QMV_STREAM64=1 / 0: force / forbid the 64-row streaming form
  bool tile_mb;                     // MLXQ_QMV_TILE_MB: M blocks of 16 rows
  bool qmv_no_tile_fused;           // MLXQ_QMV_NO_TILE_FUSED
  bool stream_set;                                      // MLXQ_QMV_TILE_STREAM given
  int stream_wv, stream_nch, stream_kh, stream_splits;  // MLXQ_QMV_TILE_STREAM=waves,chunks,K parts,splits
  int dot_sub, dot_wv;      // MLXQ_QMV_DOT=sub,waves
  int mfma_sub, mfma_wv;    // MLXQ_QMV_MFMA_CFG=sub,waves
  int qmv_sub;              // MLXQ_QMV_SUB
  int row_r, row_w;         // MLXQ_QMV_ROW_R, MLXQ_QMV_ROW_W
  int qmm_cfg, qmm_split;   // MLXQ_QMM_CFG, MLXQ_QMM_SPLIT
  bool qmm_lib, qmm_fused;  // MLXQ_QMM_LIB, MLXQ_QMM_FUSED
  int qmm_lib_algo;         // MLXQ_QMM_LIB_ALGO
};
const Overrides& overrides();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Every kernel launch of the library goes through this: recorded instead
// of launched while a route query is active on this thread.
#define MLXQ_LAUNCH(kern, ...)                                                  \
  do {                                                                          \
    if (::mlxq::route_query_active())                                           \
      ::mlxq::route_query_kernel(reinterpret_cast<const void*>(kern));          \
    else                                                                        \
      hipLaunchKernelGGL(kern, __VA_ARGS__);                                    \
  } while (0)

// ---- device scalar conversions (bit-level, independent of FP modes) ----
__device__ __forceinline__ float bits_to_f32(uint32_t u) { return __uint_as_float(u); }

// Exact binary16 -> binary32, NaNs quieted with payload kept (the conversion
// `half::f16::to_f32` performs, used by src/gguf/dequant.rs:222-225).
// Branch-free: the three encodings are formed and selected, so no per-call
// control flow is left for the compiler to repeat at every use.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  const uint32_t normal = sign | ((exp + 112u) << 23) | (man << 13);
  const uint32_t special = sign | 0x7F800000u | (man ? (0x400000u | (man << 13)) : 0u);
  // subnormal (or zero): man * 2^-24 is exact in f32
  const uint32_t sub = sign | __float_as_uint(static_cast<float>(man) * 5.9604644775390625e-08f);
  return bits_to_f32(exp == 0u ? sub : (exp == 0x1Fu ? special : normal));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return bits_to_f32(b << 16); }

// f32 -> bf16 round-to-nearest-even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- cross-lane adds on the VALU (no LDS crossbar): DPP within rows of 16
// lanes, the gfx950 row swaps across rows ----
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;

// v + v of lane ^ 16 (rows 0+1, 2+3 of 16 lanes)
__device__ __forceinline__ float add_xor16(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
// v + v of lane ^ 32 (the two halves of the wave)
__device__ __forceinline__ float add_xor32(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
// sum over the 64 lanes, every lane gets it
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowHalfMirror>(v);  // lane i <-> 7-i: the other quad of the 8
  v += dpp_f32<kDppRowMirror>(v);      // lane i <-> 15-i: the other 8 of the row
  return add_xor32(add_xor16(v));
}

}  // namespace mlxq
