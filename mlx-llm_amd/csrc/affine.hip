// Group-wise affine quantize / dequantize for gfx950.
//
// Reference: QuantizedLinear::quantize / dequantize_weight
// (src/primitives/quant.rs:38-53, :73-81) -> mlx_rs::ops::{quantize,dequantize}
// (MLX 0.31.2); the per-group arithmetic is in affine_group.hpp.
// Layout: every lane owns 8 consecutive elements; the group_size/8 lanes of a
// group reduce min/max with butterfly shuffles, then each lane packs its own
// codes into one (Q4) or two (Q8) uint32 words, so loads and stores are fully
// coalesced 16-byte accesses.  This file is compiled with -ffp-contract=off:
// codes must be bit-identical with the CPU restatement.
#include <hip/hip_runtime.h>

#include <string>

#include "affine_group.hpp"
#include "common.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));


constexpr int kThreads = 256;

template <int DT>
__device__ __forceinline__ void load8(const void* w, int64_t e, float (&v)[8]) {
  if constexpr (DT == MLXQ_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(w) + e);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + e);
    uint32_t s[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = bf16_bits_to_f32(s[i] & 0xFFFFu);
      v[2 * i + 1] = bf16_bits_to_f32(s[i] >> 16);
    }
  }
}

template <int DT>
__device__ __forceinline__ void store1(void* p, int64_t i, float v) {
  if constexpr (DT == MLXQ_F32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
}

template <int DT>
__device__ __forceinline__ float load1(const void* p, int64_t i) {
  if constexpr (DT == MLXQ_F32) return static_cast<const float*>(p)[i];
  else return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// One lane per 8 elements; LPG = group_size / 8 lanes per group.
template <int DT, int BITS, int LPG>
__global__ __launch_bounds__(kThreads) void affine_quantize_kernel(const void* __restrict__ w, int64_t n_lanes,
                                                                    uint32_t* __restrict__ wq,
                                                                    void* __restrict__ scales,
                                                                    void* __restrict__ biases) {
  const int64_t lane = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const bool active = lane < n_lanes;
  float v[8];
  if (active) {
    load8<DT>(w, lane * 8, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.f;
  }
  uint32_t codes[8];
  float scale, bias;
  quantize_group8<BITS, LPG>(v, codes, scale, bias);
  if (!active) return;
  store_codes8<BITS>(wq, lane, codes);
  if ((threadIdx.x & (LPG - 1)) == 0) {
    const int64_t g = lane / LPG;
    store1<DT>(scales, g, scale);
    store1<DT>(biases, g, bias);
  }
}

// One lane per 8 elements: out = scale*q + bias in f32, then stored in DT.
template <int DT, int BITS>
__global__ __launch_bounds__(kThreads) void affine_dequantize_kernel(const uint32_t* __restrict__ wq,
                                                                      const void* __restrict__ scales,
                                                                      const void* __restrict__ biases,
                                                                      int64_t n_lanes, int lanes_per_group,
                                                                      void* __restrict__ out) {
  const int64_t lane = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (lane >= n_lanes) return;
  const int64_t g = lane / lanes_per_group;
  const float s = load1<DT>(scales, g), b = load1<DT>(biases, g);
  uint32_t q[8];
  if constexpr (BITS == 4) {
    uint32_t word = wq[lane];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = (word >> (4 * i)) & 0xFu;
  } else {
    uint2 words = reinterpret_cast<const uint2*>(wq)[lane];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      q[i] = (words.x >> (8 * i)) & 0xFFu;
      q[4 + i] = (words.y >> (8 * i)) & 0xFFu;
    }
  }
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; i++) r[i] = s * static_cast<float>(q[i]) + b;
  if constexpr (DT == MLXQ_F32) {
    float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + lane * 8);
    o[0] = make_float4(r[0], r[1], r[2], r[3]);
    o[1] = make_float4(r[4], r[5], r[6], r[7]);
  } else {
    // v_cvt_pk_bf16_f32: two values per instruction, round to nearest even
    auto pk = [](float lo, float hi) {
      const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
      return __builtin_bit_cast(uint32_t, v);
    };
    uint4 p;
    p.x = pk(r[0], r[1]);
    p.y = pk(r[2], r[3]);
    p.z = pk(r[4], r[5]);
    p.w = pk(r[6], r[7]);
    reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + lane * 8)[0] = p;
  }
}

int check_args(int dtype, int64_t rows, int64_t cols, int group_size, int bits) {
  if (bits != 4 && bits != 8)
    return fail(MLXQ_ERR_UNSUPPORTED, "unsupported: bits=" + std::to_string(bits) + " (4 or 8)");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MLXQ_ERR_UNSUPPORTED, "unsupported: group_size=" + std::to_string(group_size) + " (32, 64, 128)");
  if (dtype != MLXQ_F32 && dtype != MLXQ_BF16)
    return fail(MLXQ_ERR_UNSUPPORTED, "unsupported: dtype " + std::to_string(dtype) + " (f32 or bf16)");
  if (rows < 0 || cols <= 0) return fail(MLXQ_ERR_INVALID, "quantize: bad shape");
  if (cols % group_size)
    return fail(MLXQ_ERR_SHAPE, "quantize: last dimension " + std::to_string(cols) +
                                    " is not divisible by group_size " + std::to_string(group_size));
  return MLXQ_OK;
}

template <int DT, int BITS>
void launch_quant(const void* w, int64_t n_lanes, int group_size, uint32_t* wq, void* s, void* b, hipStream_t st) {
  dim3 grid(ceil_div(n_lanes, kThreads));
  switch (group_size) {
    case 32: MLXQ_LAUNCH((affine_quantize_kernel<DT, BITS, 4>), grid, dim3(kThreads), 0, st, w, n_lanes, wq, s, b); break;
    case 64: MLXQ_LAUNCH((affine_quantize_kernel<DT, BITS, 8>), grid, dim3(kThreads), 0, st, w, n_lanes, wq, s, b); break;
    default: MLXQ_LAUNCH((affine_quantize_kernel<DT, BITS, 16>), grid, dim3(kThreads), 0, st, w, n_lanes, wq, s, b); break;
  }
}

}  // namespace
}  // namespace mlxq

using namespace mlxq;

extern "C" int mlxq_quantize(const void* w, int dtype, int64_t rows, int64_t cols, int group_size, int bits,
                             uint32_t* wq, void* scales, void* biases, void* stream) {
  clear_error();
  int rc = check_args(dtype, rows, cols, group_size, bits);
  if (rc) return rc;
  const int64_t n_lanes = rows * cols / 8;
  if (n_lanes == 0) return MLXQ_OK;
  if (!w || !wq || !scales || !biases) return fail(MLXQ_ERR_INVALID, "quantize: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == MLXQ_F32) {
    if (bits == 4) launch_quant<MLXQ_F32, 4>(w, n_lanes, group_size, wq, scales, biases, st);
    else launch_quant<MLXQ_F32, 8>(w, n_lanes, group_size, wq, scales, biases, st);
  } else {
    if (bits == 4) launch_quant<MLXQ_BF16, 4>(w, n_lanes, group_size, wq, scales, biases, st);
    else launch_quant<MLXQ_BF16, 8>(w, n_lanes, group_size, wq, scales, biases, st);
  }
  return check_launch("quantize");
}

extern "C" int mlxq_dequantize(const uint32_t* wq, const void* scales, const void* biases, int dtype, int64_t rows,
                               int64_t cols, int group_size, int bits, void* out, void* stream) {
  clear_error();
  int rc = check_args(dtype, rows, cols, group_size, bits);
  if (rc) return rc;
  const int64_t n_lanes = rows * cols / 8;
  if (n_lanes == 0) return MLXQ_OK;
  if (!wq || !scales || !biases || !out) return fail(MLXQ_ERR_INVALID, "dequantize: null pointer");
  hipStream_t st = as_stream(stream);
  dim3 grid(ceil_div(n_lanes, kThreads));
  const int lpg = group_size / 8;
  if (dtype == MLXQ_F32) {
    if (bits == 4) MLXQ_LAUNCH((affine_dequantize_kernel<MLXQ_F32, 4>), grid, dim3(kThreads), 0, st, wq, scales, biases, n_lanes, lpg, out);
    else MLXQ_LAUNCH((affine_dequantize_kernel<MLXQ_F32, 8>), grid, dim3(kThreads), 0, st, wq, scales, biases, n_lanes, lpg, out);
  } else {
    if (bits == 4) MLXQ_LAUNCH((affine_dequantize_kernel<MLXQ_BF16, 4>), grid, dim3(kThreads), 0, st, wq, scales, biases, n_lanes, lpg, out);
    else MLXQ_LAUNCH((affine_dequantize_kernel<MLXQ_BF16, 8>), grid, dim3(kThreads), 0, st, wq, scales, biases, n_lanes, lpg, out);
  }
  return check_launch("dequantize");
}
