// MLX group-wise affine quantization of one group, shared by the quantizer
// (affine.hip) and the fused GGUF converter (gguf_requant.hip).
//
// Reference: QuantizedLinear::quantize (src/primitives/quant.rs:38-53) ->
// mlx_rs::ops::quantize (MLX 0.31.2 semantics, restated):
//   scale = max((max - min) / n_bins, 1e-7); the edge with the larger
//   magnitude becomes the bias and the scale is snapped so that 0 is exactly
//   on the grid; code = clamp(rint((w - bias) / scale), 0, n_bins).
// Every file including this header is compiled with -ffp-contract=off: codes
// must be bit-identical with the CPU restatement.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace mlxq {
namespace {  // internal linkage: each including file has its own copy

// Lane owns 8 consecutive elements v of a group of 8 * LPG; the LPG lanes of
// the group (aligned, within one wavefront) reduce min/max with butterfly
// shuffles.  Every lane of the group must call it.
template <int BITS, int LPG>
__device__ __forceinline__ void quantize_group8(const float (&v)[8], uint32_t (&codes)[8], float& scale,
                                                float& bias) {
  float w_max = v[0], w_min = v[0];
#pragma unroll
  for (int i = 1; i < 8; i++) {
    w_max = fmaxf(w_max, v[i]);
    w_min = fminf(w_min, v[i]);
  }
  // Butterfly within the LPG lanes of this group (groups never straddle a
  // wavefront: LPG divides 64 and the lane index is group-aligned).
#pragma unroll
  for (int off = 1; off < LPG; off <<= 1) {
    w_max = fmaxf(w_max, __shfl_xor(w_max, off, 64));
    w_min = fminf(w_min, __shfl_xor(w_min, off, 64));
  }

  constexpr float n_bins = static_cast<float>((1 << BITS) - 1);
  const float eps = 1e-7f;
  const bool mask = fabsf(w_min) > fabsf(w_max);
  scale = fmaxf((w_max - w_min) / n_bins, eps);
  scale = mask ? scale : -scale;
  const float edge = mask ? w_min : w_max;
  const float q0 = __builtin_rintf(edge / scale);
  bias = 0.f;
  if (q0 != 0.f) {
    scale = edge / q0;
    bias = edge;
  }

#pragma unroll
  for (int i = 0; i < 8; i++) {
    float q = __builtin_rintf((v[i] - bias) / scale);
    q = fminf(fmaxf(q, 0.f), n_bins);
    codes[i] = static_cast<uint32_t>(q);
  }
}

// Pack 8 codes LSB-first: one word (Q4) or two (Q8) at lane index `lane`.
template <int BITS>
__device__ __forceinline__ void store_codes8(uint32_t* wq, int64_t lane, const uint32_t (&codes)[8]) {
  if constexpr (BITS == 4) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) word |= codes[i] << (4 * i);
    wq[lane] = word;
  } else {
    uint2 words;
    words.x = codes[0] | (codes[1] << 8) | (codes[2] << 16) | (codes[3] << 24);
    words.y = codes[4] | (codes[5] << 8) | (codes[6] << 16) | (codes[7] << 24);
    reinterpret_cast<uint2*>(wq)[lane] = words;
  }
}

}  // namespace
}  // namespace mlxq
