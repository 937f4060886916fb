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

// Lane owns EPL consecutive elements v of a group of EPL * LPG; the LPG
// lanes of the group (aligned, within one wavefront) reduce min/max with
// butterfly shuffles.  Every lane of the group must call it.
template <int BITS, int LPG, int EPL = 8>
__device__ __forceinline__ void quantize_group8(const float (&v)[EPL], uint32_t (&codes)[EPL], float& scale,
                                                float& bias) {
  float w_max = v[0], w_min = v[0];
#pragma unroll
  for (int i = 1; i < EPL; i++) {
    w_max = fmaxf(w_max, v[i]);
    w_min = fminf(w_min, v[i]);
  }
  // All-reduce within the LPG lanes of this group (groups never straddle a
  // 16-lane row: LPG is 4, 8 or 16 and the lane index is group-aligned) with
  // DPP moves: quad swaps, then the other quad of 8 (lane i <-> 7 - i), then
  // the other 8 of 16 (i <-> 15 - i).  Exact for max/min in any order.
  static_assert(LPG == 2 || LPG == 4 || LPG == 8 || LPG == 16, "lanes per group");
  w_max = fmaxf(w_max, dpp_f32<kDppQuadXor1>(w_max));
  w_min = fminf(w_min, dpp_f32<kDppQuadXor1>(w_min));
  if constexpr (LPG >= 4) {
    w_max = fmaxf(w_max, dpp_f32<kDppQuadXor2>(w_max));
    w_min = fminf(w_min, dpp_f32<kDppQuadXor2>(w_min));
  }
  if constexpr (LPG >= 8) {
    w_max = fmaxf(w_max, dpp_f32<kDppRowHalfMirror>(w_max));
    w_min = fminf(w_min, dpp_f32<kDppRowHalfMirror>(w_min));
  }
  if constexpr (LPG >= 16) {
    w_max = fmaxf(w_max, dpp_f32<kDppRowMirror>(w_max));
    w_min = fminf(w_min, dpp_f32<kDppRowMirror>(w_min));
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

  // code = rint(fl((w - bias) / scale)), fl the correctly rounded f32
  // division.  The compiler's division of d by scale is v_div_scale (of
  // both operands), v_rcp_f32, one Newton step of the reciprocal, the
  // quotient and two residual corrections (the last through v_div_fmas),
  // then v_div_fixup.  Where the operands need no scaling and the quotient
  // no fixing (finite, |scale| in [2^-60, 2^60], |quotient| < 1024) the
  // scalings are identities and v_div_fmas is a plain fma, so the same
  // sequence without them gives the same bits; its reciprocal step depends
  // on the scale only and is done once for the lane's elements.  Elsewhere
  // (never for weights of ordinary magnitude) the division itself runs.
  // A quotient below 1024 in magnitude but far smaller than the scale
  // (|d| << |scale|) could still meet a scaled division; its code is 0
  // either way (rint of a value far below 0.5).
  const float r0 = __builtin_amdgcn_rcpf(scale);
  const float r1 = fmaf(fmaf(-scale, r0, 1.0f), r0, r0);
  const bool ordinary = fabsf(scale) >= 0x1p-60f && fabsf(scale) <= 0x1p60f;
  bool any_other = !ordinary;  // one test for the lane's elements, one branch
#pragma unroll
  for (int i = 0; i < EPL; i++) {
    const float d = v[i] - bias;
    const float q0 = d * r1;
    const float q1 = fmaf(fmaf(-scale, q0, d), r1, q0);
    const float q2 = fmaf(fmaf(-scale, q1, d), r1, q1);
    any_other |= !(fabsf(q0) < 1024.f);
    codes[i] = static_cast<uint32_t>(fminf(fmaxf(__builtin_rintf(q2), 0.f), n_bins));
  }
  if (any_other) {
#pragma unroll
    for (int i = 0; i < EPL; i++) {
      const float d = v[i] - bias;
      if (!(ordinary && fabsf(d * r1) < 1024.f))
        codes[i] = static_cast<uint32_t>(fminf(fmaxf(__builtin_rintf(d / scale), 0.f), n_bins));
    }
  }
}

// Pack 16 codes LSB-first: two words (Q4) or four (Q8) at 16-code index
// `lane` (8-byte stores).
template <int BITS>
__device__ __forceinline__ void store_codes16(uint32_t* wq, int64_t lane, const uint32_t (&codes)[16]) {
  uint32_t w[BITS / 2];
#pragma unroll
  for (int j = 0; j < BITS / 2; j++) {
    w[j] = 0;
#pragma unroll
    for (int i = 0; i < 32 / BITS; i++) w[j] |= codes[j * (32 / BITS) + i] << (BITS * i);
  }
#pragma unroll
  for (int j = 0; j < BITS / 4; j++) reinterpret_cast<uint2*>(wq)[lane * (BITS / 4) + j] = uint2{w[2 * j], w[2 * j + 1]};
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
