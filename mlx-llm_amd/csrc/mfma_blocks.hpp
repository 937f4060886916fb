// MFMA building blocks shared by the matrix-core GEMV kernels (qmv_mfma.hip,
// qmv_tile.hip): the group-pure block layout of a 64-byte chunk of codes,
// the code -> bf16 decoders and the one-block MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlxq {
namespace mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 4 x 4 transpose of dwords across the four 16-lane rows of a wave: row r,
// register i holds D[r][i] before and D[i][r] after.
__device__ __forceinline__ void transpose_rows(uint32_t (&d)[4]) {
  auto a = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
  auto b = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
  auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  auto e = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  d[0] = c[0];
  d[1] = c[1];
  d[2] = e[0];
  d[3] = e[1];
}

// MFMA blocks of a 64-byte chunk.  Transposed layouts (Q4; Q8 with 32-code
// groups): block j = codes [B*j, B*(j+1)), lane gq supplies [B*j + B/4*gq,
// +B/4).  Q8 with groups of >= 64 codes keeps the loaded layout instead
// (natural): the chunk is one group, block t takes codes 16*gq + 8t + [0, 8)
// from each lane -- no transpose, and 16x16x32 instead of 16x16x16 MFMAs.
template <int BITS, int GS>
struct Blk {
  static constexpr bool NAT = BITS == 8 && GS >= 64;
  static constexpr bool X32 = BITS == 4 || NAT;            // v_mfma_f32_16x16x32_bf16, else 16x16x16
  static constexpr int KC = 64 * 8 / BITS;                 // codes per chunk
  static constexpr int NB = NAT ? 2 : 4;                   // blocks per chunk
  static constexpr int B = NAT ? 32 : (X32 ? 32 : 16);     // codes per block
  static constexpr int XW = X32 ? 4 : 2;                   // operand dwords per lane per block
  static constexpr int BPG = NAT ? NB : (GS / B < NB ? GS / B : NB);  // consecutive blocks of one group
  // activation offset (elements within a chunk) of lane gq's slice of block j
  static __device__ __forceinline__ int xoff(int j, int gq) { return NAT ? 16 * gq + 8 * j : B * j + (B / 4) * gq; }
  // first code of block j within the chunk (its group)
  static constexpr int code0(int j) { return NAT ? 0 : B * j; }
};

// One block's MFMA: C + A . B^T with A = 16 activation rows, B = 16 weight rows.
template <bool X32>
__device__ __forceinline__ f32x4 mma(const uint32_t* a, const uint32_t* b, f32x4 c) {
  if constexpr (X32) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, u32x4{a[0], a[1], a[2], a[3]}),
                                                   __builtin_bit_cast(bf16x8, u32x4{b[0], b[1], b[2], b[3]}), c, 0, 0,
                                                   0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, u32x2{a[0], a[1]}),
                                                     __builtin_bit_cast(s16x4, u32x2{b[0], b[1]}), c, 0, 0, 0);
  }
}

// 4 Q4 codes pairs of one dword -> bf16 (128 + c) as (c0,c4),(c1,c5),(c2,c6),(c3,c7)
__device__ __forceinline__ void decode_q4(uint32_t q, uint32_t* b) {
  b[0] = (q & 0x000F000Fu) | 0x43004300u;
  b[1] = ((q >> 4) & 0x000F000Fu) | 0x43004300u;
  b[2] = ((q >> 8) & 0x000F000Fu) | 0x43004300u;
  b[3] = ((q >> 12) & 0x000F000Fu) | 0x43004300u;
}

// 4 Q8 codes of one dword -> 4 bf16 in order (exact through f32)
__device__ __forceinline__ void decode_q8(uint32_t q, uint32_t* b) {
  const float f0 = static_cast<float>(q & 0xFFu), f1 = static_cast<float>((q >> 8) & 0xFFu);
  const float f2 = static_cast<float>((q >> 16) & 0xFFu), f3 = static_cast<float>(q >> 24);
  b[0] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  b[1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

// activations of one Q4 block (as loaded) -> the order of decode_q4
__device__ __forceinline__ void act_order_q4(const uint32_t* x, uint32_t* a) {
  a[0] = __builtin_amdgcn_perm(x[2], x[0], 0x05040100u);
  a[1] = __builtin_amdgcn_perm(x[2], x[0], 0x07060302u);
  a[2] = __builtin_amdgcn_perm(x[3], x[1], 0x05040100u);
  a[3] = __builtin_amdgcn_perm(x[3], x[1], 0x07060302u);
}

}  // namespace mfma
}  // namespace mlxq
