// GGUF block decoding shared by the dequantizer (gguf.hip) and the fused
// dequantize + requantize converter (gguf_requant.hip).
//
// Reference: the per-type block decoders of src/gguf/dequant.rs (:228-719),
// solved for one element: decode<TAG>(block, j) is element j of a block, with
// exactly the IEEE f32 operations, operand order and roundings the reference
// uses for it.  Every file that includes this header is compiled with
// -ffp-contract=off so no mul+add/sub is fused; f16 scales are decoded with
// integer bit operations.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"
#include "iq_tables.h"

namespace mlxq {
namespace {  // internal linkage: each including file has its own copy

constexpr int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                               1,    13,   25,  38,  53,  69,  89,  113};
// The codebook as four little-endian dwords of bytes, so a lookup is a
// v_perm byte select in registers instead of a per-lane memory load.
constexpr uint32_t iq4nl_word(int w) {
  return static_cast<uint32_t>(static_cast<uint8_t>(kIq4nl[4 * w])) |
         (static_cast<uint32_t>(static_cast<uint8_t>(kIq4nl[4 * w + 1])) << 8) |
         (static_cast<uint32_t>(static_cast<uint8_t>(kIq4nl[4 * w + 2])) << 16) |
         (static_cast<uint32_t>(static_cast<uint8_t>(kIq4nl[4 * w + 3])) << 24);
}
// kIq4nl[q] for q in 0..15.  Two forms, chosen per including file by what
// measured faster there: the memory-bound dequantizer defines
// MLXQ_IQ4NL_IN_REGISTERS (v_perm picks byte q & 7 of the 8-byte half
// selected by q & 8; selector values 0-3 address the second operand: 51 ->
// 44 us for a 14336x4096 IQ4_NL tensor), the VALU-bound converter keeps the
// table load (56 vs 61 us with the v_perm form).
#ifdef MLXQ_IQ4NL_IN_REGISTERS
__device__ __forceinline__ int iq4nl_value(uint32_t q) {
  const uint32_t sel = q & 7u;
  const uint32_t lo = __builtin_amdgcn_perm(iq4nl_word(1), iq4nl_word(0), sel);
  const uint32_t hi = __builtin_amdgcn_perm(iq4nl_word(3), iq4nl_word(2), sel);
  return static_cast<int8_t>((q & 8u) ? hi : lo);
}
#else
__constant__ int8_t kIq4nlDev[16] = {kIq4nl[0],  kIq4nl[1],  kIq4nl[2],  kIq4nl[3],  kIq4nl[4],  kIq4nl[5],
                                     kIq4nl[6],  kIq4nl[7],  kIq4nl[8],  kIq4nl[9],  kIq4nl[10], kIq4nl[11],
                                     kIq4nl[12], kIq4nl[13], kIq4nl[14], kIq4nl[15]};
__device__ __forceinline__ int iq4nl_value(uint32_t q) { return kIq4nlDev[q]; }
#endif

__device__ __forceinline__ float rd_f16(const uint8_t* b, int i) {
  return f16_bits_to_f32(static_cast<uint32_t>(b[i]) | (static_cast<uint32_t>(b[i + 1]) << 8));
}
__device__ __forceinline__ uint32_t rd_u32(const uint8_t* b) {
  return static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8) |
         (static_cast<uint32_t>(b[2]) << 16) | (static_cast<uint32_t>(b[3]) << 24);
}

// get_scale_min_k4 (dequant.rs:375-383).  Branch-free (j differs between
// the lanes of a wave, so a branch would run both sides): with a = q[j & 3],
// b = q[(j & 3) + 4], c = q[(j & 3) + 8], sub-blocks 0-3 take the low 6 bits
// of a / b, sub-blocks 4-7 the nibbles of c plus the top 2 bits of a / b.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint32_t& d, uint32_t& m) {
  const int j3 = j & 3;
  const uint32_t a = q[j3], b = q[j3 + 4], c = q[j3 + 8];
  const bool low = j < 4;
  d = low ? (a & 63u) : ((c & 0x0Fu) | ((a >> 6) << 4));
  m = low ? (b & 63u) : ((c >> 4) | ((b >> 6) << 4));
}

// One element j of a block at b (LDS).  Tag is a template constant.
template <int TAG>
__device__ __forceinline__ float decode(const uint8_t* b, int j);

// Q4_0 (dequant.rs:228-237): y[j]=(lo-8)*d, y[j+16]=(hi-8)*d
template <>
__device__ __forceinline__ float decode<2>(const uint8_t* b, int j) {
  float d = rd_f16(b, 0);
  uint32_t byte = b[2 + (j & 15)];
  int q = static_cast<int>(j < 16 ? (byte & 0xFu) : (byte >> 4)) - 8;
  return static_cast<float>(q) * d;
}
// Q4_1 (dequant.rs:239-247): q*d + m
template <>
__device__ __forceinline__ float decode<3>(const uint8_t* b, int j) {
  float d = rd_f16(b, 0), m = rd_f16(b, 2);
  uint32_t byte = b[4 + (j & 15)];
  uint32_t q = j < 16 ? (byte & 0xFu) : (byte >> 4);
  return static_cast<float>(q) * d + m;
}
// Q5_0 (dequant.rs:249-261)
template <>
__device__ __forceinline__ float decode<6>(const uint8_t* b, int j) {
  float d = rd_f16(b, 0);
  uint32_t qh = rd_u32(b + 2);
  int jj = j & 15;
  uint32_t byte = b[6 + jj];
  uint32_t x;
  if (j < 16) x = (byte & 0xFu) | (((qh >> jj) << 4) & 0x10u);
  else x = (byte >> 4) | ((qh >> (jj + 12)) & 0x10u);
  return static_cast<float>(static_cast<int>(x) - 16) * d;
}
// Q5_1 (dequant.rs:263-276)
template <>
__device__ __forceinline__ float decode<7>(const uint8_t* b, int j) {
  float d = rd_f16(b, 0), m = rd_f16(b, 2);
  uint32_t qh = rd_u32(b + 4);
  int jj = j & 15;
  uint32_t byte = b[8 + jj];
  uint32_t x;
  if (j < 16) x = (byte & 0xFu) | (((qh >> jj) << 4) & 0x10u);
  else x = (byte >> 4) | ((qh >> (jj + 12)) & 0x10u);
  return static_cast<float>(x) * d + m;
}
// Q8_0 (dequant.rs:278-284)
template <>
__device__ __forceinline__ float decode<8>(const uint8_t* b, int j) {
  float d = rd_f16(b, 0);
  return static_cast<float>(static_cast<int8_t>(b[2 + j])) * d;
}
// Q2_K (dequant.rs:288-318): element j -> half h (128), shift round r (32),
// 16-lane half l2/16 selecting scales[8h + 2r + l2/16].
template <>
__device__ __forceinline__ float decode<10>(const uint8_t* b, int j) {
  int h = j >> 7, r = (j >> 5) & 3, l2 = j & 31;
  uint32_t sc = b[8 * h + 2 * r + (l2 >> 4)];
  float d = rd_f16(b, 80), dmin = rd_f16(b, 82);
  float dl = d * static_cast<float>(sc & 0xFu);
  float ml = dmin * static_cast<float>(sc >> 4);
  uint32_t qb = b[16 + 32 * h + l2];
  return dl * static_cast<float>((qb >> (2 * r)) & 3u) - ml;
}
// Q3_K (dequant.rs:320-371)
template <>
__device__ __forceinline__ float decode<11>(const uint8_t* b, int j) {
  const uint32_t K1 = 0x03030303u, K2 = 0x0f0f0f0fu;
  int h = j >> 7, r = (j >> 5) & 3, l2 = j & 31;
  int is = 8 * h + 2 * r + (l2 >> 4);
  uint32_t a0 = rd_u32(b + 96), a1 = rd_u32(b + 100), tmp = rd_u32(b + 104);
  uint32_t aux;
  switch (is >> 2) {
    case 0: aux = (a0 & K2) | ((tmp & K1) << 4); break;
    case 1: aux = (a1 & K2) | (((tmp >> 2) & K1) << 4); break;
    case 2: aux = ((a0 >> 4) & K2) | (((tmp >> 4) & K1) << 4); break;
    default: aux = ((a1 >> 4) & K2) | (((tmp >> 6) & K1) << 4); break;
  }
  int sc = static_cast<int8_t>((aux >> (8 * (is & 3))) & 0xFFu);
  float d_all = rd_f16(b, 108);
  float dl = d_all * static_cast<float>(sc - 32);
  uint32_t m = 1u << (4 * h + r);
  int hbit = (b[l2] & m) ? 0 : 4;
  uint32_t qb = b[32 + 32 * h + l2];
  return dl * static_cast<float>(static_cast<int>((qb >> (2 * r)) & 3u) - hbit);
}
// Q4_K (dequant.rs:385-410)
template <>
__device__ __forceinline__ float decode<12>(const uint8_t* b, int j) {
  int c = j >> 6, hi = (j >> 5) & 1, l = j & 31;
  uint32_t sc, m;
  scale_min_k4(2 * c + hi, b + 4, sc, m);
  float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
  float d1 = d * static_cast<float>(sc);
  float m1 = dmin * static_cast<float>(m);
  uint32_t qb = b[16 + 32 * c + l];
  uint32_t q = hi ? (qb >> 4) : (qb & 0xFu);
  return d1 * static_cast<float>(q) - m1;
}
// Q5_K (dequant.rs:412-444)
template <>
__device__ __forceinline__ float decode<13>(const uint8_t* b, int j) {
  int c = j >> 6, hi = (j >> 5) & 1, l = j & 31;
  uint32_t sc, m;
  scale_min_k4(2 * c + hi, b + 4, sc, m);
  float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
  float d1 = d * static_cast<float>(sc);
  float m1 = dmin * static_cast<float>(m);
  uint32_t u = (hi ? 2u : 1u) << (2 * c);
  int hib = (b[16 + l] & u) ? 16 : 0;
  uint32_t qb = b[48 + 32 * c + l];
  int q = static_cast<int>(hi ? (qb >> 4) : (qb & 0xFu)) + hib;
  return d1 * static_cast<float>(q) - m1;
}
// Q6_K (dequant.rs:446-468): (d * scale) * q, left to right
template <>
__device__ __forceinline__ float decode<14>(const uint8_t* b, int j) {
  int idx = j >> 7, t = (j >> 5) & 3, l = j & 31;
  const uint8_t* qlp = b + 64 * idx;
  const uint8_t* qhp = b + 128 + 32 * idx;
  // branch-free: byte l or l + 32 of ql, low or high nibble
  const uint32_t lo = (static_cast<uint32_t>(qlp[l + 32 * (t & 1)]) >> (4 * (t >> 1))) & 0xFu;
  uint32_t hb = (qhp[l] >> (2 * t)) & 3u;
  int q = static_cast<int>(static_cast<int8_t>(lo | (hb << 4))) - 32;
  int sc = static_cast<int8_t>(b[192 + 8 * idx + (l >> 4) + 2 * t]);
  float d = rd_f16(b, 208);
  return d * static_cast<float>(sc) * static_cast<float>(q);
}
// IQ4_NL (dequant.rs:472-479)
template <>
__device__ __forceinline__ float decode<20>(const uint8_t* b, int j) {
  float d = rd_f16(b, 0);
  uint32_t byte = b[2 + (j & 15)];
  uint32_t q = j < 16 ? (byte & 0xFu) : (byte >> 4);
  return d * static_cast<float>(iq4nl_value(q));
}
// IQ4_XS (dequant.rs:481-497)
template <>
__device__ __forceinline__ float decode<23>(const uint8_t* b, int j) {
  int ib = j >> 5, jj = j & 31;
  float d = rd_f16(b, 0);
  uint32_t sh = static_cast<uint32_t>(b[2]) | (static_cast<uint32_t>(b[3]) << 8);
  int ls = static_cast<int>((b[4 + (ib >> 1)] >> (4 * (ib & 1))) & 0xFu) |
           static_cast<int>(((sh >> (2 * ib)) & 3u) << 4);
  float dl = d * static_cast<float>(ls - 32);
  uint32_t byte = b[8 + 16 * ib + (jj & 15)];
  uint32_t q = jj < 16 ? (byte & 0xFu) : (byte >> 4);
  return dl * static_cast<float>(iq4nl_value(q));
}

// ---- IQ grid types (dequant.rs:505-719).  Codebooks: the format's fixed
// tables (iq_tables.h).  ksigns_iq2xs is computed: entry i is i with bit 7 =
// parity of i.
__constant__ uint64_t kIq2xxs[256] = {MLXQ_IQ2XXS_GRID};
__constant__ uint64_t kIq2xs[512] = {MLXQ_IQ2XS_GRID};
__constant__ uint64_t kIq2s[1024] = {MLXQ_IQ2S_GRID};
__constant__ uint32_t kIq3xxs[256] = {MLXQ_IQ3XXS_GRID};
__constant__ uint32_t kIq3s[512] = {MLXQ_IQ3S_GRID};
__constant__ uint64_t kIq1s[2048] = {MLXQ_IQ1S_GRID};
constexpr float kIq1sDelta = 0.125f;  // dequant.rs:26-27

__device__ __forceinline__ uint32_t ksigns(uint32_t i) {
  i &= 127u;
  return i | ((__popc(i) & 1u) << 7);
}
// output lane jj's sign: -1 where bit jj of the sign byte is set (dequant.rs:508-516)
__device__ __forceinline__ float iq_sign(uint32_t s, int jj) { return (s >> jj) & 1u ? -1.0f : 1.0f; }
__device__ __forceinline__ uint32_t grid_byte(uint64_t g, int jj) {
  return static_cast<uint32_t>(g >> (8 * jj)) & 0xFFu;
}

// IQ2_XXS (dequant.rs:521-539): 32-block ib32, 8-lane group l, lane jj
template <>
__device__ __forceinline__ float decode<16>(const uint8_t* b, int j) {
  const int ib32 = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  const float d = rd_f16(b, 0);
  const uint8_t* q = b + 2 + 8 * ib32;
  const uint32_t aux1 = rd_u32(q + 4);
  const float db = d * (0.5f + static_cast<float>(aux1 >> 28)) * 0.25f;
  const uint64_t g = kIq2xxs[q[l]];
  return db * static_cast<float>(grid_byte(g, jj)) * iq_sign(ksigns(aux1 >> (7 * l)), jj);
}
// IQ2_XS (dequant.rs:543-564)
template <>
__device__ __forceinline__ float decode<17>(const uint8_t* b, int j) {
  const int ib32 = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  const float d = rd_f16(b, 0);
  const uint32_t sc = b[66 + ib32];
  const float db = d * (0.5f + static_cast<float>(l < 2 ? (sc & 0xFu) : (sc >> 4))) * 0.25f;
  const int qo = 2 + 2 * (4 * ib32 + l);
  const uint32_t q = static_cast<uint32_t>(b[qo]) | (static_cast<uint32_t>(b[qo + 1]) << 8);
  const uint64_t g = kIq2xs[q & 511u];
  return db * static_cast<float>(grid_byte(g, jj)) * iq_sign(ksigns(q >> 9), jj);
}
// IQ2_S (dequant.rs:568-591)
template <>
__device__ __forceinline__ float decode<22>(const uint8_t* b, int j) {
  const int ib32 = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  const float d = rd_f16(b, 0);
  const uint32_t sc = b[74 + ib32];
  const float db = d * (0.5f + static_cast<float>(l < 2 ? (sc & 0xFu) : (sc >> 4))) * 0.25f;
  const uint32_t idx = b[2 + 4 * ib32 + l] | ((static_cast<uint32_t>(b[66 + ib32]) << (8 - 2 * l)) & 0x300u);
  const uint64_t g = kIq2s[idx];
  return db * static_cast<float>(grid_byte(g, jj)) * iq_sign(b[34 + 4 * ib32 + l], jj);
}
// IQ3_XXS (dequant.rs:596-615): lanes 0-3 from grid point 2l, 4-7 from 2l+1
template <>
__device__ __forceinline__ float decode<18>(const uint8_t* b, int j) {
  const int ib32 = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  const float d = rd_f16(b, 0);
  const uint32_t aux = rd_u32(b + 66 + 4 * ib32);
  const float db = d * (0.5f + static_cast<float>(aux >> 28)) * 0.5f;
  const uint32_t g = kIq3xxs[b[2 + 8 * ib32 + 2 * l + (jj >> 2)]];
  return db * static_cast<float>(grid_byte(g, jj & 3)) * iq_sign(ksigns(aux >> (7 * l)), jj);
}
// IQ3_S (dequant.rs:619-651): 64-element pair k, its half, 8-lane group l
template <>
__device__ __forceinline__ float decode<21>(const uint8_t* b, int j) {
  const int k = j >> 6, half = (j >> 5) & 1, l = (j >> 3) & 3, jj = j & 7;
  const float d = rd_f16(b, 0);
  const uint32_t sc = b[106 + k];
  const float db = d * static_cast<float>(1 + 2 * static_cast<int>(half ? (sc >> 4) : (sc & 0xFu)));
  const uint32_t qhb = b[66 + 2 * k + half];
  const uint8_t* q = b + 2 + 16 * k + 8 * half;
  const uint32_t idx = jj < 4 ? (q[2 * l] | ((qhb << (8 - 2 * l)) & 256u))
                              : (q[2 * l + 1] | ((qhb << (7 - 2 * l)) & 256u));
  const uint32_t g = kIq3s[idx];
  return db * static_cast<float>(grid_byte(g, jj & 3)) * iq_sign(b[74 + 8 * k + 4 * half + l], jj);
}
// IQ1_S (dequant.rs:655-673): signed grid plus a +-delta offset
template <>
__device__ __forceinline__ float decode<19>(const uint8_t* b, int j) {
  const int ib = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  const float d = rd_f16(b, 0);
  const uint32_t h = static_cast<uint32_t>(b[34 + 2 * ib]) | (static_cast<uint32_t>(b[35 + 2 * ib]) << 8);
  const float dl = d * static_cast<float>(2 * static_cast<int>((h >> 12) & 7u) + 1);
  const float delta = (h & 0x8000u) ? -kIq1sDelta : kIq1sDelta;
  const uint32_t idx = b[2 + 4 * ib + l] | (((h >> (3 * l)) & 7u) << 8);
  const int v = static_cast<int8_t>(grid_byte(kIq1s[idx], jj));
  return dl * (static_cast<float>(v) + delta);
}
// IQ1_M (dequant.rs:678-719): f16 scale from the top nibbles of the four
// scale words, two 3-bit sub-scales per 32-block
template <>
__device__ __forceinline__ float decode<29>(const uint8_t* b, int j) {
  const int ib = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  uint32_t sc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) sc[i] = static_cast<uint32_t>(b[48 + 2 * i]) | (static_cast<uint32_t>(b[49 + 2 * i]) << 8);
  const uint32_t bits = (sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0u) | ((sc[2] >> 4) & 0x0F00u) | (sc[3] & 0xF000u);
  const float d = f16_bits_to_f32(bits);
  const uint32_t w = sc[ib >> 1];
  const int shift = 6 * (ib & 1) + (l < 2 ? 0 : 3);
  const float dl = d * static_cast<float>(2 * static_cast<int>((w >> shift) & 7u) + 1);
  const uint32_t qh = b[32 + 2 * ib + (l >> 1)];
  const uint32_t idx = b[4 * ib + l] | ((l & 1) ? ((qh << 4) & 0x700u) : ((qh << 8) & 0x700u));
  const float delta = (qh & ((l & 1) ? 0x80u : 0x08u)) ? -kIq1sDelta : kIq1sDelta;
  const int v = static_cast<int8_t>(grid_byte(kIq1s[idx], jj));
  return dl * (static_cast<float>(v) + delta);
}

template <int TAG> struct Geo;
template <> struct Geo<2> { static constexpr int E = 32, B = 18; };
template <> struct Geo<3> { static constexpr int E = 32, B = 20; };
template <> struct Geo<6> { static constexpr int E = 32, B = 22; };
template <> struct Geo<7> { static constexpr int E = 32, B = 24; };
template <> struct Geo<8> { static constexpr int E = 32, B = 34; };
template <> struct Geo<10> { static constexpr int E = 256, B = 84; };
template <> struct Geo<11> { static constexpr int E = 256, B = 110; };
template <> struct Geo<12> { static constexpr int E = 256, B = 144; };
template <> struct Geo<13> { static constexpr int E = 256, B = 176; };
template <> struct Geo<14> { static constexpr int E = 256, B = 210; };
template <> struct Geo<20> { static constexpr int E = 32, B = 18; };
template <> struct Geo<23> { static constexpr int E = 256, B = 136; };
template <> struct Geo<16> { static constexpr int E = 256, B = 66; };
template <> struct Geo<17> { static constexpr int E = 256, B = 74; };
template <> struct Geo<22> { static constexpr int E = 256, B = 82; };
template <> struct Geo<18> { static constexpr int E = 256, B = 98; };
template <> struct Geo<21> { static constexpr int E = 256, B = 110; };
template <> struct Geo<19> { static constexpr int E = 256, B = 50; };
template <> struct Geo<29> { static constexpr int E = 256, B = 56; };

}  // namespace
}  // namespace mlxq
