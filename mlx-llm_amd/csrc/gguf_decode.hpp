// GGUF block decoding shared by the dequantizer (gguf.hip) and the fused
// dequantize + requantize converter (gguf_requant.hip).
//
// Reference: the per-type block decoders of src/gguf/dequant.rs (:228-497),
// solved for one element: decode<TAG>(block, j) is element j of a block, with
// exactly the IEEE f32 operations, operand order and roundings the reference
// uses for it.  Every file that includes this header is compiled with
// -ffp-contract=off so no mul+add/sub is fused; f16 scales are decoded with
// integer bit operations.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace mlxq {
namespace {  // internal linkage: each including file has its own copy

__constant__ int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};

__device__ __forceinline__ float rd_f16(const uint8_t* b, int i) {
  return f16_bits_to_f32(static_cast<uint32_t>(b[i]) | (static_cast<uint32_t>(b[i + 1]) << 8));
}
__device__ __forceinline__ uint32_t rd_u32(const uint8_t* b) {
  return static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8) |
         (static_cast<uint32_t>(b[2]) << 16) | (static_cast<uint32_t>(b[3]) << 24);
}

// get_scale_min_k4 (dequant.rs:375-383)
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint32_t& d, uint32_t& m) {
  if (j < 4) {
    d = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    d = (q[j + 4] & 0x0Fu) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
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
  uint32_t lo = (t & 1) ? qlp[l + 32] : qlp[l];
  lo = (t & 2) ? (lo >> 4) : (lo & 0xFu);
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
  return d * static_cast<float>(kIq4nl[q]);
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
  return dl * static_cast<float>(kIq4nl[q]);
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

}  // namespace
}  // namespace mlxq
