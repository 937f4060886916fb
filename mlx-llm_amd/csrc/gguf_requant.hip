// Fused GGUF -> MLX affine requantization of a projection weight, on device.
//
// Reference: the convert chain of src/gguf/convert.rs for a projection
// tensor: dequantize (:131, dequant.rs:156-211), the llama q/k row
// un-permute (:133-137, permute_inverse_qk :232-256), the cast to bf16
// (:156, as_dtype(bf16): round to nearest even) and the snapshot writer's
// requant (:176 -> snapshot.rs:100-107 -> quant.rs:44, mlx quantize of the
// bf16 tensor).  The reference materializes the whole f32 tensor on the host
// and then the bf16 copy; here every lane gathers the 8 consecutive elements
// of its output row straight from the GGUF blocks (un-permuted source row),
// rounds them to bf16 and quantizes its share of the group in registers, so
// the only HBM traffic is the GGUF bytes in and the packed MLX tensor out.
//
// Bit-exactness: the element decode (gguf_decode.hpp) and the group
// quantization (affine_group.hpp) are the ones of mlxq_gguf_dequantize and
// mlxq_quantize; this file is compiled with -ffp-contract=off.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "affine_group.hpp"
#include "common.hpp"
#include "gguf_decode.hpp"

namespace mlxq {
namespace {

constexpr int kThreads = 256;
constexpr int kEpl = 16;  // elements per lane

// Element e of a float-typed GGUF tensor (F32 = 0, F16 = 1, BF16 = 30).
template <int TAG>
__device__ __forceinline__ float float_elem(const uint8_t* d, int64_t e) {
  if constexpr (TAG == 0) {
    return __uint_as_float(rd_u32(d + 4 * e));
  } else if constexpr (TAG == 1) {
    return f16_bits_to_f32(static_cast<uint32_t>(d[2 * e]) | (static_cast<uint32_t>(d[2 * e + 1]) << 8));
  } else {
    return bf16_bits_to_f32(static_cast<uint32_t>(d[2 * e]) | (static_cast<uint32_t>(d[2 * e + 1]) << 8));
  }
}

template <int TAG>
constexpr bool is_float_tag() {
  return TAG == 0 || TAG == 1 || TAG == 30;
}

// 16 bytes per lane from global memory straight into LDS: a wave's active
// lanes fill lane * 16 bytes from `l` (no registers held while in flight)
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}

// Source row of output row r: perm_hd > 0 un-permutes llama.cpp's q/k head
// interleave -- within head h = r / perm_hd, output row rr = r % perm_hd
// reads source row h * perm_hd + 2 * (rr % half) + rr / half (half =
// perm_hd / 2).
__device__ __forceinline__ int source_row(int r, int perm_hd) {
  if (perm_hd <= 0) return r;
  const int h = r / perm_hd, rr = r - h * perm_hd, half = perm_hd / 2;
  return h * perm_hd + 2 * (rr % half) + rr / half;
}

// The 16 consecutive elements j0 .. j0 + 15 (j0 a multiple of 16) of the
// block at b (LDS), with the per-element arithmetic of decode<TAG> in the
// same order (bit-identical), for the formats where one lane's 16 elements
// share their bytes' layout: one nibble half of 16 consecutive bytes and one
// scale.  decode<TAG> takes j at run time, so per element it re-derives the
// half, the byte and (k-quants) the sub-block scale; here they are derived
// once per lane and the bytes are read as whole 2- or 16-byte words.
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

template <int TAG>
__device__ __forceinline__ void decode16(const uint8_t* b, int j0, float (&v)[kEpl]) {
  if constexpr (TAG == 2 || TAG == 20) {
    // Q4_0 / IQ4_NL: element j0 + k is nibble (j0 / 16) of byte 2 + k
    const float d = rd_f16(b, 0);
    const int sh = (j0 >> 2) & 4;
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
      const uint32_t w = lds_u16(b + 2 + k);
      const uint32_t q0 = (w >> sh) & 0xFu, q1 = (w >> (sh + 8)) & 0xFu;
      if constexpr (TAG == 2) {
        v[k] = static_cast<float>(static_cast<int>(q0) - 8) * d;
        v[k + 1] = static_cast<float>(static_cast<int>(q1) - 8) * d;
      } else {
        v[k] = d * static_cast<float>(iq4nl_value(q0));
        v[k + 1] = d * static_cast<float>(iq4nl_value(q1));
      }
    }
  } else if constexpr (TAG == 8) {
    // Q8_0: element j0 + k is the signed byte 2 + j0 + k
    const float d = rd_f16(b, 0);
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
      const uint32_t w = lds_u16(b + 2 + j0 + k);
      v[k] = static_cast<float>(static_cast<int8_t>(w & 0xFFu)) * d;
      v[k + 1] = static_cast<float>(static_cast<int8_t>(w >> 8)) * d;
    }
  } else if constexpr (TAG == 12) {
    // Q4_K: sub-block 2c + hi; bytes 16 + 32c + (j0 & 31) .. +15 (16-byte aligned)
    const int c = j0 >> 6, hi = (j0 >> 5) & 1;
    uint32_t sc, m;
    scale_min_k4(2 * c + hi, b + 4, sc, m);
    const float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
    const float d1 = d * static_cast<float>(sc);
    const float m1 = dmin * static_cast<float>(m);
    const uint4 q = *reinterpret_cast<const uint4*>(b + 16 + 32 * c + (j0 & 31));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const int sh = 4 * hi;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t nib = (w[k >> 2] >> (8 * (k & 3) + sh)) & 0xFu;
      v[k] = d1 * static_cast<float>(nib) - m1;
    }
  } else if constexpr (TAG == 14) {
    // Q6_K: 128-half idx, quarter t, bytes l = (j0 & 31) + k of ql (at 32 (t & 1),
    // nibble t / 2) and qh (2-bit field t); one scale per 16 elements
    const int idx = j0 >> 7, t = (j0 >> 5) & 3, l0 = j0 & 31;
    const uint8_t* qlp = b + 64 * idx + 32 * (t & 1) + l0;
    const uint8_t* qhp = b + 128 + 32 * idx + l0;
    const int sc = static_cast<int8_t>(b[192 + 8 * idx + (l0 >> 4) + 2 * t]);
    const float ds = rd_f16(b, 208) * static_cast<float>(sc);
    const int shl = 4 * (t >> 1), shh = 2 * t;
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
      const uint32_t wl = lds_u16(qlp + k), wh = lds_u16(qhp + k);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const uint32_t lo = (wl >> (8 * e + shl)) & 0xFu, hb = (wh >> (8 * e + shh)) & 3u;
        const int q = static_cast<int>(static_cast<int8_t>(lo | (hb << 4))) - 32;
        v[k + e] = ds * static_cast<float>(q);
      }
    }
  } else if constexpr (TAG == 23) {
    // IQ4_XS: sub-block ib, nibble (j0 / 16) & 1 of bytes 8 + 16 ib .. +15 (8-byte aligned)
    const int ib = j0 >> 5;
    const float d = rd_f16(b, 0);
    const uint32_t shw = static_cast<uint32_t>(b[2]) | (static_cast<uint32_t>(b[3]) << 8);
    const int ls = static_cast<int>((b[4 + (ib >> 1)] >> (4 * (ib & 1))) & 0xFu) |
                   static_cast<int>(((shw >> (2 * ib)) & 3u) << 4);
    const float dl = d * static_cast<float>(ls - 32);
    const uint2 q0 = *reinterpret_cast<const uint2*>(b + 8 + 16 * ib);
    const uint2 q1 = *reinterpret_cast<const uint2*>(b + 16 + 16 * ib);
    const uint32_t w[4] = {q0.x, q0.y, q1.x, q1.y};
    const int sh = (j0 >> 2) & 4;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t nib = (w[k >> 2] >> (8 * (k & 3) + sh)) & 0xFu;
      v[k] = dl * static_cast<float>(iq4nl_value(nib));
    }
  }
}
template <int TAG>
constexpr bool has_decode16() {
  return TAG == 2 || TAG == 8 || TAG == 12 || TAG == 14 || TAG == 20 || TAG == 23;
}

// A workgroup converts `rpw` consecutive output rows.  All of their source
// rows' GGUF bytes are requested up front (direct global -> LDS loads when
// 16-byte aligned, so the bytes in flight per CU are those of every resident
// workgroup's rows), then every lane decodes 16 consecutive elements of a row
// from LDS, rounds them to bf16 and quantizes its share of the group.
// Each lane takes kEpl = 16 elements (LPG lanes per group), so the
// per-block header decode and the per-group scale arithmetic, which every
// lane of a group repeats, are shared by twice as many elements as with 8.

template <int TAG, int BITS, int LPG, bool ALIGNED16>
__global__ __launch_bounds__(kThreads) void gguf_requant_kernel(const uint8_t* __restrict__ data, int rows, int K,
                                                                 int row_bytes, int perm_hd, int rpw,
                                                                 uint32_t* __restrict__ wq,
                                                                 uint16_t* __restrict__ scales,
                                                                 uint16_t* __restrict__ biases) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int lpr = K / kEpl;  // lanes (kEpl elements each) per row
  const int r0 = blockIdx.x * rpw;
  const int nr = min(rpw, rows - r0);
  const int tid = threadIdx.x;
  if constexpr (ALIGNED16) {
    const int n16 = row_bytes >> 4;
    const int pieces = (n16 + 63) >> 6;  // 1 KB wave loads per row
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    for (int t = wave; t < nr * pieces; t += kThreads / 64) {
      const int i = t / pieces, p = t - i * pieces, q = p * 64 + lane;
      const uint8_t* src = data + static_cast<int64_t>(source_row(r0 + i, perm_hd)) * row_bytes;
      if (q < n16) lds_dma16(src + q * 16, lds + i * row_bytes + p * 1024);
    }
    __builtin_amdgcn_s_waitcnt(0);
  } else {
    for (int i = 0; i < nr; i++) {
      const uint8_t* src = data + static_cast<int64_t>(source_row(r0 + i, perm_hd)) * row_bytes;
      for (int j = tid; j < row_bytes; j += kThreads) lds[i * row_bytes + j] = src[j];
    }
  }
  __syncthreads();
  for (int i = 0; i < nr; i++) {
    const int r = r0 + i;
    const uint8_t* row = lds + i * row_bytes;
    // lanes of the row in whole groups per pass (kThreads is a multiple of LPG
    // and lpr of LPG, so a group's lanes are active together)
    for (int l0 = 0; l0 < lpr; l0 += kThreads) {
      const int l = l0 + tid;
      const bool active = l < lpr;
      float v[kEpl];
#pragma unroll
      for (int j = 0; j < kEpl; j++) v[j] = 0.f;
      if (active) {
        const int e = l * kEpl;
        if constexpr (is_float_tag<TAG>()) {
#pragma unroll
          for (int j = 0; j < kEpl; j++) v[j] = float_elem<TAG>(row, e + j);
        } else {
          constexpr int E = Geo<TAG>::E, B = Geo<TAG>::B;
          static_assert(E % kEpl == 0, "a lane's elements never straddle a block");
          const int blk = e / E;
          const uint8_t* b = row + blk * B;
          if constexpr (has_decode16<TAG>()) {
            decode16<TAG>(b, e - blk * E, v);
          } else {
#pragma unroll
            for (int j = 0; j < kEpl; j++) v[j] = decode<TAG>(b, e - blk * E + j);
          }
        }
#pragma unroll
        for (int j = 0; j < kEpl; j++) v[j] = static_cast<float>(static_cast<__bf16>(v[j]));  // as_dtype(bf16): v_cvt_pk_bf16_f32, round to nearest even (a NaN payload cannot reach a code: max/min skip NaN and a NaN quotient clamps to 0)
      }
      uint32_t codes[kEpl];
      float scale, bias;
      quantize_group8<BITS, LPG, kEpl>(v, codes, scale, bias);  // every lane of the group takes part
      if (active) {
        const int64_t lane = static_cast<int64_t>(r) * lpr + l;
        store_codes16<BITS>(wq, lane, codes);
        if ((l & (LPG - 1)) == 0) {
          const int64_t g = lane / LPG;
          scales[g] = static_cast<uint16_t>(f32_to_bf16_bits(scale));
          biases[g] = static_cast<uint16_t>(f32_to_bf16_bits(bias));
        }
      }
    }
  }
}

// Rows per workgroup: as many as fit 32 KB of LDS (at most 8), so that a
// CU's resident workgroups keep ~100 KB of GGUF bytes in flight.
inline int rows_per_workgroup(int row_bytes) {
  return std::max(1, std::min(8, (32 * 1024) / std::max(row_bytes, 1)));
}

template <int TAG, int BITS, int LPG>
int launch_lpg(int rows, int K, int row_bytes, int perm_hd, const uint8_t* d, uint32_t* wq, uint16_t* s,
               uint16_t* b, hipStream_t st) {
  const bool al = (reinterpret_cast<uintptr_t>(d) & 15u) == 0 && row_bytes % 16 == 0;
  const int rpw = rows_per_workgroup(row_bytes);
  const size_t lds = static_cast<size_t>(rpw) * row_bytes;
  const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw));
  auto kern = al ? gguf_requant_kernel<TAG, BITS, LPG, true> : gguf_requant_kernel<TAG, BITS, LPG, false>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("gguf_requantize: LDS size: ") + hipGetErrorString(e));
  }
  MLXQ_LAUNCH(kern, grid, dim3(kThreads), lds, st, d, rows, K, row_bytes, perm_hd, rpw, wq, s, b);
  return check_launch("gguf_requantize");
}

template <int TAG, int BITS>
int launch_bits(int group_size, int rows, int K, int row_bytes, int perm_hd, const uint8_t* d, uint32_t* wq,
                uint16_t* s, uint16_t* b, hipStream_t st) {
  if (group_size == 32) return launch_lpg<TAG, BITS, 32 / kEpl>(rows, K, row_bytes, perm_hd, d, wq, s, b, st);
  if (group_size == 64) return launch_lpg<TAG, BITS, 64 / kEpl>(rows, K, row_bytes, perm_hd, d, wq, s, b, st);
  return launch_lpg<TAG, BITS, 128 / kEpl>(rows, K, row_bytes, perm_hd, d, wq, s, b, st);
}

template <int TAG>
int launch_tag(int bits, int group_size, int rows, int K, int row_bytes, int perm_hd, const uint8_t* d,
               uint32_t* wq, uint16_t* s, uint16_t* b, hipStream_t st) {
  if (bits == 4) return launch_bits<TAG, 4>(group_size, rows, K, row_bytes, perm_hd, d, wq, s, b, st);
  return launch_bits<TAG, 8>(group_size, rows, K, row_bytes, perm_hd, d, wq, s, b, st);
}

}  // namespace
}  // namespace mlxq

using namespace mlxq;

extern "C" int mlxq_gguf_requantize(uint32_t tag, const void* data, int64_t data_len, int64_t rows, int64_t cols,
                                    int permute_heads, int group_size, int bits, uint32_t* wq, void* scales,
                                    void* biases, void* stream) {
  clear_error();
  if (bits != 4 && bits != 8) return fail(MLXQ_ERR_UNSUPPORTED, "gguf_requantize: bits must be 4 or 8");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MLXQ_ERR_UNSUPPORTED, "gguf_requantize: group_size must be 32, 64 or 128");
  if (rows < 0 || cols <= 0 || permute_heads < 0) return fail(MLXQ_ERR_INVALID, "gguf_requantize: bad shape");
  if (cols % group_size)
    return fail(MLXQ_ERR_SHAPE, "gguf_requantize: cols=" + std::to_string(cols) + " not divisible by group_size");
  if (cols > INT32_MAX / 2 || rows > INT32_MAX) return fail(MLXQ_ERR_INVALID, "gguf_requantize: too large");
  int64_t elems = 0, bbytes = 0;
  if (int rc = mlxq_gguf_block(tag, &elems, &bbytes)) return rc;
  const bool device_tag = tag == 0 || tag == 1 || tag == 30 || tag == 2 || tag == 3 || tag == 6 || tag == 7 ||
                          tag == 8 || tag == 10 || tag == 11 || tag == 12 || tag == 13 || tag == 14 || tag == 20 ||
                          tag == 23 || tag == 16 || tag == 17 || tag == 22 || tag == 18 || tag == 21 || tag == 19 ||
                          tag == 29;
  if (!device_tag) return fail(MLXQ_ERR_UNSUPPORTED, "gguf_requantize: GGUF type " + std::to_string(tag) +
                                                         " has no device decoder");
  if (cols % elems) return fail(MLXQ_ERR_SHAPE, "gguf_requantize: rows must hold whole blocks");
  const int64_t n = rows * cols;
  const int64_t need = n / elems * bbytes;
  if (data_len < need)
    return fail(MLXQ_ERR_SHORT_BUFFER, "gguf_requantize: need " + std::to_string(need) + " bytes of blocks, got " +
                                           std::to_string(data_len));
  int perm_hd = 0;
  if (permute_heads > 0) {
    if (rows % permute_heads) return fail(MLXQ_ERR_SHAPE, "gguf_requantize: rows not divisible by the head count");
    perm_hd = static_cast<int>(rows / permute_heads);
    if (perm_hd % 2) return fail(MLXQ_ERR_SHAPE, "gguf_requantize: odd head_dim");
  }
  if (n == 0) return MLXQ_OK;
  if (!data || !wq || !scales || !biases) return fail(MLXQ_ERR_INVALID, "gguf_requantize: null pointer");
  if ((reinterpret_cast<uintptr_t>(wq) & 7u)) return fail(MLXQ_ERR_INVALID, "gguf_requantize: wq must be 8-byte aligned");
  const int64_t row_bytes = cols / elems * bbytes;
  if (row_bytes > 160 * 1024) return fail(MLXQ_ERR_UNSUPPORTED, "gguf_requantize: row larger than LDS");
  const int K = static_cast<int>(cols), R = static_cast<int>(rows), RB = static_cast<int>(row_bytes);
  const uint8_t* d = static_cast<const uint8_t*>(data);
  uint16_t* s = static_cast<uint16_t*>(scales);
  uint16_t* b = static_cast<uint16_t*>(biases);
  hipStream_t st = as_stream(stream);
  switch (tag) {
    case 0: return launch_tag<0>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 1: return launch_tag<1>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 30: return launch_tag<30>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 2: return launch_tag<2>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 3: return launch_tag<3>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 6: return launch_tag<6>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 7: return launch_tag<7>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 8: return launch_tag<8>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 10: return launch_tag<10>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 11: return launch_tag<11>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 12: return launch_tag<12>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 13: return launch_tag<13>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 14: return launch_tag<14>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 20: return launch_tag<20>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 16: return launch_tag<16>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 17: return launch_tag<17>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 22: return launch_tag<22>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 18: return launch_tag<18>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 21: return launch_tag<21>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 19: return launch_tag<19>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    case 29: return launch_tag<29>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
    default: return launch_tag<23>(bits, group_size, R, K, RB, perm_hd, d, wq, s, b, st);
  }
}
