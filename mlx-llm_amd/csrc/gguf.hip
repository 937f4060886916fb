// GGUF block dequantization for gfx950.
//
// Reference: src/gguf/dequant.rs:156-211 (dispatcher) and the per-type block
// decoders it calls (:228-719).  The reference walks blocks one at a time on
// one host thread; here a workgroup stages a chunk of whole blocks into LDS
// with wide coalesced loads, then every thread decodes VEC consecutive output
// elements straight from LDS and writes them with one 16-byte store.
//
// Bit-exactness: each output element is computed with exactly the IEEE f32
// operations, operand order and roundings the reference uses for it (the
// per-element formulas below are the reference's block loops solved for one
// element).  This file is compiled with -ffp-contract=off so no mul+add/sub is
// fused, and f16 scales are decoded with integer bit operations.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#define MLXQ_IQ4NL_IN_REGISTERS 1  // IQ4 codebook lookups by v_perm (this kernel is memory-bound)
#include "gguf_decode.hpp"

namespace mlxq {
namespace {

constexpr int kThreads = 256;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kVec = 8;                          // outputs per thread per pass
constexpr int kChunkElems = kThreads * kVec;     // 2048 elements per chunk

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

template <bool BF16OUT>
__device__ __forceinline__ void store_vec(void* out, int64_t e, const float (&v)[kVec]) {
  if constexpr (BF16OUT) {
    // v_cvt_pk_bf16_f32: round to nearest even, two values per instruction
    // (the same bits as f32_to_bf16_bits except NaN payloads)
    uint4 p;
    p.x = pack_bf16_rne(v[0], v[1]);
    p.y = pack_bf16_rne(v[2], v[3]);
    p.z = pack_bf16_rne(v[4], v[5]);
    p.w = pack_bf16_rne(v[6], v[7]);
    // written once and not read back by this kernel: non-temporal (each
    // wave instruction covers 1 KB contiguously)
    __builtin_nontemporal_store(u32x4{p.x, p.y, p.z, p.w}, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + e));
  } else {
    float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + e);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// One workgroup per kCpw chunks of kChunkElems elements (each a whole number
// of blocks): every byte of the workgroup's chunks is requested before the
// barrier (one memory round trip per workgroup, kCpw x the bytes in flight
// of a one-chunk workgroup), then each thread decodes kVec elements of every
// chunk and writes them with 16-byte stores.  Chunk bytes are a multiple of
// 16 for every tag, so with a 16-byte aligned base every chunk start is
// 16-byte aligned and staged with uint4 loads.
constexpr int kCpw = 4;

// 16 bytes per lane from global memory straight into LDS (a wave's 64 lanes
// fill 1 KB from `l`)
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}

// f32 output in two 1 KB halves per store pass (measured, µs for a 14336 x
// 4096 tensor: Q4_0 53.3 -> 47.6, Q8_0 61 -> 51.7, Q6_K 56.5 -> 49.6,
// IQ4_NL 52 -> 47.4, IQ4_XS 52 -> 48; Q4_K with its 4-element run decoder
// 58 -> 48); the other formats keep 8 consecutive elements per thread
template <int TAG>
constexpr bool f32_halves() {
  return TAG == 2 || TAG == 8 || TAG == 12 || TAG == 14 || TAG == 20 || TAG == 23;
}

// Q4_K elements j .. j + N - 1 (one sub-block, one nibble half) with
// decode<12>'s arithmetic in its order: the sub-block's scale and min and
// the block's d, dmin derived once for the run
// (N = 4 or 8: j a multiple of N; the run's bytes are N-byte aligned)
template <int N>
__device__ __forceinline__ void q4k_run(const uint8_t* b, int j, float* v) {
  const int c = j >> 6, hi = (j >> 5) & 1, l = j & 31;
  uint32_t sc, m;
  scale_min_k4(2 * c + hi, b + 4, sc, m);
  const float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
  const float d1 = d * static_cast<float>(sc);
  const float m1 = dmin * static_cast<float>(m);
  uint32_t w[N / 4];
  if constexpr (N == 8) {
    const uint2 q = *reinterpret_cast<const uint2*>(b + 16 + 32 * c + l);
    w[0] = q.x;
    w[1] = q.y;
  } else {
    w[0] = *reinterpret_cast<const uint32_t*>(b + 16 + 32 * c + l);
  }
  const int sh = 4 * hi;
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = d1 * static_cast<float>((w[i >> 2] >> (8 * (i & 3) + sh)) & 0xFu) - m1;
}

template <int TAG, bool BF16OUT, bool ALIGNED16>
__global__ __launch_bounds__(kThreads) void gguf_dequant_kernel(const uint8_t* __restrict__ data,
                                                                 int64_t nblocks, void* __restrict__ out) {
  constexpr int E = Geo<TAG>::E, B = Geo<TAG>::B;
  constexpr int BPC = kChunkElems / E;         // blocks per chunk
  constexpr int CB = BPC * B;                  // chunk bytes
  constexpr int WB = kCpw * CB;                // workgroup bytes
  static_assert(CB % 16 == 0, "chunk bytes must be a multiple of 16");
  __shared__ __align__(16) uint8_t lds[(WB + 1023) / 1024 * 1024];

  const int64_t blk0 = static_cast<int64_t>(blockIdx.x) * kCpw * BPC;
  const int nb = static_cast<int>(min<int64_t>(kCpw * BPC, nblocks - blk0));  // blocks of this workgroup
  const int bytes = nb * B;
  const uint8_t* src = data + blk0 * B;
  const int tid = threadIdx.x;

  if constexpr (ALIGNED16) {
    // direct global -> LDS loads: each wave instruction moves 1 KB (16 B per
    // lane) into a contiguous LDS range, no registers held while in flight
    const int n16 = bytes >> 4;  // whole uint4s (bytes is a multiple of 2 at least)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    constexpr int kPieces = (WB + 1023) / 1024;  // 1 KB pieces of the workgroup
#pragma unroll
    for (int k = 0; k < (kPieces + kThreads / 64 - 1) / (kThreads / 64); k++) {
      const int piece = k * (kThreads / 64) + wave;
      if (piece < kPieces && piece * 64 + lane < n16)
        lds_dma16(src + (piece * 64 + lane) * 16, lds + piece * 1024);
    }
    for (int i = (n16 << 4) + tid; i < bytes; i += kThreads) lds[i] = src[i];
    __builtin_amdgcn_s_waitcnt(0);
  } else {
    for (int i = tid; i < bytes; i += kThreads) lds[i] = src[i];
  }
  __syncthreads();

#pragma unroll
  for (int c = 0; c < kCpw; c++) {
    if constexpr (!BF16OUT && f32_halves<TAG>()) {
      // f32 out: elements tid * 4 .. +3 and 1024 + tid * 4 .. +3 of the
      // chunk, so that each of the two 16-byte store instructions covers 1
      // KB contiguously and can go out non-temporal (with 32 bytes per lane
      // each instruction would cover every line half, and non-temporal
      // half-line stores measured nearly twice as slow)
      const int e0 = c * kChunkElems + tid * 4;
      if (e0 >= nb * E) return;  // the second half lies beyond the first
      float v[kVec];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int e = e0 + h * (kThreads * 4);
        if constexpr (TAG == 12) {
          q4k_run<4>(lds + (e / E) * B, e % E, v + 4 * h);
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++) v[4 * h + i] = decode<TAG>(lds + ((e + i) / E) * B, (e + i) % E);
        }
      }
      f32x4* o = reinterpret_cast<f32x4*>(static_cast<float*>(out) + static_cast<int64_t>(blockIdx.x) * kCpw * kChunkElems + e0);
      __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, o);
      if (e0 + kThreads * 4 < nb * E) __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, o + kThreads);
    } else {
      const int e0 = c * kChunkElems + tid * kVec;  // element within the workgroup
      if (e0 >= nb * E) return;
      float v[kVec];
      if constexpr (TAG == 12) {
        q4k_run<8>(lds + (e0 / E) * B, e0 % E, v);
      } else {
#pragma unroll
        for (int i = 0; i < kVec; i++) {
          const int e = e0 + i;
          v[i] = decode<TAG>(lds + (e / E) * B, e % E);
        }
      }
      store_vec<BF16OUT>(out, static_cast<int64_t>(blockIdx.x) * kCpw * kChunkElems + e0, v);
    }
  }
}

// F32 / F16 / BF16 pass-through (dequant.rs:174-188): one element per thread.
template <int TAG, bool BF16OUT>
__global__ __launch_bounds__(kThreads) void gguf_float_kernel(const uint8_t* __restrict__ data, int64_t n,
                                                               void* __restrict__ out) {
  int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= n) return;
  float v;
  if (TAG == 0) {
    v = bits_to_f32(rd_u32(data + 4 * e));
  } else {
    uint32_t h = static_cast<uint32_t>(data[2 * e]) | (static_cast<uint32_t>(data[2 * e + 1]) << 8);
    v = TAG == 1 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
  }
  if constexpr (BF16OUT) static_cast<uint16_t*>(out)[e] = static_cast<uint16_t>(f32_to_bf16_bits(v));
  else static_cast<float*>(out)[e] = v;
}

template <int TAG, bool BF16OUT>
void launch_blocks(const uint8_t* data, int64_t nblocks, void* out, hipStream_t st) {
  constexpr int E = Geo<TAG>::E;
  int64_t chunks = ceil_div(nblocks * E, static_cast<int64_t>(kCpw) * kChunkElems);  // workgroups
  if (chunks == 0) return;
  bool aligned = (reinterpret_cast<uintptr_t>(data) & 15u) == 0;
  if (aligned)
    MLXQ_LAUNCH((gguf_dequant_kernel<TAG, BF16OUT, true>), dim3(chunks), dim3(kThreads), 0, st, data,
                       nblocks, out);
  else
    MLXQ_LAUNCH((gguf_dequant_kernel<TAG, BF16OUT, false>), dim3(chunks), dim3(kThreads), 0, st, data,
                       nblocks, out);
}

template <int TAG, bool BF16OUT>
void launch_float(const uint8_t* data, int64_t n, void* out, hipStream_t st) {
  int64_t grid = ceil_div(n, static_cast<int64_t>(kThreads));
  if (grid == 0) return;
  MLXQ_LAUNCH((gguf_float_kernel<TAG, BF16OUT>), dim3(grid), dim3(kThreads), 0, st, data, n, out);
}

template <bool BF16OUT>
int dispatch(uint32_t tag, const uint8_t* d, int64_t nblocks, int64_t n, void* out, hipStream_t st) {
  switch (tag) {
    case 0: launch_float<0, BF16OUT>(d, n, out, st); break;
    case 1: launch_float<1, BF16OUT>(d, n, out, st); break;
    case 30: launch_float<30, BF16OUT>(d, n, out, st); break;
    case 2: launch_blocks<2, BF16OUT>(d, nblocks, out, st); break;
    case 3: launch_blocks<3, BF16OUT>(d, nblocks, out, st); break;
    case 6: launch_blocks<6, BF16OUT>(d, nblocks, out, st); break;
    case 7: launch_blocks<7, BF16OUT>(d, nblocks, out, st); break;
    case 8: launch_blocks<8, BF16OUT>(d, nblocks, out, st); break;
    case 10: launch_blocks<10, BF16OUT>(d, nblocks, out, st); break;
    case 11: launch_blocks<11, BF16OUT>(d, nblocks, out, st); break;
    case 12: launch_blocks<12, BF16OUT>(d, nblocks, out, st); break;
    case 13: launch_blocks<13, BF16OUT>(d, nblocks, out, st); break;
    case 14: launch_blocks<14, BF16OUT>(d, nblocks, out, st); break;
    case 20: launch_blocks<20, BF16OUT>(d, nblocks, out, st); break;
    case 23: launch_blocks<23, BF16OUT>(d, nblocks, out, st); break;
    case 16: launch_blocks<16, BF16OUT>(d, nblocks, out, st); break;
    case 17: launch_blocks<17, BF16OUT>(d, nblocks, out, st); break;
    case 22: launch_blocks<22, BF16OUT>(d, nblocks, out, st); break;
    case 18: launch_blocks<18, BF16OUT>(d, nblocks, out, st); break;
    case 21: launch_blocks<21, BF16OUT>(d, nblocks, out, st); break;
    case 19: launch_blocks<19, BF16OUT>(d, nblocks, out, st); break;
    case 29: launch_blocks<29, BF16OUT>(d, nblocks, out, st); break;
    default:
      return fail(MLXQ_ERR_UNSUPPORTED,
                  "unsupported: GGUF type tag " + std::to_string(tag) + " has no device dequantizer");
  }
  return check_launch("gguf_dequantize");
}

}  // namespace
}  // namespace mlxq

using namespace mlxq;

extern "C" int mlxq_gguf_dequantize(uint32_t tag, const void* data, int64_t data_len, int64_t n,
                                    int out_dtype, void* out, void* stream) {
  clear_error();
  int64_t be = 0, bb = 0;
  int rc = mlxq_gguf_block(tag, &be, &bb);
  if (rc) return rc;
  if (n < 0 || data_len < 0) return fail(MLXQ_ERR_INVALID, "gguf: negative size");
  if (n % be)  // dequant.rs:159-163
    return fail(MLXQ_ERR_SHAPE, "gguf: " + std::to_string(n) + " elements not a multiple of " +
                                    std::to_string(be) + " for tag " + std::to_string(tag));
  int64_t nblocks = n / be, need = nblocks * bb;
  if (data_len < need)  // dequant.rs:166-171
    return fail(MLXQ_ERR_SHORT_BUFFER, "gguf: tag " + std::to_string(tag) + " needs " + std::to_string(need) +
                                           " bytes for " + std::to_string(n) + " elements, got " +
                                           std::to_string(data_len));
  if (out_dtype != MLXQ_F32 && out_dtype != MLXQ_BF16)
    return fail(MLXQ_ERR_UNSUPPORTED, "gguf: output dtype must be f32 or bf16");
  if (n == 0) return MLXQ_OK;
  if (!data || !out) return fail(MLXQ_ERR_INVALID, "gguf: null pointer");
  // Block types write kVec outputs per 16-byte store (n is a multiple of 32).
  if (be > 1 && (reinterpret_cast<uintptr_t>(out) & 15u))
    return fail(MLXQ_ERR_INVALID, "gguf: output pointer must be 16-byte aligned");
  const uint8_t* d = static_cast<const uint8_t*>(data);
  hipStream_t st = as_stream(stream);
  return out_dtype == MLXQ_BF16 ? dispatch<true>(tag, d, nblocks, n, out, st)
                                : dispatch<false>(tag, d, nblocks, n, out, st);
}
