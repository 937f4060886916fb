// Prefill-shaped quantized matmul (qmm) for gfx950: y[M,N] = x[M,K] . W^T,
// W group-wise affine quantized (Q4 / Q8), any M.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul, which MLX serves with its qmm kernels when M
// is large (prefill, batched decode).
//
// Design (MFMA-bound):
//  * Workgroup tile 256 (M) x 128 (N), K step 64; 4 wavefronts in a 2x2 grid,
//    each owning 128x64 of the output as 4x2 tiles of
//    v_mfma_f32_32x32x16_bf16 (f32 accumulators).
//  * Per K step the workgroup stages the activation tile (bf16, 256x64) and the
//    weight tile into LDS.  The weight tile is dequantized once per workgroup
//    on the way in: codes -> f32 -> scale*q + bias -> bf16 (round to nearest
//    even), the same values MLX's qmm places in threadgroup memory.
//  * Two LDS stages (2 x 55 KB of gfx950's 160 KB): global loads for step k+1
//    are issued before the MFMAs of step k and written to the other stage
//    after them, one barrier per step.  Rows are padded to 72 bf16 so the
//    16-byte fragment reads of 16 consecutive rows hit distinct banks.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int LDR = BK + 8;                       // padded LDS row, bf16 elements
constexpr int kStageElems = (BM + BN) * LDR;      // bf16 per stage
constexpr int kLdsBytes = 2 * kStageElems * 2;    // two stages

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(a);  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

template <int BITS>
struct BRegs {
  static constexpr int W = BITS == 4 ? 4 : 8;  // code words per thread per K step (32 elements)
  uint32_t w[W];
  float s, b;
};

template <int BITS, int GS>
__global__ __launch_bounds__(kThreads) void qmm_kernel(const uint16_t* __restrict__ x, int M,
                                                        const uint32_t* __restrict__ wq,
                                                        const uint16_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ biases,
                                                        const uint16_t* __restrict__ bias_vec, int N, int K,
                                                        uint16_t* __restrict__ y) {
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int KT = K / BK;
  const int G = K / GS;
  const int64_t row_words = static_cast<int64_t>(K) * BITS / 32;

  // ---- activation tile loader: 8 rows x 16 B per wave instruction ----
  const int a_chunk = tid & 7;    // 8 bf16 of the 64-wide K step
  const int a_row0 = tid >> 3;    // + 32*i, i < 8
  const uint4* a_src[8];
  bool a_ok[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int m = m0 + a_row0 + 32 * i;
    a_ok[i] = m < M;
    a_src[i] = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(a_ok[i] ? m : 0) * K + a_chunk * 8);
  }
  // ---- weight tile loader: one row, 32 consecutive K per thread ----
  const int b_row = tid >> 1, b_half = tid & 1;
  const int b_n = min(n0 + b_row, N - 1);
  const uint32_t* b_src = wq + b_n * row_words + b_half * (32 * BITS / 32);
  const uint16_t* s_src = scales + static_cast<int64_t>(b_n) * G;
  const uint16_t* z_src = biases + static_cast<int64_t>(b_n) * G;

  uint4 areg[8];
  BRegs<BITS> breg;

  auto load_tiles = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < 8; i++) areg[i] = a_ok[i] ? a_src[i][k0 / 8] : make_uint4(0, 0, 0, 0);
    const uint32_t* p = b_src + static_cast<int64_t>(k0) * BITS / 32;
#pragma unroll
    for (int i = 0; i < BRegs<BITS>::W; i += 4) {
      uint4 v = *reinterpret_cast<const uint4*>(p + i);
      breg.w[i] = v.x; breg.w[i + 1] = v.y; breg.w[i + 2] = v.z; breg.w[i + 3] = v.w;
    }
    const int g = (k0 + 32 * b_half) / GS;
    breg.s = bf16_bits_to_f32(s_src[g]);
    breg.b = bf16_bits_to_f32(z_src[g]);
  };

  auto store_tiles = [&](int stage) {
    uint16_t* sa = lds + stage * kStageElems;
    uint16_t* sb = sa + BM * LDR;
#pragma unroll
    for (int i = 0; i < 8; i++)
      *reinterpret_cast<uint4*>(sa + (a_row0 + 32 * i) * LDR + a_chunk * 8) = areg[i];
    uint32_t packed[16];
    if constexpr (BITS == 4) {
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t q = breg.w[w];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float lo = breg.s * static_cast<float>((q >> (8 * j)) & 0xFu) + breg.b;
          const float hi = breg.s * static_cast<float>((q >> (8 * j + 4)) & 0xFu) + breg.b;
          packed[4 * w + j] = pack_bf16(lo, hi);
        }
      }
    } else {
#pragma unroll
      for (int w = 0; w < 8; w++) {
        const uint32_t q = breg.w[w];
        const float v0 = breg.s * static_cast<float>(q & 0xFFu) + breg.b;
        const float v1 = breg.s * static_cast<float>((q >> 8) & 0xFFu) + breg.b;
        const float v2 = breg.s * static_cast<float>((q >> 16) & 0xFFu) + breg.b;
        const float v3 = breg.s * static_cast<float>(q >> 24) + breg.b;
        packed[2 * w] = pack_bf16(v0, v1);
        packed[2 * w + 1] = pack_bf16(v2, v3);
      }
    }
    uint4* dst = reinterpret_cast<uint4*>(sb + b_row * LDR + b_half * 32);
#pragma unroll
    for (int i = 0; i < 4; i++)
      dst[i] = make_uint4(packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]);
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;

  load_tiles(0);
  store_tiles(0);
  __syncthreads();
  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) load_tiles(kt + 1);
    const uint16_t* sa = lds + cur * kStageElems + (wm * 128 + frag_row) * LDR + frag_k;
    const uint16_t* sb = lds + cur * kStageElems + BM * LDR + (wn * 64 + frag_row) * LDR + frag_k;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) {
      bf16x8 a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; i++)
        a[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sa + 32 * i * LDR + ks * 16));
#pragma unroll
      for (int j = 0; j < 2; j++)
        b[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sb + 32 * j * LDR + ks * 16));
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // C layout of a 32x32 MFMA tile: lane holds column lane%32 and rows
  // 8*(v/4) + 4*(lane/32) + v%4.
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = n0 + wn * 64 + 32 * j + (lane & 31);
    if (n >= N) continue;
    const float bb = bias_vec ? bf16_bits_to_f32(bias_vec[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + wm * 128 + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < M) y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(acc[i][j][v] + bb));
      }
  }
}

template <int BITS, int GS>
int launch(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint16_t* bias,
           int N, int K, uint16_t* y, hipStream_t st) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&qmm_kernel<BITS, GS>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmm: set LDS size: ") + hipGetErrorString(e));
    attr_set = true;
  }
  dim3 grid(ceil_div(N, BN), ceil_div(M, BM));
  hipLaunchKernelGGL((qmm_kernel<BITS, GS>), grid, dim3(kThreads), kLdsBytes, st, x, M, wq, s, b, bias, N, K, y);
  return check_launch("qmm");
}

}  // namespace

int launch_qmm(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y, hipStream_t st) {
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  if (bits == 4) {
    if (group_size == 32) return launch<4, 32>(x, m, wq, s, b, bias, n, k, y, st);
    if (group_size == 64) return launch<4, 64>(x, m, wq, s, b, bias, n, k, y, st);
    return launch<4, 128>(x, m, wq, s, b, bias, n, k, y, st);
  }
  if (group_size == 32) return launch<8, 32>(x, m, wq, s, b, bias, n, k, y, st);
  if (group_size == 64) return launch<8, 64>(x, m, wq, s, b, bias, n, k, y, st);
  return launch<8, 128>(x, m, wq, s, b, bias, n, k, y, st);
}

}  // namespace mlxq
