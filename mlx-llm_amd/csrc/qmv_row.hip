// Batch-1 quantized GEMV, whole rows per wave (gfx950).
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul at decode batch 1 (MLX's qmv).
//
// Why this shape: at M = 1 the call is a pure stream of the packed weights,
// and the fastest way this GPU reads a weight matrix is many short waves
// that each request their whole share at once, every load instruction
// covering 1 KB of one row (64 lanes x 16 B, contiguous).  Measured on the
// Llama shapes, a plain read in that form takes 5.96 us for the 29 MB gate
// matrix, against 6.3 us for 8 rows x 128 B per instruction.
//  * A wave owns R rows and the whole of K: R * NI 16-byte loads per lane
//    (NI = K*bits/8 / 1 KB), all issued before any arithmetic, after the
//    workgroup's loads of x.  No K split, no partial sums, no second launch.
//  * The workgroup stages x once in LDS: Q4 as bf16 pairs (x0,x2) (x4,x6)
//    (x1,x3) (x5,x7) of every 8 elements, the order of the Q4 decode below,
//    Q8 in natural order; plus the sum of x over every lane chunk (32 codes
//    for Q4, 16 for Q8).
//  * Q4 codes become bf16 (128 + q) pairs: the even and the odd nibbles are
//    masked into bytes and interleaved with 0x43 bytes by v_perm (0x43nn is
//    bf16 128 + nn, whose ulp is 1), 7 instructions per 8 codes; Q8 codes
//    are converted exactly through f32.
//    v_dot2_f32_bf16 accumulates; per chunk y += s*dot + (b - OFF*s)*sum(x)
//    (OFF = 128 for Q4, 0 for Q8), in f32.  One chunk never straddles a
//    group (group sizes 32/64/128 >= chunk).
//  * The 64 lanes of a row reduce with DPP adds and the gfx950 row swaps;
//    y = bf16(acc (+ bias)).
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <string>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace row {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Q8: 4 codes of one dword -> bf16 pairs (q0,q1), (q2,q3), exact through f32
__device__ __forceinline__ void decode_q8(uint32_t q, uint32_t& b0, uint32_t& b1) {
  const float f0 = static_cast<float>(q & 0xFFu), f1 = static_cast<float>((q >> 8) & 0xFFu);
  const float f2 = static_cast<float>((q >> 16) & 0xFFu), f3 = static_cast<float>(q >> 24);
  b0 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  b1 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

// BITS: 4 or 8; NI: 1 KB load instructions per row; R: rows per wave; W:
// waves per workgroup; MM: activation rows (1..4; each code is decoded once
// and dotted with every activation row)
template <int BITS, int NI, int R, int W, int MM = 1>
__global__ __launch_bounds__(64 * W) void qmv_row_kernel(const uint16_t* __restrict__ x,
                                                         const uint32_t* __restrict__ wq,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint16_t* __restrict__ bi,
                                                         const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                         int N, int gs) {
  constexpr int T = 64 * W;
  constexpr int K = NI * 8192 / BITS;   // elements per row
  constexpr int CPL = 128 / BITS;       // codes per lane per load (one chunk)
  constexpr int NP = K / 8;             // 16-byte pieces of x
  constexpr int XPT = (MM * NP + T - 1) / T; // pieces per thread (all activation rows)
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  static_assert(NP % 4 == 0, "whole chunks of x");
  __shared__ uint4 xp[MM * NP];
  __shared__ float xs[MM * (K / CPL)];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row0 = (blockIdx.x * W + wave) * R;
  const int gsh = __builtin_ctz(gs);  // group sizes are powers of two (32, 64, 128)
  const int G = K >> gsh;

  // 1. x pieces (first: the staging waits on them, the codes can keep coming)
  uint4 xv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int q = tid + i * T;
    xv[i] = q < MM * NP ? reinterpret_cast<const uint4*>(x)[q] : make_uint4(0, 0, 0, 0);
  }
  // 2. the wave's rows: codes (1 KB per instruction), then the lanes' scale/bias
  uint4 cw[R][NI];
  uint16_t sv[R][NI], bv[R][NI];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n = min(row0 + r, N - 1);  // rows past N repeat row N-1 (results dropped)
    const uint4* wr = reinterpret_cast<const uint4*>(wq) + static_cast<int64_t>(n) * (NI * 64);
#pragma unroll
    for (int t = 0; t < NI; t++) cw[r][t] = wr[t * 64 + lane];
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n = min(row0 + r, N - 1);
#pragma unroll
    for (int t = 0; t < NI; t++) {
      const int g = ((t * 64 + lane) * CPL) >> gsh;
      sv[r][t] = sc[static_cast<int64_t>(n) * G + g];
      bv[r][t] = bi[static_cast<int64_t>(n) * G + g];
    }
  }
  // 3. stage x: Q4 pair order, Q8 natural; per-chunk sums of the bf16 values
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int q = tid + i * T;
    if (i * T + T > MM * NP && q >= MM * NP) continue;  // whole 4-lane groups drop out together (NP % 4 == 0)
    const uint32_t a[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      f[2 * e] = bf16_bits_to_f32(a[e] & 0xFFFFu);
      f[2 * e + 1] = bf16_bits_to_f32(a[e] >> 16);
    }
    if (BITS == 4) {
      xp[q] = make_uint4(__builtin_amdgcn_perm(a[1], a[0], 0x05040100u), __builtin_amdgcn_perm(a[3], a[2], 0x05040100u),
                         __builtin_amdgcn_perm(a[1], a[0], 0x07060302u), __builtin_amdgcn_perm(a[3], a[2], 0x07060302u));
    } else {
      xp[q] = xv[i];
    }
    float sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    sum += dpp_f32<kDppQuadXor1>(sum);  // Q8 chunk: 2 pieces
    if (BITS == 4) {
      sum += dpp_f32<kDppQuadXor2>(sum);  // Q4 chunk: 4 pieces
      if ((lane & 3) == 0) xs[q >> 2] = sum;
    } else {
      if ((lane & 1) == 0) xs[q >> 1] = sum;
    }
  }
  __syncthreads();

  // 4. dot products: chunk ch = t*64 + lane of every row shares its x
  float acc[R][MM];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MM; m++) acc[r][m] = 0.f;
#pragma unroll
  for (int t = 0; t < NI; t++) {
    const int ch = t * 64 + lane;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t wd[4] = {cw[r][t].x, cw[r][t].y, cw[r][t].z, cw[r][t].w};
      uint32_t p[8];  // decoded bf16 pairs of the 16 bytes
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if (BITS == 4) {
          // even nibbles (k0,k2,k4,k6) and odd nibbles as bytes, interleaved
          // with 0x43: (k0,k2) (k4,k6) (k1,k3) (k5,k7); p[2k], p[2k+1] and
          // the next pair of slots of the same k are reused below
          p[2 * k] = wd[k] & 0x0F0F0F0Fu;
          p[2 * k + 1] = (wd[k] >> 4) & 0x0F0F0F0Fu;
        } else {
          decode_q8(wd[k], p[2 * k], p[2 * k + 1]);
        }
      }
      const float s = bf16_bits_to_f32(sv[r][t]), b = bf16_bits_to_f32(bv[r][t]);
#pragma unroll
      for (int m = 0; m < MM; m++) {
        const float xsum = xs[m * (K / CPL) + ch];
        float d = 0.f;
        if (BITS == 4) {
          const uint4* xq = xp + m * NP + ch * 4;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            const uint4 X = xq[k];
            const uint32_t lo = p[2 * k], hi = p[2 * k + 1], c43 = 0x43434343u;
            d = dot2(__builtin_amdgcn_perm(lo, c43, 0x00050004u), X.x, d);
            d = dot2(__builtin_amdgcn_perm(lo, c43, 0x00070006u), X.y, d);
            d = dot2(__builtin_amdgcn_perm(hi, c43, 0x00050004u), X.z, d);
            d = dot2(__builtin_amdgcn_perm(hi, c43, 0x00070006u), X.w, d);
          }
        } else {
          const uint4* xq = xp + m * NP + ch * 2;
          const uint4 X0 = xq[0], X1 = xq[1];
          const uint32_t xd[8] = {X0.x, X0.y, X0.z, X0.w, X1.x, X1.y, X1.z, X1.w};
#pragma unroll
          for (int k = 0; k < 8; k++) d = dot2(p[k], xd[k], d);
        }
        acc[r][m] += s * d + (b - OFF * s) * xsum;
      }
    }
  }
  // 5. row sums across the 64 lanes
#pragma unroll
  for (int r = 0; r < R; r++) {
#pragma unroll
    for (int m = 0; m < MM; m++) {
      float v = wave_sum(acc[r][m]);
      const int n = row0 + r;
      if (lane == 0 && n < N) {
        if (bias) v += bf16_bits_to_f32(bias[n]);
        y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(v));
      }
    }
  }
}

template <int BITS, int NI, int R, int W, int MM = 1>
int launch_rw(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint16_t* bias,
              int64_t N, int gs, uint16_t* y, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>((N + R * W - 1) / (R * W));
  hipLaunchKernelGGL((qmv_row_kernel<BITS, NI, R, W, MM>), dim3(grid), dim3(64 * W), 0, st, x, wq, s, b, bias, y,
                     static_cast<int>(N), gs);
  return check_launch("qmv_row");
}

// (rows per wave, waves per workgroup) instantiated per row length: short
// rows take several rows per wave, long rows one (registers), with more
// waves per workgroup to share the activation staging.
template <int BITS, int NI>
int launch_ni(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
              const uint16_t* bias, int64_t N, int gs, uint16_t* y, int R, int W, hipStream_t st) {
  if constexpr (NI * 8192 / BITS <= 4096) {  // several activation rows: K <= 4096 (LDS)
    if (M == 2) return launch_rw<BITS, NI, 1, 4, 2>(x, wq, s, b, bias, N, gs, y, st);
    if (M == 3) return launch_rw<BITS, NI, 1, 4, 3>(x, wq, s, b, bias, N, gs, y, st);
    if (M == 4) return launch_rw<BITS, NI, 1, 4, 4>(x, wq, s, b, bias, N, gs, y, st);
  }
  if (M != 1) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_row: M > 1 needs K <= 4096");
  if constexpr (NI <= 2) {
    if (R >= 4) return launch_rw<BITS, NI, 4, 4>(x, wq, s, b, bias, N, gs, y, st);
    if (R == 2) return launch_rw<BITS, NI, 2, 4>(x, wq, s, b, bias, N, gs, y, st);
    return launch_rw<BITS, NI, 1, 4>(x, wq, s, b, bias, N, gs, y, st);
  } else if constexpr (NI <= 4) {
    if (R >= 2) return launch_rw<BITS, NI, 2, 4>(x, wq, s, b, bias, N, gs, y, st);
    return launch_rw<BITS, NI, 1, 4>(x, wq, s, b, bias, N, gs, y, st);
  } else {
    if (W >= 16) return launch_rw<BITS, NI, 1, 16>(x, wq, s, b, bias, N, gs, y, st);
    if (W >= 8) return launch_rw<BITS, NI, 1, 8>(x, wq, s, b, bias, N, gs, y, st);
    return launch_rw<BITS, NI, 1, 4>(x, wq, s, b, bias, N, gs, y, st);
  }
}

}  // namespace row

bool qmv_row_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M < 1 || M > 4 || N < 1 || (bits != 4 && bits != 8) || group_size < 128 / bits) return false;
  if (M > 1 && K > 4096) return false;  // the activation rows share the workgroup's LDS
  if ((K * bits / 8) % 1024) return false;
  const int64_t ni = K * bits / 8 / 1024;
  // Q4 with 7 KB rows (the down projection, K = 14336) measured faster on
  // qmv_dot (10.3 vs 10.9 us): the 28 KB activation staging per workgroup of
  // 4 rows costs more than the whole-row loads save there
  if (bits == 4 && ni >= 7) return false;
  return ni == 1 || ni == 2 || ni == 4 || ni == 7 || ni == 8 || ni == 14 || ni == 16;
}

// Rows per wave and waves per workgroup, from measurements at the Llama
// shapes (MLXQ_QMV_ROW_R / MLXQ_QMV_ROW_W override them).
void qmv_row_geometry(int64_t N, int64_t K, int bits, int& R, int& W) {
  const int64_t ni = K * bits / 8 / 1024;
  R = bits == 4 && ni <= 2 && N >= 4096 ? 2 : 1;  // Q4 q/o 4.96 vs 5.18 us, gate 9.72 vs 10.48; Q8 best at 1
  W = 4;                                          // Q8 down: 15.8 us at 4 waves, 16.2 at 8, 17.6 at 16
  if (overrides().row_r) R = overrides().row_r;
  if (overrides().row_w) W = overrides().row_w;
}

int launch_qmv_row(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   hipStream_t st) {
  using namespace row;
  int R = 1, W = 4;
  qmv_row_geometry(N, K, bits, R, W);
  const int64_t ni = K * bits / 8 / 1024;
#define MLXQ_ROW_CASE(NIV)                                                                       \
  case NIV:                                                                                      \
    return bits == 4 ? launch_ni<4, NIV>(x, M, wq, s, b, bias, N, group_size, y, R, W, st)             \
                     : launch_ni<8, NIV>(x, M, wq, s, b, bias, N, group_size, y, R, W, st);
  switch (ni) {
    MLXQ_ROW_CASE(1)
    MLXQ_ROW_CASE(2)
    MLXQ_ROW_CASE(4)
    MLXQ_ROW_CASE(7)
    MLXQ_ROW_CASE(8)
    MLXQ_ROW_CASE(14)
    MLXQ_ROW_CASE(16)
    default:
      return fail(MLXQ_ERR_UNSUPPORTED, "qmv_row: K*bits/8 must be 1, 2, 4, 7, 8, 14 or 16 KB");
  }
#undef MLXQ_ROW_CASE
}

}  // namespace mlxq
