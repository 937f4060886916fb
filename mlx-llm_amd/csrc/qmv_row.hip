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
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

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

enum : int { kNorm = 1, kSwiGLU = 2, kRepeat = 4 };
constexpr int kMaxSegs = 3;

// One weight matrix of a launch; its workgroups end at tile_end (exclusive).
struct RowSeg {
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* bias;  // [N] or null
  const uint16_t* res;   // [M, N] residual or null
  uint16_t* y;           // [M, N]
  int N;
  int tile_end;
};

struct RowParams {
  const uint16_t* x;       // activations, row stride x_stride
  const uint16_t* norm_w;  // [K] RMSNorm weight (kNorm)
  float eps;
  int x_stride;
  int gsh;                 // log2(group size)
  int rep_hd8, rep;        // kRepeat: head size in 8-element pieces, query heads per KV head
  float rcp_hd8, rcp_grp;  // 1 / rep_hd8, 1 / (rep_hd8 * rep)
  int nseg;
  RowSeg seg[kMaxSegs];
};

// n / d for 0 <= n < 2^24, d >= 1, given rcp = 1/d: the f32 quotient is
// within one of the true one; one correction each way makes it exact.
__device__ __forceinline__ int div_rcp(int n, int d, float rcp) {
  int q = static_cast<int>(static_cast<float>(n) * rcp);
  q -= q * d > n;
  q += (q + 1) * d <= n;
  return q;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};  // v_cvt_pk_bf16_f32: round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// BITS: 4 or 8; NI: 1 KB load instructions per row; R: rows per wave; W:
// waves per workgroup; MM: activation rows (1..4; each code is decoded once
// and dotted with every activation row); F: fused forms.
//  * kNorm: RMSNorm of the activations while they are staged (nn.rs:35-37)
//    at MLX's rounding points, x' = bf16(w * bf16(x * inv)) with inv =
//    1/sqrt(mean(x^2) + eps) from f32 sums (one extra barrier).
//  * kRepeat: GQA head repeat (attention.rs:45-55) by remapping the staging
//    loads: query head h reads KV head h / rep.
//  * several projections of the same activations (q, k, v): the workgroups
//    are split over up to kMaxSegs weight matrices.
//  * residual epilogue (llama.rs:729-733): y = bf16(r + bf16(acc)).
//  * kSwiGLU (R = 2): a wave's two row slots are row n of the gate matrix
//    and row n of the up matrix; y = bf16(bf16(g * bf16(sigmoid(g))) * u)
//    with g, u the bf16 projection outputs (llama.rs:1040-1045).
template <int BITS, int NI, int R, int W, int MM, int F>
__global__ __launch_bounds__(64 * W) void qmv_row_kernel(const RowParams p) {
  constexpr int T = 64 * W;
  constexpr int K = NI * 8192 / BITS;   // elements per row
  constexpr int CPL = 128 / BITS;       // codes per lane per load (one chunk)
  constexpr int NP = K / 8;             // 16-byte pieces of x
  constexpr int XPT = (MM * NP + T - 1) / T; // pieces per thread (all activation rows)
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  static_assert(NP % 4 == 0, "whole chunks of x");
  static_assert(!(F & kSwiGLU) || R == 2, "SwiGLU: a gate and an up row per wave");
  __shared__ uint4 xp[MM * NP];
  __shared__ float xs[MM * (K / CPL)];
  __shared__ float ssq[(F & kNorm) ? W * MM : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gsh = p.gsh;
  const int G = K >> gsh;

  // this wave's row slots: (matrix, row) each
  int sg = 0, rbase;
  if constexpr (F & kSwiGLU) {
    rbase = blockIdx.x * W + wave;  // row n of gate (slot 0) and of up (slot 1)
  } else {
    const int t = blockIdx.x;
    while (sg + 1 < p.nseg && t >= p.seg[sg].tile_end) sg++;
    rbase = ((t - (sg ? p.seg[sg - 1].tile_end : 0)) * W + wave) * R;
  }
  auto slot_seg = [&](int r) -> const RowSeg& { return (F & kSwiGLU) ? p.seg[r] : p.seg[sg]; };
  auto slot_row = [&](int r) { return (F & kSwiGLU) ? rbase : rbase + r; };

  // 1. x pieces (first: the staging waits on them, the codes can keep coming)
  uint4 xv[XPT];
  uint4 nw[(F & kNorm) ? XPT : 1];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int q = min(tid + i * T, MM * NP - 1);  // clamped: no branch around the loads
    const int m = q / NP, k8 = q - m * NP;
    int src8 = k8;
    if constexpr (F & kRepeat) {
      const int grp = p.rep_hd8 * p.rep;
      const int hq = div_rcp(k8, grp, p.rcp_grp);
      const int r = k8 - hq * grp;
      src8 = hq * p.rep_hd8 + (r - div_rcp(r, p.rep_hd8, p.rcp_hd8) * p.rep_hd8);
    }
    xv[i] = *reinterpret_cast<const uint4*>(p.x + static_cast<int64_t>(m) * p.x_stride + src8 * 8);
    if constexpr (F & kNorm) nw[i] = reinterpret_cast<const uint4*>(p.norm_w)[k8];
  }
  // 2. the wave's rows: codes (1 KB per instruction), then the lanes' scale/bias
  uint4 cw[R][NI];
  uint16_t sv[R][NI], bv[R][NI];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const RowSeg& S = slot_seg(r);
    const int n = min(slot_row(r), S.N - 1);  // rows past N repeat row N-1 (results dropped)
    const uint4* wr = reinterpret_cast<const uint4*>(S.wq) + static_cast<int64_t>(n) * (NI * 64);
#pragma unroll
    for (int t = 0; t < NI; t++) {
      if constexpr (NI <= 4) {
        // rows of up to 4 KB: non-temporal (the codes are read once; Q4 k
        // 3.36 -> 3.07 us, q 4.80 -> 4.62, Q8 q 5.81 -> 5.59); the 7 KB
        // rows of the down projection measured slower with it (9.9 -> 10.9)
        const u32x4v q = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(wr) + t * 64 + lane);
        cw[r][t] = make_uint4(q.x, q.y, q.z, q.w);
      } else {
        cw[r][t] = wr[t * 64 + lane];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const RowSeg& S = slot_seg(r);
    const int n = min(slot_row(r), S.N - 1);
#pragma unroll
    for (int t = 0; t < NI; t++) {
      const int g = ((t * 64 + lane) * CPL) >> gsh;
      // non-temporal too (read once; Q4 k 3.03 -> 2.80 us, q 4.55 -> 4.28,
      // gate 8.9 -> 8.5-8.6, Q8 gate 13.8 -> 12.6-12.8), except for the Q4
      // 7 KB rows (down: 9.95-10.05 -> 10.05-10.26)
      if constexpr (!(BITS == 4 && NI >= 7)) {
        sv[r][t] = __builtin_nontemporal_load(S.s + static_cast<int64_t>(n) * G + g);
        bv[r][t] = __builtin_nontemporal_load(S.b + static_cast<int64_t>(n) * G + g);
      } else {
        sv[r][t] = S.s[static_cast<int64_t>(n) * G + g];
        bv[r][t] = S.b[static_cast<int64_t>(n) * G + g];
      }
    }
  }
  // 3a. RMSNorm: sums of x^2 per activation row over the workgroup, then
  //     x' = bf16(w * bf16(x * inv)) in registers
  if constexpr (F & kNorm) {
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) ss[m] = 0.f;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int q = tid + i * T;
      const uint32_t a[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float lo = bf16_bits_to_f32(a[e] & 0xFFFFu), hi = bf16_bits_to_f32(a[e] >> 16);
        sq = fmaf(lo, lo, fmaf(hi, hi, sq));
      }
#pragma unroll
      for (int m = 0; m < MM; m++) ss[m] += (q < MM * NP && q / NP == m) ? sq : 0.f;
    }
#pragma unroll
    for (int m = 0; m < MM; m++) {
      ss[m] = wave_sum(ss[m]);
      if (lane == 0) ssq[wave * MM + m] = ss[m];
    }
    __syncthreads();
    float inv[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < W; w++) t += ssq[w * MM + m];
      inv[m] = 1.0f / sqrtf(t / static_cast<float>(K) + p.eps);
    }
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int mi = min(tid + i * T, MM * NP - 1) / NP;
      float iv = inv[0];
#pragma unroll
      for (int m = 1; m < MM; m++) iv = mi == m ? inv[m] : iv;
      const uint32_t a[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      const uint32_t gw[4] = {nw[i].x, nw[i].y, nw[i].z, nw[i].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t nx = pack_bf16(bf16_bits_to_f32(a[e] & 0xFFFFu) * iv, bf16_bits_to_f32(a[e] >> 16) * iv);
        o[e] = pack_bf16(bf16_bits_to_f32(gw[e] & 0xFFFFu) * bf16_bits_to_f32(nx & 0xFFFFu),
                         bf16_bits_to_f32(gw[e] >> 16) * bf16_bits_to_f32(nx >> 16));
      }
      xv[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  // 3b. stage x: Q4 pair order, Q8 natural; per-chunk sums of the bf16 values
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
      uint32_t pr[8];  // decoded bf16 pairs of the 16 bytes (Q8), nibble bytes (Q4)
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if (BITS == 4) {
          // even nibbles (k0,k2,k4,k6) and odd nibbles as bytes, interleaved
          // with 0x43 below: (k0,k2) (k4,k6) (k1,k3) (k5,k7)
          pr[2 * k] = wd[k] & 0x0F0F0F0Fu;
          pr[2 * k + 1] = (wd[k] >> 4) & 0x0F0F0F0Fu;
        } else {
          decode_q8(wd[k], pr[2 * k], pr[2 * k + 1]);
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
            const uint32_t lo = pr[2 * k], hi = pr[2 * k + 1], c43 = 0x43434343u;
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
          for (int k = 0; k < 8; k++) d = dot2(pr[k], xd[k], d);
        }
        acc[r][m] += s * d + (b - OFF * s) * xsum;
      }
    }
  }
  // 5. row sums across the 64 lanes, epilogue
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MM; m++) acc[r][m] = wave_sum(acc[r][m]);
  if (lane != 0) return;
  if constexpr (F & kSwiGLU) {
    const RowSeg& Sg = p.seg[0];
    const RowSeg& Su = p.seg[1];
    const int n = rbase;
    if (n >= Sg.N) return;
#pragma unroll
    for (int m = 0; m < MM; m++) {
      float g = acc[0][m], u = acc[1][m];
      if (Sg.bias) g += bf16_bits_to_f32(Sg.bias[n]);
      if (Su.bias) u += bf16_bits_to_f32(Su.bias[n]);
      g = bf16_round(g);
      u = bf16_round(u);
      const float sig = bf16_round(1.0f / (1.0f + expf(-g)));
      const float a = bf16_round(g * sig);
      Sg.y[static_cast<int64_t>(m) * Sg.N + n] = static_cast<uint16_t>(f32_to_bf16_bits(a * u));
    }
  } else {
    const RowSeg& S = p.seg[sg];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int n = rbase + r;
      if (n >= S.N) continue;
#pragma unroll
      for (int m = 0; m < MM; m++) {
        float v = acc[r][m];
        if (S.bias) v += bf16_bits_to_f32(S.bias[n]);
        const int64_t o = static_cast<int64_t>(m) * S.N + n;
        if (S.res) v = bf16_bits_to_f32(S.res[o]) + bf16_round(v);
        S.y[o] = static_cast<uint16_t>(f32_to_bf16_bits(v));
      }
    }
  }
}

template <int BITS, int NI, int R, int W, int MM, int F>
int launch_rw(const RowParams& a, int64_t tiles, hipStream_t st) {
  MLXQ_LAUNCH((qmv_row_kernel<BITS, NI, R, W, MM, F>), dim3(static_cast<unsigned>(tiles)), dim3(64 * W), 0, st,
                     a);
  return check_launch("qmv_row");
}

// Workgroups of each matrix (R rows per wave, W waves), written into the
// segments' tile_end; returns the total.
int64_t set_tiles(RowParams& a, int R, int W, bool swiglu) {
  int64_t end = 0;
  for (int i = 0; i < a.nseg; i++) {
    if (!(swiglu && i)) end += ceil_div(a.seg[i].N, static_cast<int64_t>(swiglu ? W : R * W));
    a.seg[i].tile_end = static_cast<int>(end);
  }
  return end;
}

// (rows per wave, waves per workgroup) instantiated per row length: short
// rows take several rows per wave, long rows one (registers), with more
// waves per workgroup to share the activation staging.  Plain form (F = 0).
template <int BITS, int NI>
int launch_ni(RowParams& a, int64_t M, int R, int W, hipStream_t st) {
  if constexpr (NI * 8192 / BITS <= 4096) {  // several activation rows: K <= 4096 (LDS)
    if (M >= 2 && M <= 4) {
      const int64_t t = set_tiles(a, 1, 4, false);
      if (M == 2) return launch_rw<BITS, NI, 1, 4, 2, 0>(a, t, st);
      if (M == 3) return launch_rw<BITS, NI, 1, 4, 3, 0>(a, t, st);
      return launch_rw<BITS, NI, 1, 4, 4, 0>(a, t, st);
    }
  }
  if (M != 1) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_row: M > 1 needs K <= 4096");
  if constexpr (NI <= 2) {
    if (R >= 4) return launch_rw<BITS, NI, 4, 4, 1, 0>(a, set_tiles(a, 4, 4, false), st);
    if (R == 2) return launch_rw<BITS, NI, 2, 4, 1, 0>(a, set_tiles(a, 2, 4, false), st);
    return launch_rw<BITS, NI, 1, 4, 1, 0>(a, set_tiles(a, 1, 4, false), st);
  } else if constexpr (NI <= 4) {
    if (R >= 2) return launch_rw<BITS, NI, 2, 4, 1, 0>(a, set_tiles(a, 2, 4, false), st);
    return launch_rw<BITS, NI, 1, 4, 1, 0>(a, set_tiles(a, 1, 4, false), st);
  } else {
    if (R >= 2) {
      if (W >= 8) return launch_rw<BITS, NI, 2, 8, 1, 0>(a, set_tiles(a, 2, 8, false), st);
      return launch_rw<BITS, NI, 2, 4, 1, 0>(a, set_tiles(a, 2, 4, false), st);
    }
    if (W >= 16) return launch_rw<BITS, NI, 1, 16, 1, 0>(a, set_tiles(a, 1, 16, false), st);
    if (W >= 8) return launch_rw<BITS, NI, 1, 8, 1, 0>(a, set_tiles(a, 1, 8, false), st);
    return launch_rw<BITS, NI, 1, 4, 1, 0>(a, set_tiles(a, 1, 4, false), st);
  }
}

// Fused forms at M = 1 (the batch-1 decode chain), K*bits/8 of 1, 2 or 4 KB.
template <int BITS, int NI, int F>
int launch_fused_r(RowParams& a, int R, hipStream_t st) {
  // 8 waves per workgroup for the norm / SwiGLU / head-repeat forms: half
  // the workgroups stage (and normalise) the activations (config-5 batch-1
  // step 1.263 -> 1.245 and 1.232 -> 1.219 ms on two boxes); MLXQ_QMV_ROW_W=4 or 8 forces either
  const bool w8 = overrides().row_w ? overrides().row_w == 8 : F != 0;
  if constexpr (F & kSwiGLU) {
    if (w8) return launch_rw<BITS, NI, 2, 8, 1, F>(a, set_tiles(a, 2, 8, true), st);
    return launch_rw<BITS, NI, 2, 4, 1, F>(a, set_tiles(a, 2, 4, true), st);
  } else {
    if (w8) {
      if (R >= 2) return launch_rw<BITS, NI, 2, 8, 1, F>(a, set_tiles(a, 2, 8, false), st);
      return launch_rw<BITS, NI, 1, 8, 1, F>(a, set_tiles(a, 1, 8, false), st);
    }
    if (R >= 2) return launch_rw<BITS, NI, 2, 4, 1, F>(a, set_tiles(a, 2, 4, false), st);
    return launch_rw<BITS, NI, 1, 4, 1, F>(a, set_tiles(a, 1, 4, false), st);
  }
}
template <int BITS, int F>
int launch_fused_f(RowParams& a, int64_t ni, int R, hipStream_t st) {
  // the down projection (+ residual): 7 KB rows, one row x 8 waves (the plain
  // call's 2 rows x 4 waves measured 0.4% slower per batch-1 decode step here)
  if constexpr (BITS == 4 && F == 0) {
    if (ni == 7) return launch_rw<4, 7, 1, 8, 1, 0>(a, set_tiles(a, 1, 8, false), st);
  }
  if (ni == 1) return launch_fused_r<BITS, 1, F>(a, R, st);
  if (ni == 2) return launch_fused_r<BITS, 2, F>(a, R, st);
  return launch_fused_r<BITS, 4, F>(a, R, st);
}
template <int BITS>
int launch_fused_b(RowParams& a, int form, int64_t ni, int R, hipStream_t st) {
  switch (form) {
    case 0: return launch_fused_f<BITS, 0>(a, ni, R, st);
    case kNorm: return launch_fused_f<BITS, kNorm>(a, ni, R, st);
    case kNorm | kSwiGLU: return launch_fused_f<BITS, kNorm | kSwiGLU>(a, ni, R, st);
    default: return launch_fused_f<BITS, kRepeat>(a, ni, R, st);
  }
}

}  // namespace row

bool qmv_row_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M < 1 || M > 4 || N < 1 || (bits != 4 && bits != 8) || group_size < 128 / bits) return false;
  if (M > 1 && K > 4096) return false;  // the activation rows share the workgroup's LDS
  if ((K * bits / 8) % 1024) return false;
  const int64_t ni = K * bits / 8 / 1024;
  // Q4 with 7 KB rows (the down projection, K = 14336) run here, faster
  // than qmv_dot (9.92 -> 9.50 us at one row x 8 waves, less at two rows x
  // 4 waves); 14 KB and longer Q4 rows stay on qmv_dot
  if (bits == 4 && ni >= 14 && !overrides().qmv_row_all) return false;
  return ni == 1 || ni == 2 || ni == 4 || ni == 7 || ni == 8 || ni == 14 || ni == 16;
}

// Rows per wave and waves per workgroup, from measurements at the Llama
// shapes (MLXQ_QMV_ROW_R / MLXQ_QMV_ROW_W override them).
void qmv_row_geometry(int64_t N, int64_t K, int bits, int& R, int& W) {
  const int64_t ni = K * bits / 8 / 1024;
  // Q4 gate 9.72 vs 10.48 us at 2 rows (with the non-temporal loads 8.4-8.8
  // either way); q/o 4.10 at 1 row vs 4.28 at 2 (it was 4.96 vs 5.18 the
  // other way before the non-temporal loads); Q4 down (7 KB rows) 10.06 us at
  // 2 rows x 4 waves against 10.66 at 1 x 8 and 11.16 at 2 x 8 (the two rows
  // share each lane's activation reads from LDS); Q8 best at 1
  R = bits == 4 && ((ni <= 2 && N > 8192) || ni == 7) ? 2 : 1;
  W = bits == 4 && ni >= 8 ? 8 : 4;  // Q8 down: 14.2 us at 4 waves, 16.9 at 8
  if (overrides().row_r) R = overrides().row_r;
  if (overrides().row_w) W = overrides().row_w;
}

row::RowParams row_params(const QmvFused& f) {
  using namespace row;
  RowParams a{};
  a.x = f.x;
  a.norm_w = f.norm_w;
  a.eps = f.eps;
  a.x_stride = static_cast<int>(f.x_stride);
  a.gsh = __builtin_ctz(static_cast<unsigned>(f.group_size));
  a.rep = f.rep > 1 ? f.rep : 1;
  a.rep_hd8 = f.rep > 1 ? f.rep_hd / 8 : 1;
  a.rcp_hd8 = 1.0f / static_cast<float>(a.rep_hd8);
  a.rcp_grp = 1.0f / static_cast<float>(a.rep_hd8 * a.rep);
  a.nseg = f.nproj;
  for (int i = 0; i < f.nproj; i++) {
    const QmvProj& P = f.proj[i];
    a.seg[i] = RowSeg{P.wq, P.s, P.b, P.bias, P.res, P.y, static_cast<int>(P.N), 0};
  }
  return a;
}

int launch_qmv_row(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   hipStream_t st) {
  using namespace row;
  int R = 1, W = 4;
  qmv_row_geometry(N, K, bits, R, W);
  const int64_t ni = K * bits / 8 / 1024;
  QmvFused f{};
  f.x = x;
  f.M = M;
  f.K = K;
  f.x_stride = K;
  f.nproj = 1;
  f.proj[0] = QmvProj{wq, s, b, bias, nullptr, y, N};
  f.group_size = group_size;
  f.bits = bits;
  RowParams a = row_params(f);
#define MLXQ_ROW_CASE(NIV)                                                  \
  case NIV:                                                                 \
    return bits == 4 ? launch_ni<4, NIV>(a, M, R, W, st) : launch_ni<8, NIV>(a, M, R, W, st);
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

bool qmv_row_fused_eligible(const QmvFused& f) {
  if (f.M != 1 || (f.bits != 4 && f.bits != 8) || f.group_size < 128 / f.bits) return false;
  if (f.group_size != 32 && f.group_size != 64 && f.group_size != 128) return false;
  if ((f.K * f.bits / 8) % 1024) return false;
  const int64_t ni = f.K * f.bits / 8 / 1024;
  const bool plain = !f.norm_w && !f.swiglu && f.rep <= 1;
  if (ni != 1 && ni != 2 && ni != 4 && !(ni == 7 && f.bits == 4 && plain)) return false;
  if (f.nproj < 1 || f.nproj > row::kMaxSegs || (f.swiglu && f.nproj != 2)) return false;
  if (f.swiglu && f.proj[0].N != f.proj[1].N) return false;
  if (f.rep > 1 && (f.rep_hd <= 0 || f.rep_hd % 8 || f.K % (static_cast<int64_t>(f.rep_hd) * f.rep))) return false;
  if (f.rep > 1 && f.norm_w) return false;
  if (f.swiglu && !f.norm_w) return false;
  for (int i = 0; i < f.nproj; i++)
    if (f.proj[i].N < 1) return false;
  return true;
}

int launch_qmv_row_fused(const QmvFused& f, hipStream_t st) {
  using namespace row;
  if (!qmv_row_fused_eligible(f)) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_row: fused shape not supported");
  const int form = f.swiglu ? (kNorm | kSwiGLU) : f.norm_w ? kNorm : f.rep > 1 ? kRepeat : 0;
  const int64_t ni = f.K * f.bits / 8 / 1024;
  // rows per wave: 2 for Q4 over 2 KB rows (as the plain form on the taller
  // matrices), else 1; SwiGLU always takes a gate and an up row
  int R = f.bits == 4 && ni <= 2 ? 2 : 1;
  if (overrides().row_r) R = overrides().row_r;
  RowParams a = row_params(f);
  return f.bits == 4 ? launch_fused_b<4>(a, form, ni, R, st) : launch_fused_b<8>(a, form, ni, R, st);
}

}  // namespace mlxq
