// Decode GEMV for M <= 4 activation rows on the vector ALUs (gfx950):
// the kernel template, shared by the translation units that instantiate its
// plain and fused forms (qmv_dot*.hip).
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul at decode shapes (MLX's qmv family).
//
// At M <= 4 a 16-row MFMA tile would be 75-94% padding, so this kernel does
// the contraction with v_dot2_f32_bf16 instead:
//  * Streaming layout: lane (r16, gq) of a wave loads 16 bytes of codes of
//    weight row r16 (the gq-th quarter of a 64-byte chunk), so one wave
//    instruction reads 16 rows x 64 contiguous bytes -- as fast as a copy.
//  * Each lane contracts its own 32 (Q4) / 16 (Q8) codes per chunk against
//    the activations.  Q4 codes become bf16 (128 + q) pairs with two masks
//    and four v_perm per 8 codes; Q8 codes are converted exactly through f32.
//  * The activations are staged once per workgroup in LDS -- already in the
//    pair order of the Q4 unpack -- together with their sum over every lane
//    segment, so a segment's result is s * dot + (b - 128 s) * sum(x).  A
//    lane segment never straddles a quantization group (32 or 16 codes vs
//    groups of 32..128), so no masking is needed.
//  * One memory round trip: each thread first requests its activation
//    pieces, then the codes and group parameters of its wave's first round
//    (a wave owns a contiguous range of 64-byte chunks, taken 4 at a time);
//    the activation wait therefore never waits for the weights.  Each later
//    round is requested before the previous one is computed.
//  * Lanes reduce over gq with cross-lane adds, waves through LDS in fixed
//    order (deterministic), then bf16 y (+ bias) is stored.
//
// Fused forms (the decode layer chain of src/models/llama.rs:689-735 around
// the projections, at MLX's bf16 rounding points):
//  * kNorm: RMSNorm of the activations while they are staged (nn.rs:35-37),
//    at MLX's rounding points: x' = bf16(w * bf16(x * inv)), inv =
//    1/sqrt(mean(x^2) + eps) from f32 sums (one extra barrier).
//  * kRepeat: GQA head repeat of the activations (attention.rs:45-55) by
//    index remapping of the staging loads.
//  * Several projections of the same activations in one launch (q, k, v):
//    the workgroups are split over up to kMaxSegs weight matrices.
//  * residual epilogue (llama.rs:729-733): y = bf16(r + bf16(acc)).
//  * kSwiGLU: gate and up rows of the same index in one workgroup (its first
//    half of waves streams the gate rows, the second half the up rows) and
//    the epilogue y = bf16(bf16(g * bf16(sigmoid(g))) * u) with g, u the bf16
//    projection outputs (llama.rs:1040-1045).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"

namespace mlxq {
namespace dot {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxWaves = 8;  // waves per workgroup: 4 or 8 (chosen per shape)
constexpr int kRound = 4;     // chunks per round
constexpr int kMaxSegs = 3;   // weight matrices per launch

enum : int { kNorm = 1, kSwiGLU = 2, kRepeat = 4 };

// chunks per round: 4, or 2 when a wave streams 2 row sub-tiles (keeps the
// two rounds in flight within 128 registers) and a 2-chunk round still
// covers an even number of groups (whole 32-bit parameter words)
constexpr int round_chunks(int bits, int gs, int sub) {
  const int gb = gs * bits / 8;
  const int groups4 = kRound * (gb >= 64 ? 1 : 64 / gb) / (gb > 64 ? gb / 64 : 1);
  return sub >= 2 && groups4 >= 4 ? 2 : kRound;
}

struct Seg {
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* bias;  // [N] or null
  const uint16_t* res;   // [M, N] residual or null
  uint16_t* y;           // [M, N]
  int N;
  int tile_end;  // exclusive end of this matrix's workgroups (row tiles)
};

struct Params {
  const uint16_t* x;       // activations, row stride x_stride
  const uint16_t* norm_w;  // [K] RMSNorm weight (kNorm)
  float eps;
  int M;  // activation rows (the MFMA form; the vector-ALU form has M compiled in)
  int K;
  int cw;  // chunks per wave
  int x_stride;
  int rep_hd8, rep;        // kRepeat: head size in 8-element pieces, query heads per KV head
  float rcp_hd8, rcp_grp;  // 1 / rep_hd8, 1 / (rep_hd8 * rep) (division by reciprocal)
  int nseg;
  Seg seg[kMaxSegs];
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// two f32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// n / d for 0 <= n < 2^24, d >= 1, given rcp = 1/d: the f32 quotient is
// within one of the true one; one correction each way makes it exact.
__device__ __forceinline__ int div_rcp(int n, int d, float rcp) {
  int q = static_cast<int>(static_cast<float>(n) * rcp);
  q -= q * d > n;
  q += (q + 1) * d <= n;
  return q;
}

template <int BITS, int GS, int RC>
struct DotGeom {
  static constexpr int KC = 64 * 8 / BITS;             // k per 64-byte chunk
  static constexpr int KL = KC / 4;                    // k per lane per chunk (one segment)
  static constexpr int GB = GS * BITS / 8;             // bytes per group per row
  static constexpr int NGC = GB >= 64 ? 1 : 64 / GB;   // groups per chunk
  static constexpr int CPG = GB >= 64 ? GB / 64 : 1;   // chunks per group
  static constexpr int NGR = RC * NGC / CPG;           // groups per round of RC chunks
  static constexpr int NGW = (NGR + 1) / 2;            // 32-bit words holding NGR bf16
};

// Codes and group parameters of one round (RC chunks) for SUB rows.
template <int BITS, int GS, int SUB, int RC>
struct DotRound {
  using Gm = DotGeom<BITS, GS, RC>;
  uint4 w[RC][SUB];
  uint32_t s[SUB][Gm::NGW], b[SUB][Gm::NGW];
};

template <int NW>
__device__ __forceinline__ void load_param_words(const uint16_t* p, uint32_t (&v)[NW]) {
  if constexpr (NW == 1) {
    v[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (NW == 2) {
    uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = t.x; v[1] = t.y;
  } else {
#pragma unroll
    for (int i = 0; i < NW; i += 4) {
      uint4 t = *reinterpret_cast<const uint4*>(p + 2 * i);
      v[i] = t.x; v[i + 1] = t.y; v[i + 2] = t.z; v[i + 3] = t.w;
    }
  }
}

// Entry `base + j` of NGC consecutive bf16 parameters packed two per word;
// base is a compile-time index (so the words stay in registers) and j < NGC
// is the lane's group within its chunk (a select, not a dynamic index).
template <int NGC>
__device__ __forceinline__ float pick_param(const uint32_t* v, int base, int j) {
  if constexpr (NGC == 1) {
    const uint32_t w = v[base >> 1];
    return bf16_bits_to_f32((base & 1) ? (w >> 16) : (w & 0xFFFFu));
  } else if constexpr (NGC == 2) {  // base even: both entries in one word
    const uint32_t w = v[base >> 1];
    return __uint_as_float(j ? (w & 0xFFFF0000u) : (w << 16));
  } else {  // NGC == 4: two words
    const uint32_t w = j >= 2 ? v[(base >> 1) + 1] : v[base >> 1];
    return __uint_as_float((j & 1) ? (w & 0xFFFF0000u) : (w << 16));
  }
}

// PT: activation pieces (8 bf16 each) per thread in the LDS prologue;
// WV: waves per workgroup; F: fused forms (kNorm | kSwiGLU).
template <int BITS, int GS, int MV, int SUB, int RC, int PT, int WV, int F>
__global__ __launch_bounds__(64 * WV) void qmv_dot_kernel(const Params p) {
  using Gm = DotGeom<BITS, GS, RC>;
  using Rnd = DotRound<BITS, GS, SUB, RC>;
  static_assert(!(F & kSwiGLU) || SUB == 1, "SwiGLU splits the waves, not the rows");
  constexpr int R = 16 * SUB;
  constexpr int SEGP = Gm::KL / 8;  // pieces per segment
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  const int K = p.K;
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                   // [MV][K] bf16 (pair order)
  float* xsum = reinterpret_cast<float*>(smem + MV * K * 2);           // [MV][K / KL]
  float* red = xsum + MV * (K / Gm::KL);                               // [WV][MV][R]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches below
  const int r16 = lane & 15, gq = lane >> 4;
  const int G = K / GS;
  const int chunks = K * BITS / 8 / 64;
  const int64_t row_u4 = static_cast<int64_t>(K) * BITS / 128;

  // row tile of this workgroup: weight matrix `sg`, rows n0 .. n0 + R
  // (SwiGLU: rows n0 .. n0 + 16; waves [0, WV/2) stream the gate matrix,
  // waves [WV/2, WV) the up matrix, each half over the whole K)
  constexpr int KW = (F & kSwiGLU) ? WV / 2 : WV;  // waves sharing one row tile's K
  int sg = 0, n0;
  if constexpr (F & kSwiGLU) {
    n0 = blockIdx.x * 16;
    sg = wave / KW;
  } else {
    const int t = blockIdx.x;
    while (sg + 1 < p.nseg && t >= p.seg[sg].tile_end) sg++;
    n0 = (t - (sg ? p.seg[sg - 1].tile_end : 0)) * R;
  }

  // 1) activation pieces of this thread: issued first so that waiting for
  //    them never waits for the (later, slower) weight loads
  const int kp8 = K / 8;  // pieces per activation row
  const int pieces = MV * kp8;
  // activation row of piece i (M <= 4: compares instead of a division)
  auto row_of = [&](int i) {
    int m = 0;
#pragma unroll
    for (int t = 1; t < MV; t++) m += i >= t * kp8;
    return m;
  };
  uint4 xp[PT];
  uint4 nw[(F & kNorm) ? PT : 1];
#pragma unroll
  for (int j = 0; j < PT; j++) {  // clamped, unconditional: no branch, no early wait
    const int i = min(tid * PT + j, pieces - 1);
    const int m = row_of(i), k8 = i - m * kp8;
    int src8 = k8;
    if constexpr (F & kRepeat) {  // query head h reads KV head h / rep
      const int grp = p.rep_hd8 * p.rep;
      const int hq = div_rcp(k8, grp, p.rcp_grp);
      const int r = k8 - hq * grp;
      src8 = hq * p.rep_hd8 + (r - div_rcp(r, p.rep_hd8, p.rcp_hd8) * p.rep_hd8);
    }
    xp[j] = *reinterpret_cast<const uint4*>(p.x + static_cast<int64_t>(m) * p.x_stride + src8 * 8);
    if constexpr (F & kNorm) nw[j] = reinterpret_cast<const uint4*>(p.norm_w)[k8];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first

  // 2) codes and parameters of the wave's first round
  const uint4* wrow[SUB];
  const uint16_t* srow[SUB];
  const uint16_t* brow[SUB];
#pragma unroll
  for (int s = 0; s < SUB; s++) {
    const Seg& S = p.seg[sg];
    const int n = min(n0 + 16 * s + r16, S.N - 1);  // rows past N repeat row N-1
    wrow[s] = reinterpret_cast<const uint4*>(S.wq) + n * row_u4 + gq;
    srow[s] = S.s + static_cast<int64_t>(n) * G;
    brow[s] = S.b + static_cast<int64_t>(n) * G;
  }
  // The wave's chunk range [cbeg, cend) lies inside the row; its full rounds
  // end at cfull.  A round is fetched only when it ends at or before cfull,
  // so every load stays inside the row.  A wave whose range holds no full
  // round fetches none (the branches on cfull are wave-uniform).  Inside
  // fetch all register indices are compile-time, so a round stays in
  // registers.
  const int cbeg = min((wave % KW) * p.cw, chunks), cend = min(chunks, cbeg + p.cw);
  const int cfull = cbeg + ((cend - cbeg) / RC) * RC;  // end of the wave's full rounds
  auto fetch = [&](Rnd& T, int c0) {
    const int g0 = c0 * Gm::NGC / Gm::CPG;
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      load_param_words<Gm::NGW>(srow[s] + g0, T.s[s]);
      load_param_words<Gm::NGW>(brow[s] + g0, T.b[s]);
    }
#pragma unroll
    for (int u = 0; u < RC; u++)
#pragma unroll
      for (int s = 0; s < SUB; s++) T.w[u][s] = wrow[s][static_cast<int64_t>(c0 + u) * 4];
  };
  Rnd cur, nxt;
  // Unconditional: a wave with no full round fetches the row's last round
  // (unused; the host guarantees a row holds a round).  A conditional fetch
  // would make the compiler's memory-counter waits in the staging below wait
  // for these codes too, putting a second memory round trip before the math.
  fetch(cur, min(cbeg, chunks - RC));
  __builtin_amdgcn_sched_barrier(0);  // the whole first round is in flight before the prologue

  // 3a) RMSNorm: sums of x^2 per activation row over the workgroup, then
  //     x' = bf16(w * bf16(x * inv)) in registers
  if constexpr (F & kNorm) {
    float* ssq = red;  // [WV][MV]; red is next written after two more barriers
    float ss[MV];
#pragma unroll
    for (int m = 0; m < MV; m++) ss[m] = 0.f;
#pragma unroll
    for (int j = 0; j < PT; j++) {
      const int i = tid * PT + j;
      const uint32_t xs[4] = {xp[j].x, xp[j].y, xp[j].z, xp[j].w};
      float q = 0.f;
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const float a = bf16_bits_to_f32(xs[h] & 0xFFFFu), b = bf16_bits_to_f32(xs[h] >> 16);
        q = fmaf(a, a, fmaf(b, b, q));
      }
      const int mi = row_of(min(i, pieces - 1));
#pragma unroll
      for (int m = 0; m < MV; m++) ss[m] += (i < pieces && mi == m) ? q : 0.f;
    }
#pragma unroll
    for (int m = 0; m < MV; m++) {
      ss[m] = wave_sum(ss[m]);
      if (lane == 0) ssq[wave * MV + m] = ss[m];
    }
    __syncthreads();
    float inv[MV];
#pragma unroll
    for (int m = 0; m < MV; m++) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < WV; w++) t += ssq[w * MV + m];
      inv[m] = 1.0f / sqrtf(t / static_cast<float>(K) + p.eps);
    }
#pragma unroll
    for (int j = 0; j < PT; j++) {
      const int mi = row_of(min(tid * PT + j, pieces - 1));
      float iv = inv[0];
#pragma unroll
      for (int m = 1; m < MV; m++) iv = mi == m ? inv[m] : iv;
      const uint32_t xs[4] = {xp[j].x, xp[j].y, xp[j].z, xp[j].w};
      const uint32_t gw[4] = {nw[j].x, nw[j].y, nw[j].z, nw[j].w};
      uint32_t o[4];
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const uint32_t nx = pack_bf16(bf16_bits_to_f32(xs[h] & 0xFFFFu) * iv, bf16_bits_to_f32(xs[h] >> 16) * iv);
        o[h] = pack_bf16(bf16_bits_to_f32(gw[h] & 0xFFFFu) * bf16_bits_to_f32(nx & 0xFFFFu),
                         bf16_bits_to_f32(gw[h] >> 16) * bf16_bits_to_f32(nx >> 16));
      }
      xp[j] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }

  // 3b) activations -> LDS in the Q4 pair order, plus per-segment sums
  float segsum = 0.f;
#pragma unroll
  for (int j = 0; j < PT; j++) {
    const int i = tid * PT + j;
    uint4 v = xp[j];
    if constexpr (BITS == 4) {  // (x0,x1),(x2,x3),(x4,x5),(x6,x7) -> (x0,x2),(x4,x6),(x1,x3),(x5,x7)
      uint4 q;
      q.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
      q.y = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
      q.z = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
      q.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
      v = q;
    }
    const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; h++) segsum += bf16_bits_to_f32(ws[h] & 0xFFFFu) + bf16_bits_to_f32(ws[h] >> 16);
    if (i < pieces) reinterpret_cast<uint4*>(xl)[i] = v;
    if ((j + 1) % SEGP == 0) {  // PT is a multiple of SEGP: segments never straddle threads
      if (i < pieces) xsum[i / SEGP] = segsum;
      segsum = 0.f;
    }
  }
  __syncthreads();

  float acc[SUB][MV];
#pragma unroll
  for (int s = 0; s < SUB; s++)
#pragma unroll
    for (int m = 0; m < MV; m++) acc[s][m] = 0.f;

  const int jl = gq * Gm::KL / GS % Gm::NGC;  // lane's group within its chunk (NGC > 1)

  // dot products of one chunk (codes w) for SUB rows against the LDS activations
  auto chunk_dots = [&](const uint4 (&w)[SUB], int kbase, float (&dots)[SUB][MV]) {
#pragma unroll
    for (int s = 0; s < SUB; s++)
#pragma unroll
      for (int m = 0; m < MV; m++) dots[s][m] = 0.f;
#pragma unroll
    for (int t = 0; t < Gm::KL / 8; t++) {  // 8 codes per step
      uint32_t xv[MV][4];
#pragma unroll
      for (int m = 0; m < MV; m++) {
        const uint4 v = *reinterpret_cast<const uint4*>(xl + m * K + kbase + 8 * t);
        xv[m][0] = v.x; xv[m][1] = v.y; xv[m][2] = v.z; xv[m][3] = v.w;
      }
#pragma unroll
      for (int s = 0; s < SUB; s++) {
        const uint32_t wv[4] = {w[s].x, w[s].y, w[s].z, w[s].w};
        uint32_t q[4];
        if constexpr (BITS == 4) {
          // codes k0..k7 -> bf16 (128 + k) pairs (k0,k2),(k4,k6),(k1,k3),(k5,k7):
          // even / odd nibbles masked into bytes, then interleaved with 0x43
          // bytes by v_perm (0x43nn is the bf16 of 128 + nn)
          const uint32_t c = wv[t];
          const uint32_t lo = c & 0x0F0F0F0Fu, hi = (c >> 4) & 0x0F0F0F0Fu, e = 0x43434343u;
          q[0] = __builtin_amdgcn_perm(lo, e, 0x00050004u);
          q[1] = __builtin_amdgcn_perm(lo, e, 0x00070006u);
          q[2] = __builtin_amdgcn_perm(hi, e, 0x00050004u);
          q[3] = __builtin_amdgcn_perm(hi, e, 0x00070006u);
        } else {
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const uint32_t c = wv[2 * t + h];
            const float f0 = static_cast<float>(c & 0xFFu), f1 = static_cast<float>((c >> 8) & 0xFFu);
            const float f2 = static_cast<float>((c >> 16) & 0xFFu), f3 = static_cast<float>(c >> 24);
            q[2 * h] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
            q[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
          }
        }
#pragma unroll
        for (int m = 0; m < MV; m++)
          dots[s][m] = dot2(q[3], xv[m][3], dot2(q[2], xv[m][2], dot2(q[1], xv[m][1], dot2(q[0], xv[m][0], dots[s][m]))));
      }
    }
  };

  auto compute = [&](const Rnd& T, int c0) {
#pragma unroll
    for (int u = 0; u < RC; u++) {
      const int seg = (c0 + u) * 4 + gq;  // lane segment index (KL codes)
      float dots[SUB][MV];
      chunk_dots(T.w[u], seg * Gm::KL, dots);
      const int base = u * Gm::NGC / Gm::CPG;  // first group of chunk u (compile-time after unrolling)
#pragma unroll
      for (int s = 0; s < SUB; s++) {
        const float sc = pick_param<Gm::NGC>(T.s[s], base, jl);
        const float c = pick_param<Gm::NGC>(T.b[s], base, jl) - OFF * sc;
#pragma unroll
        for (int m = 0; m < MV; m++) acc[s][m] = fmaf(sc, dots[s][m], fmaf(c, xsum[m * (K / Gm::KL) + seg], acc[s][m]));
      }
    }
  };

  // 4) full rounds of RC chunks, the next one in flight while one is
  //    computed; the last round is peeled so that nothing is fetched past
  //    the wave's range (a wasted fetch would add a memory round trip to
  //    the end of every wave)
  if (cfull > cbeg) {
    int c0 = cbeg;
    for (; c0 + RC < cfull; c0 += RC) {
      fetch(nxt, c0 + RC);
      __builtin_amdgcn_sched_barrier(0);  // next round in flight before this one is computed
      compute(cur, c0);
      cur = nxt;
    }
    compute(cur, c0);
  }
  // ragged end of the wave's range (< RC chunks): each lane gathers its own
  // group's parameters
  for (int c = cfull; c < cend; c++) {
    const int seg = c * 4 + gq;
    const int g = seg * Gm::KL / GS;
    uint4 w[SUB];
    float sc[SUB], bb[SUB];
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      w[s] = wrow[s][static_cast<int64_t>(c) * 4];
      sc[s] = bf16_bits_to_f32(srow[s][g]);
      bb[s] = bf16_bits_to_f32(brow[s][g]);
    }
    float dots[SUB][MV];
    chunk_dots(w, seg * Gm::KL, dots);
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      const float c2 = bb[s] - OFF * sc[s];
#pragma unroll
      for (int m = 0; m < MV; m++) acc[s][m] = fmaf(sc[s], dots[s][m], fmaf(c2, xsum[m * (K / Gm::KL) + seg], acc[s][m]));
    }
  }

  // 5) reduce over the 4 lane groups (same row, other k segments), then waves
#pragma unroll
  for (int s = 0; s < SUB; s++)
#pragma unroll
    for (int m = 0; m < MV; m++) {
      float v = acc[s][m];
      v = add_xor32(add_xor16(v));
      if (gq == 0) red[(wave * MV + m) * R + 16 * s + r16] = v;
    }
  __syncthreads();
  auto wave_sum = [&](int m, int r, int w0) {  // waves w0 .. w0 + KW
    float sum = red[(w0 * MV + m) * R + r];
#pragma unroll
    for (int w = 1; w < KW; w++) sum += red[((w0 + w) * MV + m) * R + r];
    return sum;
  };
  if constexpr (F & kSwiGLU) {
    const Seg& Sg = p.seg[0];
    const Seg& Su = p.seg[1];
    for (int i = tid; i < MV * 16; i += 64 * WV) {
      const int m = i / 16, r = i % 16, n = n0 + r;
      if (n >= Sg.N) continue;
      float g = wave_sum(m, r, 0), u = wave_sum(m, r, KW);
      if (Sg.bias) g += bf16_bits_to_f32(Sg.bias[n]);
      if (Su.bias) u += bf16_bits_to_f32(Su.bias[n]);
      g = bf16_round(g);
      u = bf16_round(u);
      const float sig = bf16_round(1.0f / (1.0f + expf(-g)));
      const float a = bf16_round(g * sig);
      Sg.y[static_cast<int64_t>(m) * Sg.N + n] = static_cast<uint16_t>(f32_to_bf16_bits(a * u));
    }
  } else {
    const Seg& S = p.seg[sg];
    for (int i = tid; i < MV * R; i += 64 * WV) {
      const int m = i / R, r = i % R, n = n0 + r;
      if (n >= S.N) continue;
      float sum = wave_sum(m, r, 0);
      if (S.bias) sum += bf16_bits_to_f32(S.bias[n]);
      const int64_t o = static_cast<int64_t>(m) * S.N + n;
      if (S.res) sum = bf16_bits_to_f32(S.res[o]) + bf16_round(sum);
      S.y[o] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
    }
  }
}

// ---------------------------------------------------------------- launch

struct Cfg {
  int sub = 1, wv = 8, pt = 0;
  int64_t tiles = 0;
  size_t lds = 0;
};

// query != nullptr: report resident workgroups per CU for this configuration
// instead of launching (the choice between configurations needs it).
template <int BITS, int GS, int MV, int SUB, int PT, int WV, int F>
int run(const Cfg& c, const Params& a, hipStream_t st, int* query) {
  auto kern = qmv_dot_kernel<BITS, GS, MV, SUB, round_chunks(BITS, GS, SUB), PT, WV, F>;
  static bool raised = false;  // once per process; the attribute is per function
  if (c.lds > 64 * 1024 && !raised) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmv_dot: LDS size: ") + hipGetErrorString(e));
    raised = true;
  }
  if (query) {
    static int cached = -1;  // the kernel's registers fix it; LDS is part of the key
    static size_t cached_lds = 0;
    if (cached < 0 || cached_lds != c.lds) {
      int nb = 0;
      hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), 64 * WV,
                                                                  c.lds);
      if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmv_dot: occupancy: ") + hipGetErrorString(e));
      cached = nb;
      cached_lds = c.lds;
    }
    *query = cached;
    return MLXQ_OK;
  }
  MLXQ_LAUNCH(kern, dim3(c.tiles), dim3(64 * WV), c.lds, st, a);
  return check_launch("qmv_dot");
}

template <int BITS, int GS, int MV, int SUB, int WV, int F>
int run_pt(const Cfg& c, const Params& a, hipStream_t st, int* q) {
  constexpr int SEGP = 64 * 8 / BITS / 4 / 8;
  if (c.pt <= SEGP) return run<BITS, GS, MV, SUB, SEGP, WV, F>(c, a, st, q);
  if (c.pt <= 2 * SEGP) return run<BITS, GS, MV, SUB, 2 * SEGP, WV, F>(c, a, st, q);
  if constexpr (4 * SEGP <= 8) {
    if (c.pt <= 4 * SEGP) return run<BITS, GS, MV, SUB, 4 * SEGP, WV, F>(c, a, st, q);
  }
  return fail(MLXQ_ERR_INVALID, "qmv_dot: activation prologue too large");
}

template <int BITS, int GS, int SUB, int WV, int F>
int run_m(int64_t M, const Cfg& c, const Params& a, hipStream_t st, int* q) {
  switch (M) {
    case 1: return run_pt<BITS, GS, 1, SUB, WV, F>(c, a, st, q);
    case 2: return run_pt<BITS, GS, 2, SUB, WV, F>(c, a, st, q);
    case 3: return run_pt<BITS, GS, 3, SUB, WV, F>(c, a, st, q);
    default: return run_pt<BITS, GS, 4, SUB, WV, F>(c, a, st, q);
  }
}

template <int BITS, int GS, int F>
int run_cfg(int64_t M, const Cfg& c, const Params& a, hipStream_t st, int* q) {
  if constexpr (F & kSwiGLU) {
    return c.wv == 4 ? run_m<BITS, GS, 1, 4, F>(M, c, a, st, q) : run_m<BITS, GS, 1, 8, F>(M, c, a, st, q);
  } else {
    if (c.sub == 1) return c.wv == 4 ? run_m<BITS, GS, 1, 4, F>(M, c, a, st, q) : run_m<BITS, GS, 1, 8, F>(M, c, a, st, q);
    return c.wv == 4 ? run_m<BITS, GS, 2, 4, F>(M, c, a, st, q) : run_m<BITS, GS, 2, 8, F>(M, c, a, st, q);
  }
}

// One instantiation per fused form F, each in its own translation unit.
template <int F>
int dispatch(int64_t M, int group_size, int bits, const Cfg& c, const Params& a, hipStream_t st, int* q) {
  if (bits == 4) {
    if (group_size == 32) return run_cfg<4, 32, F>(M, c, a, st, q);
    if (group_size == 64) return run_cfg<4, 64, F>(M, c, a, st, q);
    return run_cfg<4, 128, F>(M, c, a, st, q);
  }
  if (group_size == 32) return run_cfg<8, 32, F>(M, c, a, st, q);
  if (group_size == 64) return run_cfg<8, 64, F>(M, c, a, st, q);
  return run_cfg<8, 128, F>(M, c, a, st, q);
}

extern template int dispatch<0>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);
extern template int dispatch<kNorm>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);
extern template int dispatch<kNorm | kSwiGLU>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);
extern template int dispatch<kRepeat>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);

}  // namespace dot
}  // namespace mlxq
