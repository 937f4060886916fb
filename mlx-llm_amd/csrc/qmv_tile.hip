// Batched-decode quantized GEMV on the matrix cores (gfx950): 5..32
// activation rows, the activations shared through LDS.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul at batched-decode shapes (MLX's qmv / small
// qmm kernels).
//
// A wave that streams 16 weight rows and reads its own activations moves
// 4M/16 bytes of activations per byte of Q4 codes (8x at M = 32): the
// activation reads, not the weights, then fill the memory pipeline.  Here:
//  * A workgroup of 4 or 8 waves covers 64 or 128 weight rows (16 per wave)
//    over one slice of K (4, 8 or 16 64-byte chunks per row).  The slice's
//    activations (16 * MT rows) are loaded once by the workgroup and staged
//    in LDS (rows padded by 16 bytes, so the 16 rows of an MFMA operand read
//    hit distinct banks; Q4 pairs pre-permuted to the code order), and every
//    wave reads its MFMA A operands from there.
//  * Every load of the slice is issued up front (activations, group
//    parameters, then the codes chunk by chunk): one memory round trip, and
//    the math on chunk c waits only for chunks <= c.
//  * Math per chunk: lane (r16, gq) holds 16 bytes of weight row r16; a
//    4 x 4 dword transpose across the lane rows gives group-pure MFMA
//    blocks; P = sum x (OFF + q) per group, acc += s P in f32.  The rest of
//    the affine term, sum_g S_g (b - OFF s) with S_g the group's sum of x,
//    is one MFMA (two for Q4) per slice: the group sums are formed once per
//    workgroup while staging (not per wave and chunk) and fed as bf16 hi/lo
//    halves against the bf16 biases (and scales).
//  * Split K: blockIdx.y picks the slice.  With more than one slice the
//    workgroups store f32 partial tiles in the caller's workspace and a
//    second, elementwise kernel adds them in slice order (deterministic),
//    adds the bias and stores bf16 y.  A hand-off inside the first kernel
//    (last-arriving workgroup reduces) was measured slower: its device-scope
//    stores, counter atomic and loads are three serial trips past the L2.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "common.hpp"
#include "mfma_blocks.hpp"
#include "qmatmul.hpp"
#include "qmv_dot_kernel.hpp"

namespace mlxq {
namespace tile {

using dot::DotGeom;
using dot::load_param_words;
using mfma::Blk;
using mfma::decode_q8;
using mfma::f32x4;
using mfma::mma;
using mfma::transpose_rows;
using mfma::u32x4;

struct TileParams {
  const uint16_t* x;
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* bias;
  uint16_t* y;
  float* part;  // [splits][M][N] partial sums (splits > 1)
  int M, N, K;
  int splits;
  int steps;  // K slices per workgroup (streaming form)
  // fused forms (whole-K form only, no K split): residual epilogue
  // y = bf16(res + bf16(acc + bias)); GQA head repeat by remapping the
  // activation loads; up to three weight matrices of the same activations,
  // each its own run of tiles (segment) of blockIdx.x
  const uint16_t* res;     // [M, N] or null
  // SwiGLU (streaming form): even row groups read the gate matrix (wq, s, b,
  // bias), odd ones the up matrix (wq2, s2, b2, bias2) for the same outputs;
  // y = bf16(bf16(g * bf16(sigmoid(g))) * u) of the bf16 projections
  const uint32_t* wq2;
  const uint16_t* s2;
  const uint16_t* b2;
  const uint16_t* bias2;
  int x_stride;            // activation row stride (elements)
  int rep_hd8, rep;        // head repeat: piece k8 reads (k8 / (rep_hd8 rep)) rep_hd8 + k8 % rep_hd8
  float rcp_hd8, rcp_grp;
  int rep_sh_hd8, rep_sh_grp;  // log2 of rep_hd8 and rep_hd8 rep when both are powers of two, else -1
};

// One weight matrix of a fused launch; its tiles end at tile_end (exclusive).
struct TileSeg {
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* bias;
  const uint16_t* res;
  uint16_t* y;
  int N;
  int tile_end;
};
struct TileFused {
  TileParams p;  // x, M, K and the fused-form fields; the matrix fields come from seg
  int nseg;
  TileSeg seg[3];
};

// n / d for 0 <= n < 2^24, d >= 1, given rcp = 1/d: the f32 quotient is
// within one of the true one; one correction each way makes it exact.
__device__ __forceinline__ int div_rcp(int n, int d, float rcp) {
  int q = static_cast<int>(static_cast<float>(n) * rcp);
  q -= q * d > n;
  q += (q + 1) * d <= n;
  return q;
}

// First activation row of this workgroup's M block (blockIdx.z): a call with
// more activation rows than one workgroup stages runs the blocks side by
// side, each over the same weight rows.
template <int MT>
__device__ __forceinline__ int m_block0() {
  return static_cast<int>(blockIdx.z) * 16 * MT;
}

constexpr int kMaxSplitsK = 16;  // most K splits of one call

// Q4 codes of one dword (k0..k7, LSB first) -> bf16 (128 + k) pairs
// (k0,k2),(k4,k6),(k1,k3),(k5,k7): two masks pick the even / odd nibbles
// into bytes, then v_perm interleaves them with 0x43 bytes (0x43nn is the
// bf16 of 128 + nn).  7 operations per dword.
__device__ __forceinline__ void decode_q4_bytes(uint32_t q, uint32_t* b) {
  const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu, c = 0x43434343u;
  b[0] = __builtin_amdgcn_perm(lo, c, 0x00050004u);
  b[1] = __builtin_amdgcn_perm(lo, c, 0x00070006u);
  b[2] = __builtin_amdgcn_perm(hi, c, 0x00050004u);
  b[3] = __builtin_amdgcn_perm(hi, c, 0x00070006u);
}

// 8 activations x0..x7 (4 dwords as loaded) -> the order of decode_q4_bytes:
// (x0,x2),(x4,x6),(x1,x3),(x5,x7)
__device__ __forceinline__ void act_order_q4_bytes(const uint32_t* x, uint32_t* a) {
  a[0] = __builtin_amdgcn_perm(x[1], x[0], 0x05040100u);
  a[1] = __builtin_amdgcn_perm(x[3], x[2], 0x05040100u);
  a[2] = __builtin_amdgcn_perm(x[1], x[0], 0x07060302u);
  a[3] = __builtin_amdgcn_perm(x[3], x[2], 0x07060302u);
}

// Geometry of a workgroup: WV waves in RG = WV / KH row groups of 16 weight
// rows times KH parts of the workgroup's K slice, NCH chunks per wave.
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
struct TileGeom {
  using Bk = Blk<BITS, GS>;
  static constexpr int T = 64 * WV;                  // threads
  static constexpr int RG = WV / KH;                 // row groups (16 weight rows each)
  static constexpr int MR = 16 * MT;                 // activation rows staged (padded)
  static constexpr int KS = NCH * Bk::KC;            // k per wave slice
  static constexpr int KW = KH * KS;                 // k per workgroup slice
  static constexpr int ROW16 = KW / 8 + 1;           // 16-byte slots per staged row (one of padding)
  static constexpr int XP = MR * (KW / 8) / T;       // 16-byte activation pieces per thread
  static constexpr int NG = KS / GS;                 // groups per wave slice
  static constexpr int NGW = NG / 2;                 // parameter words per row and wave slice
  // group sums of the staged activations, as MFMA A operands of the bias
  // term: per row and K part [hi(0..NGP), lo(0..NGP), zeros] in bf16, KB
  // blocks of 32 k
  static constexpr int NGP = NG < 8 ? 8 : NG;        // groups padded to whole 8-lane slices
  static constexpr int KB = (2 * NGP + 31) / 32;     // bias-term MFMAs per M tile
  static constexpr int SXP = 32 * KB;                // bf16 per K part
  static constexpr int SXS = KH * SXP + 8;           // bf16 per row (8 of padding)
  // codes loaded row-contiguous across lanes (tile_load_w)
  static constexpr bool COAL = Bk::NAT && MT == 2 && NCH <= 4;
  static_assert(WV % KH == 0, "K parts divide the waves");
  static_assert(XP >= 1 && MR * (KW / 8) % T == 0, "activation pieces must divide over the threads");
  static_assert(NG % 2 == 0 && (NGW == 2 || NGW % 4 == 0), "parameters load as whole vectors");
  static_assert(NGP % 8 == 0 && (KW / 8) % 8 == 0, "a group's eight pieces sit in eight consecutive lanes");
};

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// One work item (16 RG weight rows x one workgroup K slice): its global
// data, held in registers from the loads until they are used -- the
// activation pieces until the LDS staging, the parameters and codes until
// the math.
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
struct TileX {
  u32x4 xg[TileGeom<BITS, GS, MT, WV, NCH, KH>::XP];  // activation pieces of the slice
};
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
struct TileW {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  uint32_t sw[Tg::NGW], bw[Tg::NGW];  // this lane's row's scales / biases over the wave's slice
  u32x4 w[NCH];                       // this lane's 16 bytes of its row, per chunk
};

// The activation loads of the workgroup's slice: piece i of this thread is
// 16-byte slot tid + T i of the slice's rows of C slots; its row and column
// follow from tid at compile-time steps.
template <int BITS, int GS, int MT, int WV, int NCH, int KH, bool FUSED = false>
__device__ __forceinline__ void tile_load_x(const TileParams& p, int split, TileX<BITS, GS, MT, WV, NCH, KH>& X) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  const int tid = threadIdx.x;
  constexpr int C = Tg::KW / 8;
  const uint16_t* xs0 = p.x + split * Tg::KW;  // slice start (element offsets stay below 2^31)
#pragma unroll
  for (int i = 0; i < Tg::XP; i++) {  // rows past M read row M-1: they only feed output rows >= M
    const int row = Tg::T >= C ? tid / C + i * (Tg::T / C) : i / (C / Tg::T);
    const int col = Tg::T >= C ? tid % C : tid + Tg::T * (i % (C / Tg::T));
    int src = col;
    if constexpr (FUSED) {
      if (p.rep > 1) {  // query head hq reads KV head hq / rep (whole-K form: col is the piece of the row)
        if (p.rep_sh_grp >= 0) {  // powers of two (Llama: 16 pieces per head, 4 query heads per KV head)
          src = ((col >> p.rep_sh_grp) << p.rep_sh_hd8) + (col & (p.rep_hd8 - 1));
        } else {
          const int grp = p.rep_hd8 * p.rep;
          const int hq = div_rcp(col, grp, p.rcp_grp);
          const int r = col - hq * grp;
          src = hq * p.rep_hd8 + (r - div_rcp(r, p.rep_hd8, p.rcp_hd8) * p.rep_hd8);
        }
      }
    }
    X.xg[i] = *reinterpret_cast<const u32x4*>(xs0 + min(m_block0<MT>() + row, p.M - 1) * (FUSED ? p.x_stride : p.K) +
                                              src * 8);
  }
}

// The group parameters, then the codes chunk by chunk (the math on chunk c
// waits only for chunks <= c), of this lane's weight row over this wave's
// part of the slice.
template <int BITS, int GS, int MT, int WV, int NCH, int KH, bool SW = false>
__device__ __forceinline__ void tile_load_w(const TileParams& p, int tile, int split,
                                            TileW<BITS, GS, MT, WV, NCH, KH>& W) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  using Bk = typename Tg::Bk;
  const int K = p.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave % Tg::RG, kh = wave / Tg::RG;
  const int r16 = lane & 15, gq = lane >> 4;
  const int G = K / GS;
  const int64_t row_u4 = static_cast<int64_t>(K) * BITS / 128;
  const int c0 = (split * KH + kh) * NCH;  // first chunk of the wave's part
  // rows past N repeat row N-1 (results dropped); SwiGLU: row group rg
  // reads matrix rg & 1 at output block rg / 2
  const bool up = SW && (rg & 1);
  const int n = SW ? min(tile * 8 * Tg::RG + (rg >> 1) * 16 + r16, p.N - 1)
                   : min(tile * 16 * Tg::RG + rg * 16 + r16, p.N - 1);
  load_param_words<Tg::NGW>((up ? p.s2 : p.s) + static_cast<int64_t>(n) * G + c0 * Bk::KC / GS, W.sw);
  load_param_words<Tg::NGW>((up ? p.b2 : p.b) + static_cast<int64_t>(n) * G + c0 * Bk::KC / GS, W.bw);
  // Q8 (natural block layout) with 32 activation rows: lanes 4r..4r+3 load
  // row r's 64 contiguous bytes of a chunk (adjacent lanes on one piece of a
  // row), and the math moves them to lane (row, quarter) = r + 16 q with
  // ds_bpermute.  Measured (Q8 M = 32, µs): gate 21.88 -> 21.36, down 23.11
  // -> 22.57; with 16 rows the bpermutes cost more than they save (gate
  // 18.18 -> 18.44), and so they do with 8 chunks per wave (q 10.70 ->
  // 10.97), so those keep the row-per-lane-group loads.
  if constexpr (Tg::COAL) {
    const int rc = lane >> 2, qc = lane & 3;
    const int nc = SW ? min(tile * 8 * Tg::RG + (rg >> 1) * 16 + rc, p.N - 1)
                      : min(tile * 16 * Tg::RG + rg * 16 + rc, p.N - 1);
    const u32x4* wrc = reinterpret_cast<const u32x4*>(up ? p.wq2 : p.wq) + nc * row_u4 + qc;
#pragma unroll
    for (int c = 0; c < NCH; c++) W.w[c] = wrc[static_cast<int64_t>(c0 + c) * 4];
    return;
  }
  const u32x4* wrow = reinterpret_cast<const u32x4*>(up ? p.wq2 : p.wq) + n * row_u4 + gq;
#pragma unroll
  for (int c = 0; c < NCH; c++) W.w[c] = wrow[static_cast<int64_t>(c0 + c) * 4];
}

// Stage the workgroup slice's activations in LDS (and their group sums),
// then a barrier.
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
__device__ __forceinline__ void tile_stage(const TileX<BITS, GS, MT, WV, NCH, KH>& X, u32x4* xs, uint16_t* sx,
                                           bool pad = true) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  const int tid = threadIdx.x;
  constexpr int C = Tg::KW / 8;
  // staged in the order of the Q4 decode (pairs (x0,x2),(x4,x6),...): the
  // permutation is done once here instead of by every wave per block.  The
  // sum of x over each group (row m, group g) is formed here once for the
  // workgroup: a piece's 8 values with v_dot2 against ones, then the group's
  // 8 pieces (8 consecutive lanes) with DPP adds; it is stored as the bf16
  // pair hi + lo (hi = bf16(S), lo = bf16(S - hi): S to about 2^-16).
  const uint32_t one2 = 0x3F803F80u;  // bf16 (1, 1)
#pragma unroll
  for (int i = 0; i < Tg::XP; i++) {
    float ps = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) ps = dot::dot2(X.xg[i][w], one2, ps);
    ps += dpp_f32<kDppQuadXor1>(ps);
    ps += dpp_f32<kDppQuadXor2>(ps);
    ps += dpp_f32<kDppRowHalfMirror>(ps);  // the 8 lanes of the group now hold its sum
    const int row = Tg::T >= C ? tid / C + i * (Tg::T / C) : i / (C / Tg::T);
    const int col = Tg::T >= C ? tid % C : tid + Tg::T * (i % (C / Tg::T));
    if constexpr (BITS == 4) {
      const uint32_t xv[4] = {X.xg[i][0], X.xg[i][1], X.xg[i][2], X.xg[i][3]};
      uint32_t a[4];
      act_order_q4_bytes(xv, a);
      xs[row * Tg::ROW16 + col] = u32x4{a[0], a[1], a[2], a[3]};
    } else {
      xs[row * Tg::ROW16 + col] = X.xg[i];
    }
    // the group's 8 lanes store the same value (no branch)
    const int gw = col / (GS / 8);  // group within the workgroup slice
    const uint32_t hi = bf16_rne_bits(ps);
    uint16_t* sr = sx + row * Tg::SXS + (gw / Tg::NG) * Tg::SXP + gw % Tg::NG;
    sr[0] = static_cast<uint16_t>(hi);
    sr[Tg::NGP] = static_cast<uint16_t>(bf16_rne_bits(ps - __uint_as_float(hi << 16)));
  }
  // zeros in the padding of the group-sum rows (groups NG..NGP of each
  // half, and past 2 NGP, in every K part)
  if (pad)
  for (int e = tid; e < Tg::MR * KH * Tg::SXP; e += Tg::T) {
    const int row = e / (KH * Tg::SXP), t = e % Tg::SXP, part = (e / Tg::SXP) % KH;
    if (t >= 2 * Tg::NGP || t % Tg::NGP >= Tg::NG) sx[row * Tg::SXS + part * Tg::SXP + t] = 0;
  }
  __syncthreads();
}

// The math of one K slice from the staged activations and the wave's
// parameters and codes: group-pure MFMAs and per-group folds, then the bias
// term, added into the wave's accumulators acc (16 weight rows x 16 MT
// activation rows).
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
__device__ __forceinline__ void tile_accum(f32x4 (&acc)[MT], const TileW<BITS, GS, MT, WV, NCH, KH>& L,
                                           const u32x4* xs, const uint16_t* sx) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  using Bk = typename Tg::Bk;
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = wave / Tg::RG;
  const int r16 = lane & 15, gq = lane >> 4;
  const int xc0 = kh * NCH;  // the wave's first chunk within the staged slice

#pragma unroll
  for (int c = 0; c < NCH; c++) {
    uint32_t d[4] = {L.w[c][0], L.w[c][1], L.w[c][2], L.w[c][3]};
    if constexpr (Tg::COAL) {  // from the loading lane 4 r16 + gq (tile_load_w)
      const int src = (4 * r16 + gq) * 4;
#pragma unroll
      for (int i = 0; i < 4; i++) d[i] = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(d[i]));
    }
    if constexpr (!Bk::NAT) transpose_rows(d);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 P[MT];
#pragma unroll
    for (int j = 0; j < Bk::NB; j++) {
      const bool first = j % Bk::BPG == 0;
      uint32_t bq[4];
      if constexpr (BITS == 4) {
        decode_q4_bytes(d[j], bq);
      } else if constexpr (Bk::NAT) {
        decode_q8(d[2 * j], bq);
        decode_q8(d[2 * j + 1], bq + 2);
      } else {
        decode_q8(d[j], bq);
      }
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        // A operand: activation row 16 mt + r16, this lane's slice of block j
        const u32x4* rowp = xs + (16 * mt + r16) * Tg::ROW16;
        const int e = (xc0 + c) * Bk::KC + Bk::xoff(j, gq);
        uint32_t a[4];
        if constexpr (Bk::XW == 4) {
          const u32x4 v = rowp[e / 8];
          a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
        } else {
          const uint2 v = reinterpret_cast<const uint2*>(rowp)[e / 4];
          a[0] = v.x; a[1] = v.y;
        }
        P[mt] = mma<Bk::X32>(a, bq, first ? zero : P[mt]);
      }
      if (j % Bk::BPG == Bk::BPG - 1) {
        const int g = (c * Bk::KC + Bk::code0(j)) / GS;  // group within the wave slice (compile-time)
        const float sc = __uint_as_float((g & 1) ? (L.sw[g >> 1] & 0xFFFF0000u) : (L.sw[g >> 1] << 16));
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int v = 0; v < 4; v++) acc[mt][v] = fmaf(sc, P[mt][v], acc[mt][v]);
      }
    }
  }

  // The bias term sum_g S[m, g] (b[n, g] - OFF s[n, g]) of the wave slice on
  // the matrix cores: A = the staged group sums (hi and lo halves), B = this
  // row's biases (and scales) over the same k positions, both halves.  Lane
  // (r16, gq) supplies k = 32 kb + 8 gq + [0, 8): groups g0.. of one half.
  {
    f32x4 ab[MT], as[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) ab[mt] = as[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < Tg::KB; kb++) {
      const int t0 = 32 * kb + 8 * gq;
      const bool valid = t0 < 2 * Tg::NGP;
      const int g0 = t0 % Tg::NGP;
      uint32_t bb[4] = {0u, 0u, 0u, 0u}, bs[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int cg = 0; cg < Tg::NGP / 8; cg++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (4 * cg + i < Tg::NGW) {
            const bool take = valid && g0 == 8 * cg;
            bb[i] = take ? L.bw[4 * cg + i] : bb[i];
            if constexpr (BITS == 4) bs[i] = take ? L.sw[4 * cg + i] : bs[i];
          }
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const u32x4 av =
            *reinterpret_cast<const u32x4*>(sx + (16 * mt + r16) * Tg::SXS + kh * Tg::SXP + t0);
        const uint32_t a[4] = {av[0], av[1], av[2], av[3]};
        ab[mt] = mma<true>(a, bb, ab[mt]);
        if constexpr (BITS == 4) as[mt] = mma<true>(a, bs, as[mt]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++)
        acc[mt][v] += BITS == 4 ? fmaf(-OFF, as[mt][v], ab[mt][v]) : ab[mt][v];
  }
}

// The end of a workgroup item: K parts 1.. hand their sums to part 0 through
// LDS (added in part order), then y (one K split) or the split's f32 partial
// tile.
// The residual values this lane adds in tile_finish<RES> (rows past M read
// row M - 1, columns past N column N - 1: no branch around the loads),
// loaded when the workgroup starts so that their latency hides under the
// math instead of following it.
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
__device__ __forceinline__ void tile_load_res(const TileParams& p, int tile, float (&rv)[MT][4]) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave % Tg::RG;
  const int nn = min(tile * 16 * Tg::RG + rg * 16 + (lane & 15), p.N - 1);
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int m = min(m_block0<MT>() + 16 * mt + 4 * (lane >> 4) + v, p.M - 1);
      rv[mt][v] = bf16_bits_to_f32((p.res ? p.res : p.y)[static_cast<int64_t>(m) * p.N + nn]);
    }
}

template <int BITS, int GS, int MT, int WV, int NCH, int KH, bool RES = false>
__device__ __forceinline__ void tile_finish(const TileParams& p, int tile, int split, f32x4 (&acc)[MT], f32x4* red,
                                            const float (*rv)[4] = nullptr) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  const int M = p.M, N = p.N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave % Tg::RG, kh = wave / Tg::RG;
  const int r16 = lane & 15, gq = lane >> 4;
  const int n0 = tile * 16 * Tg::RG + rg * 16;  // this wave's 16 weight rows
  const int mb = m_block0<MT>();

  // K parts 1.. hand their sums to part 0 through LDS (added in part order)
  if constexpr (KH > 1) {
    if (kh > 0)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) red[(((kh - 1) * Tg::RG + rg) * MT + mt) * 64 + lane] = acc[mt];
    __syncthreads();
    if (kh > 0) return;
#pragma unroll
    for (int h = 1; h < KH; h++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const f32x4 o = red[(((h - 1) * Tg::RG + rg) * MT + mt) * 64 + lane];
#pragma unroll
        for (int v = 0; v < 4; v++) acc[mt][v] += o[v];
      }
  }

  // C layout of a 16x16 MFMA tile: lane holds column (weight row) r16 and
  // activation rows 4 gq + v of the M-tile.
  const int nn = n0 + r16;
  if (nn >= N) return;
  if (p.splits == 1) {
    const float bb = p.bias ? bf16_bits_to_f32(p.bias[nn]) : 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int m = mb + 16 * mt + 4 * gq + v;
        if (m >= M) continue;
        const int64_t o = static_cast<int64_t>(m) * N + nn;
        uint32_t r = f32_to_bf16_bits(acc[mt][v] + bb);
        if (RES && p.res)  // residual: bf16(r + bf16(v))
          r = f32_to_bf16_bits((rv ? rv[mt][v] : bf16_bits_to_f32(p.res[o])) + bf16_bits_to_f32(r));
        p.y[o] = static_cast<uint16_t>(r);
      }
    return;
  }
  // partial tile of this slice; split_reduce4_kernel adds the slices
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int m = mb + 16 * mt + 4 * gq + v;
      if (m < M) p.part[(static_cast<int64_t>(split) * M + m) * N + nn] = acc[mt][v];
    }
}

// SwiGLU end of a streaming item (one K split): K parts add up in LDS as in
// tile_finish, then each up row group hands its sums to the gate row group
// of the same outputs, which stores y = bf16(bf16(g * bf16(sigmoid(g))) * u)
// with g, u the bf16 projection outputs (llama.rs:1040-1045 at MLX's
// rounding points).  Every wave reaches both barriers.
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
__device__ __forceinline__ void tile_finish_swiglu(const TileParams& p, int tile, f32x4 (&acc)[MT], f32x4* red,
                                                   f32x4* hand) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  static_assert(Tg::RG % 2 == 0, "SwiGLU: gate and up row groups in pairs");
  const int M = p.M, N = p.N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave % Tg::RG, kh = wave / Tg::RG;
  const int r16 = lane & 15, gq = lane >> 4;
  if constexpr (KH > 1) {
    if (kh > 0)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) red[(((kh - 1) * Tg::RG + rg) * MT + mt) * 64 + lane] = acc[mt];
    __syncthreads();
    if (kh == 0)
#pragma unroll
      for (int h = 1; h < KH; h++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          const f32x4 o = red[(((h - 1) * Tg::RG + rg) * MT + mt) * 64 + lane];
#pragma unroll
          for (int v = 0; v < 4; v++) acc[mt][v] += o[v];
        }
  }
  if (kh == 0 && (rg & 1))
#pragma unroll
    for (int mt = 0; mt < MT; mt++) hand[((rg >> 1) * MT + mt) * 64 + lane] = acc[mt];
  __syncthreads();
  if (kh != 0 || (rg & 1)) return;
  const int nn = tile * 8 * Tg::RG + (rg >> 1) * 16 + r16;
  if (nn >= N) return;
  const float bg = p.bias ? bf16_bits_to_f32(p.bias[nn]) : 0.f, bu = p.bias2 ? bf16_bits_to_f32(p.bias2[nn]) : 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const f32x4 u4 = hand[((rg >> 1) * MT + mt) * 64 + lane];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int m = m_block0<MT>() + 16 * mt + 4 * gq + v;
      if (m >= M) continue;
      const float g = bf16_bits_to_f32(f32_to_bf16_bits(acc[mt][v] + bg));
      const float u = bf16_bits_to_f32(f32_to_bf16_bits(u4[v] + bu));
      const float sig = bf16_bits_to_f32(f32_to_bf16_bits(1.0f / (1.0f + expf(-g))));
      const float a = bf16_bits_to_f32(f32_to_bf16_bits(g * sig));
      p.y[static_cast<int64_t>(m) * N + nn] = static_cast<uint16_t>(f32_to_bf16_bits(a * u));
    }
  }
}

// One item per workgroup: blockIdx.x = tile of 16 RG rows, blockIdx.y = K
// slice, blockIdx.z = M block.
template <int BITS, int GS, int MT, int WV, int NCH, int KH>
__global__ __launch_bounds__(64 * WV) void qmv_tile_kernel(const TileParams p) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  __shared__ u32x4 xs[Tg::MR * Tg::ROW16];
  __shared__ __align__(16) uint16_t sx[Tg::MR * Tg::SXS];
  __shared__ f32x4 red[KH > 1 ? (KH - 1) * Tg::RG * MT * 64 : 1];
  TileX<BITS, GS, MT, WV, NCH, KH> X;
  TileW<BITS, GS, MT, WV, NCH, KH> W;
  tile_load_x(p, blockIdx.y, X);
  tile_load_w(p, blockIdx.x, blockIdx.y, W);
  __builtin_amdgcn_sched_barrier(0);  // every load is issued before the first wait
  tile_stage(X, xs, sx);
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  tile_accum(acc, W, xs, sx);
  tile_finish<BITS, GS, MT, WV, NCH, KH>(p, blockIdx.x, blockIdx.y, acc, red);
}

// Fused forms on the whole-K single-slice kernel: blockIdx.x picks the
// segment (weight matrix) and its tile, blockIdx.z the M block; no K split.
template <int BITS, int GS, int MT, int WV, int NCH, int KH, bool RES>
__global__ __launch_bounds__(64 * WV) void qmv_tile_fused_kernel(const TileFused f) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  __shared__ u32x4 xs[Tg::MR * Tg::ROW16];
  __shared__ __align__(16) uint16_t sx[Tg::MR * Tg::SXS];
  __shared__ f32x4 red[KH > 1 ? (KH - 1) * Tg::RG * MT * 64 : 1];
  int sg = 0;
  const int t = blockIdx.x;
  while (sg + 1 < f.nseg && t >= f.seg[sg].tile_end) sg++;
  const TileSeg& S = f.seg[sg];
  TileParams p = f.p;
  p.wq = S.wq;
  p.s = S.s;
  p.b = S.b;
  p.bias = S.bias;
  p.res = S.res;
  p.y = S.y;
  p.N = S.N;
  const int tile = t - (sg ? f.seg[sg - 1].tile_end : 0);
  TileX<BITS, GS, MT, WV, NCH, KH> X;
  TileW<BITS, GS, MT, WV, NCH, KH> W;
  tile_load_x<BITS, GS, MT, WV, NCH, KH, true>(p, 0, X);
  tile_load_w(p, tile, 0, W);
  // RES (some segment has a residual): loaded on every path (from y in a
  // segment without one, values unused) -- a load issued on one side of a
  // branch would make the compiler wait for every earlier load where the
  // paths join
  float rv[MT][4] = {};
  if constexpr (RES) tile_load_res<BITS, GS, MT, WV, NCH, KH>(p, tile, rv);
  __builtin_amdgcn_sched_barrier(0);  // every load is issued before the first wait
  tile_stage(X, xs, sx);
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  tile_accum(acc, W, xs, sx);
  tile_finish<BITS, GS, MT, WV, NCH, KH, RES>(p, tile, 0, acc, red, rv);
}

// Streaming form: a workgroup owns its 16 RG weight rows over `steps`
// consecutive K slices (blockIdx.y picks the run of slices when K is split).
// While the waves work on slice s from one LDS buffer, the codes of slices
// s + 1 and s + 2 and the activations of s + 1 are already in flight, and s + 1
// is staged into the other buffer: the memory stream of the workgroup keeps
// going under its arithmetic instead of alternating with it, and a whole
// projection needs no second pass over partial sums.
// SW: the SwiGLU form (gate / up row groups in pairs, tile_finish_swiglu).
template <int BITS, int GS, int MT, int WV, int NCH, int KH, bool SW = false>
__global__ __launch_bounds__(64 * WV) void qmv_stream_kernel(const TileParams p) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH, KH>;
  __shared__ u32x4 xs[2][Tg::MR * Tg::ROW16];
  __shared__ __align__(16) uint16_t sx[2][Tg::MR * Tg::SXS];
  __shared__ f32x4 red[KH > 1 ? (KH - 1) * Tg::RG * MT * 64 : 1];
  __shared__ f32x4 hand[SW ? Tg::RG / 2 * MT * 64 : 1];
  const int steps = p.steps, s0 = blockIdx.y * steps, tile = blockIdx.x;
  // Every load below is issued on every path (a slice past the run re-reads
  // the last one): the memory counter then holds the same loads wherever
  // control flow joins, so each wait names exactly the loads it needs.  A
  // load issued only on some paths made the compiler wait at the join as
  // if it were absent, i.e. for the just-issued prefetch of slice s + 2 too.
  const int last = s0 + steps - 1;
  TileX<BITS, GS, MT, WV, NCH, KH> X0, X1;
  TileW<BITS, GS, MT, WV, NCH, KH> W0, W1;
  tile_load_x(p, s0, X0);
  tile_load_w<BITS, GS, MT, WV, NCH, KH, SW>(p, tile, s0, W0);
  tile_load_x(p, min(s0 + 1, last), X1);
  tile_load_w<BITS, GS, MT, WV, NCH, KH, SW>(p, tile, min(s0 + 1, last), W1);
  __builtin_amdgcn_sched_barrier(0);
  tile_stage(X0, xs[0], sx[0]);
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // slice s: codes W0 / buffer 0 (s even), W1 / buffer 1 (s odd); each
  // register set and buffer is refilled as soon as its slice is used.
  // Steady state while slices s + 2 and s + 3 exist; then a tail of 1..3.
  int s = 0;
  for (; s + 3 < steps; s += 2) {
    tile_load_x(p, s0 + s + 2, X0);
    tile_accum(acc, W0, xs[0], sx[0]);
    tile_load_w<BITS, GS, MT, WV, NCH, KH, SW>(p, tile, s0 + s + 2, W0);
    tile_stage(X1, xs[1], sx[1], s == 0);
    tile_load_x(p, s0 + s + 3, X1);
    tile_accum(acc, W1, xs[1], sx[1]);
    tile_load_w<BITS, GS, MT, WV, NCH, KH, SW>(p, tile, s0 + s + 3, W1);
    tile_stage(X0, xs[0], sx[0], false);
  }
  const int rest = steps - s;  // 1 only when steps == 1
  if (rest == 3) {
    tile_load_x(p, s0 + s + 2, X0);
    tile_accum(acc, W0, xs[0], sx[0]);
    tile_load_w<BITS, GS, MT, WV, NCH, KH, SW>(p, tile, s0 + s + 2, W0);
    tile_stage(X1, xs[1], sx[1], s == 0);
    tile_accum(acc, W1, xs[1], sx[1]);
    tile_stage(X0, xs[0], sx[0], false);
    tile_accum(acc, W0, xs[0], sx[0]);
  } else if (rest == 2) {
    tile_accum(acc, W0, xs[0], sx[0]);
    tile_stage(X1, xs[1], sx[1], s == 0);
    tile_accum(acc, W1, xs[1], sx[1]);
  } else {
    tile_accum(acc, W0, xs[0], sx[0]);
  }
  if constexpr (SW)
    tile_finish_swiglu<BITS, GS, MT, WV, NCH, KH>(p, tile, acc, red, hand);
  else
    tile_finish<BITS, GS, MT, WV, NCH, KH>(p, tile, blockIdx.y, acc, red);
}

// y[m, n] = bf16(sum over splits of part[s, m, n] (in split order) + bias[n])
__global__ __launch_bounds__(256) void qmv_tile_reduce_kernel(const float* __restrict__ part,
                                                              const uint16_t* __restrict__ bias,
                                                              uint16_t* __restrict__ y, int64_t MN, int N,
                                                              int splits) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MN) return;
  float sum = 0.f;
  for (int sp = 0; sp < splits; sp++) sum += part[sp * MN + i];
  if (bias) sum += bf16_bits_to_f32(bias[i % N]);
  y[i] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
}

// The same sum, four consecutive outputs per thread (N % 4 == 0, y 8-byte
// aligned): 16-byte partial loads, one 8-byte store.  S > 0: the split count
// at compile time, every partial load issued before the first add (one
// memory round trip instead of one per split); S = 0: any count.
template <int S>
__global__ __launch_bounds__(256) void split_reduce4_kernel(const float4* __restrict__ part,
                                                            const uint16_t* __restrict__ bias,
                                                            uint2* __restrict__ y, int64_t MN4, int N,
                                                            int splits) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MN4) return;
  float4 sum;
  if constexpr (S > 0) {
    float4 v[S];
#pragma unroll
    for (int sp = 0; sp < S; sp++) v[sp] = part[sp * MN4 + i];
    sum = v[0];
#pragma unroll
    for (int sp = 1; sp < S; sp++) {
      sum.x += v[sp].x; sum.y += v[sp].y; sum.z += v[sp].z; sum.w += v[sp].w;
    }
  } else {
    sum = part[i];
    for (int sp = 1; sp < splits; sp++) {
      const float4 v = part[sp * MN4 + i];
      sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
    }
  }
  if (bias) {
    const int n = static_cast<int>((4 * i) % N);
    sum.x += bf16_bits_to_f32(bias[n]);
    sum.y += bf16_bits_to_f32(bias[n + 1]);
    sum.z += bf16_bits_to_f32(bias[n + 2]);
    sum.w += bf16_bits_to_f32(bias[n + 3]);
  }
  y[i] = make_uint2(f32_to_bf16_bits(sum.x) | (f32_to_bf16_bits(sum.y) << 16),
                    f32_to_bf16_bits(sum.z) | (f32_to_bf16_bits(sum.w) << 16));
}

// The split sum as split_reduce4_kernel (split order, then the bias, then
// bf16), then the residual add and RMSNorm of mlxq_add_rms_norm on the row
// (same per-thread pieces and reduction order): one workgroup per row.
template <int PT>
__global__ __launch_bounds__(256) void split_add_norm_kernel(const float* __restrict__ part,
                                                             const uint16_t* __restrict__ bias,
                                                             const uint16_t* __restrict__ res,
                                                             const uint16_t* __restrict__ w, int64_t MN, int N,
                                                             int splits, float eps, uint16_t* __restrict__ s,
                                                             uint16_t* __restrict__ y) {
  // PT pieces of 8 per thread at most (pieces i = t, t + 256, ...), all
  // loaded before any arithmetic and kept in registers between the passes
  __shared__ float wpart[4];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * N;
  const uint4* rr = reinterpret_cast<const uint4*>(res + off);
  uint4* sr = reinterpret_cast<uint4*>(s + off);
  uint4* yr = reinterpret_cast<uint4*>(y + off);
  const uint4* wv = reinterpret_cast<const uint4*>(w);
  const int pieces = N / 8;
  float4 lo[PT], hi[PT];
  uint4 r[PT], g[PT];
#pragma unroll
  for (int k = 0; k < PT; k++) {
    const int i = min(static_cast<int>(threadIdx.x) + 256 * k, pieces - 1);  // clamped: no branch around the loads
    const float4* p0 = reinterpret_cast<const float4*>(part + off) + 2 * i;
    lo[k] = p0[0];
    hi[k] = p0[1];
    r[k] = rr[i];
    g[k] = wv[i];
  }
  for (int sp = 1; sp < splits; sp++)
#pragma unroll
    for (int k = 0; k < PT; k++) {
      const int i = min(static_cast<int>(threadIdx.x) + 256 * k, pieces - 1);
      const float4* pp = reinterpret_cast<const float4*>(part + sp * MN + off) + 2 * i;
      const float4 u = pp[0], v = pp[1];
      lo[k].x += u.x; lo[k].y += u.y; lo[k].z += u.z; lo[k].w += u.w;
      hi[k].x += v.x; hi[k].y += v.y; hi[k].z += v.z; hi[k].w += v.w;
    }
  float ss = 0.f;
  uint32_t o[PT][4];
#pragma unroll
  for (int k = 0; k < PT; k++) {
    const int i = static_cast<int>(threadIdx.x) + 256 * k;
    if (i >= pieces) break;
    float d[8] = {lo[k].x, lo[k].y, lo[k].z, lo[k].w, hi[k].x, hi[k].y, hi[k].z, hi[k].w};
    if (bias)
#pragma unroll
      for (int e = 0; e < 8; e++) d[e] += bf16_bits_to_f32(bias[8 * i + e]);
    const uint32_t ra[4] = {r[k].x, r[k].y, r[k].z, r[k].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float d0 = bf16_bits_to_f32(f32_to_bf16_bits(d[2 * j]));
      const float d1 = bf16_bits_to_f32(f32_to_bf16_bits(d[2 * j + 1]));
      o[k][j] = f32_to_bf16_bits(bf16_bits_to_f32(ra[j] & 0xFFFFu) + d0) |
                (f32_to_bf16_bits(bf16_bits_to_f32(ra[j] >> 16) + d1) << 16);
      const float u = bf16_bits_to_f32(o[k][j] & 0xFFFFu), v = bf16_bits_to_f32(o[k][j] >> 16);
      ss = fmaf(u, u, ss);
      ss = fmaf(v, v, ss);
    }
    sr[i] = make_uint4(o[k][0], o[k][1], o[k][2], o[k][3]);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) wpart[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) tot += wpart[i];
  const float inv = 1.0f / sqrtf(tot / static_cast<float>(N) + eps);
#pragma unroll
  for (int k = 0; k < PT; k++) {
    const int i = static_cast<int>(threadIdx.x) + 256 * k;
    if (i >= pieces) break;
    const uint32_t gw[4] = {g[k].x, g[k].y, g[k].z, g[k].w};
    uint32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float n0 = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(o[k][j] & 0xFFFFu) * inv));
      const float n1 = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(o[k][j] >> 16) * inv));
      q[j] = f32_to_bf16_bits(bf16_bits_to_f32(gw[j] & 0xFFFFu) * n0) |
             (f32_to_bf16_bits(bf16_bits_to_f32(gw[j] >> 16) * n1) << 16);
    }
    yr[i] = make_uint4(q[0], q[1], q[2], q[3]);
  }
}

}  // namespace tile

int launch_split_add_norm(const float* part, const uint16_t* bias, int64_t M, int64_t N, int splits,
                          const AddNormEpilogue& ep, hipStream_t st) {
  // pieces of 8 per thread (the same assignment as mlxq_add_rms_norm)
  const int64_t pt = ceil_div(N / 8, int64_t(256));
  auto kern = pt <= 1 ? tile::split_add_norm_kernel<1>
              : pt <= 2 ? tile::split_add_norm_kernel<2>
              : pt <= 4 ? tile::split_add_norm_kernel<4>
                        : tile::split_add_norm_kernel<8>;
  if (pt > 8) return fail(MLXQ_ERR_UNSUPPORTED, "split_add_norm: rows longer than 16384");
  MLXQ_LAUNCH(kern, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, part, bias, ep.res, ep.norm_w, M * N,
                     static_cast<int>(N), splits, ep.eps, ep.sum_out, ep.y_norm);
  return check_launch("split_add_norm");
}

int launch_split_reduce(const float* part, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int splits,
                        hipStream_t st) {
  const int64_t mn = M * N;
  if (N % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
    const int64_t mn4 = mn / 4;
    auto kern = splits == 2 ? tile::split_reduce4_kernel<2>
                : splits == 4 ? tile::split_reduce4_kernel<4>
                : splits == 8 ? tile::split_reduce4_kernel<8>
                              : tile::split_reduce4_kernel<0>;
    MLXQ_LAUNCH(kern, dim3(static_cast<unsigned>(ceil_div(mn4, 256))), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(part), bias, reinterpret_cast<uint2*>(y), mn4,
                       static_cast<int>(N), splits);
  } else {
    MLXQ_LAUNCH(tile::qmv_tile_reduce_kernel, dim3(static_cast<unsigned>(ceil_div(mn, 256))), dim3(256), 0,
                       st, part, bias, y, mn, static_cast<int>(N), splits);
  }
  return check_launch("split_reduce");
}

namespace tile {

// ---------------------------------------------------------------- launch

constexpr int kMaxSplits = kMaxSplitsK;

struct Cfg {
  int mt = 1, wv = 4, nch = 8, kh = 1;
};

template <int BITS, int MT, int WV, int NCH, int KH>
int run(const TileParams& a, int tiles, int mblocks, hipStream_t st, int* query) {
  auto kern = qmv_tile_kernel<BITS, 64, MT, WV, NCH, KH>;
  if (query) {
    static int cached = -1;
    if (cached < 0) {
      int nb = 0;
      hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), 64 * WV, 0);
      if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmv_tile: occupancy: ") + hipGetErrorString(e));
      cached = nb;
    }
    *query = cached;
    return MLXQ_OK;
  }
  MLXQ_LAUNCH(kern, dim3(tiles, a.splits, mblocks), dim3(64 * WV), 0, st, a);
  return check_launch("qmv_tile");
}

template <int BITS, int MT, int WV, int NCH, int KH, bool SW = false>
int run_stream(const TileParams& a, int tiles, int mblocks, hipStream_t st) {
  MLXQ_LAUNCH((qmv_stream_kernel<BITS, 64, MT, WV, NCH, KH, SW>), dim3(tiles, a.splits, mblocks),
                     dim3(64 * WV), 0, st, a);
  return check_launch("qmv_stream");
}

// The streaming forms: (waves, Q4 chunks per wave and slice, K parts); Q8
// takes twice the chunks, so a slice covers the same K either way.  Eight K
// parts (one row group of 16 rows per workgroup, for short matrices) only
// with 16 activation rows per workgroup: two such LDS buffers of 2048 k are
// the most that fit.
struct SCfg {
  int wv = 8, nch = 2, kh = 2;
};
bool scfg_known(const SCfg& c, int mt) {
  if (c.wv == 8 && (c.kh == 1 || c.kh == 2)) return c.nch == 2 || c.nch == 4;
  if (c.wv == 8 && c.kh == 4) return c.nch == 2;
  if (c.wv == 8 && c.kh == 8) return c.nch == 2 && mt == 1;
  if (c.wv == 4 && c.kh == 1) return c.nch == 2 || c.nch == 4;
  return false;
}
template <int BITS, int MT>
int dispatch_stream_mt(const SCfg& c, const TileParams& a, int tiles, int mb, hipStream_t st) {
  constexpr int F = BITS == 4 ? 1 : 2;
  if (c.wv == 8 && c.kh == 2)
    return c.nch == 2 ? run_stream<BITS, MT, 8, 2 * F, 2>(a, tiles, mb, st)
                      : run_stream<BITS, MT, 8, 4 * F, 2>(a, tiles, mb, st);
  if (c.wv == 8 && c.kh == 4) return run_stream<BITS, MT, 8, 2 * F, 4>(a, tiles, mb, st);
  if constexpr (MT == 1)
    if (c.wv == 8 && c.kh == 8) return run_stream<BITS, MT, 8, 2 * F, 8>(a, tiles, mb, st);
  if (c.wv == 4)
    return c.nch == 2 ? run_stream<BITS, MT, 4, 2 * F, 1>(a, tiles, mb, st)
                      : run_stream<BITS, MT, 4, 4 * F, 1>(a, tiles, mb, st);
  return c.nch == 2 ? run_stream<BITS, MT, 8, 2 * F, 1>(a, tiles, mb, st)
                    : run_stream<BITS, MT, 8, 4 * F, 1>(a, tiles, mb, st);
}
// Where the streaming form is the default, from interleaved A/B timings
// against the single-slice form at the Llama-3-8B shapes (weights streamed
// from HBM, clocks warmed): large gate/up-like matrices (K < N) from M = 8:
// Q4 M = 32 19.9 -> 17.4 us, Q8 24.3 -> 23.1, Q4 M = 16 14.5 -> 13.8, Q8 21.2
// -> 19.5; down-like (K > N) with 4 K splits: M = 32 Q4 21.2 -> 19.6, Q8 25.8
// -> 24.1, Q8 M = 16 23.1 -> 21.1 (Q4 M = 16 at parity).  The shorter
// matrices (q/o, k/v) stay on the single-slice form (parity or slower).
bool stream_preferred(int64_t M, int64_t N, int64_t K, int bits, SCfg& c, int& splits) {
  const bool large = N * K >= (int64_t(1) << 25);
  // gate/up-like from M = 3 (M = 4: Q4 13.20 -> 12.40 us, Q8 19.10 -> 18.47)
  if (!large || M < (K < N ? 3 : 8)) return false;
  // (re-measured with every load issued on every path: Q4 M = 32 gate 17.33
  // -> 16.58 on {8, 2, 2}, Q8 M = 16 19.34 -> 18.41 on {4, 4, 1}, Q4 M = 16
  // down 15.94 -> 15.56 on {4, 4, 1} with 4 splits)
  if (K < N && N >= 65536) {
    // very tall (an lm_head: 128256 rows, thousands of 64-row tiles): 4-wave
    // workgroups, several per CU (Q4 M = 4 / 8 / 16 / 32: 85.6 / 91.5 /
    // 95.6 / 119.8 -> 74.1 / 77.0 / 81.1 / 102.4 us; Q8 M = 4 132.0 -> 115.7,
    // M = 32 161.3 -> 146.0 on {4, 2, 1})
    c = bits == 8 && M > 16 ? SCfg{4, 2, 1} : SCfg{4, 4, 1};
    splits = 1;
    return true;
  }
  if (K < N) {
    if (bits == 4) c = M > 16 || M <= 4 ? SCfg{8, 2, 2} : SCfg{8, 4, 2};
    else c = M > 16 ? SCfg{8, 2, 2} : SCfg{4, 4, 1};  // Q8 M = 4 too: 18.44 -> 17.64 us against {8, 4, 2}
    splits = 1;
    return true;
  }
  if (M > 16) {
    c = SCfg{8, 2, 2};
    splits = 4;
    return true;
  }
  if (M == 16 || (bits == 8 && M > 8)) {  // Q8 M = 9 / 12 / 15: 20.59 / 23.51 / 24.71 -> 19.56 / 19.79 / 19.76 us
    c = SCfg{4, 4, 1};
    splits = 4;
    return true;
  }
  return false;
}

int dispatch_stream(int bits, int mt, const SCfg& c, const TileParams& a, int tiles, int mb, hipStream_t st) {
  if (bits == 4) return mt == 1 ? dispatch_stream_mt<4, 1>(c, a, tiles, mb, st) : dispatch_stream_mt<4, 2>(c, a, tiles, mb, st);
  return mt == 1 ? dispatch_stream_mt<8, 1>(c, a, tiles, mb, st) : dispatch_stream_mt<8, 2>(c, a, tiles, mb, st);
}

// The instantiated (waves, chunks per wave, K parts) forms: slices of 16
// chunks only with 8 waves and one K part (<= 16 activation pieces per
// thread); K parts of 2 (4 or 8 chunks) and 4 (4 chunks) with 8 waves, so a
// workgroup slice stays within 16 chunks.  Eight K parts (one row group of 16
// rows) of 4 chunks, or 8 for Q8, with 16 activation rows per workgroup: a
// slice of 4096 k, the whole K of a Llama-3-8B q/k/v/o row, in 128 KB of LDS.
bool cfg_known(const Cfg& c, int bits) {
  if (c.kh == 1) return (c.wv == 4 && (c.nch == 4 || c.nch == 8)) || (c.wv == 8 && (c.nch == 4 || c.nch == 8 || c.nch == 16));
  if (c.kh == 8) return c.wv == 8 && c.mt == 1 && (c.nch == 4 || (c.nch == 8 && bits == 8));
  if (c.kh == 4 && c.mt == 1 && c.wv == 8 && c.nch == (bits == 4 ? 8 : 16)) return true;  // whole-K, 32 rows
  return c.wv == 8 && ((c.kh == 2 && (c.nch == 4 || c.nch == 8)) || (c.kh == 4 && c.nch == 4));
}

template <int BITS, int MT>
int run_wn(const Cfg& c, const TileParams& a, int tiles, int mb, hipStream_t st, int* q) {
  if (c.kh == 2) return c.nch == 4 ? run<BITS, MT, 8, 4, 2>(a, tiles, mb, st, q) : run<BITS, MT, 8, 8, 2>(a, tiles, mb, st, q);
  if (c.kh == 4) {
    if constexpr (MT == 1)
      if (c.nch == (BITS == 4 ? 8 : 16)) return run<BITS, MT, 8, BITS == 4 ? 8 : 16, 4>(a, tiles, mb, st, q);
    return run<BITS, MT, 8, 4, 4>(a, tiles, mb, st, q);
  }
  if constexpr (MT == 1) {
    if (c.kh == 8) {
      if constexpr (BITS == 8)
        if (c.nch == 8) return run<BITS, MT, 8, 8, 8>(a, tiles, mb, st, q);
      return run<BITS, MT, 8, 4, 8>(a, tiles, mb, st, q);
    }
  }
  if (c.wv == 4) return c.nch == 4 ? run<BITS, MT, 4, 4, 1>(a, tiles, mb, st, q) : run<BITS, MT, 4, 8, 1>(a, tiles, mb, st, q);
  if (c.nch == 4) return run<BITS, MT, 8, 4, 1>(a, tiles, mb, st, q);
  return c.nch == 8 ? run<BITS, MT, 8, 8, 1>(a, tiles, mb, st, q) : run<BITS, MT, 8, 16, 1>(a, tiles, mb, st, q);
}

int dispatch(int bits, const Cfg& c, const TileParams& a, int tiles, int mb, hipStream_t st, int* q) {
  if (bits == 4) return c.mt == 1 ? run_wn<4, 1>(c, a, tiles, mb, st, q) : run_wn<4, 2>(c, a, tiles, mb, st, q);
  return c.mt == 1 ? run_wn<8, 1>(c, a, tiles, mb, st, q) : run_wn<8, 2>(c, a, tiles, mb, st, q);
}

int cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

int64_t chunks_of(int64_t K, int bits) { return K * bits / 8 / 64; }

}  // namespace tile

using namespace tile;

namespace {
// Short matrices whose whole K one workgroup stages (8 waves as 8 K parts of
// one 16-row group, 16 activation rows per M block): one workgroup per CU
// (the LDS holds 16 x K activations), taken while tiles x M blocks fill at
// most one round of CUs, so no K split and no second launch.  Measured at
// the Llama-3-8B shapes (interleaved A/B, weights streamed from HBM): k/v
// Q4 M = 6..32 6.6-8.2 -> 6.4-6.5 us, Q8 7.6-8.2 -> 7.1-7.2; q/o Q4 from M
// = 8 (6.93 -> 6.69, M = 16 8.51 -> 6.84), Q8 from M = 12 (8.53 -> 8.25, M
// = 16 9.54 -> 8.31); two M blocks of q/o take two rounds of CUs and are
// slower than the 32-row forms.
bool short_fullk(int64_t M, int64_t N, int64_t K, int bits, Cfg* c) {
  if (N * K >= (int64_t(1) << 25) || M < (N <= 2048 ? 6 : bits == 4 ? 8 : 12)) return false;
  const int64_t ch = chunks_of(K, bits);
  const Cfg f{1, 8, static_cast<int>(ch / 8), 8};
  if (ch % 8 || !cfg_known(f, bits)) return false;
  if (ceil_div(N, 16) * ceil_div(M, 16) > cu_count()) {
    // past one round: 32 rows per workgroup (two row groups x four K parts)
    // in one round, Q4 (q/o at M = 17 / 24 / 32: 9.02 / 9.29 / 9.39 -> 7.98 /
    // 8.01 / 8.05 us; Q8 10.16 -> 10.41 at M = 17, 10.76 -> 10.49 at 32)
    const Cfg f2{1, 8, static_cast<int>(ch / 4), 4};
    if (bits != 4 || overrides().tile_fused_rg == 1 || !cfg_known(f2, bits) ||
        ceil_div(N, 32) * ceil_div(M, 16) > cu_count())
      return false;
    if (c) *c = f2;
    return true;
  }
  if (c) *c = f;
  return true;
}
}  // namespace

bool qmv_tile_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M < 1 || M > kQmvMaxM || N < 1 || group_size != 64) return false;
  if ((K * bits / 8) % 64) return false;
  const int64_t ch = chunks_of(K, bits);
  if (ch % 4 || ch > 16 * kMaxSplits) return false;  // whole slices of 4, 8 or 16 chunks, <= 16 slices
  return static_cast<int64_t>(kMaxSplits) * M * N < (int64_t(1) << 31);
}

size_t qmv_tile_workspace_bytes(int64_t M, int64_t N) { return static_cast<size_t>(kMaxSplits) * M * N * 4; }

// Short prefills of gate/up-like matrices (33..256 rows): the streaming form
// with 64 activation rows per workgroup (4 MFMA row tiles x 8 row groups of
// one K part, slices of 256 k), grid z = blocks of 64 rows; one launch, no
// K split.
// Down-like matrices (K > N) split K in four (f32 partial sums in the
// workspace, added by the second launch) so that their fewer row tiles fill
// the CUs.
int qmv_stream64_splits(int64_t N, int64_t K) { return K > N ? 4 : 1; }

bool qmv_stream64_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M <= kQmvMaxM || M > 256 || group_size != 64 || (bits != 4 && bits != 8)) return false;
  const int splits = qmv_stream64_splits(N, K);
  if (N * K < (int64_t(1) << 25) || K % (256 * splits) || N > (int64_t(1) << 24) || M * K >= (int64_t(1) << 31) ||
      (splits > 1 && N % 4))
    return false;
  return true;
}

size_t qmv_stream64_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int splits = qmv_stream64_splits(N, K);
  return splits > 1 ? static_cast<size_t>(splits) * M * N * 4 : 0;
}

int launch_qmv_stream64(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                        const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                        void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (!qmv_stream64_eligible(M, N, K, group_size, bits))
    return fail(MLXQ_ERR_UNSUPPORTED, "qmv_stream64: shape not supported");
  const int splits = qmv_stream64_splits(N, K);
  const size_t need = qmv_stream64_workspace_bytes(M, N, K);
  if (need && (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255u)))
    return fail(MLXQ_ERR_UNSUPPORTED, "qmv_stream64: workspace too small for the K split");
  TileParams a{};
  a.x = x;
  a.wq = wq;
  a.s = s;
  a.b = b;
  a.bias = bias;
  a.y = y;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.splits = splits;
  a.steps = static_cast<int>(K / 256 / splits);
  a.part = splits > 1 ? static_cast<float*>(workspace) : nullptr;
  const int tiles = static_cast<int>(ceil_div(N, 16 * 8));
  const int mb = static_cast<int>(ceil_div(M, 64));
  const int rc = bits == 4 ? run_stream<4, 4, 8, 2, 1>(a, tiles, mb, st) : run_stream<8, 4, 8, 4, 1>(a, tiles, mb, st);
  if (rc || splits == 1) return rc;
  return launch_split_reduce(a.part, bias, y, M, N, splits, st);
}

bool qmv_tile_preferred(int64_t M, int64_t N, int64_t K, int bits) {
  // Measured against the block kernel (qmv.hip) and the vector-ALU kernel
  // (qmv_dot) at the Llama-3-8B projection shapes: the tile kernel wins on
  // the large projections from M = 8 (Q4) / 16 (Q8),
  // on gate/up already from M = 3 (Q4) / 4 (Q8), on short matrices (N <= 2048) from
  // M = 16, and on the other small projections above 16 rows.
  const bool large = N * K >= (int64_t(1) << 25);
  if (M <= 4) return large && K < N && M >= (bits == 4 ? 3 : 4);
  if (short_fullk(M, N, K, bits, nullptr)) return true;
  if (large) return K < N || M >= (bits == 4 ? 8 : 9);  // gate/up-like: the streaming form (Q8 M = 8 20.4 -> 19.0)
  if (N <= 2048) return M >= 16;  // k/v: M = 16 Q4 8.28 -> 7.93 us, Q8 9.27 -> 8.06; Q8 M = 24 11.07 -> 8.93
  return M > 16;  // q/o-like: Q4 M = 20 10.16 -> 9.21 us, Q8 M = 24 11.36 -> 10.42 against the block kernel
}

bool qmv_dot_preferred(int64_t M, int64_t N, int64_t K, int bits) {
  // M = 1 always; M = 2 on gate/up-like shapes (large N*K, K < N); the block
  // kernel is faster for the other shapes at M = 2..4.
  (void)bits;
  return M == 1 || (M == 2 && N * K >= (int64_t(1) << 25) && K < N);
}

int launch_qmv_tile(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                    const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                    void* workspace, size_t workspace_bytes, hipStream_t st, AddNormEpilogue* ep) {
  if (!qmv_tile_eligible(M, N, K, group_size, bits))
    return fail(MLXQ_ERR_UNSUPPORTED, "qmv_tile: shape not supported");
  TileParams a{};
  a.x = x;
  a.wq = wq;
  a.s = s;
  a.b = b;
  a.bias = bias;
  a.y = y;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  const int64_t ch = chunks_of(K, bits);
  const bool ws_ok = workspace && !(reinterpret_cast<uintptr_t>(workspace) & 255u);
  const int64_t fit = ws_ok ? static_cast<int64_t>(workspace_bytes / (M * N * 4)) : 1;  // slices that fit

  // streaming form: where stream_preferred says (or MLXQ_QMV_TILE_STREAM=
  // waves,chunks,K parts,K splits; =0 keeps the single-slice form)
  {
    const Overrides& ov = overrides();
    SCfg c;
    int splits = 1;
    bool use = false;
    if (ov.stream_set) {
      use = ov.stream_wv > 0;
      c.wv = ov.stream_wv; c.nch = ov.stream_nch; c.kh = ov.stream_kh;
      splits = ov.stream_splits > 0 ? ov.stream_splits : 1;
    } else {
      use = stream_preferred(M, N, K, bits, c, splits);
    }
    const int64_t per = c.nch * (bits == 4 ? 1 : 2) * c.kh;  // chunks per K slice
    // one M block of up to 32 rows, or (eight K parts, or MLXQ_QMV_TILE_MB)
    // blocks of 16
    const int mt = M <= 16 || c.kh == 8 || ov.tile_mb ? 1 : 2;
    if (use && scfg_known(c, mt) && ch % per == 0 && (ch / per) % splits == 0 && splits <= kMaxSplits &&
        (splits == 1 || splits <= fit)) {
      a.splits = splits;
      a.steps = static_cast<int>(ch / per / splits);
      a.part = splits > 1 ? static_cast<float*>(workspace) : nullptr;
      const int64_t tiles = ceil_div(N, 16 * (c.wv / c.kh));
      const int mb = static_cast<int>(ceil_div(M, 16 * mt));
      if (int rc = dispatch_stream(bits, mt, c, a, static_cast<int>(tiles), mb, st)) return rc;
      if (splits == 1) return MLXQ_OK;
      if (ep && N % 8 == 0 && N <= 16384) {
        ep->applied = true;
        return launch_split_add_norm(a.part, bias, M, N, splits, *ep, st);
      }
      return launch_split_reduce(a.part, bias, y, M, N, splits, st);
    }
  }

  // (waves, chunks per wave, K parts).  Measured best at the Llama-3-8B
  // shapes (M = 16 / 32, weights streamed from HBM): large N*K (gate, up,
  // down): 8 waves as 4 row groups x 2 K parts of 8 chunks (Q8 M = 32 gate
  // 25.6 -> 24.0 us, down 28.4 -> 25.7; Q4 M = 32 down 22.1 -> 20.8 against
  // one K part); q/o: Q8 M = 32 the same (12.7 -> 10.7 us), else 2 row
  // groups x 4 K parts of 4 chunks; k/v: that too (Q8 M = 32 8.5 -> 8.1 us)
  // except Q4 M = 32, 4 waves, 4 chunks, one part.  Taken when it divides K
  // into at most 16 slices that fit the workspace, else the first such of
  // the others.
  const bool large = N * K >= (int64_t(1) << 25);
  Cfg pref;
  pref.mt = M <= 16 || overrides().tile_mb ? 1 : 2;
  if (short_fullk(M, N, K, bits, &pref)) {
  } else if (large || (bits == 8 && M > 16 && N > 2048)) {
    pref.wv = 8; pref.nch = 8; pref.kh = 2;
  } else if (N <= 2048 && bits == 4 && M > 16) {
    pref.wv = 4; pref.nch = 4; pref.kh = 1;
  } else {
    pref.wv = 8; pref.nch = 4; pref.kh = 4;
  }
  const int fwv = overrides().tile_wv, fnch = overrides().tile_nch, fkh = overrides().tile_kh;
  if (fwv) pref.wv = fwv;
  if (fnch) pref.nch = fnch;
  if (fkh) pref.kh = fkh;
  if (pref.kh == 8) pref.mt = 1;  // eight K parts: M blocks of 16 rows
  const Cfg order[] = {pref,           {pref.mt, 8, 16, 1}, {pref.mt, 8, 8, 1}, {pref.mt, 4, 8, 1},
                       {pref.mt, 4, 4, 1}, {pref.mt, 8, 4, 1}};
  const Cfg* pick = nullptr;
  for (const Cfg& c : order) {
    if (!cfg_known(c, bits)) continue;
    if (ch % (c.nch * c.kh)) continue;
    const int64_t splits = ch / (c.nch * c.kh);
    if (splits > kMaxSplits || (splits > 1 && splits > fit)) continue;
    pick = &c;
    break;
  }
  if (!pick) return MLXQ_ERR_UNSUPPORTED;  // no slicing fits the workspace: the caller picks another kernel
  a.splits = static_cast<int>(ch / (pick->nch * pick->kh));
  a.part = a.splits > 1 ? static_cast<float*>(workspace) : nullptr;
  const int64_t tiles = ceil_div(N, 16 * (pick->wv / pick->kh));
  // split K: the slices are added by a second launch (split_reduce4_kernel).
  // A hand-off inside this kernel (the last arriving slice of a tile adds the
  // slices) was measured slower at the Llama-3-8B shapes (Q8 M = 32 gate
  // 26.1 -> 26.9 us): its agent-coherent partial stores and serial tail cost
  // more than the launch it saves.
  const int mb = static_cast<int>(ceil_div(M, 16 * pick->mt));
  if (int rc = dispatch(bits, *pick, a, static_cast<int>(tiles), mb, st, nullptr)) return rc;
  if (a.splits == 1) return MLXQ_OK;
  if (ep && N % 8 == 0 && N <= 16384) {
    ep->applied = true;
    return launch_split_add_norm(a.part, bias, M, N, a.splits, *ep, st);
  }
  return launch_split_reduce(a.part, bias, y, M, N, a.splits, st);
}

namespace tile {

template <int BITS, bool RES>
int run_fused_r(const Cfg& c, const TileFused& f, int tiles, int mb, hipStream_t st) {
  if (c.kh == 4) {  // two row groups x four K parts (32 rows per workgroup)
    MLXQ_LAUNCH((qmv_tile_fused_kernel<BITS, 64, 1, 8, BITS == 4 ? 8 : 16, 4, RES>), dim3(tiles, 1, mb),
                       dim3(512), 0, st, f);
  } else if (c.nch == 4) {
    MLXQ_LAUNCH((qmv_tile_fused_kernel<BITS, 64, 1, 8, 4, 8, RES>), dim3(tiles, 1, mb), dim3(512), 0, st, f);
  } else {
    if constexpr (BITS == 8)
      MLXQ_LAUNCH((qmv_tile_fused_kernel<BITS, 64, 1, 8, 8, 8, RES>), dim3(tiles, 1, mb), dim3(512), 0, st, f);
  }
  return check_launch("qmv_tile_fused");
}
template <int BITS>
int run_fused(const Cfg& c, const TileFused& f, int tiles, int mb, hipStream_t st) {
  bool res = false;
  for (int i = 0; i < f.nseg; i++) res = res || f.seg[i].res;
  return res ? run_fused_r<BITS, true>(c, f, tiles, mb, st) : run_fused_r<BITS, false>(c, f, tiles, mb, st);
}

}  // namespace tile

namespace tile {

template <int BITS, int MT>
int run_swiglu(const SCfg& c, const TileParams& a, int tiles, int mb, hipStream_t st) {
  constexpr int F = BITS == 4 ? 1 : 2;
  if (c.wv == 8 && c.kh == 2)
    return c.nch == 2 ? run_stream<BITS, MT, 8, 2 * F, 2, true>(a, tiles, mb, st)
                      : run_stream<BITS, MT, 8, 4 * F, 2, true>(a, tiles, mb, st);
  return run_stream<BITS, MT, 4, 4 * F, 1, true>(a, tiles, mb, st);  // {4, 4, 1}
}

}  // namespace tile

// SwiGLU of two projections (gate, up) of the same activations in one
// streaming launch, for 5..32 rows: the configurations stream_preferred
// takes for gate/up-like shapes (one K split), gate and up row groups
// paired in each workgroup.
bool qmv_tile_swiglu_eligible(const QmvFused& f) {
  if (!f.swiglu || f.norm_w || f.rep > 1 || f.nproj != 2 || f.M < 5 || f.M > kQmvMaxM || f.group_size != 64)
    return false;
  if (f.proj[0].N != f.proj[1].N || f.proj[0].res || f.proj[1].res || f.x_stride != f.K) return false;
  const int64_t N = f.proj[0].N, K = f.K;
  if (!qmv_tile_eligible(f.M, N, K, 64, f.bits)) return false;
  SCfg c;
  int splits = 1;
  if (!stream_preferred(f.M, N, K, f.bits, c, splits) || splits != 1) return false;
  const bool known = (c.wv == 8 && c.kh == 2 && (c.nch == 2 || c.nch == 4)) || (c.wv == 4 && c.kh == 1 && c.nch == 4);
  const int64_t per = c.nch * (f.bits == 4 ? 1 : 2) * c.kh;
  return known && chunks_of(K, f.bits) % per == 0;
}

int launch_qmv_tile_swiglu(const QmvFused& f, hipStream_t st) {
  if (!qmv_tile_swiglu_eligible(f)) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_tile_swiglu: shape not supported");
  const int64_t N = f.proj[0].N, K = f.K;
  SCfg c;
  int splits = 1;
  stream_preferred(f.M, N, K, f.bits, c, splits);
  TileParams a{};
  a.x = f.x;
  a.M = static_cast<int>(f.M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.wq = f.proj[0].wq;
  a.s = f.proj[0].s;
  a.b = f.proj[0].b;
  a.bias = f.proj[0].bias;
  a.wq2 = f.proj[1].wq;
  a.s2 = f.proj[1].s;
  a.b2 = f.proj[1].b;
  a.bias2 = f.proj[1].bias;
  a.y = f.proj[0].y;
  a.splits = 1;
  const int64_t per = c.nch * (f.bits == 4 ? 1 : 2) * c.kh;
  a.steps = static_cast<int>(chunks_of(K, f.bits) / per);
  const int tiles = static_cast<int>(ceil_div(N, 8 * (c.wv / c.kh)));  // 16 outputs per gate/up pair of row groups
  const int mt = f.M <= 16 ? 1 : 2;
  if (f.bits == 4) return mt == 1 ? run_swiglu<4, 1>(c, a, tiles, 1, st) : run_swiglu<4, 2>(c, a, tiles, 1, st);
  return mt == 1 ? run_swiglu<8, 1>(c, a, tiles, 1, st) : run_swiglu<8, 2>(c, a, tiles, 1, st);
}

// The whole-K form carries the fused decode forms for 5..32 activation rows:
// group size 64, K one slice of 8 waves x 4 chunks (Q4 K = 4096, Q8 K = 2048
// or 4096), up to three projections, a head repeat, residuals;
// no SwiGLU (gate/up go through plain calls there).
bool qmv_tile_fused_eligible(const QmvFused& f) {
  if (f.M < 5 || f.M > kQmvMaxM || f.group_size != 64 || f.swiglu || f.nproj < 1 || f.nproj > 3) return false;
  const int64_t ch = chunks_of(f.K, f.bits);
  if (ch % 8) return false;
  const Cfg c{1, 8, static_cast<int>(ch / 8), 8};
  if (!cfg_known(c, f.bits)) return false;
  // No RMSNorm: every workgroup would normalise the same activations again
  // (measured with the norm while staging: qkv at M = 16 26 us against 4.5 +
  // 13.5 for the norm kernel and the fused projections; a 128256-row
  // lm_head 379 us)
  if (f.norm_w) return false;
  int64_t tiles = 0, tiles32 = 0;
  for (int i = 0; i < f.nproj; i++) {
    tiles += ceil_div(f.proj[i].N, 16);
    tiles32 += ceil_div(f.proj[i].N, 32);
  }
  // one workgroup per CU: at most two rounds (of 32-row workgroups where
  // launch_qmv_tile_fused takes them)
  const bool rg2 = ch / 4 == (f.bits == 4 ? 8 : 16) && overrides().tile_fused_rg != 1;
  if ((rg2 && tiles * ceil_div(f.M, 16) > cu_count() ? tiles32 : tiles) * ceil_div(f.M, 16) > 2 * cu_count())
    return false;
  for (int i = 0; i < f.nproj; i++)
    if (f.proj[i].N < 1 || f.proj[i].N > (int64_t(1) << 24)) return false;
  return f.x_stride * f.M < (int64_t(1) << 31) && f.K * f.M < (int64_t(1) << 31);
}

int launch_qmv_tile_fused(const QmvFused& f, hipStream_t st) {
  if (!qmv_tile_fused_eligible(f)) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_tile_fused: shape not supported");
  TileFused a{};
  a.p.x = f.x;
  a.p.M = static_cast<int>(f.M);
  a.p.K = static_cast<int>(f.K);
  a.p.splits = 1;
  a.p.steps = 1;
  a.p.x_stride = static_cast<int>(f.x_stride);
  a.p.rep = f.rep > 1 ? f.rep : 1;
  a.p.rep_hd8 = f.rep > 1 ? f.rep_hd / 8 : 1;
  if (f.rep > 1 && f.rep_hd % 8) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_tile_fused: head size not a multiple of 8");
  a.p.rcp_hd8 = 1.0f / static_cast<float>(a.p.rep_hd8);
  a.p.rcp_grp = 1.0f / static_cast<float>(a.p.rep_hd8 * a.p.rep);
  {
    auto lg = [](int v) { return v > 0 && (v & (v - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(v)) : -1; };
    const int sh = lg(a.p.rep_hd8), sg = lg(a.p.rep_hd8 * a.p.rep);
    a.p.rep_sh_hd8 = sh;
    a.p.rep_sh_grp = sh >= 0 && sg >= 0 ? sg : -1;
  }
  a.nseg = f.nproj;
  const int64_t ch = chunks_of(f.K, f.bits);
  const int mb = static_cast<int>(ceil_div(f.M, 16));
  // 16-row tiles past one round of CUs: 32 rows per workgroup (two row
  // groups x four K parts) in one round instead
  int64_t tiles16 = 0;
  for (int i = 0; i < f.nproj; i++) tiles16 += ceil_div(f.proj[i].N, 16);
  const bool rg2 = tiles16 * mb > cu_count() && ch % 4 == 0 && ch / 4 == (f.bits == 4 ? 8 : 16) &&
                   overrides().tile_fused_rg != 1;
  const Cfg c = rg2 ? Cfg{1, 8, static_cast<int>(ch / 4), 4} : Cfg{1, 8, static_cast<int>(ch / 8), 8};
  const int rows = rg2 ? 32 : 16;
  int tiles = 0;
  for (int i = 0; i < f.nproj; i++) {
    const QmvProj& P = f.proj[i];
    tiles += static_cast<int>(ceil_div(P.N, rows));
    a.seg[i] = TileSeg{P.wq, P.s, P.b, P.bias, P.res, P.y, static_cast<int>(P.N), tiles};
  }
  return f.bits == 4 ? run_fused<4>(c, a, tiles, mb, st) : run_fused<8>(c, a, tiles, mb, st);
}

}  // namespace mlxq
