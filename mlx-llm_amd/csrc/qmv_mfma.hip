// Small-M quantized GEMV on the matrix cores (gfx950): 5..32 activation rows
// (batched decode), the streaming structure of the vector-ALU decode kernel
// (qmv_dot_kernel.hpp) with v_mfma_f32_16x16x32_bf16 (Q4) /
// v_mfma_f32_16x16x16_bf16 (Q8) as the contraction.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul at batched-decode shapes (MLX's qmv / small
// qmm kernels).
//
//  * Streaming: lane (r16, gq) of a wave loads 16 bytes of codes of weight
//    row r16 (quarter gq of a 64-byte chunk): one instruction reads 16 rows x
//    64 contiguous bytes.  A wave owns a contiguous range of chunks, taken RC
//    at a time; the next round is in flight while one is computed, and the
//    last round is peeled (nothing is fetched past the wave's range).
//  * Group-pure MFMA blocks: a 4 x 4 transpose of the code dwords across the
//    four 16-lane rows (v_permlane32_swap + v_permlane16_swap) gives lane gq
//    the codes [B*j + B/4*gq, +B/4) of every block j of B = 32 (Q4) / 16 (Q8)
//    consecutive codes, which is exactly the B-operand slice of an MFMA over
//    that block.  A block never straddles a quantization group (B <= 32 <=
//    group), so each MFMA result is one group's partial sum.
//  * A = activations (16 rows per M-tile), read from L2 in the same block
//    order (16 rows x 64 contiguous bytes per instruction); B = codes as
//    bf16 (Q4: (128 + q) pairs from one and-or per pair, activations permuted
//    to the same order with v_perm; Q8: exact through f32).  Per block:
//    P = sum x (OFF + q), S = sum x (one more MFMA against ones, shared by the
//    row sub-tiles), acc += s P + (b - OFF s) S in f32, with s, b the
//    lane's own row's group parameters (the C layout gives lane l column
//    l % 16 = its weight row).
//  * Waves reduce through LDS in fixed order (deterministic), then y (+ bias)
//    (+ residual) is stored as bf16.  No workspace.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "qmatmul.hpp"
#include "mfma_blocks.hpp"
#include "qmv_dot_kernel.hpp"

namespace mlxq {
namespace mfma {

using dot::DotGeom;
using dot::load_param_words;
using dot::Params;
using dot::Seg;

template <int BITS, int GS, int MT, int SUB, int RC, int NGW>
struct Round {
  uint4 w[RC][SUB];
  uint32_t x[RC][MT][Blk<BITS, GS>::NB][Blk<BITS, GS>::XW];
  uint32_t s[SUB][NGW], b[SUB][NGW];
};

template <int BITS, int GS, int MT, int SUB, int RC, int WV>
__global__ __launch_bounds__(64 * WV) void qmv_mfma_kernel(const Params p) {
  using Gm = DotGeom<BITS, GS, RC>;
  using Bk = Blk<BITS, GS>;
  using Rnd = Round<BITS, GS, MT, SUB, RC, Gm::NGW>;
  constexpr int R = 16 * SUB;
  constexpr int MR = 16 * MT;  // activation rows held (padded)
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  extern __shared__ __align__(16) float red[];  // [WV][MR][R]

  const int K = p.K, M = p.M;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, gq = lane >> 4;
  const int G = K / GS;
  const int chunks = K * BITS / 8 / 64;
  const int64_t row_u4 = static_cast<int64_t>(K) * BITS / 128;

  int sg = 0;
  const int t = blockIdx.x;
  while (sg + 1 < p.nseg && t >= p.seg[sg].tile_end) sg++;
  const int n0 = (t - (sg ? p.seg[sg - 1].tile_end : 0)) * R;
  const Seg& S = p.seg[sg];

  const uint4* wrow[SUB];
  const uint16_t* srow[SUB];
  const uint16_t* brow[SUB];
#pragma unroll
  for (int s = 0; s < SUB; s++) {
    const int n = min(n0 + 16 * s + r16, S.N - 1);  // rows past N repeat row N-1 (results dropped)
    wrow[s] = reinterpret_cast<const uint4*>(S.wq) + n * row_u4 + gq;
    srow[s] = S.s + static_cast<int64_t>(n) * G;
    brow[s] = S.b + static_cast<int64_t>(n) * G;
  }
  // activation row 16 mt + r16 (rows past M read row 0: they only feed
  // output rows >= M, which are never stored); this lane's slice of a block
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int m = 16 * mt + r16;
    xrow[mt] = p.x + static_cast<int64_t>(m < M ? m : 0) * p.x_stride;
  }

  // Rounds are dealt to the waves in turn (round r to wave r % WV), so at
  // any time the workgroup's waves read neighbouring 64-byte chunks of the
  // same rows; the chunks past the last full round go one per wave.
  const int nfull = chunks / RC;

  auto load_x = [&](uint32_t (&xv)[MT][Bk::NB][Bk::XW], int c) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < Bk::NB; j++) {
        const uint16_t* src = xrow[mt] + static_cast<int64_t>(c) * Bk::KC + Bk::xoff(j, gq);
        if constexpr (Bk::XW == 4) {
          const uint4 v = *reinterpret_cast<const uint4*>(src);
          xv[mt][j][0] = v.x; xv[mt][j][1] = v.y; xv[mt][j][2] = v.z; xv[mt][j][3] = v.w;
        } else {
          const uint2 v = *reinterpret_cast<const uint2*>(src);
          xv[mt][j][0] = v.x; xv[mt][j][1] = v.y;
        }
      }
  };
  auto fetch = [&](Rnd& T, int c0) {
    const int g0 = c0 * Gm::NGC / Gm::CPG;
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      if constexpr (Gm::NGR == 1) {  // one group per round: a single bf16 each
        T.s[s][0] = srow[s][g0];
        T.b[s][0] = brow[s][g0];
      } else {
        load_param_words<Gm::NGW>(srow[s] + g0, T.s[s]);
        load_param_words<Gm::NGW>(brow[s] + g0, T.b[s]);
      }
    }
#pragma unroll
    for (int u = 0; u < RC; u++) {
      load_x(T.x[u], c0 + u);
#pragma unroll
      for (int s = 0; s < SUB; s++) T.w[u][s] = wrow[s][static_cast<int64_t>(c0 + u) * 4];
    }
  };

  f32x4 acc[SUB][MT];
#pragma unroll
  for (int s = 0; s < SUB; s++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[s][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint32_t ones[4];
#pragma unroll
  for (int i = 0; i < 4; i++) ones[i] = 0x3F803F80u;  // bf16 1.0 pairs

  // one chunk: codes w (per sub-tile), activations xv.  MFMA results of
  // consecutive blocks of one group accumulate in P / SX; at the group's last
  // block the group's scale / bias, from par(s, j), fold them into acc.
  auto chunk = [&](const uint4 (&w)[SUB], const uint32_t (&xv)[MT][Bk::NB][Bk::XW], auto&& par) {
    uint32_t d[SUB][4];
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      d[s][0] = w[s].x; d[s][1] = w[s].y; d[s][2] = w[s].z; d[s][3] = w[s].w;
      if constexpr (!Bk::NAT) transpose_rows(d[s]);
    }
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 P[SUB][MT], SX[MT];
#pragma unroll
    for (int j = 0; j < Bk::NB; j++) {
      const bool first = j % Bk::BPG == 0;
      uint32_t a[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        if constexpr (BITS == 4) {
          act_order_q4(xv[mt][j], a[mt]);
        } else {
#pragma unroll
          for (int i = 0; i < Bk::XW; i++) a[mt][i] = xv[mt][j][i];
        }
        SX[mt] = mma<Bk::X32>(a[mt], ones, first ? zero : SX[mt]);
      }
#pragma unroll
      for (int s = 0; s < SUB; s++) {
        uint32_t b[4];
        if constexpr (BITS == 4) {
          decode_q4(d[s][j], b);
        } else if constexpr (Bk::NAT) {
          decode_q8(d[s][2 * j], b);
          decode_q8(d[s][2 * j + 1], b + 2);
        } else {
          decode_q8(d[s][j], b);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) P[s][mt] = mma<Bk::X32>(a[mt], b, first ? zero : P[s][mt]);
      }
      if (j % Bk::BPG == Bk::BPG - 1) {
#pragma unroll
        for (int s = 0; s < SUB; s++) {
          float sc, bb;
          par(s, j, sc, bb);
          const float c = bb - OFF * sc;
#pragma unroll
          for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[s][mt][v] = fmaf(sc, P[s][mt][v], fmaf(c, SX[mt][v], acc[s][mt][v]));
        }
      }
    }
  };

  auto compute = [&](const Rnd& T) {
#pragma unroll
    for (int u = 0; u < RC; u++) {
      chunk(T.w[u], T.x[u], [&](int s, int j, float& sc, float& bb) {
        // group of block j of chunk u, relative to the round's first group
        // (compile-time after unrolling)
        const int gi = (u * Bk::KC + Bk::code0(j)) / GS;
        float vs = 0.f, vb = 0.f;
#pragma unroll
        for (int g = 0; g < Gm::NGR; g++)
          if (g == gi) {
            vs = __uint_as_float((g & 1) ? (T.s[s][g >> 1] & 0xFFFF0000u) : (T.s[s][g >> 1] << 16));
            vb = __uint_as_float((g & 1) ? (T.b[s][g >> 1] & 0xFFFF0000u) : (T.b[s][g >> 1] << 16));
          }
        sc = vs;
        bb = vb;
      });
    }
  };

  Rnd cur, nxt;
  if (wave < nfull) {
    int r = wave;
    fetch(cur, r * RC);
    for (; r + WV < nfull; r += WV) {
      fetch(nxt, (r + WV) * RC);
      __builtin_amdgcn_sched_barrier(0);  // next round in flight before this one is computed
      compute(cur);
      cur = nxt;
    }
    compute(cur);
  }
  // chunks past the last full round (< RC <= WV): one per wave
  if (nfull * RC + wave < chunks) {
    const int c = nfull * RC + wave;
    uint4 w[SUB];
    uint32_t xv[MT][Bk::NB][Bk::XW];
    load_x(xv, c);
#pragma unroll
    for (int s = 0; s < SUB; s++) w[s] = wrow[s][static_cast<int64_t>(c) * 4];
    chunk(w, xv, [&](int s, int j, float& sc, float& bb) {
      const int g = (c * Bk::KC + Bk::code0(j)) / GS;
      sc = bf16_bits_to_f32(srow[s][g]);
      bb = bf16_bits_to_f32(brow[s][g]);
    });
  }

  // C layout of a 16x16 MFMA tile: lane holds column (weight row) r16 and
  // activation rows 4*gq + v of the M-tile
#pragma unroll
  for (int s = 0; s < SUB; s++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++) red[(wave * MR + 16 * mt + 4 * gq + v) * R + 16 * s + r16] = acc[s][mt][v];
  __syncthreads();
  for (int i = tid; i < M * R; i += 64 * WV) {
    const int m = i / R, r = i % R, n = n0 + r;
    if (n >= S.N) continue;
    float sum = red[m * R + r];
#pragma unroll
    for (int w = 1; w < WV; w++) sum += red[(w * MR + m) * R + r];
    if (S.bias) sum += bf16_bits_to_f32(S.bias[n]);
    const int64_t o = static_cast<int64_t>(m) * S.N + n;
    if (S.res) sum = bf16_bits_to_f32(S.res[o]) + dot::bf16_round(sum);
    S.y[o] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
  }
}

// ---------------------------------------------------------------- launch

struct Cfg {
  int mt = 1, sub = 1, wv = 8;
  int64_t tiles = 0;
  size_t lds = 0;
};

// chunks per round: 2 (activations and codes of two rounds stay in registers)
constexpr int kRC = 2;

template <int BITS, int GS, int MT, int SUB, int WV>
int run(const Cfg& c, const Params& a, hipStream_t st, int* query) {
  auto kern = qmv_mfma_kernel<BITS, GS, MT, SUB, kRC, WV>;
  if (query) {
    static int cached = -1;
    static size_t cached_lds = 0;
    if (cached < 0 || cached_lds != c.lds) {
      int nb = 0;
      hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), 64 * WV,
                                                                  c.lds);
      if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmv_mfma: occupancy: ") + hipGetErrorString(e));
      cached = nb;
      cached_lds = c.lds;
    }
    *query = cached;
    return MLXQ_OK;
  }
  MLXQ_LAUNCH(kern, dim3(c.tiles), dim3(64 * WV), c.lds, st, a);
  return check_launch("qmv_mfma");
}

template <int BITS, int GS, int MT>
int run_sw(const Cfg& c, const Params& a, hipStream_t st, int* q) {
  if constexpr (MT == 1) {
    if (c.sub == 2) return c.wv == 4 ? run<BITS, GS, MT, 2, 4>(c, a, st, q) : run<BITS, GS, MT, 2, 8>(c, a, st, q);
  }
  return c.wv == 4 ? run<BITS, GS, MT, 1, 4>(c, a, st, q) : run<BITS, GS, MT, 1, 8>(c, a, st, q);
}

template <int BITS, int GS>
int run_mt(const Cfg& c, const Params& a, hipStream_t st, int* q) {
  return c.mt == 1 ? run_sw<BITS, GS, 1>(c, a, st, q) : run_sw<BITS, GS, 2>(c, a, st, q);
}

int dispatch(int group_size, int bits, const Cfg& c, const Params& a, hipStream_t st, int* q) {
  if (bits == 4) {
    if (group_size == 32) return run_mt<4, 32>(c, a, st, q);
    if (group_size == 64) return run_mt<4, 64>(c, a, st, q);
    return run_mt<4, 128>(c, a, st, q);
  }
  if (group_size == 32) return run_mt<8, 32>(c, a, st, q);
  if (group_size == 64) return run_mt<8, 64>(c, a, st, q);
  return run_mt<8, 128>(c, a, st, q);
}

int cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

}  // namespace mfma

bool qmv_mfma_eligible(int64_t M, int64_t K, int group_size, int bits) {
  if (M < 1 || M > kQmvMaxM) return false;
  if ((K * bits / 8) % 64) return false;  // whole 64-byte chunks per row
  const int64_t gb = static_cast<int64_t>(group_size) * bits / 8;
  const int64_t ngr = 4 * (gb >= 64 ? 1 : 64 / gb) / (gb > 64 ? gb / 64 : 1);  // groups per 4-chunk round
  return (K / group_size) % std::min<int64_t>(ngr, 8) == 0;                 // aligned vector loads of round params
}

int launch_qmv_mfma(const QmvFused& f, hipStream_t st) {
  using namespace mfma;
  const int64_t M = f.M, K = f.K;
  if (f.nproj < 1 || f.nproj > dot::kMaxSegs || f.swiglu || f.norm_w || f.rep > 1)
    return fail(MLXQ_ERR_UNSUPPORTED, "qmv_mfma: form not supported");
  if (!qmv_mfma_eligible(M, K, f.group_size, f.bits))
    return fail(MLXQ_ERR_UNSUPPORTED, "qmv_mfma: shape not supported");
  if ((reinterpret_cast<uintptr_t>(f.x) & 15u) || (f.x_stride % 8))
    return fail(MLXQ_ERR_INVALID, "qmv_mfma: activations must be 16-byte aligned rows");
  Params a{};
  a.x = f.x;
  a.M = static_cast<int>(M);
  a.K = static_cast<int>(K);
  a.x_stride = static_cast<int>(f.x_stride);
  a.nseg = f.nproj;
  for (int i = 0; i < f.nproj; i++) {
    const QmvProj& P = f.proj[i];
    a.seg[i] = Seg{P.wq, P.s, P.b, P.bias, P.res, P.y, static_cast<int>(P.N), 0};
  }
  static const int cus = cu_count();
  const int mt = M > 16 ? 2 : 1;
  const int64_t chunks = K * f.bits / 8 / 64;
  Cfg best;
  int64_t best_pass = -1, best_waves = 0;
  const int forced_sub = overrides().mfma_sub, forced_wv = overrides().mfma_wv;
  for (int sub = 1; sub <= (mt == 1 ? 2 : 1); sub++)  // two M-tiles: one row sub-tile (registers)
    for (int wv = 4; wv <= 8; wv += 4) {
      if ((forced_sub && sub != forced_sub) || (forced_wv && wv != forced_wv)) continue;
      Cfg c;
      c.mt = mt;
      c.sub = sub;
      c.wv = wv;
      c.lds = static_cast<size_t>(wv) * 16 * mt * 16 * sub * 4;
      for (int i = 0; i < f.nproj; i++) c.tiles += ceil_div(f.proj[i].N, 16 * sub);
      int nb = 0;
      if (int rc = dispatch(f.group_size, f.bits, c, a, st, &nb)) return rc;
      const int64_t slots = std::max<int64_t>(1, static_cast<int64_t>(nb) * cus);
      const int64_t pass = ceil_div(c.tiles, slots);
      const int64_t waves = std::min(c.tiles, slots) * wv;
      if (best_pass < 0 || pass < best_pass || (pass == best_pass && waves > best_waves)) {
        best = c;
        best_pass = pass;
        best_waves = waves;
      }
    }
  if (best_pass < 0) return fail(MLXQ_ERR_INVALID, "qmv_mfma: no configuration fits this shape");
  a.cw = static_cast<int>(ceil_div(ceil_div(chunks, best.wv), kRC) * kRC);
  int64_t end = 0;
  for (int i = 0; i < f.nproj; i++) {
    end += ceil_div(f.proj[i].N, 16 * best.sub);
    a.seg[i].tile_end = static_cast<int>(end);
  }
  return dispatch(f.group_size, f.bits, best, a, st, nullptr);
}

}  // namespace mlxq
