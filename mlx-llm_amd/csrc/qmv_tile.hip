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
//    blocks; P = sum x (OFF + q), S = sum x (MFMA against ones),
//    acc += s P + (b - OFF s) S per group in f32.
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
};

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

template <int BITS, int GS, int MT, int WV, int NCH>
struct TileGeom {
  using Bk = Blk<BITS, GS>;
  static constexpr int T = 64 * WV;                  // threads
  static constexpr int MR = 16 * MT;                 // activation rows staged (padded)
  static constexpr int KS = NCH * Bk::KC;            // k per slice
  static constexpr int ROW16 = KS / 8 + 1;           // 16-byte slots per staged row (one of padding)
  static constexpr int XP = MR * (KS / 8) / T;       // 16-byte activation pieces per thread
  static constexpr int NG = KS / GS;                 // groups per slice
  static constexpr int NGW = NG / 2;                 // parameter words per row and slice
  static_assert(XP >= 1 && MR * (KS / 8) % T == 0, "activation pieces must divide over the threads");
  static_assert(NG % 2 == 0 && (NGW == 2 || NGW % 4 == 0), "parameters load as whole vectors");
};

template <int BITS, int GS, int MT, int WV, int NCH>
__global__ __launch_bounds__(64 * WV) void qmv_tile_kernel(const TileParams p) {
  using Tg = TileGeom<BITS, GS, MT, WV, NCH>;
  using Bk = typename Tg::Bk;
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  __shared__ u32x4 xs[Tg::MR * Tg::ROW16];

  const int K = p.K, M = p.M, N = p.N;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, gq = lane >> 4;
  const int G = K / GS;
  const int64_t row_u4 = static_cast<int64_t>(K) * BITS / 128;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int n0 = tile * 16 * WV + wave * 16;  // this wave's 16 weight rows
  const int c0 = split * NCH;                 // first chunk of the slice
  const int n = min(n0 + r16, N - 1);         // rows past N repeat row N-1 (results dropped)

  // 1. activations of the slice (issued first: the LDS staging waits on them)
  u32x4 xg[Tg::XP];
  int xdst[Tg::XP];
#pragma unroll
  for (int i = 0; i < Tg::XP; i++) {
    const int q = tid + Tg::T * i;
    const int row = q / (Tg::KS / 8), col = q % (Tg::KS / 8);
    // rows past M read row M-1: they only feed output rows >= M
    xg[i] = *reinterpret_cast<const u32x4*>(p.x + static_cast<int64_t>(min(row, M - 1)) * K +
                                            static_cast<int64_t>(c0) * Bk::KC + col * 8);
    xdst[i] = row * Tg::ROW16 + col;
  }
  // 2. this lane's row's group parameters over the slice, then 3. its codes,
  // chunk by chunk (the math on chunk c waits only for chunks <= c)
  uint32_t sw[Tg::NGW], bw[Tg::NGW];
  load_param_words<Tg::NGW>(p.s + static_cast<int64_t>(n) * G + c0 * Bk::KC / GS, sw);
  load_param_words<Tg::NGW>(p.b + static_cast<int64_t>(n) * G + c0 * Bk::KC / GS, bw);
  u32x4 w[NCH];
  const u32x4* wrow = reinterpret_cast<const u32x4*>(p.wq) + n * row_u4 + gq;
#pragma unroll
  for (int c = 0; c < NCH; c++) w[c] = wrow[static_cast<int64_t>(c0 + c) * 4];
  __builtin_amdgcn_sched_barrier(0);  // every load is issued before the first wait

  // staged in the order of the Q4 decode (pairs (x0,x2),(x4,x6),...): the
  // permutation is done once here instead of by every wave per block
#pragma unroll
  for (int i = 0; i < Tg::XP; i++) {
    if constexpr (BITS == 4) {
      const uint32_t xv[4] = {xg[i][0], xg[i][1], xg[i][2], xg[i][3]};
      uint32_t a[4];
      act_order_q4_bytes(xv, a);
      xs[xdst[i]] = u32x4{a[0], a[1], a[2], a[3]};
    } else {
      xs[xdst[i]] = xg[i];
    }
  }
  __syncthreads();

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint32_t ones[4];
#pragma unroll
  for (int i = 0; i < 4; i++) ones[i] = 0x3F803F80u;  // bf16 1.0 pairs

#pragma unroll
  for (int c = 0; c < NCH; c++) {
    uint32_t d[4] = {w[c][0], w[c][1], w[c][2], w[c][3]};
    if constexpr (!Bk::NAT) transpose_rows(d);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 P[MT], SX[MT];
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
        const int e = c * Bk::KC + Bk::xoff(j, gq);
        uint32_t a[4];
        if constexpr (Bk::XW == 4) {
          const u32x4 v = rowp[e / 8];
          a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
        } else {
          const uint2 v = reinterpret_cast<const uint2*>(rowp)[e / 4];
          a[0] = v.x; a[1] = v.y;
        }
        SX[mt] = mma<Bk::X32>(a, ones, first ? zero : SX[mt]);
        P[mt] = mma<Bk::X32>(a, bq, first ? zero : P[mt]);
      }
      if (j % Bk::BPG == Bk::BPG - 1) {
        const int g = (c * Bk::KC + Bk::code0(j)) / GS;  // group within the slice (compile-time)
        const float sc = __uint_as_float((g & 1) ? (sw[g >> 1] & 0xFFFF0000u) : (sw[g >> 1] << 16));
        const float bb = __uint_as_float((g & 1) ? (bw[g >> 1] & 0xFFFF0000u) : (bw[g >> 1] << 16));
        const float cf = bb - OFF * sc;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int v = 0; v < 4; v++) acc[mt][v] = fmaf(sc, P[mt][v], fmaf(cf, SX[mt][v], acc[mt][v]));
      }
    }
  }

  // C layout of a 16x16 MFMA tile: lane holds column (weight row) r16 and
  // activation rows 4 gq + v of the M-tile.
  const int nn = n0 + r16;
  if (p.splits == 1) {
    if (nn < N) {
      const float bb = p.bias ? bf16_bits_to_f32(p.bias[nn]) : 0.f;
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
          const int m = 16 * mt + 4 * gq + v;
          if (m < M) p.y[static_cast<int64_t>(m) * N + nn] = static_cast<uint16_t>(f32_to_bf16_bits(acc[mt][v] + bb));
        }
    }
    return;
  }

  // partial tile of this slice; split_reduce4_kernel adds the slices
  if (nn < N) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int m = 16 * mt + 4 * gq + v;
        if (m < M) p.part[(static_cast<int64_t>(split) * M + m) * N + nn] = acc[mt][v];
      }
  }
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
// aligned): 16-byte partial loads, one 8-byte store.
__global__ __launch_bounds__(256) void split_reduce4_kernel(const float4* __restrict__ part,
                                                            const uint16_t* __restrict__ bias,
                                                            uint2* __restrict__ y, int64_t MN4, int N,
                                                            int splits) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MN4) return;
  float4 sum = part[i];
  for (int sp = 1; sp < splits; sp++) {
    const float4 v = part[sp * MN4 + i];
    sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
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

}  // namespace tile

int launch_split_reduce(const float* part, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int splits,
                        hipStream_t st) {
  const int64_t mn = M * N;
  if (N % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
    const int64_t mn4 = mn / 4;
    hipLaunchKernelGGL(tile::split_reduce4_kernel, dim3(static_cast<unsigned>(ceil_div(mn4, 256))), dim3(256), 0,
                       st, reinterpret_cast<const float4*>(part), bias, reinterpret_cast<uint2*>(y), mn4,
                       static_cast<int>(N), splits);
  } else {
    hipLaunchKernelGGL(tile::qmv_tile_reduce_kernel, dim3(static_cast<unsigned>(ceil_div(mn, 256))), dim3(256), 0,
                       st, part, bias, y, mn, static_cast<int>(N), splits);
  }
  return check_launch("split_reduce");
}

namespace tile {

// ---------------------------------------------------------------- launch

constexpr int kMaxSplits = kMaxSplitsK;

struct Cfg {
  int mt = 1, wv = 4, nch = 8;
};

template <int BITS, int MT, int WV, int NCH>
int run(const TileParams& a, int tiles, hipStream_t st, int* query) {
  auto kern = qmv_tile_kernel<BITS, 64, MT, WV, NCH>;
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
  hipLaunchKernelGGL(kern, dim3(tiles, a.splits), dim3(64 * WV), 0, st, a);
  return check_launch("qmv_tile");
}

// (waves, chunks per slice): slices of 16 chunks only with 8 waves, which
// keeps the activation staging at <= 16 pieces per thread
template <int BITS, int MT>
int run_wn(const Cfg& c, const TileParams& a, int tiles, hipStream_t st, int* q) {
  if (c.wv == 4) return c.nch == 4 ? run<BITS, MT, 4, 4>(a, tiles, st, q) : run<BITS, MT, 4, 8>(a, tiles, st, q);
  if (c.nch == 4) return run<BITS, MT, 8, 4>(a, tiles, st, q);
  return c.nch == 8 ? run<BITS, MT, 8, 8>(a, tiles, st, q) : run<BITS, MT, 8, 16>(a, tiles, st, q);
}

int dispatch(int bits, const Cfg& c, const TileParams& a, int tiles, hipStream_t st, int* q) {
  if (bits == 4) return c.mt == 1 ? run_wn<4, 1>(c, a, tiles, st, q) : run_wn<4, 2>(c, a, tiles, st, q);
  return c.mt == 1 ? run_wn<8, 1>(c, a, tiles, st, q) : run_wn<8, 2>(c, a, tiles, st, q);
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

bool qmv_tile_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M < 1 || M > kQmvMaxM || N < 1 || group_size != 64) return false;
  if ((K * bits / 8) % 64) return false;
  const int64_t ch = chunks_of(K, bits);
  if (ch % 4 || ch > 16 * kMaxSplits) return false;  // whole slices of 4, 8 or 16 chunks, <= 16 slices
  return static_cast<int64_t>(kMaxSplits) * M * N < (int64_t(1) << 31);
}

size_t qmv_tile_workspace_bytes(int64_t M, int64_t N) { return static_cast<size_t>(kMaxSplits) * M * N * 4; }

bool qmv_tile_preferred(int64_t M, int64_t N, int64_t K, int bits) {
  // Measured against the block kernel (qmv.hip) and the vector-ALU kernel
  // (qmv_dot) at the Llama-3-8B projection shapes: the tile kernel wins on
  // the large projections from M = 8 (Q4) / 16 (Q8),
  // on Q4 gate/up already from M = 3, on short matrices (N <= 2048) from
  // M = 16, and on the other small projections from M = 24 (Q4) / 32 (Q8).
  const bool large = N * K >= (int64_t(1) << 25);
  if (M <= 4) return large && K < N && bits == 4 && M >= 3;
  if (large) return M >= (bits == 4 ? 8 : 16);
  if (N <= 2048) return M >= 16;  // k/v: M = 16 Q4 8.28 -> 7.93 us, Q8 9.27 -> 8.06; Q8 M = 24 11.07 -> 8.93
  return M >= (bits == 4 ? 24 : 32);
}

bool qmv_dot_preferred(int64_t M, int64_t N, int64_t K, int bits) {
  // M = 1 always; M = 2 on gate/up-like shapes (large N*K, K < N); the block
  // kernel is faster for the other shapes at M = 2..4.
  (void)bits;
  return M == 1 || (M == 2 && N * K >= (int64_t(1) << 25) && K < N);
}

int launch_qmv_tile(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                    const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                    void* workspace, size_t workspace_bytes, hipStream_t st) {
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

  // (waves, chunks per slice).  Measured best at the Llama-3-8B shapes
  // (M = 8..32): large N*K with K >= 2N (down): 8 waves, 16-chunk slices;
  // other large N*K: Q4 8 waves / 8 chunks, Q8 4 waves / 8 chunks; small
  // N*K: 4 waves, 8 chunks (4 for Q4 with N < 2048).  Taken when it divides
  // K into at most 16 slices that fit the workspace, else the first such of
  // the others.
  const bool large = N * K >= (int64_t(1) << 25);
  Cfg pref;
  pref.mt = M <= 16 ? 1 : 2;
  if (large && K >= 2 * N) {
    pref.wv = 8; pref.nch = 16;
  } else if (large) {
    pref.wv = bits == 4 ? 8 : 4; pref.nch = 8;
  } else {
    pref.wv = 4; pref.nch = bits == 4 && N < 2048 ? 4 : 8;
  }
  const int fwv = overrides().tile_wv, fnch = overrides().tile_nch;
  if (fwv) pref.wv = fwv;
  if (fnch) pref.nch = fnch;
  const Cfg order[] = {pref, {pref.mt, 8, 16}, {pref.mt, 8, 8}, {pref.mt, 4, 8}, {pref.mt, 4, 4}, {pref.mt, 8, 4}};
  const Cfg* pick = nullptr;
  for (const Cfg& c : order) {
    if ((c.wv != 4 && c.wv != 8) || (c.nch != 4 && c.nch != 8 && c.nch != 16) || (c.nch == 16 && c.wv != 8))
      continue;
    if (ch % c.nch) continue;
    const int64_t splits = ch / c.nch;
    if (splits > kMaxSplits || (splits > 1 && splits > fit)) continue;
    pick = &c;
    break;
  }
  if (!pick) return MLXQ_ERR_UNSUPPORTED;  // no slicing fits the workspace: the caller picks another kernel
  a.splits = static_cast<int>(ch / pick->nch);
  a.part = a.splits > 1 ? static_cast<float*>(workspace) : nullptr;
  const int64_t tiles = ceil_div(N, 16 * pick->wv);
  // split K: the slices are added by a second launch (split_reduce4_kernel).
  // A hand-off inside this kernel (the last arriving slice of a tile adds the
  // slices) was measured slower at the Llama-3-8B shapes (Q8 M = 32 gate
  // 26.1 -> 26.9 us): its agent-coherent partial stores and serial tail cost
  // more than the launch it saves.
  if (int rc = dispatch(bits, *pick, a, static_cast<int>(tiles), st, nullptr)) return rc;
  if (a.splits == 1) return MLXQ_OK;
  return launch_split_reduce(a.part, bias, y, M, N, a.splits, st);
}

}  // namespace mlxq
