// Decode-shaped quantized matmul (qmv) for gfx950: y[M,N] = x[M,K] . W^T with
// W group-wise affine quantized (Q4 / Q8), M <= 32.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul(x, w, scales, biases, transpose=true, g, bits),
// which MLX serves with its qmv kernels for small M.
//
// Design (HBM-bound: the packed weights are read exactly once):
//  * A workgroup of 4 wavefronts owns a tile of 64 weight rows and one K-split;
//    its waves take interleaved blocks of U consecutive groups, so each wave
//    reads U*group_size*bits/8 contiguous bytes per row per block.
//  * The contraction runs on the matrix cores with v_mfma_f32_16x16x32_bf16:
//    A = activations (M padded to 16 rows per M-tile), B = 16 weight rows.
//    Q4 codes become bf16 (128 + q) with one and-or per pair of nibbles
//    (0x4300 | q is exactly 128 + q in bf16); Q8 codes are converted exactly
//    through f32.  A-operand activations are permuted with v_perm to the same
//    nibble order, so the products pair up correctly.
//  * Per group, the MFMA partial P = sum x*(OFF+q) is folded into f32
//    accumulators: acc += s*P + (b - OFF*s) * sum(x), with sum(x) produced by
//    one extra MFMA against an all-ones operand (shared by the 4 sub-tiles).
//  * The 4 waves reduce through LDS; with several K-splits each workgroup
//    writes an f32 partial to the workspace and the last one to arrive (atomic
//    ticket) sums the splits in fixed order, so results are deterministic.  It
//    then resets its ticket to zero, leaving the workspace ready for reuse.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 64;  // weight rows per workgroup (4 sub-tiles of 16)
constexpr int kSub = 4;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Load NW consecutive 32-bit words (NW in {1,2,4,8}), naturally aligned.
template <int NW>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t (&w)[NW]) {
  if constexpr (NW == 1) {
    w[0] = *p;
  } else if constexpr (NW == 2) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < NW; i += 4) {
      uint4 v = *reinterpret_cast<const uint4*>(p + i);
      w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
  }
}

// B operand for one MFMA step from the lane's codes.
template <int BITS>
__device__ __forceinline__ bf16x8 weights_to_bf16(const uint32_t* w) {
  u32x4 r;
  if constexpr (BITS == 4) {
    // nibbles k0..k7 -> bf16 pairs (k0,k4),(k1,k5),(k2,k6),(k3,k7), value 128+q
    const uint32_t q = w[0];
    r[0] = (q & 0x000F000Fu) | 0x43004300u;
    r[1] = ((q >> 4) & 0x000F000Fu) | 0x43004300u;
    r[2] = ((q >> 8) & 0x000F000Fu) | 0x43004300u;
    r[3] = ((q >> 12) & 0x000F000Fu) | 0x43004300u;
  } else {
    // bytes k0..k7 (two words) -> exact bf16 of 0..255 in natural order; the
    // f32 of an integer <= 255 has zero low half, so the high half is exact.
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t q = w[i];
      float f0 = static_cast<float>(q & 0xFFu), f1 = static_cast<float>((q >> 8) & 0xFFu);
      float f2 = static_cast<float>((q >> 16) & 0xFFu), f3 = static_cast<float>(q >> 24);
      r[2 * i] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
      r[2 * i + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
    }
  }
  return as_bf16x8(r);
}

// A operand for one MFMA step from 8 consecutive bf16 activations (4 words).
template <int BITS>
__device__ __forceinline__ bf16x8 acts_to_bf16(const uint32_t* d) {
  u32x4 r;
  if constexpr (BITS == 4) {
    // (x0,x1),(x2,x3),(x4,x5),(x6,x7) -> (x0,x4),(x1,x5),(x2,x6),(x3,x7)
    r[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
    r[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
    r[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
    r[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
  } else {
    r[0] = d[0]; r[1] = d[1]; r[2] = d[2]; r[3] = d[3];
  }
  return as_bf16x8(r);
}

// Load U consecutive bf16 scales (or biases) starting at a U-aligned group.
template <int U>
__device__ __forceinline__ void load_group_params(const uint16_t* p, float (&v)[U]) {
  if constexpr (U == 4) {
    uint2 w = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_bits_to_f32(w.x & 0xFFFFu); v[1] = bf16_bits_to_f32(w.x >> 16);
    v[2] = bf16_bits_to_f32(w.y & 0xFFFFu); v[3] = bf16_bits_to_f32(w.y >> 16);
  } else if constexpr (U == 2) {
    uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    v[0] = bf16_bits_to_f32(w & 0xFFFFu); v[1] = bf16_bits_to_f32(w >> 16);
  } else {
    v[0] = bf16_bits_to_f32(*p);
  }
}

// The per-wave state of one qmv workgroup: row pointers and accumulators.
template <int BITS, int GS, int MT>
struct QmvWave {
  static constexpr int T = GS / 32;      // MFMA steps per group
  static constexpr int WPS = BITS / 4;   // code words per lane per MFMA step
  static constexpr int WPG = T * WPS;    // code words per lane per group
  static constexpr int XW = GS / 8;      // activation words (bf16 pairs) per lane per group
  static constexpr float OFF = BITS == 4 ? 128.f : 0.f;

  const uint32_t* wrow[kSub];
  const uint16_t* srow[kSub];
  const uint16_t* brow[kSub];
  const uint32_t* xrow[MT];
  bool xvalid[MT];
  f32x4 acc[kSub][MT];

  // U consecutive groups starting at g0 (U-aligned): every load is issued
  // before any use, with no divergent control flow, so they all overlap.
  template <int U>
  __device__ __forceinline__ void block(int g0) {
    uint32_t wb[U][kSub][WPG];
    uint32_t xa[U][MT][XW];
    float sv[kSub][U], bv[kSub][U];
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int s = 0; s < kSub; s++)
        load_words<WPG>(wrow[s] + static_cast<int64_t>(g0 + u) * (GS * BITS / 32), wb[u][s]);
#pragma unroll
    for (int s = 0; s < kSub; s++) {
      load_group_params<U>(srow[s] + g0, sv[s]);
      load_group_params<U>(brow[s] + g0, bv[s]);
    }
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) load_words<XW>(xrow[mt] + static_cast<int64_t>(g0 + u) * (GS / 2), xa[u][mt]);

    const bf16x8 ones = as_bf16x8(u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
#pragma unroll
    for (int u = 0; u < U; u++) {
      bf16x8 A[MT][T];
      f32x4 xs[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int i = 0; i < XW; i++) xa[u][mt][i] = xvalid[mt] ? xa[u][mt][i] : 0u;  // rows >= M
        xs[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < T; t++) {
          A[mt][t] = acts_to_bf16<BITS>(&xa[u][mt][4 * t]);
          xs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][t], ones, xs[mt], 0, 0, 0);
        }
      }
#pragma unroll
      for (int s = 0; s < kSub; s++) {
        f32x4 P[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) P[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < T; t++) {
          const bf16x8 B = weights_to_bf16<BITS>(&wb[u][s][t * WPS]);
#pragma unroll
          for (int mt = 0; mt < MT; mt++)
            P[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][t], B, P[mt], 0, 0, 0);
        }
        const float sc = sv[s][u];
        const float c = bv[s][u] - OFF * sc;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int v = 0; v < 4; v++) acc[s][mt][v] = fmaf(sc, P[mt][v], fmaf(c, xs[mt][v], acc[s][mt][v]));
      }
    }
  }
};

template <int BITS, int GS, int MT, int U>
__global__ __launch_bounds__(kThreads) void qmv_kernel(const uint16_t* __restrict__ x, int M,
                                                        const uint32_t* __restrict__ wq,
                                                        const uint16_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ biases,
                                                        const uint16_t* __restrict__ bias_vec, int N, int K,
                                                        int gps, uint16_t* __restrict__ y,
                                                        float* __restrict__ partial,
                                                        uint32_t* __restrict__ tickets) {
  using W = QmvWave<BITS, GS, MT>;
  __shared__ float red[kWaves][MT * 16][kRows];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, gq = lane >> 4;
  const int n0 = blockIdx.x * kRows;
  const int S = gridDim.y, split = blockIdx.y;
  const int G = K / GS;
  const int gs = split * gps, ge = min(G, gs + gps);
  const int64_t row_words = static_cast<int64_t>(K) * BITS / 32;

  W w;
#pragma unroll
  for (int s = 0; s < kSub; s++) {
    const int n = min(n0 + 16 * s + r16, N - 1);  // rows past N repeat row N-1 (results dropped)
    w.wrow[s] = wq + n * row_words + gq * W::WPG;
    w.srow[s] = scales + static_cast<int64_t>(n) * G;
    w.brow[s] = biases + static_cast<int64_t>(n) * G;
  }
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int m = 16 * mt + r16;
    w.xvalid[mt] = m < M;  // rows past M load row 0 and are zeroed before use
    w.xrow[mt] = reinterpret_cast<const uint32_t*>(x + static_cast<int64_t>(m < M ? m : 0) * K) + gq * W::XW;
  }
#pragma unroll
  for (int s = 0; s < kSub; s++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) w.acc[s][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // whole U-blocks, interleaved over the 4 waves, then single-group tail
  int g0 = gs + wave * U;
  for (; g0 + U <= ge; g0 += kWaves * U) w.template block<U>(g0);
  if constexpr (U > 1) {
    for (int g = g0; g < min(g0 + U, ge); g++) w.template block<1>(g);
  }

  // C layout of a 16x16 MFMA tile: lane holds column (weight row) r16 and
  // activation rows 4*gq + v.
#pragma unroll
  for (int s = 0; s < kSub; s++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++) red[wave][16 * mt + 4 * gq + v][16 * s + r16] = w.acc[s][mt][v];
  __syncthreads();

  const int outs = M * kRows;
  if (S == 1) {
    for (int i = tid; i < outs; i += kThreads) {
      const int m = i / kRows, r = i % kRows, n = n0 + r;
      if (n >= N) continue;
      float sum = ((red[0][m][r] + red[1][m][r]) + red[2][m][r]) + red[3][m][r];
      if (bias_vec) sum += bf16_bits_to_f32(bias_vec[n]);
      y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
    }
    return;
  }

  // Split-K hand-off without flushing or invalidating L2: partials are
  // written with device-scope atomic stores (write-through), completed with
  // s_waitcnt before the ticket increment, and read back by the last
  // workgroup with device-scope atomic loads (which bypass L2).
  for (int i = tid; i < outs; i += kThreads) {
    const int m = i / kRows, r = i % kRows, n = n0 + r;
    if (n >= N) continue;
    __hip_atomic_store(&partial[(static_cast<int64_t>(split) * M + m) * N + n],
                       ((red[0][m][r] + red[1][m][r]) + red[2][m][r]) + red[3][m][r], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    last_flag = __hip_atomic_fetch_add(&tickets[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                static_cast<uint32_t>(S - 1);
  __syncthreads();
  if (!last_flag) return;
  for (int i = tid; i < outs; i += kThreads) {
    const int m = i / kRows, r = i % kRows, n = n0 + r;
    if (n >= N) continue;
    float sum = 0.f;
    for (int sp = 0; sp < S; sp++)
      sum += __hip_atomic_load(&partial[(static_cast<int64_t>(sp) * M + m) * N + n], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    if (bias_vec) sum += bf16_bits_to_f32(bias_vec[n]);
    y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
  }
  if (tid == 0) __hip_atomic_store(&tickets[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int BITS, int GS, int MT>
void launch_u(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
              const uint16_t* bias, int N, int K, uint16_t* y, float* partial, uint32_t* tickets, hipStream_t st) {
  dim3 grid(p.row_tiles, p.splits);
  switch (p.unroll) {
    case 1: hipLaunchKernelGGL((qmv_kernel<BITS, GS, MT, 1>), grid, dim3(kThreads), 0, st, x, M, wq, s, b, bias, N, K, p.groups_per_split, y, partial, tickets); break;
    case 2: hipLaunchKernelGGL((qmv_kernel<BITS, GS, MT, 2>), grid, dim3(kThreads), 0, st, x, M, wq, s, b, bias, N, K, p.groups_per_split, y, partial, tickets); break;
    default: hipLaunchKernelGGL((qmv_kernel<BITS, GS, MT, 4>), grid, dim3(kThreads), 0, st, x, M, wq, s, b, bias, N, K, p.groups_per_split, y, partial, tickets); break;
  }
}

template <int BITS, int GS>
void launch_mt(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int N, int K, uint16_t* y, float* partial, uint32_t* tickets, hipStream_t st) {
  if (M <= 16) launch_u<BITS, GS, 1>(p, x, M, wq, s, b, bias, N, K, y, partial, tickets, st);
  else launch_u<BITS, GS, 2>(p, x, M, wq, s, b, bias, N, K, y, partial, tickets, st);
}

}  // namespace

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  QmvPlan p{};
  const int64_t G = K / group_size;
  p.row_tiles = ceil_div(N, kRows);
  // Aim for ~512 workgroups (2 per CU on 256 CUs) with at least one group
  // per wave in each split.
  int64_t splits = std::max<int64_t>(1, (512 + p.row_tiles / 2) / p.row_tiles);
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, G / kWaves));
  int64_t gps = ceil_div(G, splits);
  // groups per wave-block: keep U dividing the per-wave share when possible
  int unroll = 4;
  while (unroll > 1 && (gps < kWaves * unroll || G % unroll)) unroll >>= 1;
  gps = ceil_div(gps, unroll) * unroll;
  splits = ceil_div(G, gps);
  p.unroll = unroll;
  if (p.row_tiles > kMaxRowTiles) {  // too many tiles for the ticket area: no split
    splits = 1;
    gps = G;
  }
  p.splits = splits;
  p.groups_per_split = gps;
  p.partial_bytes = splits > 1 ? static_cast<size_t>(splits * M * N) * sizeof(float) : 0;
  (void)bits;
  return p;
}

int launch_qmv(const QmvPlan& p, const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s,
               const uint16_t* b, const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
               void* workspace, hipStream_t st) {
  // workspace layout: [tickets: kTicketBytes] [partials f32]
  uint32_t* tickets = static_cast<uint32_t*>(workspace);
  float* partial = p.splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kTicketBytes) : nullptr;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  if (bits == 4) {
    if (group_size == 32) launch_mt<4, 32>(p, x, m, wq, s, b, bias, n, k, y, partial, tickets, st);
    else if (group_size == 64) launch_mt<4, 64>(p, x, m, wq, s, b, bias, n, k, y, partial, tickets, st);
    else launch_mt<4, 128>(p, x, m, wq, s, b, bias, n, k, y, partial, tickets, st);
  } else {
    if (group_size == 32) launch_mt<8, 32>(p, x, m, wq, s, b, bias, n, k, y, partial, tickets, st);
    else if (group_size == 64) launch_mt<8, 64>(p, x, m, wq, s, b, bias, n, k, y, partial, tickets, st);
    else launch_mt<8, 128>(p, x, m, wq, s, b, bias, n, k, y, partial, tickets, st);
  }
  return check_launch("qmv");
}

}  // namespace mlxq
