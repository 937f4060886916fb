// Decode-shaped quantized matmul (qmv) for gfx950: y[M,N] = x[M,K] . W^T with
// W group-wise affine quantized (Q4 / Q8), M <= 32.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul(x, w, scales, biases, transpose=true, g, bits),
// which MLX serves with its qmv kernels for small M.
//
// Design (HBM-bound: the packed weights are read exactly once).  A decode
// GEMV of 2-60 MB lasts a few microseconds, so the kernel is built around
// memory latency as much as bandwidth: one round trip for the weights, one
// store for y, nothing in between.
//  * A workgroup of 8 wavefronts owns 16*SUB weight rows (SUB = 1, 2 or 4
//    MFMA sub-tiles, chosen per shape so the grid covers the 256 CUs) and the
//    whole K range.  Its waves take interleaved blocks of U consecutive
//    groups; all loads of a block are issued before any of them is used.
//  * The contraction runs on the matrix cores with v_mfma_f32_16x16x32_bf16:
//    A = activations (M padded to 16 rows per M-tile), B = 16 weight rows.
//    Q4 codes become bf16 (128 + q) with one and-or per pair of nibbles
//    (0x4300 | q is exactly 128 + q in bf16); Q8 codes are converted exactly
//    through f32.  A-operand activations are permuted with v_perm to the same
//    nibble order, so the products pair up correctly.
//  * Per group, the MFMA partial P = sum x*(OFF+q) is folded into f32
//    accumulators: acc += s*P + (b - OFF*s) * sum(x), with sum(x) produced by
//    one extra MFMA against an all-ones operand (shared by the 4 sub-tiles).
//  * The 8 waves reduce through LDS in a fixed order (deterministic results),
//    add the optional bias and store bf16 y.  No workspace is used.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include <string>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


constexpr int kWaves = 8;                // wavefronts per workgroup, splitting K
constexpr int kThreads = kWaves * 64;

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

// A operand for one MFMA step with per-lane byte selectors: the same v_perm
// that reorders the activations (Q4 nibble order) also zeroes the lanes that
// belong to another quantization group (selector byte 0x0C yields 0x00).
template <int BITS>
__device__ __forceinline__ bf16x8 acts_to_bf16_sel(const uint32_t* d, uint32_t sel_lo, uint32_t sel_hi) {
  u32x4 r;
  if constexpr (BITS == 4) {
    r[0] = __builtin_amdgcn_perm(d[2], d[0], sel_lo);
    r[1] = __builtin_amdgcn_perm(d[2], d[0], sel_hi);
    r[2] = __builtin_amdgcn_perm(d[3], d[1], sel_lo);
    r[3] = __builtin_amdgcn_perm(d[3], d[1], sel_hi);
  } else {
    r[0] = __builtin_amdgcn_perm(0u, d[0], sel_lo);
    r[1] = __builtin_amdgcn_perm(0u, d[1], sel_lo);
    r[2] = __builtin_amdgcn_perm(0u, d[2], sel_lo);
    r[3] = __builtin_amdgcn_perm(0u, d[3], sel_lo);
  }
  return as_bf16x8(r);
}

// Load U consecutive bf16 scales (or biases) starting at a U-aligned group.
template <int U>
__device__ __forceinline__ void load_group_params(const uint16_t* p, float (&v)[U]) {
  if constexpr (U == 16 || U == 8) {
#pragma unroll
    for (int i = 0; i < U; i += 8) {
      uint4 w = *reinterpret_cast<const uint4*>(p + i);
      uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        v[i + 2 * j] = bf16_bits_to_f32(ws[j] & 0xFFFFu);
        v[i + 2 * j + 1] = bf16_bits_to_f32(ws[j] >> 16);
      }
    }
  } else if constexpr (U == 4) {
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

// Per-wave state when every lane loads 8 bytes of codes per group (one group
// per 32-bit-word set): groups never straddle a load.  Used for any K; the
// unit of work is one quantization group.
template <int BITS, int GS, int MT, int SUB, int MV>
struct QmvWaveNarrow {
  static constexpr int T = GS / 32;      // MFMA steps per group
  static constexpr int WPS = BITS / 4;   // code words per lane per MFMA step
  static constexpr int WPG = T * WPS;    // code words per lane per group
  static constexpr int XW = GS / 8;      // activation words (bf16 pairs) per lane per group
  static constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  static constexpr int UNIT_ALIGN = 1;   // block starts must be multiples of this

  const uint32_t* wrow[SUB];
  const uint16_t* srow[SUB];
  const uint16_t* brow[SUB];
  const uint32_t* xrow[MT];
  f32x4 acc[SUB][MT];

  static __device__ __forceinline__ int units(int K) { return K / GS; }

  __device__ __forceinline__ void init(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* scales,
                                       const uint16_t* biases, int N, int K, int n0, int r16, int gq) {
    const int G = K / GS;
    const int64_t row_words = static_cast<int64_t>(K) * BITS / 32;
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      const int n = min(n0 + 16 * s + r16, N - 1);  // rows past N repeat row N-1 (results dropped)
      wrow[s] = wq + n * row_words + gq * WPG;
      srow[s] = scales + static_cast<int64_t>(n) * G;
      brow[s] = biases + static_cast<int64_t>(n) * G;
    }
    // activation rows past M load row 0; they only feed discarded outputs
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const int m = 16 * mt + r16;
      xrow[mt] = reinterpret_cast<const uint32_t*>(x + static_cast<int64_t>(m < M ? m : 0) * K) + gq * XW;
    }
#pragma unroll
    for (int s = 0; s < SUB; s++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) acc[s][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // U consecutive groups starting at g0 (U-aligned): every load is issued
  // before any use, with no divergent control flow, so they all overlap.
  template <int U>
  __device__ __forceinline__ void block(int g0) {
    uint32_t wb[U][SUB][WPG];
    uint32_t xa[U][MT][XW];
    float sv[SUB][U], bv[SUB][U];
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int s = 0; s < SUB; s++)
        load_words<WPG>(wrow[s] + static_cast<int64_t>(g0 + u) * (GS * BITS / 32), wb[u][s]);
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      load_group_params<U>(srow[s] + g0, sv[s]);
      load_group_params<U>(brow[s] + g0, bv[s]);
    }
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) load_words<XW>(xrow[mt] + static_cast<int64_t>(g0 + u) * (GS / 2), xa[u][mt]);
    // keep every load of the block ahead of the first use (no sinking)
    __builtin_amdgcn_sched_barrier(0);

    const bf16x8 ones = as_bf16x8(u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
#pragma unroll
    for (int u = 0; u < U; u++) {
      bf16x8 A[MT][T];
      f32x4 xs[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        xs[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < T; t++) {
          A[mt][t] = acts_to_bf16<BITS>(&xa[u][mt][4 * t]);
          xs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][t], ones, xs[mt], 0, 0, 0);
        }
      }
#pragma unroll
      for (int s = 0; s < SUB; s++) {
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
          for (int v = 0; v < MV; v++) acc[s][mt][v] = fmaf(sc, P[mt][v], fmaf(c, xs[mt][v], acc[s][mt][v]));
      }
    }
  }
};

// Per-wave state when every lane loads 16 bytes (the 64-byte chunk of a row
// is split over the 4 lane groups): one wave instruction reads 16 rows x 64
// contiguous bytes, which streams from HBM as fast as a plain copy.  A chunk
// can hold 1, 2 or 4 quantization groups (NGC) or be half of one (CPG = 2);
// MFMA partials must not mix groups, so with NGC > 1 the activation operand
// is masked to the lanes of one group and the MFMA is issued once per group.
// Needs K*bits/8 to be a multiple of 64 (the dispatcher checks).
template <int BITS, int GS, int MT, int SUB, int MV>
struct QmvWaveWide {
  static constexpr int GB = GS * BITS / 8;            // bytes per group per row
  static constexpr int NGC = GB >= 64 ? 1 : 64 / GB;  // groups per chunk
  static constexpr int CPG = GB >= 64 ? GB / 64 : 1;  // chunks per group
  static constexpr int KC = 64 * 8 / BITS;            // k per chunk
  static constexpr int KL = KC / 4;                   // k per lane per chunk
  static constexpr int STEPS = KL / 8;                // MFMA steps per chunk
  static constexpr int WPS = BITS / 4;                // code words per MFMA step
  static constexpr int XW = KL / 2;                   // activation words per lane per chunk
  static constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  static constexpr int UNIT_ALIGN = CPG;

  const uint4* wrow[SUB];
  const uint16_t* srow[SUB];
  const uint16_t* brow[SUB];
  const uint32_t* xrow[MT];
  uint32_t sel_lo[NGC], sel_hi[NGC];  // v_perm selectors: group j's lanes, others zeroed
  f32x4 acc[SUB][MT];

  static __device__ __forceinline__ int units(int K) { return K * BITS / 8 / 64; }

  __device__ __forceinline__ void init(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* scales,
                                       const uint16_t* biases, int N, int K, int n0, int r16, int gq) {
    const int G = K / GS;
    const int64_t row_u4 = static_cast<int64_t>(K) * BITS / 128;
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      const int n = min(n0 + 16 * s + r16, N - 1);
      wrow[s] = reinterpret_cast<const uint4*>(wq) + n * row_u4 + gq;
      srow[s] = scales + static_cast<int64_t>(n) * G;
      brow[s] = biases + static_cast<int64_t>(n) * G;
    }
    // Activation rows past M load row 0: they only feed output rows >= M,
    // which are never stored.
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const int m = 16 * mt + r16;
      xrow[mt] = reinterpret_cast<const uint32_t*>(x + static_cast<int64_t>(m < M ? m : 0) * K) + gq * XW;
    }
    const uint32_t lo = BITS == 4 ? 0x05040100u : 0x03020100u, hi = BITS == 4 ? 0x07060302u : 0x03020100u;
#pragma unroll
    for (int j = 0; j < NGC; j++) {
      const bool mine = NGC == 1 || gq * NGC / 4 == j;
      sel_lo[j] = mine ? lo : 0x0C0C0C0Cu;
      sel_hi[j] = mine ? hi : 0x0C0C0C0Cu;
    }
#pragma unroll
    for (int s = 0; s < SUB; s++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) acc[s][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // U chunks starting at chunk c0 (c0 and U multiples of CPG).
  template <int U>
  __device__ __forceinline__ void block(int c0) {
    constexpr int NG = U * NGC / CPG;  // groups in the block
    uint4 wb[U][SUB];
    uint32_t xa[U][MT][XW];
    float sv[SUB][NG], bv[SUB][NG];
    const int g0 = c0 * NGC / CPG;
    // Issue order = consumption order (vmcnt retires in order): activations
    // and scales first, then the code chunks, so the math on chunk 0 can
    // start while the later chunks are still in flight.
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
        load_words<XW>(xrow[mt] + static_cast<int64_t>(c0 + u) * (KC / 2), xa[u][mt]);
#pragma unroll
    for (int s = 0; s < SUB; s++) {
      load_group_params<NG>(srow[s] + g0, sv[s]);
      load_group_params<NG>(brow[s] + g0, bv[s]);
    }
    // Q4 codes non-temporal (read once; M = 4 q 6.2 -> 6.0 us, down 14.5 ->
    // 14.4); Q8 measured slower with it (q 7.2 -> 7.6, down 19.8 -> 21.9)
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int s = 0; s < SUB; s++) {
        if constexpr (BITS == 4) {
          const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[s] + static_cast<int64_t>(c0 + u) * 4));
          wb[u][s] = make_uint4(q[0], q[1], q[2], q[3]);
        } else {
          wb[u][s] = wrow[s][static_cast<int64_t>(c0 + u) * 4];
        }
      }
    __builtin_amdgcn_sched_barrier(0);

    const bf16x8 ones = as_bf16x8(u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    f32x4 P[SUB][NGC][MT], xs[NGC][MT];
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (u % CPG == 0) {
#pragma unroll
        for (int j = 0; j < NGC; j++)
#pragma unroll
          for (int mt = 0; mt < MT; mt++) {
            xs[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < SUB; s++) P[s][j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      }
      uint32_t w[SUB][4];
#pragma unroll
      for (int s = 0; s < SUB; s++) {
        w[s][0] = wb[u][s].x; w[s][1] = wb[u][s].y; w[s][2] = wb[u][s].z; w[s][3] = wb[u][s].w;
      }
#pragma unroll
      for (int t = 0; t < STEPS; t++) {
        bf16x8 A[NGC][MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
          for (int j = 0; j < NGC; j++) {
            if constexpr (NGC == 1) A[j][mt] = acts_to_bf16<BITS>(&xa[u][mt][4 * t]);
            else A[j][mt] = acts_to_bf16_sel<BITS>(&xa[u][mt][4 * t], sel_lo[j], sel_hi[j]);
            xs[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j][mt], ones, xs[j][mt], 0, 0, 0);
          }
        }
#pragma unroll
        for (int s = 0; s < SUB; s++) {
          const bf16x8 B = weights_to_bf16<BITS>(&w[s][t * WPS]);
#pragma unroll
          for (int j = 0; j < NGC; j++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
              P[s][j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j][mt], B, P[s][j][mt], 0, 0, 0);
        }
      }
      if (u % CPG == CPG - 1) {
#pragma unroll
        for (int j = 0; j < NGC; j++) {
          const int gi = (u / CPG) * NGC + j;  // group index within the block
#pragma unroll
          for (int s = 0; s < SUB; s++) {
            const float sc = sv[s][gi];
            const float c = bv[s][gi] - OFF * sc;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
              for (int v = 0; v < MV; v++)  // rows 4*gq + v; only v < MV can be < M
                acc[s][mt][v] = fmaf(sc, P[s][j][mt][v], fmaf(c, xs[j][mt][v], acc[s][mt][v]));
          }
        }
      }
    }
  }
};

template <template <int, int, int, int, int> class WAVE, int BITS, int GS, int MT, int SUB, int MV, int U>
__global__ __launch_bounds__(kThreads) void qmv_kernel(const uint16_t* __restrict__ x, int M,
                                                        const uint32_t* __restrict__ wq,
                                                        const uint16_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ biases,
                                                        const uint16_t* __restrict__ bias_vec, int N, int K,
                                                        uint16_t* __restrict__ y) {
  using W = WAVE<BITS, GS, MT, SUB, MV>;
  constexpr int R = 16 * SUB;  // weight rows per workgroup
  __shared__ float red[kWaves][MT * 16][R];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, gq = lane >> 4;
  const int n0 = blockIdx.x * R;

  W w;
  w.init(x, M, wq, scales, biases, N, K, n0, r16, gq);
  // whole U-unit blocks interleaved over the waves, then the tail in the
  // smallest aligned steps
  const int units = W::units(K);
  int u0 = wave * U;
  for (; u0 + U <= units; u0 += kWaves * U) w.template block<U>(u0);
  if constexpr (U > W::UNIT_ALIGN) {
    for (int u = u0; u < min(u0 + U, units); u += W::UNIT_ALIGN) w.template block<W::UNIT_ALIGN>(u);
  }

  // C layout of a 16x16 MFMA tile: lane holds column (weight row) r16 and
  // activation rows 4*gq + v.
#pragma unroll
  for (int s = 0; s < SUB; s++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++) red[wave][16 * mt + 4 * gq + v][16 * s + r16] = w.acc[s][mt][v];
  __syncthreads();

  for (int i = tid; i < M * R; i += kThreads) {
    const int m = i / R, r = i % R, n = n0 + r;
    if (n >= N) continue;
    float sum = red[0][m][r];
#pragma unroll
    for (int wv = 1; wv < kWaves; wv++) sum += red[wv][m][r];
    if (bias_vec) sum += bf16_bits_to_f32(bias_vec[n]);
    y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
  }
}

template <int BITS, int GS, int MT, int SUB>
void launch_narrow(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s,
                   const uint16_t* b, const uint16_t* bias, int N, int K, uint16_t* y, hipStream_t st) {
  dim3 grid(p.row_tiles);
  switch (p.unroll) {
    case 1: MLXQ_LAUNCH((qmv_kernel<QmvWaveNarrow, BITS, GS, MT, SUB, 4, 1>), grid, dim3(kThreads), 0, st, x, M, wq, s, b, bias, N, K, y); break;
    case 2: MLXQ_LAUNCH((qmv_kernel<QmvWaveNarrow, BITS, GS, MT, SUB, 4, 2>), grid, dim3(kThreads), 0, st, x, M, wq, s, b, bias, N, K, y); break;
    default: MLXQ_LAUNCH((qmv_kernel<QmvWaveNarrow, BITS, GS, MT, SUB, 4, 4>), grid, dim3(kThreads), 0, st, x, M, wq, s, b, bias, N, K, y); break;
  }
}

template <int BITS, int GS, int MT, int SUB, int MV>
void launch_wide(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                 const uint16_t* bias, int N, int K, uint16_t* y, hipStream_t st) {
  // blocks of 4 chunks (256 bytes of codes per row); 2 for 128-byte groups
  // and where 4 chunks of Q4 activations would not fit in registers
  constexpr int U = (QmvWaveWide<BITS, GS, MT, SUB, MV>::CPG == 2 ||
                     (BITS == 4 && (MT == 2 || SUB >= 2 || GS == 32))) ? 2 : 4;
  static_assert(SUB <= 2, "wide qmv: at most 2 sub-tiles");
  MLXQ_LAUNCH((qmv_kernel<QmvWaveWide, BITS, GS, MT, SUB, MV, U>), dim3(p.row_tiles), dim3(kThreads), 0, st, x,
                     M, wq, s, b, bias, N, K, y);
}

template <int BITS, int GS, int MT, int SUB>
void launch_u(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
              const uint16_t* bias, int N, int K, uint16_t* y, hipStream_t st) {
  if (!p.wide) {
    launch_narrow<BITS, GS, MT, SUB>(p, x, M, wq, s, b, bias, N, K, y, st);
  } else if (MT == 1 && M == 1) {
    launch_wide<BITS, GS, MT, SUB, 1>(p, x, M, wq, s, b, bias, N, K, y, st);
  } else if (MT == 1 && M == 2) {
    launch_wide<BITS, GS, MT, SUB, 2>(p, x, M, wq, s, b, bias, N, K, y, st);
  } else {
    launch_wide<BITS, GS, MT, SUB, 4>(p, x, M, wq, s, b, bias, N, K, y, st);
  }
}

template <int BITS, int GS, int MT>
void launch_sub(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                const uint16_t* bias, int N, int K, uint16_t* y, hipStream_t st) {
  switch (p.sub) {
    case 1: launch_u<BITS, GS, MT, 1>(p, x, M, wq, s, b, bias, N, K, y, st); break;
    case 2: launch_u<BITS, GS, MT, 2>(p, x, M, wq, s, b, bias, N, K, y, st); break;
    default: launch_narrow<BITS, GS, MT, 4>(p, x, M, wq, s, b, bias, N, K, y, st); break;
  }
}

template <int BITS, int GS>
void launch_mt(const QmvPlan& p, const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int N, int K, uint16_t* y, hipStream_t st) {
  if (M <= 16) launch_sub<BITS, GS, 1>(p, x, M, wq, s, b, bias, N, K, y, st);
  else launch_sub<BITS, GS, 2>(p, x, M, wq, s, b, bias, N, K, y, st);
}

}  // namespace

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  QmvPlan p{};
  const int64_t G = K / group_size;
  // Rows per workgroup: the largest of 64 / 32 / 16 that still gives every CU
  // a workgroup (more rows per workgroup = more reuse of each activation load).
  // Rows per workgroup (16 * sub): keep every wave of the grid resident at
  // once (about two 8-wave workgroups per CU), since these kernels last a
  // few microseconds and a second round of workgroups would pay the memory
  // latency twice.
  int sub = 1;
  while (sub < 4 && ceil_div(N, 16 * sub) > 512) sub <<= 1;
  if (const int o = overrides().qmv_sub; o == 1 || o == 2 || o == 4) sub = o;
  p.sub = sub;
  p.row_tiles = ceil_div(N, 16 * sub);
  // 16-byte-per-lane loads need whole 64-byte chunks per row, and the
  // block's scales (U chunks' groups) aligned for one vector load.
  const int64_t row_bytes = K * bits / 8;
  const int64_t gb = static_cast<int64_t>(group_size) * bits / 8;
  const int64_t groups_per_block = gb >= 64 ? 4 * 64 / gb : 4 * 64 / gb;  // upper bound over U in {2, 4}
  if (sub > 2 && row_bytes % 64 == 0) sub = 2;  // the wide loader tops out at 2 sub-tiles
  p.sub = sub;
  p.row_tiles = ceil_div(N, 16 * sub);
  p.wide = sub <= 2 && row_bytes % 64 == 0 && G % std::max<int64_t>(1, groups_per_block) == 0 &&
           !overrides().qmv_narrow;
  int unroll = 4;
  while (unroll > 1 && G % unroll) unroll >>= 1;
  p.unroll = unroll;
  (void)M;
  (void)bits;
  return p;
}

int launch_qmv(const QmvPlan& p, const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s,
               const uint16_t* b, const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
               hipStream_t st) {
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  if (bits == 4) {
    if (group_size == 32) launch_mt<4, 32>(p, x, m, wq, s, b, bias, n, k, y, st);
    else if (group_size == 64) launch_mt<4, 64>(p, x, m, wq, s, b, bias, n, k, y, st);
    else launch_mt<4, 128>(p, x, m, wq, s, b, bias, n, k, y, st);
  } else {
    if (group_size == 32) launch_mt<8, 32>(p, x, m, wq, s, b, bias, n, k, y, st);
    else if (group_size == 64) launch_mt<8, 64>(p, x, m, wq, s, b, bias, n, k, y, st);
    else launch_mt<8, 128>(p, x, m, wq, s, b, bias, n, k, y, st);
  }
  return check_launch("qmv");
}

}  // namespace mlxq
