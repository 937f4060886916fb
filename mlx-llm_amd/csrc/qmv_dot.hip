// Decode GEMV for M <= 4 activation rows on the vector ALUs (gfx950).
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
//    the activations.  Q4 codes become bf16 (128 + q) pairs with one and-or
//    per pair; Q8 codes are converted exactly through f32.
//  * The activations are staged once per workgroup in LDS -- already in the
//    pair order of the Q4 unpack -- together with their sum over every lane
//    segment, so a segment's result is s * dot + (b - 128 s) * sum(x).  A
//    lane segment never straddles a quantization group (32 or 16 codes vs
//    groups of 32..128), so no masking is needed.
//  * One memory round trip: each thread first requests its activation
//    pieces, then the codes and group parameters of its wave's first two
//    rounds (a wave owns a contiguous range of 64-byte chunks, taken 4 at a
//    time); the activation wait therefore never waits for the weights.  Each
//    later round is requested before the previous one is computed.
//  * Lanes reduce over gq with cross-lane adds, waves through LDS in fixed
//    order (deterministic), then bf16 y (+ bias) is stored.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxWaves = 8;  // waves per workgroup: 4 or 8 (chosen per shape)

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
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
// WV: waves per workgroup.
template <int BITS, int GS, int MV, int SUB, int RC, int PT, int WV>
__global__ __launch_bounds__(64 * WV) void qmv_dot_kernel(const uint16_t* __restrict__ x,
                                                            const uint32_t* __restrict__ wq,
                                                            const uint16_t* __restrict__ scales,
                                                            const uint16_t* __restrict__ biases,
                                                            const uint16_t* __restrict__ bias_vec, int N, int K,
                                                            int cw, uint16_t* __restrict__ y) {
  using Gm = DotGeom<BITS, GS, RC>;
  using Rnd = DotRound<BITS, GS, SUB, RC>;
  constexpr int R = 16 * SUB;
  constexpr int SEGP = Gm::KL / 8;  // pieces per segment
  constexpr float OFF = BITS == 4 ? 128.f : 0.f;
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem);                   // [MV][K] bf16 (pair order)
  float* xsum = reinterpret_cast<float*>(smem + MV * K * 2);           // [MV][K / KL]
  float* red = xsum + MV * (K / Gm::KL);                               // [WV][MV][R]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches below
  const int r16 = lane & 15, gq = lane >> 4;
  const int n0 = blockIdx.x * R;
  const int G = K / GS;
  const int chunks = K * BITS / 8 / 64;
  const int64_t row_u4 = static_cast<int64_t>(K) * BITS / 128;

  // 1) activation pieces of this thread: issued first so that waiting for
  //    them never waits for the (later, slower) weight loads
  const int pieces = MV * K / 8;
  uint4 xp[PT];
#pragma unroll
  for (int j = 0; j < PT; j++) {  // clamped, unconditional: no branch, no early wait
    xp[j] = reinterpret_cast<const uint4*>(x)[min(tid * PT + j, pieces - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first

  // 2) codes and parameters of the wave's first round
  const uint4* wrow[SUB];
  const uint16_t* srow[SUB];
  const uint16_t* brow[SUB];
#pragma unroll
  for (int s = 0; s < SUB; s++) {
    const int n = min(n0 + 16 * s + r16, N - 1);  // rows past N repeat row N-1 (results dropped)
    wrow[s] = reinterpret_cast<const uint4*>(wq) + n * row_u4 + gq;
    srow[s] = scales + static_cast<int64_t>(n) * G;
    brow[s] = biases + static_cast<int64_t>(n) * G;
  }
  // The wave's chunk range [cbeg, cend) lies inside the row; its full rounds
  // end at cfull.  A round is fetched only when it ends at or before cfull,
  // so every load stays inside the row.  A wave whose range holds no full
  // round fetches none (the branches on cfull are wave-uniform).  Inside
  // fetch all register indices are compile-time, so a round stays in
  // registers.
  const int cbeg = min(wave * cw, chunks), cend = min(chunks, cbeg + cw);
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
  if (cfull > cbeg) fetch(cur, cbeg);
  __builtin_amdgcn_sched_barrier(0);  // the whole first round is in flight before the prologue

  // 3) activations -> LDS in the Q4 pair order, plus per-segment sums
  float segsum = 0.f;
#pragma unroll
  for (int j = 0; j < PT; j++) {
    const int i = tid * PT + j;
    uint4 v = xp[j];
    if constexpr (BITS == 4) {  // (x0,x1),(x2,x3),(x4,x5),(x6,x7) -> (x0,x4),(x1,x5),(x2,x6),(x3,x7)
      uint4 p;
      p.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
      p.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
      p.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
      p.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
      v = p;
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
        uint32_t p[4];
        if constexpr (BITS == 4) {
          const uint32_t q = wv[t];
          p[0] = (q & 0x000F000Fu) | 0x43004300u;
          p[1] = ((q >> 4) & 0x000F000Fu) | 0x43004300u;
          p[2] = ((q >> 8) & 0x000F000Fu) | 0x43004300u;
          p[3] = ((q >> 12) & 0x000F000Fu) | 0x43004300u;
        } else {
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const uint32_t q = wv[2 * t + h];
            const float f0 = static_cast<float>(q & 0xFFu), f1 = static_cast<float>((q >> 8) & 0xFFu);
            const float f2 = static_cast<float>((q >> 16) & 0xFFu), f3 = static_cast<float>(q >> 24);
            p[2 * h] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
            p[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
          }
        }
#pragma unroll
        for (int m = 0; m < MV; m++)
          dots[s][m] = dot2(p[3], xv[m][3], dot2(p[2], xv[m][2], dot2(p[1], xv[m][1], dot2(p[0], xv[m][0], dots[s][m]))));
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
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (gq == 0) red[(wave * MV + m) * R + 16 * s + r16] = v;
    }
  __syncthreads();
  for (int i = tid; i < MV * R; i += 64 * WV) {
    const int m = i / R, r = i % R, n = n0 + r;
    if (n >= N) continue;
    float sum = red[m * R + r];
#pragma unroll
    for (int wv = 1; wv < WV; wv++) sum += red[(wv * MV + m) * R + r];
    if (bias_vec) sum += bf16_bits_to_f32(bias_vec[n]);
    y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(sum));
  }
}

constexpr int kRound = 4;  // chunks per round

// Pieces (8 activations) per thread in the prologue: whole segments.
int prologue_pieces(int64_t M, int64_t K, int bits, int wv) {
  const int64_t segp = 64 * 8 / bits / 4 / 8;
  int64_t pt = ceil_div(M * K / 8, 64 * wv);
  pt = ceil_div(std::max<int64_t>(pt, segp), segp) * segp;
  return static_cast<int>(pt);
}

struct DotArgs {
  const uint16_t* x;
  const uint32_t* wq;
  const uint16_t *s, *b, *bias;
  int N, K;
  uint16_t* y;
  hipStream_t st;
};

struct DotCfg {
  int sub = 1, wv = 8, pt = 0, cw = 0;
  int64_t tiles = 0;
  size_t lds = 0;
};

// query: report resident workgroups per CU for this configuration instead of
// launching (the choice between configurations needs it).
template <int BITS, int GS, int MV, int SUB, int PT, int WV>
int run(const DotCfg& c, const DotArgs& a, int* query) {
  auto kern = qmv_dot_kernel<BITS, GS, MV, SUB, kRound, PT, WV>;
  static bool raised = false;  // once per process; the attribute is per function
  if (c.lds > 64 * 1024 && !raised) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmv_dot: LDS size: ") + hipGetErrorString(e));
    raised = true;
  }
  if (query) {
    static int cached = -1;  // the kernel's registers fix it; LDS is checked per call below
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
  hipLaunchKernelGGL(kern, dim3(c.tiles), dim3(64 * WV), c.lds, a.st, a.x, a.wq, a.s, a.b, a.bias, a.N, a.K, c.cw, a.y);
  return check_launch("qmv_dot");
}

template <int BITS, int GS, int MV, int SUB, int WV>
int run_pt(const DotCfg& c, const DotArgs& a, int* q) {
  constexpr int SEGP = 64 * 8 / BITS / 4 / 8;
  if (c.pt <= SEGP) return run<BITS, GS, MV, SUB, SEGP, WV>(c, a, q);
  if (c.pt <= 2 * SEGP) return run<BITS, GS, MV, SUB, 2 * SEGP, WV>(c, a, q);
  if constexpr (4 * SEGP <= 8) {
    if (c.pt <= 4 * SEGP) return run<BITS, GS, MV, SUB, 4 * SEGP, WV>(c, a, q);
  }
  return fail(MLXQ_ERR_INVALID, "qmv_dot: activation prologue too large");
}

template <int BITS, int GS, int SUB, int WV>
int run_m(int64_t M, const DotCfg& c, const DotArgs& a, int* q) {
  switch (M) {
    case 1: return run_pt<BITS, GS, 1, SUB, WV>(c, a, q);
    case 2: return run_pt<BITS, GS, 2, SUB, WV>(c, a, q);
    case 3: return run_pt<BITS, GS, 3, SUB, WV>(c, a, q);
    default: return run_pt<BITS, GS, 4, SUB, WV>(c, a, q);
  }
}

template <int BITS, int GS>
int run_cfg(int64_t M, const DotCfg& c, const DotArgs& a, int* q) {
  if (c.sub == 1) return c.wv == 4 ? run_m<BITS, GS, 1, 4>(M, c, a, q) : run_m<BITS, GS, 1, 8>(M, c, a, q);
  return c.wv == 4 ? run_m<BITS, GS, 2, 4>(M, c, a, q) : run_m<BITS, GS, 2, 8>(M, c, a, q);
}

int dispatch(int64_t M, int group_size, int bits, const DotCfg& c, const DotArgs& a, int* q) {
  if (bits == 4) {
    if (group_size == 32) return run_cfg<4, 32>(M, c, a, q);
    if (group_size == 64) return run_cfg<4, 64>(M, c, a, q);
    return run_cfg<4, 128>(M, c, a, q);
  }
  if (group_size == 32) return run_cfg<8, 32>(M, c, a, q);
  if (group_size == 64) return run_cfg<8, 64>(M, c, a, q);
  return run_cfg<8, 128>(M, c, a, q);
}

size_t lds_bytes(int64_t M, int64_t K, int bits, int sub, int wv) {
  const int64_t kl = 64 * 8 / bits / 4;
  return static_cast<size_t>(M * K * 2 + M * (K / kl) * 4 + wv * M * 16 * sub * 4);
}

DotCfg make_cfg(int64_t M, int64_t N, int64_t K, int bits, int sub, int wv) {
  DotCfg c;
  c.sub = sub;
  c.wv = wv;
  c.pt = prologue_pieces(M, K, bits, wv);
  c.tiles = ceil_div(N, 16 * sub);
  c.lds = lds_bytes(M, K, bits, sub, wv);
  // each wave owns a contiguous range of whole rounds of chunks
  const int64_t chunks = K * bits / 8 / 64;
  c.cw = static_cast<int>(ceil_div(ceil_div(chunks, wv), kRound) * kRound);
  return c;
}

bool cfg_ok(const DotCfg& c) { return c.pt <= 8 && c.lds <= 160 * 1024; }

int cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

}  // namespace

size_t qmv_dot_lds_bytes(int64_t M, int64_t K, int bits, int sub) { return lds_bytes(M, K, bits, sub, kMaxWaves); }

bool qmv_dot_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M < 1 || M > kQmvDotMaxM) return false;
  if ((K * bits / 8) % 64) return false;  // whole 64-byte chunks per row
  const int64_t gb = static_cast<int64_t>(group_size) * bits / 8;
  const int64_t ngr = kRound * (gb >= 64 ? 1 : 64 / gb) / (gb > 64 ? gb / 64 : 1);  // groups per round
  if ((K / group_size) % std::min<int64_t>(ngr, 8)) return false;  // aligned vector loads of round params
  return cfg_ok(make_cfg(M, N, K, bits, 2, kMaxWaves));             // activations staged through registers
}

int launch_qmv_dot(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   hipStream_t st) {
  const DotArgs a{x, wq, s, b, bias, static_cast<int>(N), static_cast<int>(K), y, st};
  // Pick rows per workgroup (16 or 32) and waves per workgroup (4 or 8) so
  // that the whole grid is resident at once (no second, partly filled pass
  // of workgroups), preferring the most waves in flight.
  static const int cus = cu_count();
  DotCfg best;
  int64_t best_pass = -1, best_waves = 0;
  int forced_sub = 0, forced_wv = 0;
  if (const char* e = getenv("MLXQ_QMV_DOT")) sscanf(e, "%d,%d", &forced_sub, &forced_wv);
  for (int sub = 1; sub <= 2; sub++)
    for (int wv = 4; wv <= 8; wv += 4) {
      if ((forced_sub && sub != forced_sub) || (forced_wv && wv != forced_wv)) continue;
      const DotCfg c = make_cfg(M, N, K, bits, sub, wv);
      if (!cfg_ok(c)) continue;
      int nb = 0;
      if (int rc = dispatch(M, group_size, bits, c, a, &nb)) return rc;
      const int64_t slots = std::max<int64_t>(1, static_cast<int64_t>(nb) * cus);
      const int64_t pass = ceil_div(c.tiles, slots);
      const int64_t waves = std::min(c.tiles, slots) * wv;
      if (best_pass < 0 || pass < best_pass || (pass == best_pass && waves > best_waves)) {
        best = c;
        best_pass = pass;
        best_waves = waves;
      }
    }
  if (best_pass < 0) return fail(MLXQ_ERR_INVALID, "qmv_dot: no configuration fits this shape");
  return dispatch(M, group_size, bits, best, a, nullptr);
}

}  // namespace mlxq
