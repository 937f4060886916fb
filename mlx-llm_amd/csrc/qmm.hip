// Prefill-shaped quantized matmul (qmm) for gfx950: y[M,N] = x[M,K] . W^T,
// W group-wise affine quantized (Q4 / Q8), any M.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul, which MLX serves with its qmm kernels when M
// is large (prefill, batched decode).
//
// Design (MFMA-bound):
//  * Workgroup tile BM x BN, K step 64, WM x WN wavefronts each owning
//    (BM/WM) x (BN/WN) of the output as tiles of v_mfma_f32_32x32x16_bf16
//    with f32 accumulators.  256 x 256 tiles of 8 wavefronts (2 per SIMD) or
//    128 x 128 tiles of 4 (two workgroups per CU), chosen from the grid size.
//  * One or two threads own each weight row of the tile per K step: they load
//    the row's 64 codes and scale/bias, dequantize them once for the whole
//    workgroup (codes -> f32 -> scale*q + bias -> bf16, round to nearest
//    even: the values MLX's qmm places in threadgroup memory) and write them
//    to LDS.  Activations are copied to LDS as they are.
//  * Latency: two LDS stages and two register stages.  The global loads of
//    K step k+2 are issued before the MFMAs of step k; step k+1, already in
//    registers, is written to the other LDS stage after them; one barrier per
//    step.  Rows are padded to 72 bf16 so the 16-byte fragment reads of 16
//    consecutive rows hit distinct banks.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include <string>
#include <type_traits>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;
constexpr int LDR = BK + 8;  // padded LDS row, bf16 elements

// Tile BM x BN, WM x WN wavefronts (each (BM/WM) x (BN/WN) of the output)
// in MF x MF MFMA tiles (32: v_mfma_f32_32x32x16_bf16, 16:
// v_mfma_f32_16x16x32_bf16).
template <int BM, int BN, int WM, int WN, int BITS, int MF>
struct QmmGeom {
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int PARTS = THREADS >= 2 * BN ? 2 : 1;  // threads per weight row
  // rows the weight loader covers: BN, or more when BN does not divide the
  // threads (the extra rows repeat clamped weights into spare LDS rows, so
  // no thread branches around its loads)
  static constexpr int LROWS = THREADS / PARTS;
  static constexpr int STAGE = (BM + LROWS) * LDR;         // bf16 per LDS stage
  static constexpr int LDS_BYTES = 2 * STAGE * 2;          // two stages
  static constexpr int TM = BM / WM / MF;                  // MFMA row tiles per wave
  static constexpr int TN = BN / WN / MF;                  // MFMA column tiles per wave
  static constexpr int NV = MF * MF / 64;                  // accumulator floats per lane per tile
  static constexpr int KS = 512 / MF;                      // k per MFMA
  static constexpr int AU4 = BM * 8 / THREADS;             // activation uint4 per thread per step
  static constexpr int CPT = BK / PARTS;                   // codes per thread per step
  static constexpr int BU4 = CPT * BITS / 128;             // code uint4 per thread per step
  static_assert(MF == 16 || MF == 32, "MFMA shape");
  static_assert(LROWS >= BN && THREADS % PARTS == 0, "weight rows map onto threads");
  static_assert((BM / WM) % MF == 0 && (BN / WN) % MF == 0, "wave tiles are whole MFMA tiles");
  static_assert(BM * 8 % THREADS == 0, "activation chunks map onto threads");
  static_assert(LDS_BYTES <= 160 * 1024, "two stages fit in LDS");
};

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(a);  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

// One K step of global data held in registers by one thread.
template <typename Gm, int NSG>
struct Stage {
  u32x4 a[Gm::AU4];  // native vectors (not uint4 structs) so the stage stays in registers
  u32x4 b[Gm::BU4];
  // scale/bias bits of the thread's codes (two groups only for g32 with 64
  // codes).  Kept as loaded: converting at load time would make the
  // compiler wait for these loads -- and, since loads retire in order, for
  // the whole step's loads -- right after issuing them.
  uint16_t s[NSG], z[NSG];
};

template <int BITS, int GS, int BM, int BN, int WM, int WN, int MF, int PP>
__global__ __launch_bounds__(64 * WM * WN, 1) void qmm_kernel(const uint16_t* __restrict__ x, int M,
                                                               const uint32_t* __restrict__ wq,
                                                               const uint16_t* __restrict__ scales,
                                                               const uint16_t* __restrict__ biases,
                                                               const uint16_t* __restrict__ bias_vec, int N, int K,
                                                               uint16_t* __restrict__ y, float* __restrict__ part,
                                                               int k_len) {
  using Gm = QmmGeom<BM, BN, WM, WN, BITS, MF>;
  using AccT = std::conditional_t<MF == 32, f32x16, f32x4>;
  static_assert(!PP || (WM == 4 && WN == 2 && BM == 256), "ping-pong: two groups of four waves");
  // scale/bias groups per thread per step: two only for g32 with 64 codes
  constexpr int NSG = (GS == 32 && Gm::CPT == 64) ? 2 : 1;
  using St = Stage<Gm, NSG>;
  constexpr int T = Gm::THREADS;
  extern __shared__ __align__(16) uint16_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  // split K: slice blockIdx.z covers k_len codes from k_base (k_len = K unsplit)
  const int k_base = blockIdx.z * k_len;
  const int KT = k_len / BK;
  const int G = K / GS;
  const int64_t row_words = static_cast<int64_t>(K) * BITS / 32;

  // activation loader: 8 threads per row (16 B each), rows tid/8 + (T/8) i;
  // ping-pong: each half of the threads loads the rows its own waves
  // multiply (half h: rows 128 h + (tid % 256)/8 + 32 i)
  const int a_chunk = tid & 7;
  const int a_row0 = PP != 0 ? (tid >> 8) * (BM / 2) + ((tid & (T / 2 - 1)) >> 3) : (tid >> 3);
  constexpr int A_STRIDE = PP != 0 ? T / 16 : T / 8;
  const u32x4* a_src = reinterpret_cast<const u32x4*>(x) + a_chunk;
  int a_off[Gm::AU4];  // uint4 offset of each row (rows past M repeat row M-1; results dropped)
#pragma unroll
  for (int i = 0; i < Gm::AU4; i++) a_off[i] = min(m0 + a_row0 + A_STRIDE * i, M - 1) * (K / 8);
  // weight loader: PARTS threads per row, each CPT consecutive codes
  const int b_row = tid / Gm::PARTS, b_part = tid % Gm::PARTS;
  const int b_n = min(n0 + b_row, N - 1);
  const u32x4* b_src = reinterpret_cast<const u32x4*>(wq + b_n * row_words) + b_part * Gm::BU4;
  const uint16_t* s_src = scales + static_cast<int64_t>(b_n) * G;
  const uint16_t* z_src = biases + static_cast<int64_t>(b_n) * G;

  auto load_a = [&](St& r, int kt) __attribute__((always_inline)) {
    const int k0 = k_base + kt * BK;
#pragma unroll
    for (int i = 0; i < Gm::AU4; i++) r.a[i] = a_src[a_off[i] + k0 / 8];
  };
  auto load_b = [&](St& r, int kt) __attribute__((always_inline)) {
    const int k0 = k_base + kt * BK;
#pragma unroll
    for (int i = 0; i < Gm::BU4; i++) r.b[i] = b_src[k0 * BITS / 128 + i];
    const int kc = k0 + b_part * Gm::CPT;  // first code of this thread
#pragma unroll
    for (int g = 0; g < NSG; g++) {
      r.s[g] = s_src[kc / GS + g];
      r.z[g] = z_src[kc / GS + g];
    }
  };
  auto load = [&](St& r, int kt) __attribute__((always_inline)) {
    load_a(r, kt);
    load_b(r, kt);
  };

  // activations from ra, weights from r (the same stage)
  auto store2 = [&](const St& ra, const St& r, int stage) __attribute__((always_inline)) {
    uint16_t* sa = lds + stage * Gm::STAGE;
    uint16_t* sb = sa + BM * LDR;
#pragma unroll
    for (int i = 0; i < Gm::AU4; i++)
      *reinterpret_cast<u32x4*>(sa + (a_row0 + A_STRIDE * i) * LDR + a_chunk * 8) = ra.a[i];
    constexpr int NW = Gm::BU4 * 4;  // code words
    uint32_t w[NW];
#pragma unroll
    for (int i = 0; i < Gm::BU4; i++) {
      w[4 * i] = r.b[i][0]; w[4 * i + 1] = r.b[i][1]; w[4 * i + 2] = r.b[i][2]; w[4 * i + 3] = r.b[i][3];
    }
    uint32_t packed[Gm::CPT / 2];
    if constexpr (BITS == 4) {
#pragma unroll
      for (int wi = 0; wi < NW; wi++) {  // word wi: codes 8 wi .. 8 wi + 7
        const int g = NSG == 2 ? wi / 4 : 0;
        const float sc = bf16_bits_to_f32(r.s[g]), zz = bf16_bits_to_f32(r.z[g]);
        // even codes to the bytes of lo, odd codes to the bytes of hi: each
        // code is then one v_cvt_f32_ubyte
        uint32_t lo = w[wi] & 0x0F0F0F0Fu, hi = (w[wi] >> 4) & 0x0F0F0F0Fu;
        // opaque to the optimizer (an empty asm, no instruction): otherwise
        // it folds the masks back into one bit-field extract per code
        asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int j = 0; j < 4; j++)
          packed[4 * wi + j] = pack_bf16(sc * static_cast<float>((lo >> (8 * j)) & 0xFFu) + zz,
                                         sc * static_cast<float>((hi >> (8 * j)) & 0xFFu) + zz);
      }
    } else {
#pragma unroll
      for (int wi = 0; wi < NW; wi++) {  // word wi: codes 4 wi .. 4 wi + 3
        const int g = NSG == 2 ? wi / 8 : 0;
        const float sc = bf16_bits_to_f32(r.s[g]), zz = bf16_bits_to_f32(r.z[g]);
        const uint32_t q = w[wi];
        packed[2 * wi] = pack_bf16(sc * static_cast<float>(q & 0xFFu) + zz, sc * static_cast<float>((q >> 8) & 0xFFu) + zz);
        packed[2 * wi + 1] = pack_bf16(sc * static_cast<float>((q >> 16) & 0xFFu) + zz, sc * static_cast<float>(q >> 24) + zz);
      }
    }
    u32x4* dst = reinterpret_cast<u32x4*>(sb + b_row * LDR + b_part * Gm::CPT);
#pragma unroll
    for (int i = 0; i < Gm::CPT / 8; i++)
      dst[i] = u32x4{packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]};
  };
  auto store = [&](const St& r, int stage) __attribute__((always_inline)) { store2(r, r, stage); };

  AccT acc[Gm::TM][Gm::TN];
#pragma unroll
  for (int i = 0; i < Gm::TM; i++)
#pragma unroll
    for (int j = 0; j < Gm::TN; j++)
#pragma unroll
      for (int v = 0; v < Gm::NV; v++) acc[i][j][v] = 0.f;

  // A/B fragment of an MF x MF tile: lane holds row lane % MF and 8
  // consecutive k from (lane / MF) * 8
  const int frag_row = lane & (MF - 1);
  const int frag_k = (lane / MF) * 8;
  constexpr int WROWS = BM / WM, WCOLS = BN / WN;

  St r0, r1;
  load(r0, 0);
  load(r1, min(1, KT - 1));
  __builtin_amdgcn_sched_barrier(0);
  store(r0, 0);
  if constexpr ((PP & 8) != 0) load_b(r0, min(2, KT - 1));  // the weights run one step further ahead
  __syncthreads();
  // One K step: LDS stage kt&1 holds step kt, `ready` holds step kt+1 and
  // `target` receives step kt+2.  Called with (r0, r1) and (r1, r0) in turn
  // so that the register roles are static.
  auto step = [&](int kt, St& target, St& ready) __attribute__((always_inline)) {
    const int cur = kt & 1;
    // unconditional (past the end: the last step again, its lines are on
    // chip): a conditional load would make the compiler's memory-counter wait
    // before `store(ready)` drain every load in flight, this step's included
    load(target, min(kt + 2, KT - 1));
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t* sa = lds + cur * Gm::STAGE + (wm * WROWS + frag_row) * LDR + frag_k;
    const uint16_t* sb = lds + cur * Gm::STAGE + BM * LDR + (wn * WCOLS + frag_row) * LDR + frag_k;  // weights
#pragma unroll
    for (int ks = 0; ks < BK / Gm::KS; ks++) {
      bf16x8 a[Gm::TM], b[Gm::TN];
#pragma unroll
      for (int i = 0; i < Gm::TM; i++)
        a[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sa + MF * i * LDR + ks * Gm::KS));
#pragma unroll
      for (int j = 0; j < Gm::TN; j++)
        b[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sb + MF * j * LDR + ks * Gm::KS));
#pragma unroll
      for (int i = 0; i < Gm::TM; i++)
#pragma unroll
        for (int j = 0; j < Gm::TN; j++) {
          if constexpr (MF == 32)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < KT) store(ready, cur ^ 1);
    __syncthreads();
  };
  if constexpr (PP != 0) {
    // Ping-pong: waves 0-3 (group 0, output rows 0-127) and 4-7 (group 1,
    // rows 128-255) take turns between barriers.  While one group runs its
    // MFMAs on stage kt, the other writes its half of stage kt+1 (loaded two
    // phases earlier) and requests its half of stage kt+2; each SIMD (one
    // wave of each group) so has one wave on the matrix core and one on
    // the vector ALU and LDS.  Stage (kt+1)&1 was last read in the previous
    // step, which both groups have left.
    const int grp = __builtin_amdgcn_readfirstlane((PP & 3) == 1 ? wave >> 2 : wave & 1);
    auto mma = [&](int kt) __attribute__((always_inline)) {
      if constexpr ((PP & 4) != 0) __builtin_amdgcn_s_setprio(1);
      const int cur = kt & 1;
      const uint16_t* sa = lds + cur * Gm::STAGE + (wm * WROWS + frag_row) * LDR + frag_k;
      const uint16_t* sb = lds + cur * Gm::STAGE + BM * LDR + (wn * WCOLS + frag_row) * LDR + frag_k;
#pragma unroll
      for (int ks = 0; ks < BK / Gm::KS; ks++) {
        bf16x8 a[Gm::TM], b[Gm::TN];
#pragma unroll
        for (int i = 0; i < Gm::TM; i++)
          a[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sa + MF * i * LDR + ks * Gm::KS));
#pragma unroll
        for (int j = 0; j < Gm::TN; j++)
          b[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sb + MF * j * LDR + ks * Gm::KS));
#pragma unroll
        for (int i = 0; i < Gm::TM; i++)
#pragma unroll
          for (int j = 0; j < Gm::TN; j++) {
            if constexpr (MF == 32)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            else
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
          }
      }
      if constexpr ((PP & 4) != 0) __builtin_amdgcn_s_setprio(0);
    };
    // r1 holds this thread's part of stage 1; past the end a stage nobody
    // reads is written (unconditional: no branch around the loads)
    auto fill = [&](int kt) __attribute__((always_inline)) {
      store(r1, (kt + 1) & 1);
      load(r1, min(kt + 2, KT - 1));
    };
    // deep form (PP & 8, KT even): the weights of stage kt+1 alternate
    // between r1 and r0 and are requested three steps ahead, the
    // activations (mostly L2 hits) two
    auto fill_e = [&](int kt) __attribute__((always_inline)) {
      store2(r1, r1, (kt + 1) & 1);
      load_a(r1, min(kt + 2, KT - 1));
      load_b(r1, min(kt + 3, KT - 1));
    };
    auto fill_o = [&](int kt) __attribute__((always_inline)) {
      store2(r1, r0, (kt + 1) & 1);
      load_a(r1, min(kt + 2, KT - 1));
      load_b(r0, min(kt + 3, KT - 1));
    };
    // one loop per group (a wave-uniform branch): both run two barriers per
    // step, so the barriers pair up with the groups half a step apart
    if constexpr ((PP & 8) != 0) {
      if (grp == 0) {
        for (int kt = 0; kt < KT; kt += 2) {
          mma(kt);
          __syncthreads();
          fill_e(kt);
          __syncthreads();
          mma(kt + 1);
          __syncthreads();
          fill_o(kt + 1);
          __syncthreads();
        }
      } else {
        for (int kt = 0; kt < KT; kt += 2) {
          fill_e(kt);
          __syncthreads();
          mma(kt);
          __syncthreads();
          fill_o(kt + 1);
          __syncthreads();
          mma(kt + 1);
          __syncthreads();
        }
      }
    } else if (grp == 0) {
      for (int kt = 0; kt < KT; kt++) {
        mma(kt);
        __syncthreads();
        fill(kt);
        __syncthreads();
      }
    } else {
      for (int kt = 0; kt < KT; kt++) {
        fill(kt);
        __syncthreads();
        mma(kt);
        __syncthreads();
      }
    }
  } else {
    for (int kt = 0; kt < KT; kt += 2) {
      step(kt, r0, r1);
      if (kt + 1 < KT) step(kt + 1, r1, r0);
    }
  }

  // C layout of an MFMA tile: lane holds column lane % MF and, for 32x32,
  // rows 8*(v/4) + 4*(lane/32) + v%4; for 16x16, rows 4*(lane/16) + v.
  auto row_of = [&](int i, int v) {
    return m0 + wm * WROWS + MF * i +
           (MF == 32 ? 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3) : 4 * (lane >> 4) + v);
  };
  if (part) {  // split K: this slice's f32 partial sums, added by the reduce kernel
    float* dst = part + static_cast<int64_t>(blockIdx.z) * M * N;
#pragma unroll
    for (int j = 0; j < Gm::TN; j++) {
      const int n = n0 + wn * WCOLS + MF * j + (lane & (MF - 1));
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < Gm::TM; i++)
#pragma unroll
        for (int v = 0; v < Gm::NV; v++) {
          const int m = row_of(i, v);
          if (m < M) dst[static_cast<int64_t>(m) * N + n] = acc[i][j][v];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < Gm::TN; j++) {
    const int n = n0 + wn * WCOLS + MF * j + (lane & (MF - 1));
    if (n >= N) continue;
    const float bb = bias_vec ? bf16_bits_to_f32(bias_vec[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < Gm::TM; i++)
#pragma unroll
      for (int v = 0; v < Gm::NV; v++) {
        const int m = row_of(i, v);
        if (m < M) y[static_cast<int64_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_bits(acc[i][j][v] + bb));
      }
  }
}

template <int BITS, int GS, int BM, int BN, int WM, int WN, int MF = 32, int PP = 0>
int launch(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint16_t* bias,
           int N, int K, uint16_t* y, float* part, int splits, hipStream_t st) {
  using Gm = QmmGeom<BM, BN, WM, WN, BITS, MF>;
  auto kern = qmm_kernel<BITS, GS, BM, BN, WM, WN, MF, PP>;
  static bool attr_set = false;  // once per process; the attribute is per function
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       Gm::LDS_BYTES);
    if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmm: set LDS size: ") + hipGetErrorString(e));
    attr_set = true;
  }
  dim3 grid(ceil_div(N, BN), ceil_div(M, BM), splits);
  hipLaunchKernelGGL(kern, grid, dim3(Gm::THREADS), Gm::LDS_BYTES, st, x, M, wq, s, b, bias, N, K, y,
                     splits > 1 ? part : nullptr, K / splits);
  if (int rc = check_launch("qmm")) return rc;
  if (splits == 1) return MLXQ_OK;
  return launch_split_reduce(part, bias, y, M, N, splits, st);
}

int cu_count() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    return n;
  }();
  return cus;
}

template <int BITS, int GS>
int launch_cfg(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint16_t* bias,
               int N, int K, uint16_t* y, float* part, int splits, hipStream_t st) {
  // Configurations measured at the Llama-3-8B projection shapes for M from
  // 256 to 4096; MLXQ_QMM_CFG overrides (tuning).
  const int64_t tiles256 = ceil_div(N, 256) * ceil_div(M, 256);
  const int64_t cus = cu_count();
  // Ping-pong 256-row tiles (two groups of four waves take turns on the
  // matrix cores) when the grid fills the CUs or K is split; the deep form
  // (weights three K steps ahead) needs an even number of K steps.  For N a
  // multiple of 224 (gate/up: 14336 = 64 x 224) Q4 takes 256 x 224 tiles,
  // which make whole rounds of CUs where 256-wide ones leave a partial one.
  // Grids too small for either: 128 x 128 tiles, two workgroups per CU.
  const bool even_steps = (K / splits / BK) % 2 == 0;
  int cfg = 6;
  if (tiles256 * splits * 8 >= cus * 7) cfg = even_steps ? 14 : 9;
  if (BITS == 4 && splits == 1 && N % 224 == 0 && (N / 224) * ceil_div(M, 256) * 8 >= cus * 7)
    cfg = even_steps ? 15 : 10;
  if (overrides().qmm_cfg) cfg = overrides().qmm_cfg;
  switch (cfg) {
    case 1: return launch<BITS, GS, 256, 256, 2, 4>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 2: return launch<BITS, GS, 256, 128, 2, 2>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 3: return launch<BITS, GS, 128, 256, 2, 4>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 4: return launch<BITS, GS, 256, 256, 4, 2>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 6: return launch<BITS, GS, 128, 128, 2, 2>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 7: return launch<BITS, GS, 256, 224, 4, 2, 16>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 9: return launch<BITS, GS, 256, 256, 4, 2, 32, 1>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 10: return launch<BITS, GS, 256, 224, 4, 2, 16, 1>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 14: return launch<BITS, GS, 256, 256, 4, 2, 32, 9>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    case 15: return launch<BITS, GS, 256, 224, 4, 2, 16, 9>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
    default: return launch<BITS, GS, 128, 256, 2, 2>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
  }
}

}  // namespace

int qmm_split_k(int64_t M, int64_t N, int64_t K) {
  // 256 x 256 tiles times splits should fill about one round of workgroups
  // (one per CU) when the unsplit grid leaves most CUs idle; each slice
  // keeps at least 16 K steps and whole groups (K / splits % 128 == 0).
  // MLXQ_QMM_SPLIT overrides (tuning).
  if (const int sp = overrides().qmm_split) {
    return sp >= 1 && sp <= kQmmMaxSplits && K % (128 * sp) == 0 ? sp : 1;
  }
  const int64_t cus = cu_count();
  const int64_t tiles = ceil_div(N, 256) * ceil_div(M, 256);
  if (tiles * 8 >= cus * 7) return 1;
  for (int sp = 2; sp <= kQmmMaxSplits; sp++) {
    if (tiles * sp > cus) break;
    if (tiles * sp * 8 >= cus * 7 && K % (128 * sp) == 0 && K / sp >= 16 * 64) return sp;
  }
  // grids that no split of 256 x 256 tiles fills (short matrices or few
  // rows): 128 x 128 tiles (two workgroups per CU), K split as far as the
  // CUs and the 16-step minimum allow (launch_cfg takes the 128 x 128 form
  // whenever the split 256-wide grid would still leave CUs idle).  Measured
  // (Q4, µs): q/o M = 128 63.6 -> 28.8, M = 512 65.7 -> 40.5; k/v M = 512
  // 64.3 -> 27.3; down M = 128 195 -> 39.9, M = 256 197 -> 56.7
  const int64_t t128 = ceil_div(N, 128) * ceil_div(M, 128);
  int best = 1;
  for (int sp = 2; sp <= kQmmMaxSplits; sp++)
    if (t128 * sp <= 2 * cus && K % (128 * sp) == 0 && K / sp >= 16 * 64) best = sp;
  return best;
}

size_t qmm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int sp = qmm_split_k(M, N, K);
  return sp > 1 ? static_cast<size_t>(sp) * M * N * sizeof(float) : 0;
}

int launch_qmm(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y, void* workspace,
               size_t workspace_bytes, hipStream_t st) {
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  // split K only when the caller's workspace holds the partials
  int splits = qmm_split_k(M, N, K);
  if (splits > 1 && (!workspace || workspace_bytes < static_cast<size_t>(splits) * M * N * sizeof(float) ||
                     (reinterpret_cast<uintptr_t>(workspace) & 255u)))
    splits = 1;
  float* part = static_cast<float*>(workspace);
  if (bits == 4) {
    if (group_size == 32) return launch_cfg<4, 32>(x, m, wq, s, b, bias, n, k, y, part, splits, st);
    if (group_size == 64) return launch_cfg<4, 64>(x, m, wq, s, b, bias, n, k, y, part, splits, st);
    return launch_cfg<4, 128>(x, m, wq, s, b, bias, n, k, y, part, splits, st);
  }
  if (group_size == 32) return launch_cfg<8, 32>(x, m, wq, s, b, bias, n, k, y, part, splits, st);
  if (group_size == 64) return launch_cfg<8, 64>(x, m, wq, s, b, bias, n, k, y, part, splits, st);
  return launch_cfg<8, 128>(x, m, wq, s, b, bias, n, k, y, part, splits, st);
}

}  // namespace mlxq
