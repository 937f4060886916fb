// Prefill-shaped quantized matmul (qmm) for gfx950: y[M,N] = x[M,K] . W^T,
// W group-wise affine quantized (Q4 / Q8), any M; K a multiple of 512 and
// of 8 groups.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul, which MLX serves with its qmm kernels when M
// is large (prefill, batched decode).
//
// Design (MFMA-bound at prefill sizes):
//  * Workgroup tile BM x 256 (BM = 256 or 128), four waves side by side
//    along N; each wave owns BM x 64 of the output as (BM/32) x 2 tiles of
//    v_mfma_f32_32x32x16_bf16 with f32 accumulators (up to 256 per lane, in
//    the accumulator registers).  K advances 64 per step.
//  * Everything arrives by LDS DMA (global_load_lds_dwordx4: no VGPRs, no
//    VALU), in whole 128-byte lines: the memory path pays per line touched,
//    so a 32-byte slice of a code row costs as much as a full line.
//      - activations: the BM x 64 bf16 tile of one step (one line per row),
//        two stages, requested one step ahead;
//      - codes: 128 bytes of each of the 256 weight rows (4 steps at Q4, 2
//        at Q8), two buffers;
//      - scales and biases: 16 bytes per row and array (8 steps of groups),
//        two buffers.
//    Rows are stored with their 16-byte chunks permuted (chunk c of row r at
//    c ^ swz(r)), which makes the 16-byte fragment reads bank-conflict free.
//  * Weights are dequantized straight into the MFMA B-operand layout in
//    registers, by the wave that multiplies them: lane (n, h) of a 32-column
//    tile takes the 32 codes k0 + 32h .. +32 of weight row n (one 16-byte LDS
//    read at Q4), and for sub-step j the 8 codes 32h + 8j .. +8 become its
//    bf16x8 operand (bf16(s * q + b): f32 FMA, round to nearest even).  The
//    activation fragment of sub-step j is the 16-byte chunk 4h + j of the
//    row: both operands follow the same k order, which the MFMA sums over.
//    No weight tile is written to LDS.
//  * Step k's MFMAs use the operands decoded during step k-1: the wave
//    alternates one MFMA (32 cycles on the matrix core) with a few decode
//    instructions and LDS reads, in a fixed per-step schedule.
//  * Tiles are ordered so that each XCD (workgroups round-robin over the 8
//    XCDs) takes a contiguous, M-major run of tiles: the workgroups of one
//    XCD share activation rows in that XCD's L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <utility>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;      // K per step
constexpr int PERIOD = 8;   // steps per unrolled period (one scale batch)

template <int BITS, int GS, int TM, int TN>
struct QmmGeom {
  static constexpr int WAVES = 4, THREADS = 64 * WAVES;
  static constexpr int BN = 256;               // weight rows per workgroup
  static constexpr int WN = BN / (32 * TN);    // waves along N (each TN 32-column tiles)
  static constexpr int WM = WAVES / WN;        // waves along M (each TM 32-row tiles)
  static constexpr int BM = WM * TM * 32;
  static constexpr int A_BYTES = BM * BK * 2;  // activation tile of one step
  static constexpr int CROW = BK * BITS / 8;   // code bytes per weight row per step
  static constexpr int CB = 128 / CROW;        // steps per code batch (one 128-byte line per row)
  static constexpr int C_BYTES = BN * 128;
  static constexpr int SROW = GS == 32 ? 32 : 16;  // scale bytes per row per batch (and bias bytes)
  static constexpr int S_BYTES = BN * 2 * SROW;
  static constexpr int A_OFF = 0, C_OFF = 2 * A_BYTES, S_OFF = C_OFF + 2 * C_BYTES;
  static constexpr int LDS_BYTES = S_OFF + 2 * S_BYTES;
  // DMA instructions per wave: activations per step, codes / scales per batch
  static constexpr int A_DMA = A_BYTES / 1024 / WAVES;
  static constexpr int C_DMA = C_BYTES / 1024 / WAVES;
  static constexpr int S_DMA = S_BYTES / 1024 / WAVES;
  static constexpr int CW = BITS == 4 ? 1 : 2;  // 16-byte code reads per lane per tile per step
  static_assert(A_BYTES % (1024 * WAVES) == 0 && C_BYTES % (1024 * WAVES) == 0 && S_BYTES % (1024 * WAVES) == 0,
                "whole DMA chunks");
  static_assert(PERIOD % CB == 0, "code batches tile the period");
  static_assert(WM * WN == WAVES && TM % 2 == 0 && TN % 2 == 0, "wave grid");
  static_assert(4 * TM * TN >= 3 * TM * TN + 2 + A_DMA && 4 * TM * TN >= C_DMA + S_DMA, "DMA slots");
  static_assert(LDS_BYTES <= 160 * 1024, "fits in LDS");
  static_assert(CB >= 2, "a code batch is needed two boundaries after its request");
  // DMA instructions a boundary issues after its activations: codes when a
  // batch starts two steps later, scales at boundary 6 of the period
  static constexpr int after(int b) { return ((b + 2) % CB == 0 ? C_DMA : 0) + (b == PERIOD - 2 ? S_DMA : 0); }
};

// LDS DMA of 16 bytes per lane (global_load_lds_dwordx4): lane l's bytes
// land at lds + 16 l.  Written out rather than through the compiler's
// builtin: the builtin only emits the 64-bit per-lane address form, while
// the SGPR-base form (wave-uniform base + 32-bit per-lane offset) carries
// half the per-lane address data, which the issuing wave pays for.  Every
// LDS DMA of this kernel goes through these two functions, so M0 (the LDS
// destination) is only ever written here, right before its use; the caller
// accounts for them in its own s_waitcnt vmcnt (the compiler does not count
// inline assembly).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_to_lds_sbase(const void* base, uint32_t off, unsigned char* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_to_lds(const void* g, unsigned char* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt with only the vector-memory counter limited to n (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// 16-byte chunk position of logical chunk c in 128-byte LDS row r is
// c ^ swz(r): a bijection within the row under which rows 0..15 at one c
// hit distinct banks
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v;
  v[0] = static_cast<__bf16>(a);  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

template <int BITS, int GS, int TM, int TN>
__global__ __launch_bounds__(256, 1) void qmm_kernel(const uint16_t* __restrict__ x, int M,
                                                     const uint32_t* __restrict__ wq,
                                                     const uint16_t* __restrict__ scales,
                                                     const uint16_t* __restrict__ biases,
                                                     const uint16_t* __restrict__ bias_vec, int N, int K,
                                                     uint16_t* __restrict__ y, float* __restrict__ part, int k_len) {
  using Gm = QmmGeom<BITS, GS, TM, TN>;
  constexpr int BM = Gm::BM, BN = Gm::BN, CB = Gm::CB;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % Gm::WN, wm = wave / Gm::WN;  // this wave's column / row block

  // tile of this workgroup: XCD blockIdx.x % 8 takes tiles [xcd * per, (xcd + 1) * per)
  const int nbn = (N + BN - 1) / BN, nbm = (M + BM - 1) / BM;
  const int tiles = nbn * nbm, per = (tiles + 7) / 8;
  const int t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (t >= tiles) return;
  const int m0 = (t / nbn) * BM, n0 = (t % nbn) * BN;
  const int kb = blockIdx.y * k_len;  // first K of this slice (split K)
  const int KT = k_len / BK;          // a multiple of PERIOD
  const int G = K / GS;
  const uint32_t row_bytes = static_cast<uint32_t>(K) * BITS / 8;

  // ---- DMA sources: per-lane byte offsets (32-bit: the host checks sizes)
  // activations: 1 KB chunk q = 8 rows; lane -> row 8q + lane/8, chunk position lane % 8
  uint32_t a_off[Gm::A_DMA];
#pragma unroll
  for (int i = 0; i < Gm::A_DMA; i++) {
    const int r = 8 * (wave * Gm::A_DMA + i) + (lane >> 3), c = (lane & 7) ^ swz(r);
    a_off[i] = (static_cast<uint32_t>(min(m0 + r, M - 1)) * K + kb + 8 * c) * 2;
  }
  // codes: the same row / chunk mapping over 128-byte code lines
  uint32_t c_off[Gm::C_DMA];
#pragma unroll
  for (int i = 0; i < Gm::C_DMA; i++) {
    const int r = 8 * (wave * Gm::C_DMA + i) + (lane >> 3), c = (lane & 7) ^ swz(r);
    c_off[i] = static_cast<uint32_t>(min(n0 + r, N - 1)) * row_bytes + kb * BITS / 8 + 16 * c;
  }
  // scales / biases: per row [scales SROW bytes][biases SROW bytes]; lanes
  // (row, array, 16-byte part)
  constexpr int SPR = 2 * Gm::SROW / 16;  // lanes per row
  uint32_t s_off[Gm::S_DMA];
#pragma unroll
  for (int i = 0; i < Gm::S_DMA; i++) {
    const int r = (wave * Gm::S_DMA + i) * (64 / SPR) + lane / SPR;
    const int part = lane % (Gm::SROW / 16);
    s_off[i] = (static_cast<uint32_t>(min(n0 + r, N - 1)) * G + kb / GS) * 2 + 16 * part;
  }
  const char* sb_base = reinterpret_cast<const char*>((lane % SPR) >= SPR / 2 ? biases : scales);

  // DMA of the activations of step kt / code batch c / scale batch sb into
  // stage / buffer `buf` (the index is clamped past the end, the buffer not)
  // instruction i of this wave's share of a DMA
  auto dma_a1 = [&](int kt, int buf, int i) __attribute__((always_inline)) {
    dma16_to_lds_sbase(reinterpret_cast<const char*>(x) + kt * (BK * 2), a_off[i],
                 lds + Gm::A_OFF + buf * Gm::A_BYTES + (wave * Gm::A_DMA + i) * 1024);
  };
  auto dma_c1 = [&](int c, int buf, int i) __attribute__((always_inline)) {  // steps CB c .. CB c + CB - 1
    dma16_to_lds_sbase(reinterpret_cast<const char*>(wq) + c * 128, c_off[i],
                 lds + Gm::C_OFF + buf * Gm::C_BYTES + (wave * Gm::C_DMA + i) * 1024);
  };
  auto dma_s1 = [&](int sb, int buf, int i) __attribute__((always_inline)) {  // steps 8 sb .. 8 sb + 7
    // groups from 8 * floor(first group / 8): 16 bytes of 8 groups (GS = 128:
    // the batch's 4 groups are one half of them)
    dma16_to_lds(sb_base + ((sb * PERIOD * BK / GS) & ~7) * 2 + s_off[i],
                 lds + Gm::S_OFF + buf * Gm::S_BYTES + (wave * Gm::S_DMA + i) * 1024);
  };
  auto dma_a = [&](int kt, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Gm::A_DMA; i++) dma_a1(kt, buf, i);
  };
  auto dma_c = [&](int c, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Gm::C_DMA; i++) dma_c1(c, buf, i);
  };
  auto dma_s = [&](int sb, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < Gm::S_DMA; i++) dma_s1(sb, buf, i);
  };

  // ---- fragment addressing (bytes within a stage / buffer)
  const int fr = lane & 31, h = lane >> 5;
  const int sw0 = (fr & 7) ^ (fr >> 3);  // swz(32 i + fr) = sw0 ^ 4 (i & 1)
  int a_rd[4][2];
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int p = 0; p < 2; p++) a_rd[j][p] = (wm * TM * 32 + fr) * 128 + 16 * ((4 * h + j) ^ sw0 ^ (4 * p));
  // codes of step s (s % CB = u) for tile tt: logical chunks CW (u * 2 + h) + v
  int c_rd[CB][TN][Gm::CW];
#pragma unroll
  for (int u = 0; u < CB; u++)
#pragma unroll
    for (int tt = 0; tt < TN; tt++)
#pragma unroll
      for (int v = 0; v < Gm::CW; v++)
        c_rd[u][tt][v] = (wn * TN * 32 + tt * 32 + fr) * 128 +
                         16 * ((Gm::CW * (2 * u + h) + v) ^ swz(wn * TN * 32 + tt * 32 + fr));
  const int s_rd = (wn * TN * 32 + fr) * 2 * Gm::SROW;  // + tt * 32 rows

  bf16x8 bop[2][TN][4];  // decoded weight operands, double-buffered over steps
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int tt = 0; tt < TN; tt++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][tt][v] = 0.f;

  // codes and scale/bias bits of one step for this lane, read from LDS
  struct Raw {
    uint32_t w[TN][4 * Gm::CW];
    uint32_t s[TN], z[TN];
  };
  // step s = k0 + u (k0 % PERIOD == 0, u compile-time, may reach PERIOD + 1)
  auto read_raw = [&](int k0, auto uc, Raw& r) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    const unsigned char* cs = lds + Gm::C_OFF + ((u / CB) & 1) * Gm::C_BYTES;  // k0 / CB is even
    const int sbuf = ((k0 / PERIOD + u / PERIOD) & 1);
    const unsigned char* ss = lds + Gm::S_OFF + sbuf * Gm::S_BYTES + s_rd;
    // element of this step's group within the row's 16 / 32 bytes
    int e;
    if constexpr (GS == 32) e = 2 * (u % PERIOD) + h;
    else if constexpr (GS == 64) e = u % PERIOD;
    else e = 4 * ((k0 / PERIOD + u / PERIOD) & 1) + (u % PERIOD) / 2;
#pragma unroll
    for (int tt = 0; tt < TN; tt++) {
      r.s[tt] = *reinterpret_cast<const uint16_t*>(ss + tt * 32 * 2 * Gm::SROW + 2 * e);
      r.z[tt] = *reinterpret_cast<const uint16_t*>(ss + tt * 32 * 2 * Gm::SROW + Gm::SROW + 2 * e);
#pragma unroll
      for (int v = 0; v < Gm::CW; v++) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(cs + c_rd[u % CB][tt][v]);
        r.w[tt][4 * v] = q[0];
        r.w[tt][4 * v + 1] = q[1];
        r.w[tt][4 * v + 2] = q[2];
        r.w[tt][4 * v + 3] = q[3];
      }
    }
  };
  auto read_a = [&](const unsigned char* as, int j, int i) __attribute__((always_inline)) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(as + i * 32 * 128 + a_rd[j][i & 1]));
  };
  // Decode piece p (0..31) of raw codes into `dst`: word w = p / 4 (tile
  // w / 4, sub-step w % 4), bf16 pair p % 4 of its operand.
  float sc[TN], zz[TN], sc16[TN];
  uint32_t lo = 0, hi = 0, d[4];
  auto piece = [&](const Raw& r, auto pc, bf16x8 (&dst)[TN][4]) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value;
    constexpr int w = p >> 2, tt = w >> 2, jj = w & 3, pp = p & 3;
    if constexpr (jj == 0 && pp == 0) {
      sc[tt] = __uint_as_float(r.s[tt] << 16);
      zz[tt] = __uint_as_float(r.z[tt] << 16);
      sc16[tt] = sc[tt] * 0.0625f;
    }
    if constexpr (BITS == 4) {
      if constexpr (pp == 0) {
        // even codes in the bytes of lo, odd codes (x16) in the bytes of hi
        lo = r.w[tt][jj] & 0x0F0F0F0Fu;
        hi = r.w[tt][jj] & 0xF0F0F0F0u;
        asm("" : "+v"(lo), "+v"(hi));  // keep the byte form (one v_cvt_f32_ubyte per code)
      }
      d[pp] = pack_bf16(__builtin_fmaf(sc[tt], static_cast<float>((lo >> (8 * pp)) & 0xFFu), zz[tt]),
                        __builtin_fmaf(sc16[tt], static_cast<float>((hi >> (8 * pp)) & 0xFFu), zz[tt]));
    } else {
      const uint32_t q = r.w[tt][2 * jj + (pp >> 1)];
      const int b0 = 16 * (pp & 1);
      d[pp] = pack_bf16(__builtin_fmaf(sc[tt], static_cast<float>((q >> b0) & 0xFFu), zz[tt]),
                        __builtin_fmaf(sc[tt], static_cast<float>((q >> (b0 + 8)) & 0xFFu), zz[tt]));
    }
    if constexpr (pp == 3) dst[tt][jj] = __builtin_bit_cast(bf16x8, u32x4{d[0], d[1], d[2], d[3]});
  };

  // One K step (kt = k0 + u) as a fixed instruction schedule: slot s issues
  // MFMA s (sub-step j = s / (TM TN), row tile i, column tile tt); after the
  // last MFMA of row tile i the LDS read of its fragment for sub-step j + 1
  // (for j = 3: the next step's first sub-step) into the same registers;
  // then decode pieces of the next step's operands.  Each slot is fenced, so
  // the wave alternates between the matrix core and the vector ALU.  In the
  // last sub-step, once every activation read of the step has been issued,
  // sits the step boundary: wait for this wave's DMA of the next step's
  // activations, barrier, issue the DMA that the schedule places here, read
  // the codes of the step after next.  With 256-row tiles the decode pieces
  // all come before the boundary, so one set of raw-code registers serves
  // (the boundary refills it); with 128-row tiles they spread over the whole
  // step and the raw codes are double-buffered.
  constexpr int S = 4 * TM * TN, NP = 4 * 4 * TN, BOUNDARY = 3 * TM * TN + 1;
  constexpr bool ONE_RAW = NP <= BOUNDARY;
  constexpr int PIECE_SLOTS = ONE_RAW ? BOUNDARY : S;
  constexpr int NRAW = ONE_RAW ? 1 : 2;
  const int KTL = KT - 1;
  auto step = [&](int k0, auto uc, const bf16x8 (&cur)[TN][4], bf16x8 (&nxt)[TN][4], const Raw& rcur, Raw& rnext,
                  bf16x8 (&a)[TM]) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    const int kt = k0 + u;
    const unsigned char* as = lds + Gm::A_OFF + (u & 1) * Gm::A_BYTES;
    const unsigned char* an = lds + Gm::A_OFF + ((u + 1) & 1) * Gm::A_BYTES;
    static_for<S>([&](auto sc_) __attribute__((always_inline)) {
      constexpr int s = decltype(sc_)::value;
      constexpr int j = s / (TM * TN), r = s % (TM * TN), i = r / TN, tt = r % TN;
      if constexpr (s == BOUNDARY) {
        wait_lgkm0();  // this wave's reads of stage kt & 1 are done
        // activations of step kt + 1 (issued at the previous boundary, before
        // the codes / scales that boundary issued)
        wait_vm<Gm::after((u + PERIOD - 1) % PERIOD)>();
        __builtin_amdgcn_s_barrier();
        read_raw(k0, std::integral_constant<int, u + 2>{}, rnext);
        __builtin_amdgcn_sched_barrier(0);
      }
      // weights as the first operand: the output tile comes out transposed,
      // lane = activation row, 4 consecutive output columns per register quad
      acc[i][tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[tt][j], a[i], acc[i][tt], 0, 0, 0);
      if constexpr (tt == TN - 1) a[i] = read_a(j < 3 ? as : an, (j + 1) & 3, i);
      // DMA, one instruction per slot so the requests do not queue up
      // behind each other: after the boundary the activations of step kt + 2
      // into stage kt & 1 (read by every wave before the barrier); in the
      // first slots, when the previous boundary scheduled them (after its
      // activations), code batch (kt + 1) / CB + 1 (when step kt + 1 starts a
      // batch) and scale batch (kt + 9) / 8 (at u = 7).  Past the end: the
      // last step / batch again, into buffers nobody reads.
      if constexpr (s > BOUNDARY && s <= BOUNDARY + Gm::A_DMA) dma_a1(min(kt + 2, KTL), u & 1, s - BOUNDARY - 1);
      if constexpr (u > 0 && (u + 1) % CB == 0 && s < Gm::C_DMA)
        dma_c1(min((kt + 1) / CB + 1, KTL / CB), ((u + 1) / CB + 1) & 1, s);
      if constexpr (u == PERIOD - 1 && s >= Gm::C_DMA && s < Gm::C_DMA + Gm::S_DMA)
        dma_s1(min((kt + 9) / PERIOD, KTL / PERIOD), (k0 / PERIOD) & 1, s - Gm::C_DMA);
      // pieces p with p * PIECE_SLOTS / NP == s
      constexpr int P_LO = (s * NP + PIECE_SLOTS - 1) / PIECE_SLOTS;
      constexpr int P_HI = ((s + 1) * NP + PIECE_SLOTS - 1) / PIECE_SLOTS;
      static_for<(NP + PIECE_SLOTS - 1) / PIECE_SLOTS>([&](auto qc) __attribute__((always_inline)) {
        constexpr int p = P_LO + decltype(qc)::value;
        if constexpr (p < P_HI && p < NP) piece(rcur, std::integral_constant<int, p>{}, nxt);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- prologue: code batches 0 and 1, scale batches 0 and 1, activations
  // of steps 0 and 1; the operands of step 0 decoded here
  bf16x8 a[TM];
  Raw raw[NRAW];
  dma_c(0, 0);
  dma_s(0, 0);
  dma_a(0, 0);
  dma_c(min(1, KTL / CB), 1);
  dma_s(min(1, KTL / PERIOD), 1);
  dma_a(min(1, KTL), 1);
  wait_vm<Gm::A_DMA + Gm::C_DMA + Gm::S_DMA>();
  __builtin_amdgcn_s_barrier();
  read_raw(0, std::integral_constant<int, 0>{}, raw[0]);
#pragma unroll
  for (int i = 0; i < TM; i++) a[i] = read_a(lds + Gm::A_OFF, 0, i);
  static_for<NP>([&](auto pc) __attribute__((always_inline)) { piece(raw[0], pc, bop[0]); });
  read_raw(0, std::integral_constant<int, 1>{}, raw[NRAW - 1]);

  for (int k0 = 0; k0 < KT; k0 += PERIOD) {
    static_for<PERIOD / 2>([&](auto vc) __attribute__((always_inline)) {
      constexpr int u = 2 * decltype(vc)::value;
      step(k0, std::integral_constant<int, u>{}, bop[0], bop[1], raw[NRAW - 1], raw[0], a);
      step(k0, std::integral_constant<int, u + 1>{}, bop[1], bop[0], raw[0], raw[NRAW - 1], a);
    });
  }
  wait_vm<0>();  // no DMA may land after the workgroup's LDS is released

  // Output layout of a 32x32 tile (weights x activations^T): lane holds
  // activation row m = lane % 32 and output columns n = 8 (v / 4) + 4 (lane /
  // 32) + v % 4 for accumulator v.  Pairs of column groups are exchanged
  // between the wave halves (permlane32 swap) so that every lane ends with 8
  // consecutive columns: one 16-byte store (bf16) or two (f32 partials).
  const int mrow0 = m0 + wm * TM * 32 + fr;
  const int ncol0 = n0 + wn * TN * 32;
  if (part) {  // split K: this slice's f32 partial sums, added by the reduce kernel
    float* dst = part + static_cast<int64_t>(blockIdx.y) * M * N;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int m = mrow0 + i * 32;
      if (m >= M) continue;
#pragma unroll
      for (int tt = 0; tt < TN; tt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int n = ncol0 + tt * 32 + 8 * g + 4 * h;
          float* q = dst + static_cast<int64_t>(m) * N + n;
          if (n + 3 < N && (N & 3) == 0) {
            *reinterpret_cast<f32x4*>(q) = f32x4{acc[i][tt][4 * g], acc[i][tt][4 * g + 1], acc[i][tt][4 * g + 2],
                                                 acc[i][tt][4 * g + 3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (n + e < N) q[e] = acc[i][tt][4 * g + e];
          }
        }
    }
  } else {
#pragma unroll
    for (int tt = 0; tt < TN; tt++) {
#pragma unroll
      for (int gp = 0; gp < 2; gp++) {
        // columns ncol0 + tt 32 + 16 gp + 8 h + [0, 8) after the exchange;
        // before it this lane holds groups 2 gp + q (q = 0, 1) at columns
        // ncol0 + tt 32 + 16 gp + 8 q + 4 h + [0, 4)
        const int n = ncol0 + tt * 32 + 16 * gp + 8 * h;
        float bb[2][4];
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int nb = ncol0 + tt * 32 + 16 * gp + 8 * q + 4 * h + e;
            bb[q][e] = bias_vec && nb < N ? bf16_bits_to_f32(bias_vec[nb]) : 0.f;
          }
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const f32x16& c = acc[i][tt];
          const uint32_t lo0 = pack_bf16(c[8 * gp + 0] + bb[0][0], c[8 * gp + 1] + bb[0][1]);
          const uint32_t lo1 = pack_bf16(c[8 * gp + 2] + bb[0][2], c[8 * gp + 3] + bb[0][3]);
          const uint32_t hi0 = pack_bf16(c[8 * gp + 4] + bb[1][0], c[8 * gp + 5] + bb[1][1]);
          const uint32_t hi1 = pack_bf16(c[8 * gp + 6] + bb[1][2], c[8 * gp + 7] + bb[1][3]);
          // lanes 0-31 keep group 2 gp and receive the other half's group
          // 2 gp; lanes 32-63 keep group 2 gp + 1 and receive the first
          // half's group 2 gp + 1
          const auto s0 = __builtin_amdgcn_permlane32_swap(lo0, hi0, false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(lo1, hi1, false, false);
          const uint32_t w0 = s0[0], w1 = s1[0], w2 = s0[1], w3 = s1[1];
          const int m = mrow0 + i * 32;
          if (m >= M) continue;
          uint16_t* q = y + static_cast<int64_t>(m) * N + n;
          if (n + 7 < N && (N & 7) == 0) {
            *reinterpret_cast<u32x4*>(q) = u32x4{w0, w1, w2, w3};
          } else {
            const uint32_t ww[4] = {w0, w1, w2, w3};
#pragma unroll
            for (int e = 0; e < 8; e++)
              if (n + e < N) q[e] = static_cast<uint16_t>(ww[e >> 1] >> (16 * (e & 1)));
          }
        }
      }
    }
  }
}

template <int BITS, int GS, int TM, int TN>
int launch(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint16_t* bias,
           int N, int K, uint16_t* y, float* part, int splits, hipStream_t st) {
  using Gm = QmmGeom<BITS, GS, TM, TN>;
  auto kern = qmm_kernel<BITS, GS, TM, TN>;
  static bool attr_set = false;  // once per process; the attribute is per function
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       Gm::LDS_BYTES);
    if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmm: set LDS size: ") + hipGetErrorString(e));
    attr_set = true;
  }
  const int64_t tiles = ceil_div(N, Gm::BN) * ceil_div(M, Gm::BM);
  dim3 grid(static_cast<unsigned>(8 * ceil_div(tiles, 8)), splits);
  MLXQ_LAUNCH(kern, grid, dim3(Gm::THREADS), Gm::LDS_BYTES, st, x, M, wq, s, b, bias, N, K, y,
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

// Workgroup tile of a launch: 256 rows (four waves of 256 x 64) when those
// tiles give at least one full round of workgroups, else 128 rows (four
// waves of 128 x 64: half the MFMAs per decoded code, twice the workgroups).
// MLXQ_QMM_CFG = 82 / 42 forces one (tests, tuning).  Measured and not kept
// (Llama-3-8B prefill, M = 2048): 2 x 2 waves of 128 x 128 (each column
// decoded twice), and two 128-row workgroups per CU.
int qmm_cfg(int64_t M, int64_t N, int splits) {
  if (const int c = overrides().qmm_cfg) return c == 42 ? 42 : 82;
  return ceil_div(N, 256) * ceil_div(M, 256) * splits >= cu_count() ? 82 : 42;
}

template <int BITS, int GS>
int launch_cfg(const uint16_t* x, int M, const uint32_t* wq, const uint16_t* s, const uint16_t* b, const uint16_t* bias,
               int N, int K, uint16_t* y, float* part, int splits, hipStream_t st) {
  if (qmm_cfg(M, N, splits) == 42) return launch<BITS, GS, 4, 2>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
  return launch<BITS, GS, 8, 2>(x, M, wq, s, b, bias, N, K, y, part, splits, st);
}

}  // namespace

bool qmm_eligible(int64_t K, int group_size) { return K % (PERIOD * BK) == 0 && K % (8 * group_size) == 0; }

int qmm_split_k(int64_t M, int64_t N, int64_t K, int group_size) {
  // split K when even 128-row tiles leave most CUs idle; every slice is a
  // whole number of unrolled periods and of 8-group scale batches.
  // MLXQ_QMM_SPLIT overrides (tests, tuning).
  const int64_t grain = std::max<int64_t>(PERIOD * BK, 8 * group_size);
  if (const int sp = overrides().qmm_split) {
    return sp >= 1 && sp <= kQmmMaxSplits && K % (grain * sp) == 0 ? sp : 1;
  }
  const int64_t cus = cu_count();
  const int64_t t128 = ceil_div(N, 256) * ceil_div(M, 128);
  if (t128 * 4 >= cus * 3) return 1;
  int best = 1;
  for (int sp = 2; sp <= kQmmMaxSplits; sp++)
    if (t128 * sp <= cus && K % (grain * sp) == 0) best = sp;
  return best;
}

size_t qmm_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size) {
  const int sp = qmm_split_k(M, N, K, group_size);
  return sp > 1 ? static_cast<size_t>(sp) * M * N * sizeof(float) : 0;
}

int launch_qmm(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y, void* workspace,
               size_t workspace_bytes, hipStream_t st) {
  // the DMA offsets are 32-bit byte offsets from the array bases
  if (M * K * 2 >= (int64_t(1) << 32) || N * K * bits / 8 >= (int64_t(1) << 32) || !qmm_eligible(K, group_size))
    return fail(MLXQ_ERR_UNSUPPORTED, "qmm: activations and codes must each be below 4 GiB, K a multiple of " +
                                          std::to_string(PERIOD * BK) + " and of 8 groups");
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  // split K only when the caller's workspace holds the partials
  int splits = qmm_split_k(M, N, K, group_size);
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
