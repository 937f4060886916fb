// Persistent decode step: the whole quantized layer chain of one batch-1
// decode step (src/models/llama.rs:689-735 per layer, q/k/v/o at :806-835,
// the MLP at :1040-1045, final norm + lm_head at :595-603) in ONE launch.
//
// Why one launch: a batch-1 projection is a pure weight stream, and every
// launch pays a ramp (the first loads of a fresh grid take a full memory
// latency to return, and the grid's tail drains before the next launch
// starts), ~2 us per projection against 1.6-11 us of streaming.  Here the
// weights of the NEXT stage are requested before the stage that needs them
// can start, so HBM keeps streaming across the dependency between stages.
//
// Structure (one workgroup per CU, all resident; grid barrier between the
// stages, stage = a set of projections of the same input):
//  * 8 compute waves.  Each streams its share of every stage's weight rows
//    through a D-slot register ring that runs ahead across stage
//    boundaries: a round is 8 rows x 128 contiguous bytes of Q4 codes
//    (8 lanes per row, 16 B each) plus the lanes' scale/bias.  These waves
//    issue no other global memory operation, so the memory-counter waits the
//    compiler places before each ring slot is used never wait for anything
//    but older ring loads.  Codes become bf16 (128+q) pairs with one
//    and-or each; v_dot2_f32_bf16 against the stage input held in LDS
//    (pre-permuted to the pair order, with per-32 sums) gives
//    y += s*dot + (b - 128 s) * sum(x).
//  * 1 stager wave.  Everything that crosses workgroups: it sums the
//    compute waves' partial rows in a fixed order, applies the epilogue
//    (residual add, SwiGLU, bf16 rounding at MLX's points), stores the
//    outputs with agent-coherent stores, arrives at the grid barrier
//    (release: L2 write-back of dirty lines + wait), waits for the other
//    workgroups, then loads the next stage's input with agent-coherent
//    direct-to-LDS loads, applies RMSNorm or the GQA head repeat and
//    writes the permuted copy the compute waves read.
//  * Work split per stage: a task is a fixed set of 8-row octets and K
//    slices covering all 8 compute waves (S slices per octet, 8/S octets
//    per task; SwiGLU pairs a gate and an up octet of the same outputs in one
//    task).  Workgroup g takes tasks g, g+G, ...; S is chosen on the host to
//    minimise the longest wave's rounds.
//  * Grid barrier: one monotonically increasing 64-bit arrival counter in
//    the plan's header (target = next multiple of the grid size), so no
//    reset between launches or graph replays.  The wait is bounded by the
//    wall clock: on time-out the workgroup sets the header's error word and
//    every wave leaves the kernel (the host reports it).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <string>
#include <vector>

#include "common.hpp"

using namespace mlxq;

namespace {

constexpr int kWaves = 8;                      // compute waves per workgroup
constexpr int kThreads = 64 * (kWaves + 1);    // + the stager wave
constexpr int kMaxMat = 3;
constexpr int kMaxResTasks = 8;                // residual stages: tasks per workgroup held in LDS
constexpr int kTraceWgs = 1024;                // profiling stamps kept for this many workgroups
constexpr int kRing = 8;                       // ring depth (rounds in flight per wave; 8 measured faster than 16 or 20)
constexpr int kLdsFloor = 96 * 1024;           // > half the CU's LDS: one workgroup per CU
constexpr long long kTimeoutTicks = 50000000ll;  // default barrier wait limit: 0.5 s at the 100 MHz wall clock

enum : int32_t { ST_QKV = 0, ST_O = 1, ST_MLP = 2, ST_DOWN = 3, ST_HEAD = 4 };
enum : int32_t { F_X_ARG = 1, F_RES_ARG = 2, F_Y_ARG = 4 };

struct DStage {
  int32_t kind, K, S, RT, n_tasks, nmat;
  int32_t oct_end[kMaxMat];  // cumulative octet ends of the matrices (MLP: gate's octets)
  int32_t kin;               // input elements before the head repeat
  int32_t groups, head_dim;  // O stage: input = repeat_kv(v)
  int32_t flags;             // F_*: pointers that are the call's x / logits
  float eps;
  const uint16_t* xin;
  const uint16_t* norm_w;
  const uint16_t* res;
  const uint32_t* wq[kMaxMat];
  const uint16_t* sc[kMaxMat];
  const uint16_t* bi[kMaxMat];
  uint16_t* y[kMaxMat];
};

static_assert(sizeof(DStage) % 16 == 0, "the stage table is copied in 16-byte pieces");

// Grid barrier state, every word in its own 256-byte block (no two
// contended words share a memory line).  Two levels: workgroup g arrives on
// group counter g % kGroups; the last of a group arrives on the top counter;
// the last group's last workgroup raises the epoch, replicated once per
// group, and each workgroup polls its own group's copy.  All counters only
// grow (no reset between launches or graph replays).
constexpr int kGroups = 8;
struct alignas(256) DLine {
  unsigned long long v;
  uint32_t pad[62];
};
struct DHeader {
  DLine group[kGroups];     // arrivals per group
  DLine top;                // groups complete
  DLine epoch[kGroups];     // barrier epoch, one copy per group
  DLine error;              // 1: a grid barrier timed out
};
static_assert(sizeof(DLine) == 256, "one line per word");

struct Lds {
  int raw, wraw, xp, xs, red, resl, tab, total;
};

__host__ __device__ inline Lds lds_layout(int max_kin, int max_k, int hidden, int ns) {
  Lds L{};
  auto up = [](int v, int a) { return (v + a - 1) / a * a; };
  L.raw = 0;
  L.wraw = up(max_kin * 2, 1024);
  L.xp = L.wraw + up(hidden * 2, 1024);
  L.xs = L.xp + max_k * 2;
  L.red = L.xs + up(max_k / 32 * 4, 16);
  L.resl = L.red + 2 * kWaves * 8 * 4;
  L.tab = L.resl + kMaxResTasks * 64 * 4;
  L.total = L.tab + ns * static_cast<int>(sizeof(DStage));
  if (L.total < kLdsFloor) L.total = kLdsFloor;
  return L;
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}
__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
__device__ __forceinline__ int wg_tasks(int n_tasks, int g, int G) { return n_tasks > g ? (n_tasks - 1 - g) / G + 1 : 0; }
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Weight pointers of compute wave wv for task T of stage s (lane's row and
// 16-byte chunk of the first round); kb = first code index of the slice.
// Global address space: the table that holds the pointers lives in LDS, and
// generic (flat) loads would count on the LDS counter as well, so every LDS
// wait would drain the ring.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4v gu4;
typedef __attribute__((address_space(1))) uint16_t gw16;  // stager's coherent loads/stores
typedef const __attribute__((address_space(1))) uint16_t gu16;

struct RowPtr {
  gu4* w;
  gu16* s;
  gu16* b;
};

__device__ __forceinline__ RowPtr task_ptr(const DStage* st, int s, int T, int wv, int lane) {
  const int S = st[s].S, RT = st[s].RT, K = st[s].K;
  const int sl = wv & (S - 1);
  int mat = 0, oct;
  if (st[s].kind == ST_MLP) {
    mat = (wv / S) & 1;
    oct = T * (4 / S) + wv / (2 * S);
    const int n = st[s].oct_end[0];
    oct = oct < n ? oct : n - 1;
  } else {
    oct = T * (8 / S) + wv / S;
    const int nm = st[s].nmat;
    const int n = st[s].oct_end[nm - 1];
    oct = oct < n ? oct : n - 1;
    int base = 0;
    for (int m = 0; m < nm - 1; m++)
      if (oct >= st[s].oct_end[m]) {
        mat = m + 1;
        base = st[s].oct_end[m];
      }
    oct -= base;
  }
  mat = uni(mat);
  const int64_t row = static_cast<int64_t>(oct) * 8 + (lane >> 3);
  const int kb = sl * RT * 256 + (lane & 7) * 32;
  RowPtr p;
  p.w = (gu4*)(st[s].wq[mat] + row * (K / 8) + kb / 8);
  p.s = (gu16*)(st[s].sc[mat] + row * (K / 64) + kb / 64);
  p.b = (gu16*)(st[s].bi[mat] + row * (K / 64) + kb / 64);
  return p;
}

template <int D>
__global__ __launch_bounds__(kThreads, 1) void decode_step_kernel(const DStage* st_g, int NS,
                                                                  const uint16_t* __restrict__ x_arg,
                                                                  uint16_t* __restrict__ logits, DHeader* hdr,
                                                                  int max_kin, int max_k, int hidden, int vocab,
                                                                  int trace_on, unsigned long long timeout_ticks) {
  extern __shared__ __align__(16) unsigned char smem[];
  const Lds L = lds_layout(max_kin, max_k, hidden, NS);
  uint16_t* raw = reinterpret_cast<uint16_t*>(smem + L.raw);
  uint16_t* wraw = reinterpret_cast<uint16_t*>(smem + L.wraw);
  uint4* xp = reinterpret_cast<uint4*>(smem + L.xp);
  float* xs = reinterpret_cast<float*>(smem + L.xs);
  float* red = reinterpret_cast<float*>(smem + L.red);    // [2][kWaves][8]
  float* resl = reinterpret_cast<float*>(smem + L.resl);  // [kMaxResTasks][64]
  DStage* st = reinterpret_cast<DStage*>(smem + L.tab);   // the stage table, copied once
  __shared__ int abort_flag;  // set by the stager before a stage-entry barrier
  __shared__ float norm_inv;  // RMSNorm scale of the stage input

  const int G = gridDim.x, g = blockIdx.x;
  const int wv = uni(threadIdx.x >> 6), lane = threadIdx.x & 63;
  {
    const uint4* src = reinterpret_cast<const uint4*>(st_g);
    uint4* dst = reinterpret_cast<uint4*>(st);
    const int n = NS * static_cast<int>(sizeof(DStage)) / 16;
    for (int i = threadIdx.x; i < n; i += kThreads) dst[i] = src[i];
  }
  if (threadIdx.x == 0) abort_flag = 0;
  __syncthreads();

  if (wv == kWaves) {
    // ------------------------------ stager ------------------------------
    unsigned long long* trace = reinterpret_cast<unsigned long long*>(hdr + 1);
    auto stamp = [&](int s, int k) {
      if (trace_on && lane == 0 && g < kTraceWgs) trace[(static_cast<size_t>(s) * kTraceWgs + g) * 4 + k] = wall_clock64();
    };
    for (int s = 0; s < NS; s++) {
      const int kind = st[s].kind, flags = st[s].flags;
      stamp(s, 0);
      if (s > 0) {
        // grid barrier.  Every value that crosses workgroups (stage outputs,
        // their reads in the next stage, the barrier words) is an agent-scope
        // atomic store or load, so it is coherent across the XCDs without an
        // L2 write-back; what the barrier must order is completion: the
        // s_waitcnt(0) below returns only once this workgroup's output stores
        // (retired by the compute waves before the workgroup barrier that
        // ended the previous stage) are acknowledged at agent scope, and only
        // then is the arrival counted.  Agent-scope release / acquire fences
        // around the barrier give the same order by the memory model, but
        // each writes back and invalidates the whole L2: measured 1.63 ->
        // 2.28 ms per batch-1 step (129 barriers).
        int ok = 1;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) {
          const int grp = g % kGroups, ngroups = G < kGroups ? G : kGroups;
          const int gsize = (G - grp + kGroups - 1) / kGroups;  // workgroups with g % kGroups == grp
          unsigned long long* ep = &hdr->epoch[grp].v;
          const unsigned long long target = __hip_atomic_load(ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
          const unsigned long long a = __hip_atomic_fetch_add(&hdr->group[grp].v, 1ull, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
          if (a % gsize == static_cast<unsigned long long>(gsize - 1)) {
            const unsigned long long b = __hip_atomic_fetch_add(&hdr->top.v, 1ull, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT);
            if (b % ngroups == static_cast<unsigned long long>(ngroups - 1))
              for (int k = 0; k < ngroups; k++)
                __hip_atomic_store(&hdr->epoch[k].v, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          const unsigned long long t0 = wall_clock64();
          while (__hip_atomic_load(ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (__hip_atomic_load(&hdr->error.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
              ok = 0;
              break;
            }
            if (wall_clock64() - t0 > timeout_ticks) {
              __hip_atomic_store(&hdr->error.v, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              ok = 0;
              break;
            }
          }
        }
        ok = uni(__shfl(ok, 0));
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (!ok) {
          // a step that times out leaves NaN logits (each workgroup its
          // share), never the previous step's values
          for (int i = g * 64 + lane; i < vocab; i += G * 64) logits[i] = 0x7FC0u;
          if (lane == 0) abort_flag = 1;
          __syncthreads();  // meets the compute waves' next stage-entry barrier: they read the flag and leave
          return;
        }
      }
      stamp(s, 1);
      // a stage without tasks here needs no input (the compute waves skip its barriers too)
      const int nt = wg_tasks(st[s].n_tasks, g, G);
      if (nt == 0) continue;
      // ---- stage input: agent-coherent direct-to-LDS loads (16 B per lane)
      const int K = st[s].K, kin = st[s].kin;
      const uint16_t* xin = (flags & F_X_ARG) ? x_arg : st[s].xin;
      const uint16_t* nw = st[s].norm_w;
      const int nx = (kin * 2 + 1023) / 1024;  // wave-wide 1 KB pieces (buffers are padded)
      for (int i = 0; i < nx; i++)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const unsigned char*>(xin) + (i * 64 + lane) * 16,
                                         reinterpret_cast<unsigned char*>(raw) + i * 1024, 16, 0, 16);
      if (nw) {
        const int nn = (K * 2 + 1023) / 1024;
        for (int i = 0; i < nn; i++)
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const unsigned char*>(nw) + (i * 64 + lane) * 16,
                                           reinterpret_cast<unsigned char*>(wraw) + i * 1024, 16, 0, 0);
      }
      // residual values of this workgroup's outputs (O, DOWN); loads issued
      // unconditionally (clamped) so they overlap instead of waiting one by one
      float rv[kMaxResTasks];
      const uint16_t* res = (flags & F_RES_ARG) ? x_arg : st[s].res;
      if (res) {
        const int S = st[s].S, opt = 8 / S, n = st[s].oct_end[st[s].nmat - 1];
#pragma unroll
        for (int t = 0; t < kMaxResTasks; t++) {
          const int slot = lane >> 3, oct = min((g + t * G) * opt + slot, n - 1);
          const uint16_t v = __hip_atomic_load((gw16*)(res) + oct * 8 + (lane & 7), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
          rv[t] = bf16_bits_to_f32(v);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      if (res) {
#pragma unroll
        for (int t = 0; t < kMaxResTasks; t++) resl[t * 64 + lane] = rv[t];
      }
      // ---- RMSNorm statistic (f32 sum of squares over the bf16 input)
      if (nw) {
        float ss = 0.f;
        for (int j = lane; j < K / 8; j += 64) {
          const uint4 v = reinterpret_cast<const uint4*>(raw)[j];
          const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float lo = bf16_bits_to_f32(a[e] & 0xFFFFu), hi = bf16_bits_to_f32(a[e] >> 16);
            ss += lo * lo;
            ss += hi * hi;
          }
        }
        ss = wave_sum(ss);
        if (lane == 0) norm_inv = 1.0f / sqrtf(ss / static_cast<float>(K) + st[s].eps);
      }
      __syncthreads();  // B1a: raw input, norm statistic and residuals in LDS
      stamp(s, 2);
      __syncthreads();  // B1b: the compute waves wrote the permuted input
      // ---- per task: sum the slices in order, epilogue, coherent store
      const int S = st[s].S;
      for (int t = 0; t < nt; t++) {
        __syncthreads();  // B2: the compute waves' partial rows of task t are in red[t & 1]
        const float* r = red + (t & 1) * kWaves * 8;
        const int slot = lane >> 3, rr = lane & 7, T = g + t * G;
        if (kind == ST_MLP) {
          const int n = st[s].oct_end[0], oct = T * (4 / S) + slot;
          if (slot < 4 / S && oct < n) {
            float gs = 0.f, us = 0.f;
            for (int q = 0; q < S; q++) {
              gs += r[((2 * slot) * S + q) * 8 + rr];
              us += r[((2 * slot + 1) * S + q) * 8 + rr];
            }
            const float gg = bf16r(gs), uu = bf16r(us);
            const float sig = bf16r(1.0f / (1.0f + expf(-gg)));
            const float a = bf16r(gg * sig);
            __hip_atomic_store((gw16*)(st[s].y[0]) + oct * 8 + rr, static_cast<uint16_t>(f32_to_bf16_bits(a * uu)),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        } else {
          const int nm = st[s].nmat, n = st[s].oct_end[nm - 1], oct = T * (8 / S) + slot;
          if (slot < 8 / S && oct < n) {
            float acc = 0.f;
            for (int q = 0; q < S; q++) acc += r[(slot * S + q) * 8 + rr];
            int mat = 0, base = 0;
            for (int m = 0; m < nm - 1; m++)
              if (oct >= st[s].oct_end[m]) {
                mat = m + 1;
                base = st[s].oct_end[m];
              }
            float yv = acc;
            if (res) yv = resl[t * 64 + lane] + bf16r(acc);
            uint16_t* y = (flags & F_Y_ARG) ? logits : st[s].y[0];
            if (nm > 1) y = mat == 1 ? st[s].y[1] : (mat == 2 ? st[s].y[2] : st[s].y[0]);
            __hip_atomic_store((gw16*)(y) + (oct - base) * 8 + rr, static_cast<uint16_t>(f32_to_bf16_bits(yv)),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      stamp(s, 3);
    }
    return;
  }

  // ---------------------------- compute waves ----------------------------
  // Each stage's rounds on this wave (tasks x RT) are padded to a multiple of
  // the ring depth D with idle rounds (they re-read the last real round's
  // address, a cache hit, and compute nothing).  Stage changes then fall on
  // the boundary of the unrolled D-slot block, so the stage-entry code
  // exists once, outside the unrolled slots.
  auto padded = [&](int s) {
    const int r = wg_tasks(st[s].n_tasks, g, G) * st[s].RT;
    return (r + D - 1) / D * D;
  };
  auto next_stage = [&](int s) {  // first stage after s with tasks here
    s++;
    while (s < NS && wg_tasks(st[s].n_tasks, g, G) == 0) s++;
    return s;
  };
  // prefetch cursor: stage, position in the stage's padded rounds, task and
  // round within the task (real positions come first, then idle ones)
  int pst = next_stage(-1), pk = 0, pt = 0, pi = 0;
  int preal = 0, ppad = 0, pRT = 1;
  if (pst < NS) {
    pRT = st[pst].RT;
    preal = wg_tasks(st[pst].n_tasks, g, G) * pRT;
    ppad = padded(pst);
  }
  RowPtr P = task_ptr(st, pst < NS ? pst : 0, pst < NS ? g : 0, wv, lane);
  auto issue = [&](u32x4v& w, uint16_t& sv, uint16_t& bv) {
    w = *P.w;
    sv = *P.s;
    bv = *P.b;
    if (pst < NS) {
      if (++pk < preal) {
        if (++pi == pRT) {
          pi = 0;
          P = task_ptr(st, pst, g + (++pt) * G, wv, lane);
        } else {
          P.w += 8;
          P.s += 4;
          P.b += 4;
        }
      } else if (pk == ppad) {
        pst = next_stage(pst);
        if (pst < NS) {
          pk = pt = pi = 0;
          pRT = st[pst].RT;
          preal = wg_tasks(st[pst].n_tasks, g, G) * pRT;
          ppad = padded(pst);
          P = task_ptr(st, pst, g, wv, lane);
        }
      }
      // positions preal..ppad-1 are idle: P stays on the stage's last real round
    }
  };

  u32x4v rw[D];
  uint16_t rs[D], rb[D];
#pragma unroll
  for (int j = 0; j < D; j++) issue(rw[j], rs[j], rb[j]);

  // compute cursor.  Stage entry (outside the unrolled slots): meet the
  // stager at its input barrier, write this wave's share of the permuted
  // input (word j holds the pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7) of
  // x[8j..8j+7] with RMSNorm or the head repeat applied, plus per-32 sums),
  // then the second barrier.  Only LDS: no global access may join the
  // weight ring's memory counter.
  int cst = next_stage(-1), ck = 0, ci = 0, creal = 0, cpad = 0, cRT = 1, ckb = 0, par = 0;
  const int c = lane & 7;
  float acc = 0.f;
  while (cst < NS) {
    if (ck == 0) {
      __syncthreads();  // B1a
      if (uni(abort_flag)) break;
      const int K = st[cst].K, groups = st[cst].groups, hd = st[cst].head_dim;
      const bool nrm = st[cst].norm_w != nullptr;
      const float inv = norm_inv;
      for (int j0 = wv * 64; j0 < K / 8; j0 += kWaves * 64) {
        const int j = j0 + lane;
        int src = 8 * j;
        if (groups > 1) src = ((8 * j / hd) / groups) * hd + (8 * j) % hd;
        const uint4 v = reinterpret_cast<const uint4*>(raw)[src / 8];
        const uint32_t a[4] = {v.x, v.y, v.z, v.w};
        float f[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          f[2 * e] = bf16_bits_to_f32(a[e] & 0xFFFFu);
          f[2 * e + 1] = bf16_bits_to_f32(a[e] >> 16);
        }
        if (nrm) {
          const uint4 w = reinterpret_cast<const uint4*>(wraw)[j];
          const uint32_t b[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            f[2 * e] = bf16r(bf16_bits_to_f32(b[e] & 0xFFFFu) * bf16r(f[2 * e] * inv));
            f[2 * e + 1] = bf16r(bf16_bits_to_f32(b[e] >> 16) * bf16r(f[2 * e + 1] * inv));
          }
        }
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = f32_to_bf16_bits(f[e]);
        xp[j] = make_uint4(h[0] | (h[4] << 16), h[1] | (h[5] << 16), h[2] | (h[6] << 16), h[3] | (h[7] << 16));
        float sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
        sum += dpp_f32<kDppQuadXor1>(sum);
        sum += dpp_f32<kDppQuadXor2>(sum);
        if ((lane & 3) == 0) xs[j >> 2] = sum;
      }
      __syncthreads();  // B1b
      cRT = st[cst].RT;
      creal = wg_tasks(st[cst].n_tasks, g, G) * cRT;
      cpad = padded(cst);
      ckb = (wv & (st[cst].S - 1)) * cRT * 256;
      ci = par = 0;
    }
#pragma unroll
    for (int j = 0; j < D; j++) {
      if (ck < creal) {
        const int kx = ckb + ci * 256 + c * 32;
        const uint4* xq = xp + kx / 8;
        const float xsum = xs[kx / 32];
        const uint32_t wd[4] = {rw[j].x, rw[j].y, rw[j].z, rw[j].w};
        float d = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint4 X = xq[q];
          const uint32_t w = wd[q];
          d = dot2((w & 0x000F000Fu) | 0x43004300u, X.x, d);
          d = dot2(((w >> 4) & 0x000F000Fu) | 0x43004300u, X.y, d);
          d = dot2(((w >> 8) & 0x000F000Fu) | 0x43004300u, X.z, d);
          d = dot2(((w >> 12) & 0x000F000Fu) | 0x43004300u, X.w, d);
        }
        const float sc = bf16_bits_to_f32(rs[j]), bi = bf16_bits_to_f32(rb[j]);
        acc += sc * d + (bi - 128.f * sc) * xsum;
        if (++ci == cRT) {
          acc += dpp_f32<kDppQuadXor1>(acc);  // the 8 lanes of a row: quads, then the other quad
          acc += dpp_f32<kDppQuadXor2>(acc);
          acc += dpp_f32<kDppRowHalfMirror>(acc);
          if (c == 0) red[(par * kWaves + wv) * 8 + (lane >> 3)] = acc;
          __syncthreads();  // B2
          acc = 0.f;
          par ^= 1;
          ci = 0;
        }
      }
      ck++;
      issue(rw[j], rs[j], rb[j]);
    }
    if (ck == cpad) {
      cst = next_stage(cst);
      ck = 0;
    }
  }
}

// Trace for profiling (plans made with MLXQ_DECODE_TRACE set): every
// workgroup's stager records 4 wall-clock stamps per stage (barrier arrival,
// barrier passed, input staged, last output stored), [stage][workgroup][4]
// for up to kTraceWgs workgroups, after the header.
size_t trace_bytes(int ns) { return static_cast<size_t>(ns) * kTraceWgs * 4 * 8; }

const DStage* stage_table(void* ws, int ns) {
  return reinterpret_cast<const DStage*>(static_cast<unsigned char*>(ws) + sizeof(DHeader) + trace_bytes(ns));
}

size_t up1k(size_t v) { return (v + 1023) / 1024 * 1024; }

struct Dims {
  int64_t hidden, inter, qd, kvd, vocab;
};

// Workspace: header | stage table | per layer q, k, v, h, a, x_out (each padded to 1 KB)
size_t table_bytes(int ns) { return (ns * sizeof(DStage) + 255) / 256 * 256; }
size_t layer_bytes(const Dims& d) {
  return up1k(d.qd * 2) + 2 * up1k(d.kvd * 2) + 2 * up1k(d.hidden * 2) + up1k(d.inter * 2);
}

int check_cfg(const mlxq_decode_config* c, Dims& d) {
  if (!c) return fail(MLXQ_ERR_INVALID, "decode_step: null config");
  if (c->layers < 1 || c->hidden <= 0 || c->intermediate <= 0 || c->heads <= 0 || c->kv_heads <= 0 ||
      c->head_dim <= 0 || c->vocab <= 0 || !(c->eps >= 0.f))
    return fail(MLXQ_ERR_INVALID, "decode_step: bad config");
  if (c->bits != 4 || c->group_size != 64)
    return fail(MLXQ_ERR_UNSUPPORTED, "decode_step: the persistent kernel covers Q4 g64");
  if (c->heads % c->kv_heads) return fail(MLXQ_ERR_SHAPE, "decode_step: heads % kv_heads != 0");
  d.hidden = c->hidden;
  d.inter = c->intermediate;
  d.qd = static_cast<int64_t>(c->heads) * c->head_dim;
  d.kvd = static_cast<int64_t>(c->kv_heads) * c->head_dim;
  d.vocab = c->vocab;
  // inputs: K % 512 (whole 64-lane passes of the stager), outputs: whole octets
  if (d.hidden % 512 || d.inter % 512 || d.qd % 512 || c->head_dim % 8 || d.kvd % 8 || d.vocab % 8 ||
      d.hidden > (1 << 16) || d.inter > (1 << 16) || d.qd > (1 << 16))
    return fail(MLXQ_ERR_UNSUPPORTED, "decode_step: widths outside the persistent kernel's layout");
  return MLXQ_OK;
}

// Slices per octet for a stage: the least work on the busiest wave, counting
// each task's workgroup barrier as half a round, scaled up when the tasks do
// not cover every workgroup (idle CUs stream nothing); fewer slices on a tie.
bool choose_split(DStage& S, int64_t octs, int G, bool mlp, bool residual) {
  const int kr = S.K / 256;
  int best = -1;
  int64_t best_rounds = 0;
  for (int sp = 1; sp <= (mlp ? 4 : 8); sp *= 2) {
    if (kr % sp) continue;
    const int64_t per = mlp ? 4 / sp : 8 / sp;
    const int64_t tasks = (octs + per - 1) / per;
    const int64_t tpw = (tasks + G - 1) / G;
    if (residual && tpw > kMaxResTasks) continue;
    int64_t rounds = tpw * (2 * (kr / sp) + 1);
    if (tasks < G) rounds = rounds * G / tasks;
    if (best < 0 || rounds < best_rounds) {
      best = sp;
      best_rounds = rounds;
    }
  }
  if (best < 0) return false;
  S.S = best;
  S.RT = kr / best;
  const int64_t per = mlp ? 4 / best : 8 / best;
  S.n_tasks = static_cast<int32_t>((octs + per - 1) / per);
  return true;
}

int device_grid(int& G) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MLXQ_ERR_DEVICE, "decode_step: hipGetDevice failed");
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return fail(MLXQ_ERR_DEVICE, "decode_step: CU count query failed");
  G = cus;
  return MLXQ_OK;
}

}  // namespace

extern "C" int mlxq_decode_plan_size(const mlxq_decode_config* cfg, size_t* bytes) {
  clear_error();
  Dims d;
  if (int rc = check_cfg(cfg, d)) return rc;
  if (!bytes) return fail(MLXQ_ERR_INVALID, "decode_plan_size: null output");
  const int ns = 4 * cfg->layers + 1;
  *bytes = sizeof(DHeader) + trace_bytes(ns) + table_bytes(ns) + static_cast<size_t>(cfg->layers) * layer_bytes(d);
  return MLXQ_OK;
}

extern "C" int mlxq_decode_plan(const mlxq_decode_config* cfg, const mlxq_decode_layer* layers,
                                const void* final_norm, const mlxq_qweight* lm_head, void* workspace,
                                size_t workspace_bytes, mlxq_decode_plan_t* plan, void* stream) {
  clear_error();
  Dims d;
  if (int rc = check_cfg(cfg, d)) return rc;
  if (!layers || !final_norm || !lm_head || !workspace || !plan)
    return fail(MLXQ_ERR_INVALID, "decode_plan: null pointer");
  size_t need = 0;
  mlxq_decode_plan_size(cfg, &need);
  if (workspace_bytes < need) return fail(MLXQ_ERR_WORKSPACE, "decode_plan: workspace too small");
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(MLXQ_ERR_INVALID, "decode_plan: workspace alignment");
  int G = 0;
  if (int rc = device_grid(G)) return rc;

  const int NS = 4 * cfg->layers + 1;
  std::vector<DStage> tab(NS);
  unsigned char* act = static_cast<unsigned char*>(workspace) + sizeof(DHeader) + trace_bytes(NS) + table_bytes(NS);
  auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
  const uint16_t* prev_x = nullptr;  // nullptr: the call's x
  auto set_mats = [](DStage& S, std::initializer_list<const mlxq_qweight*> ws) {
    int m = 0;
    for (const mlxq_qweight* w : ws) {
      S.wq[m] = w->wq;
      S.sc[m] = static_cast<const uint16_t*>(w->scales);
      S.bi[m] = static_cast<const uint16_t*>(w->biases);
      m++;
    }
    S.nmat = m;
  };
  for (int l = 0; l < cfg->layers; l++) {
    const mlxq_decode_layer& Ly = layers[l];
    const mlxq_qweight* ws[7] = {&Ly.q, &Ly.k, &Ly.v, &Ly.o, &Ly.gate, &Ly.up, &Ly.down};
    for (const mlxq_qweight* w : ws)
      if (!w->wq || !w->scales || !w->biases) return fail(MLXQ_ERR_INVALID, "decode_plan: null weight");
    if (!Ly.ln1 || !Ly.ln2) return fail(MLXQ_ERR_INVALID, "decode_plan: null norm weight");
    unsigned char* p = act + l * layer_bytes(d);
    uint16_t* q = reinterpret_cast<uint16_t*>(p);
    uint16_t* k = reinterpret_cast<uint16_t*>(p += up1k(d.qd * 2));
    uint16_t* v = reinterpret_cast<uint16_t*>(p += up1k(d.kvd * 2));
    uint16_t* h = reinterpret_cast<uint16_t*>(p += up1k(d.kvd * 2));
    uint16_t* a = reinterpret_cast<uint16_t*>(p += up1k(d.hidden * 2));
    uint16_t* xo = reinterpret_cast<uint16_t*>(p += up1k(d.inter * 2));
    DStage& A = tab[4 * l];
    A = DStage{};
    A.kind = ST_QKV;
    A.K = A.kin = static_cast<int32_t>(d.hidden);
    A.groups = 1;
    A.head_dim = cfg->head_dim;
    A.eps = cfg->eps;
    A.xin = prev_x;
    A.flags = prev_x ? 0 : F_X_ARG;
    A.norm_w = u16(Ly.ln1);
    set_mats(A, {&Ly.q, &Ly.k, &Ly.v});
    A.oct_end[0] = static_cast<int32_t>(d.qd / 8);
    A.oct_end[1] = A.oct_end[0] + static_cast<int32_t>(d.kvd / 8);
    A.oct_end[2] = A.oct_end[1] + static_cast<int32_t>(d.kvd / 8);
    A.y[0] = q;
    A.y[1] = k;
    A.y[2] = v;
    DStage& O = tab[4 * l + 1];
    O = DStage{};
    O.kind = ST_O;
    O.K = static_cast<int32_t>(d.qd);
    O.kin = static_cast<int32_t>(d.kvd);
    O.groups = cfg->heads / cfg->kv_heads;
    O.head_dim = cfg->head_dim;
    O.xin = v;
    O.res = prev_x;
    O.flags = prev_x ? 0 : F_RES_ARG;
    set_mats(O, {&Ly.o});
    O.oct_end[0] = static_cast<int32_t>(d.hidden / 8);
    O.y[0] = h;
    DStage& Mp = tab[4 * l + 2];
    Mp = DStage{};
    Mp.kind = ST_MLP;
    Mp.K = Mp.kin = static_cast<int32_t>(d.hidden);
    Mp.groups = 1;
    Mp.head_dim = cfg->head_dim;
    Mp.eps = cfg->eps;
    Mp.xin = h;
    Mp.norm_w = u16(Ly.ln2);
    set_mats(Mp, {&Ly.gate, &Ly.up});
    Mp.oct_end[0] = Mp.oct_end[1] = static_cast<int32_t>(d.inter / 8);
    Mp.y[0] = a;
    DStage& Dn = tab[4 * l + 3];
    Dn = DStage{};
    Dn.kind = ST_DOWN;
    Dn.K = Dn.kin = static_cast<int32_t>(d.inter);
    Dn.groups = 1;
    Dn.head_dim = cfg->head_dim;
    Dn.xin = a;
    Dn.res = h;
    set_mats(Dn, {&Ly.down});
    Dn.oct_end[0] = static_cast<int32_t>(d.hidden / 8);
    Dn.y[0] = xo;
    prev_x = xo;
    if (!choose_split(A, A.oct_end[2], G, false, false) || !choose_split(O, O.oct_end[0], G, false, true) ||
        !choose_split(Mp, Mp.oct_end[0], G, true, false) || !choose_split(Dn, Dn.oct_end[0], G, false, true))
      return fail(MLXQ_ERR_UNSUPPORTED, "decode_plan: no K split fits the persistent kernel");
  }
  if (!lm_head->wq || !lm_head->scales || !lm_head->biases)
    return fail(MLXQ_ERR_INVALID, "decode_plan: null lm_head");
  DStage& H = tab[NS - 1];
  H = DStage{};
  H.kind = ST_HEAD;
  H.K = H.kin = static_cast<int32_t>(d.hidden);
  H.groups = 1;
  H.head_dim = cfg->head_dim;
  H.eps = cfg->eps;
  H.xin = prev_x;
  H.norm_w = u16(final_norm);
  H.flags = F_Y_ARG;
  set_mats(H, {lm_head});
  H.oct_end[0] = static_cast<int32_t>(d.vocab / 8);
  if (!choose_split(H, H.oct_end[0], G, false, false))
    return fail(MLXQ_ERR_UNSUPPORTED, "decode_plan: no K split fits the persistent kernel");

  hipStream_t st = as_stream(stream);
  DHeader h0{};
  if (hipMemcpyAsync(workspace, &h0, sizeof(h0), hipMemcpyHostToDevice, st) != hipSuccess ||
      hipMemcpyAsync(const_cast<DStage*>(stage_table(workspace, NS)), tab.data(), NS * sizeof(DStage),
                     hipMemcpyHostToDevice, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return fail(MLXQ_ERR_DEVICE, "decode_plan: upload failed");

  const int max_k = static_cast<int>(std::max(d.hidden, std::max(d.inter, d.qd)));
  const int max_kin = max_k;
  const Lds L = lds_layout(max_kin, max_k, static_cast<int>(d.hidden), NS);
  if (L.total > 160 * 1024) return fail(MLXQ_ERR_UNSUPPORTED, "decode_plan: too many layers for the LDS stage table");
  auto kern = decode_step_kernel<kRing>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          L.total) != hipSuccess)
    return fail(MLXQ_ERR_UNSUPPORTED, "decode_plan: LDS request refused");
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(kern), kThreads, L.total) !=
          hipSuccess ||
      occ < 1)
    return fail(MLXQ_ERR_UNSUPPORTED, "decode_plan: the persistent kernel does not fit a CU");
  plan->workspace = workspace;
  plan->stages = NS;
  plan->grid = G;
  plan->lds_bytes = L.total;
  plan->max_k = max_k;
  plan->hidden = static_cast<int32_t>(d.hidden);
  plan->vocab = static_cast<int32_t>(d.vocab);
  plan->trace = getenv("MLXQ_DECODE_TRACE") ? 1 : 0;
  plan->timeout_ticks = kTimeoutTicks;
  if (const char* e = getenv("MLXQ_DECODE_TIMEOUT_TICKS")) plan->timeout_ticks = atoll(e);
  return MLXQ_OK;
}

extern "C" int mlxq_decode_step(const mlxq_decode_plan_t* plan, const void* x, void* logits, void* stream) {
  clear_error();
  if (!plan || !plan->workspace || !x || !logits) return fail(MLXQ_ERR_INVALID, "decode_step: null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16) return fail(MLXQ_ERR_INVALID, "decode_step: x must be 16-byte aligned");
  auto kern = decode_step_kernel<kRing>;
  hipLaunchKernelGGL(kern, dim3(plan->grid), dim3(kThreads), plan->lds_bytes,
                     as_stream(stream), stage_table(plan->workspace, plan->stages), plan->stages, static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(logits), static_cast<DHeader*>(plan->workspace), plan->max_k,
                     plan->max_k, plan->hidden, plan->vocab, plan->trace,
                     static_cast<unsigned long long>(plan->timeout_ticks > 0 ? plan->timeout_ticks : 1));
  return check_launch("decode_step");
}

extern "C" int mlxq_decode_status(const mlxq_decode_plan_t* plan, int* timed_out) {
  clear_error();
  if (!plan || !plan->workspace || !timed_out) return fail(MLXQ_ERR_INVALID, "decode_status: null pointer");
  uint32_t e = 0;
  if (hipMemcpy(&e, reinterpret_cast<const unsigned char*>(plan->workspace) + offsetof(DHeader, error), sizeof(e),
                hipMemcpyDeviceToHost) != hipSuccess)
    return fail(MLXQ_ERR_DEVICE, "decode_status: copy failed");
  *timed_out = e != 0;
  return MLXQ_OK;
}
