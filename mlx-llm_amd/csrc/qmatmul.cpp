// C ABI of the quantized matmul: argument checks, workspace sizing and the
// qmv / qmm choice (MLX makes the same choice from M inside quantized_matmul).
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "common.hpp"
#include "qmatmul.hpp"

using namespace mlxq;

namespace {

int check_shape(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (bits != 4 && bits != 8)
    return fail(MLXQ_ERR_UNSUPPORTED, "unsupported: bits=" + std::to_string(bits) + " (4 or 8)");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MLXQ_ERR_UNSUPPORTED, "unsupported: group_size=" + std::to_string(group_size) + " (32, 64, 128)");
  if (M < 0 || N <= 0 || K <= 0) return fail(MLXQ_ERR_INVALID, "qmatmul: bad shape");
  if (K % group_size)
    return fail(MLXQ_ERR_SHAPE, "qmatmul: K=" + std::to_string(K) + " is not divisible by group_size " +
                                    std::to_string(group_size));
  if (N > INT32_MAX / 2 || K > INT32_MAX / 2 || M > INT32_MAX / 2)
    return fail(MLXQ_ERR_INVALID, "qmatmul: dimension too large");
  return MLXQ_OK;
}

QmvPlan qmv_plan_for(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  return plan_qmv(std::min<int64_t>(std::max<int64_t>(M, 1), kQmvMaxM), N, K, group_size, bits);
}

// The kernel route of a call with more than 32 activation rows
// (MLXQ_ALGO_AUTO), from graph-timed A/B runs of every route at the
// Llama-3-8B shapes, M = 64 .. 4096, Q4 and Q8 (µs, Q4: qmm / library GEMM):
//  * up to 64 rows: the batched-decode kernels over 32-row chunks;
//  * the hand-written qmm kernel (qmm.hip) up to 2048 rows on down-like
//    matrices (K > N: down M = 2048 206 / 217, M = 1024 123 / 142), up to
//    512 rows on gate/up-like ones (K < N: M = 512 62 / 80) and up to 512
//    rows on square ones;
//  * the library GEMM on the dequantized weight (qmm_lib.hip) above that
//    (gate/up M = 1024 128 / 114, M = 2048 219 / 197; q/o M = 1024 50 / 46;
//    every shape at M = 4096, e.g. down 360 / 325).
enum class Route { Fused, Lib, Chunks };

// Short prefills of gate/up-like matrices on the 64-row streaming form: 65..128
// rows (two row blocks, one round of CUs), measured against the other routes
// (µs, one box): Q4 M = 96 46.7 -> 34.5, M = 128 48.0 -> 35.2, Q8 M = 128
// 47.1 -> 41.5; slower at 64 rows and below (two 32-row decode calls) and from
// 192 (two rounds).  MLXQ_QMV_STREAM64=1 / 0 forces / forbids it.
bool stream64_route(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  const int ov = overrides().stream64;
  if (ov == 0 || !qmv_stream64_eligible(M, N, K, group_size, bits)) return false;
  // default: gate/up-like only (down-like ones at 65..128 rows, with four K
  // splits, measured slower than the library route: Q4 M = 128 41.4 vs 37.1)
  return ov == 1 || (K < N && M > 2 * kQmvMaxM && M <= 4 * kQmvMaxM);
}

Route prefill_route(int64_t M, int64_t N, int64_t K, int group_size) {
  const Overrides& ov = overrides();
  if (ov.qmm_fused) return Route::Fused;
  if (ov.qmm_lib) return Route::Lib;
  if (N <= 16384 && M <= 2 * kQmvMaxM) return Route::Chunks;
  if (!qmm_eligible(K, group_size)) return Route::Lib;
  if (K > N) return M >= 4096 ? Route::Lib : Route::Fused;
  return M >= 1024 ? Route::Lib : Route::Fused;
}

// Workspace of the library's own kernels: split-K partials of the decode
// kernels (also for the 32-row chunks of a longer call) and of the fused
// prefill kernel.
size_t fused_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  const int64_t mq = std::min<int64_t>(M, kQmvMaxM);
  size_t bytes = qmv_plan_for(mq, N, K, group_size, bits).workspace_bytes();
  if (mq >= 2 && qmv_tile_eligible(mq, N, K, group_size, bits))
    bytes = qmv_tile_workspace_bytes(mq, N);  // split-K partials (the M = 1 decode kernel needs none)
  if (M > kQmvMaxM) {
    const size_t qmm = qmm_eligible(K, group_size) ? qmm_workspace_bytes(M, N, K, group_size) : 0;
    bytes = prefill_route(M, N, K, group_size) == Route::Chunks ? std::max(bytes, qmm) : qmm;
  }
  return bytes;
}

int qmatmul_dispatch(const void* x, int64_t M, const uint32_t* wq, const void* scales, const void* biases,
                     const void* bias_vec, int64_t N, int64_t K, int group_size, int bits, void* y, void* workspace,
                     size_t workspace_bytes, int algo, bool allow_lib, void* stream);

}  // namespace

extern "C" int mlxq_qmatmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                           size_t* bytes) {
  clear_error();
  int rc = check_shape(M, N, K, group_size, bits);
  if (rc) return rc;
  if (!bytes) return fail(MLXQ_ERR_INVALID, "qmatmul: null output pointer");
  *bytes = fused_workspace_bytes(M, N, K, group_size, bits);
  if (M > kQmvMaxM && prefill_route(M, N, K, group_size) == Route::Lib)
    *bytes = std::max(*bytes, qmm_lib_workspace_bytes(N, K));
  if (M > kQmvMaxM && stream64_route(M, N, K, group_size, bits)) *bytes = qmv_stream64_workspace_bytes(M, N, K);
  return MLXQ_OK;
}

extern "C" int mlxq_qmatmul_algo(const void* x, int64_t M, const uint32_t* wq, const void* scales,
                                 const void* biases, const void* bias_vec, int64_t N, int64_t K, int group_size,
                                 int bits, void* y, void* workspace, size_t workspace_bytes, int algo,
                                 void* stream) {
  clear_error();
  return qmatmul_dispatch(x, M, wq, scales, biases, bias_vec, N, K, group_size, bits, y, workspace, workspace_bytes,
                          algo, true, stream);
}

namespace {

int qmatmul_dispatch(const void* x, int64_t M, const uint32_t* wq, const void* scales, const void* biases,
                     const void* bias_vec, int64_t N, int64_t K, int group_size, int bits, void* y, void* workspace,
                     size_t workspace_bytes, int algo, bool allow_lib, void* stream) {
  int rc = check_shape(M, N, K, group_size, bits);
  if (rc) return rc;
  if (algo < MLXQ_ALGO_AUTO || algo > MLXQ_ALGO_QMM_LIB)
    return fail(MLXQ_ERR_INVALID, "qmatmul: unknown algo " + std::to_string(algo));
  if (M == 0) return MLXQ_OK;
  if (!x || !wq || !scales || !biases || !y) return fail(MLXQ_ERR_INVALID, "qmatmul: null pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(wq)) & 15u)
    return fail(MLXQ_ERR_INVALID, "qmatmul: x and wq must be 16-byte aligned");
  if (algo == MLXQ_ALGO_QMM_LIB)
    return launch_qmm_lib(static_cast<const uint16_t*>(x), M, wq, static_cast<const uint16_t*>(scales),
                          static_cast<const uint16_t*>(biases), static_cast<const uint16_t*>(bias_vec), N, K,
                          group_size, bits, static_cast<uint16_t*>(y), workspace, workspace_bytes,
                          as_stream(stream));
  if (algo == MLXQ_ALGO_AUTO && M > kQmvMaxM) {
    if (stream64_route(M, N, K, group_size, bits) && x && wq && scales && biases && y) {
      rc = launch_qmv_stream64(static_cast<const uint16_t*>(x), M, wq, static_cast<const uint16_t*>(scales),
                               static_cast<const uint16_t*>(biases), static_cast<const uint16_t*>(bias_vec), N, K,
                               group_size, bits, static_cast<uint16_t*>(y), workspace, workspace_bytes,
                               as_stream(stream));
      if (rc != MLXQ_ERR_UNSUPPORTED) return rc;  // else (workspace too small for the K split): the other routes
      clear_error();
    }
    const Route r = prefill_route(M, N, K, group_size);
    if (r == Route::Lib && allow_lib && workspace && workspace_bytes >= qmm_lib_workspace_bytes(N, K)) {
      rc = launch_qmm_lib(static_cast<const uint16_t*>(x), M, wq, static_cast<const uint16_t*>(scales),
                          static_cast<const uint16_t*>(biases), static_cast<const uint16_t*>(bias_vec), N, K,
                          group_size, bits, static_cast<uint16_t*>(y), workspace, workspace_bytes,
                          as_stream(stream));
      if (rc != MLXQ_ERR_UNSUPPORTED) return rc;  // else (no library algorithm): the fused kernel
      clear_error();
    }
    if (r == Route::Chunks && (!fused_workspace_bytes(kQmvMaxM, N, K, group_size, bits) ||
                               (workspace && workspace_bytes >= fused_workspace_bytes(kQmvMaxM, N, K, group_size, bits)))) {
      for (int64_t m0 = 0; m0 < M; m0 += kQmvMaxM) {
        rc = qmatmul_dispatch(static_cast<const uint16_t*>(x) + m0 * K, std::min<int64_t>(kQmvMaxM, M - m0), wq,
                              scales, biases, bias_vec, N, K, group_size, bits, static_cast<uint16_t*>(y) + m0 * N,
                              workspace, workspace_bytes, MLXQ_ALGO_QMV, false, stream);
        if (rc) return rc;
      }
      return MLXQ_OK;
    }
  }
  if (algo == MLXQ_ALGO_AUTO) algo = M <= kQmvMaxM ? MLXQ_ALGO_QMV : MLXQ_ALGO_QMM;
  if (algo == MLXQ_ALGO_QMM && !qmm_eligible(K, group_size)) algo = MLXQ_ALGO_QMV;  // 32-row chunks

  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* sp = static_cast<const uint16_t*>(scales);
  const uint16_t* bp = static_cast<const uint16_t*>(biases);
  const uint16_t* bias = static_cast<const uint16_t*>(bias_vec);
  uint16_t* yp = static_cast<uint16_t*>(y);
  hipStream_t st = as_stream(stream);

  if (algo == MLXQ_ALGO_QMM)
    return launch_qmm(xp, M, wq, sp, bp, bias, N, K, group_size, bits, yp, workspace, workspace_bytes, st);

  // Kernel per shape, from measurements at the Llama-3-8B projection shapes:
  // the vector-ALU kernel at M = 1 (and M = 2 on gate/up), the LDS-shared
  // tile kernel where qmv_tile_preferred says, the block kernel otherwise.
  // MLXQ_QMV_MFMA=1 never takes the vector-ALU kernel, MLXQ_QMV_DOT_ALL=1
  // takes it for every eligible M <= 4.
  // whole rows per wave (qmv_row.hip) where K*bits/8 is a whole number of
  // 1 KB load instructions: at M = 1, and at M = 2..4 for short matrices (N
  // <= 2048: k/v 6.1 -> 5.6 us Q4, 6.9 -> 5.1 Q8 at M = 4; on taller ones
  // its per-row decode and LDS reads make it slower than the kernels below).
  // MLXQ_QMV_NO_ROW=1 skips it, MLXQ_QMV_ROW_ALL=1 takes it for every M <= 4.
  const Overrides& ov = overrides();
  // M = 2: also on the taller matrices except Q4 gate/up-like ones (Q8 gate
  // 17.0 -> 14.4 us, Q8 q 7.0 -> 6.3, Q4 q 6.0 -> 5.7; Q4 gate stays on qmv_dot)
  const bool gate_like = K < N && N * K >= (int64_t(1) << 25);
  // M = 3: Q8 gate/up-like ones too (19.42 -> 16.82 us; the other shapes at parity or slower)
  const bool row_m2 = (M == 2 && !(bits == 4 && gate_like)) || (M == 3 && bits == 8 && gate_like);
  if (qmv_row_eligible(M, N, K, group_size, bits) && (M == 1 || row_m2 || N <= 2048 || ov.qmv_row_all) &&
      !ov.qmv_no_row && !ov.qmv_mfma)
    return launch_qmv_row(xp, M, wq, sp, bp, bias, N, K, group_size, bits, yp, st);
  if (M <= kQmvDotMaxM && qmv_dot_eligible(M, N, K, group_size, bits) && !ov.qmv_mfma &&
      (qmv_dot_preferred(M, N, K, bits) || ov.qmv_dot_all))
    return launch_qmv_dot(xp, M, wq, sp, bp, bias, N, K, group_size, bits, yp, st);

  // batched decode: activations shared through LDS, K split across
  // workgroups (qmv_tile.hip), where measured faster than the block kernel
  // below.  MLXQ_QMV_TILE_ALL=1 takes it for every eligible shape,
  // MLXQ_QMV_LEGACY=1 never.
  if (M <= kQmvMaxM && qmv_tile_eligible(M, N, K, group_size, bits) &&
      (qmv_tile_preferred(M, N, K, bits) || ov.qmv_tile_all) && !ov.qmv_legacy) {
    rc = launch_qmv_tile(xp, M, wq, sp, bp, bias, N, K, group_size, bits, yp, workspace, workspace_bytes, st);
    if (rc != MLXQ_ERR_UNSUPPORTED) return rc;  // else: no split fits the workspace, use the block kernel
  }

  // qmv in chunks of at most 32 activation rows (one launch for decode shapes)
  const QmvPlan full = qmv_plan_for(M, N, K, group_size, bits);
  if (full.workspace_bytes() > 0) {
    if (!workspace || workspace_bytes < full.workspace_bytes())
      return fail(MLXQ_ERR_WORKSPACE, "qmatmul: workspace of " + std::to_string(full.workspace_bytes()) +
                                          " bytes required, got " + std::to_string(workspace_bytes));
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
      return fail(MLXQ_ERR_WORKSPACE, "qmatmul: workspace must be 256-byte aligned");
  }
  for (int64_t m0 = 0; m0 < M; m0 += kQmvMaxM) {
    const int64_t mc = std::min<int64_t>(kQmvMaxM, M - m0);
    const QmvPlan p = plan_qmv(mc, N, K, group_size, bits);
    rc = launch_qmv(p, xp + m0 * K, mc, wq, sp, bp, bias, N, K, group_size, bits, yp + m0 * N, st);
    if (rc) return rc;
  }
  return MLXQ_OK;
}

}  // namespace

extern "C" int mlxq_qmatmul(const void* x, int64_t M, const uint32_t* wq, const void* scales, const void* biases,
                            const void* bias_vec, int64_t N, int64_t K, int group_size, int bits, void* y,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return mlxq_qmatmul_algo(x, M, wq, scales, biases, bias_vec, N, K, group_size, bits, y, workspace,
                           workspace_bytes, MLXQ_ALGO_AUTO, stream);
}

extern "C" int mlxq_qmatmul_fused(const void* x, int64_t M, int64_t K, const void* norm_weight, float eps,
                                  int kv_heads, int head_dim, int groups, const mlxq_projection* proj, int nproj,
                                  int swiglu, int group_size, int bits, void* stream) {
  clear_error();
  if (!proj || nproj < 1 || nproj > 3) return fail(MLXQ_ERR_INVALID, "qmatmul_fused: 1 to 3 projections");
  if (swiglu && nproj != 2) return fail(MLXQ_ERR_UNSUPPORTED, "qmatmul_fused: SwiGLU needs gate and up");
  if (swiglu && !norm_weight && M <= kQmvDotMaxM)
    return fail(MLXQ_ERR_UNSUPPORTED, "qmatmul_fused: SwiGLU without a norm needs more than 4 rows");
  if (norm_weight && groups > 1) return fail(MLXQ_ERR_UNSUPPORTED, "qmatmul_fused: norm and head repeat together");
  for (int i = 0; i < nproj; i++) {
    int rc = check_shape(M, proj[i].N, K, group_size, bits);
    if (rc) return rc;
    if (!proj[i].wq || !proj[i].scales || !proj[i].biases || !proj[i].y)
      return fail(MLXQ_ERR_INVALID, "qmatmul_fused: null projection pointer");
    if (reinterpret_cast<uintptr_t>(proj[i].wq) & 15u)
      return fail(MLXQ_ERR_INVALID, "qmatmul_fused: wq must be 16-byte aligned");
  }
  if (M == 0) return MLXQ_OK;
  if (!x || (reinterpret_cast<uintptr_t>(x) & 15u)) return fail(MLXQ_ERR_INVALID, "qmatmul_fused: bad x");
  if (norm_weight && (reinterpret_cast<uintptr_t>(norm_weight) & 15u))
    return fail(MLXQ_ERR_INVALID, "qmatmul_fused: norm_weight must be 16-byte aligned");
  if (norm_weight && !(eps >= 0.f)) return fail(MLXQ_ERR_INVALID, "qmatmul_fused: eps must be >= 0");
  if (K % 8) return fail(MLXQ_ERR_SHAPE, "qmatmul_fused: K must be a multiple of 8");
  QmvFused f{};
  f.x = static_cast<const uint16_t*>(x);
  f.M = M;
  f.K = K;
  f.x_stride = K;
  f.norm_w = static_cast<const uint16_t*>(norm_weight);
  f.eps = eps;
  if (groups > 1) {
    if (kv_heads <= 0 || head_dim <= 0 || static_cast<int64_t>(kv_heads) * head_dim * groups != K)
      return fail(MLXQ_ERR_SHAPE, "qmatmul_fused: kv_heads * head_dim * groups must equal K");
    f.rep = groups;
    f.rep_hd = head_dim;
    f.x_stride = K / groups;
  }
  f.nproj = nproj;
  for (int i = 0; i < nproj; i++)
    f.proj[i] = QmvProj{proj[i].wq, static_cast<const uint16_t*>(proj[i].scales),
                        static_cast<const uint16_t*>(proj[i].biases), static_cast<const uint16_t*>(proj[i].bias),
                        static_cast<const uint16_t*>(proj[i].residual), static_cast<uint16_t*>(proj[i].y),
                        proj[i].N};
  f.swiglu = swiglu != 0;
  f.group_size = group_size;
  f.bits = bits;
  // 5..32 rows: the whole-K tile form where it covers the shape (every form
  // but SwiGLU); MLXQ_QMV_LEGACY=1 or MLXQ_QMV_NO_TILE_FUSED=1 skips it
  if (M > kQmvDotMaxM && qmv_tile_fused_eligible(f) && !overrides().qmv_legacy && !overrides().qmv_no_tile_fused)
    return launch_qmv_tile_fused(f, as_stream(stream));
  // 5..32 rows, SwiGLU without a norm: gate/up pairs on the streaming form
  if (M > kQmvDotMaxM && qmv_tile_swiglu_eligible(f) && !overrides().qmv_legacy && !overrides().qmv_no_tile_fused)
    return launch_qmv_tile_swiglu(f, as_stream(stream));
  if (M > kQmvDotMaxM) {  // matrix-core form: plain, residual and multi-projection only
    if (f.norm_w || f.swiglu || f.rep > 1 || M > kQmvMaxM)
      return fail(MLXQ_ERR_UNSUPPORTED, "qmatmul_fused: for M > " + std::to_string(kQmvDotMaxM) +
                                            " only the residual / multi-projection forms (M <= 32) are fused");
    return launch_qmv_mfma(f, as_stream(stream));
  }
  // whole-row kernel where it covers the shape (M = 1, rows of 1, 2 or 4 KB:
  // the batch-1 chain's q/k/v, o and gate/up); MLXQ_QMV_NO_ROW=1 skips it
  if (qmv_row_fused_eligible(f) && !overrides().qmv_no_row) return launch_qmv_row_fused(f, as_stream(stream));
  return launch_qmv_dot_fused(f, as_stream(stream));
}

// Down projection + residual add + the next layer's RMSNorm (llama.rs:729-733
// then :698): at 5..32 rows on the tile kernels the split-K sum, the residual
// and the norm share the second launch; elsewhere the unfused calls.
extern "C" int mlxq_qmatmul_add_rms_norm(const void* x, int64_t M, const uint32_t* wq, const void* scales,
                                         const void* biases, const void* bias_vec, int64_t N, int64_t K,
                                         int group_size, int bits, const void* residual, const void* norm_weight,
                                         float eps, void* sum_out, void* y, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  clear_error();
  int rc = check_shape(M, N, K, group_size, bits);
  if (rc) return rc;
  if (M == 0) return MLXQ_OK;
  if (!residual || !norm_weight || !sum_out || !y) return fail(MLXQ_ERR_INVALID, "qmatmul_add_rms_norm: null pointer");
  auto mis = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) != 0; };
  if (mis(residual) || mis(norm_weight) || mis(sum_out) || mis(y))
    return fail(MLXQ_ERR_INVALID, "qmatmul_add_rms_norm: pointers must be 16-byte aligned");
  if (N % 8) return fail(MLXQ_ERR_SHAPE, "qmatmul_add_rms_norm: N must be a multiple of 8");
  if (!(eps >= 0.f)) return fail(MLXQ_ERR_INVALID, "qmatmul_add_rms_norm: eps must be >= 0");
  const Overrides& ov = overrides();
  const uint16_t* res = static_cast<const uint16_t*>(residual);
  uint16_t* so = static_cast<uint16_t*>(sum_out);
  if (M > kQmvDotMaxM && M <= kQmvMaxM && qmv_tile_eligible(M, N, K, group_size, bits) &&
      (qmv_tile_preferred(M, N, K, bits) || ov.qmv_tile_all) && !ov.qmv_legacy &&
      !ov.qmv_no_tile_fused && x && wq && scales && biases) {
    AddNormEpilogue ep{res, static_cast<const uint16_t*>(norm_weight), eps, so, static_cast<uint16_t*>(y), false};
    rc = launch_qmv_tile(static_cast<const uint16_t*>(x), M, wq, static_cast<const uint16_t*>(scales),
                         static_cast<const uint16_t*>(biases), static_cast<const uint16_t*>(bias_vec), N, K,
                         group_size, bits, so, workspace, workspace_bytes, as_stream(stream), &ep);
    if (rc == MLXQ_OK && ep.applied) return MLXQ_OK;
    if (rc == MLXQ_OK) {  // one K slice: the projection is in sum_out
      if ((rc = mlxq_add(res, so, M * N, so, stream))) return rc;
      return mlxq_rms_norm(so, norm_weight, M, N, eps, y, stream);
    }
    if (rc != MLXQ_ERR_UNSUPPORTED) return rc;
    clear_error();
  }
  rc = qmatmul_dispatch(x, M, wq, scales, biases, bias_vec, N, K, group_size, bits, so, workspace, workspace_bytes,
                        MLXQ_ALGO_AUTO, true, stream);
  if (rc) return rc;
  if ((rc = mlxq_add(res, so, M * N, so, stream))) return rc;  // element-wise, in place
  return mlxq_rms_norm(so, norm_weight, M, N, eps, y, stream);
}

// ---------------------------------------------------------------- route query

extern "C" int mlxq_qmatmul_route(int64_t M, int64_t N, int64_t K, int group_size, int bits, size_t workspace_bytes,
                                  int algo, int noalloc, char* buf, size_t buf_len) {
  clear_error();
  // dummy 256-byte-aligned pointers: nothing is launched or dereferenced
  void* const p = reinterpret_cast<void*>(uintptr_t(1) << 20);
  const uint32_t* const wq = static_cast<const uint32_t*>(p);
  if (noalloc) {
    if (int rc = check_shape(M, N, K, group_size, bits)) return rc;
    const size_t need = fused_workspace_bytes(M, N, K, group_size, bits);
    if (need > mlxq_qmatmul_noalloc_max_scratch())  // the call itself refuses such shapes before any launch
      return fail(MLXQ_ERR_WORKSPACE, "qmatmul_route: the no-alloc call refuses this shape (" + std::to_string(need) +
                                          " bytes of scratch needed)");
    return run_route_query([&] { return qmatmul_dispatch(p, M, wq, p, p, nullptr, N, K, group_size, bits, p,
                                                         need ? p : nullptr, need, MLXQ_ALGO_AUTO, false, nullptr); },
                           buf, buf_len);
  }
  return run_route_query([&] { return qmatmul_dispatch(p, M, wq, p, p, nullptr, N, K, group_size, bits, p,
                                                       workspace_bytes ? p : nullptr, workspace_bytes, algo, true,
                                                       nullptr); },
                         buf, buf_len);
}

// ---------------------------------------------------------------- no-alloc

namespace {

// Library-owned scratch of the allocation-free entry point: the split-K
// partial sums mlxq_qmatmul keeps in the caller's workspace.  Each device
// holds its own copy for the life of the process.  In host code `scratch`
// is only a handle for hipGetSymbolAddress: kernels receive the per-device
// address it returns.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// This device's address of `scratch`, looked up once per device (with that
// device current) and kept.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MLXQ_ERR_DEVICE, std::string("qmatmul_noalloc: hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MLXQ_ERR_DEVICE, "qmatmul_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MLXQ_ERR_DEVICE, std::string("qmatmul_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MLXQ_OK;
}

}  // namespace

extern "C" size_t mlxq_qmatmul_noalloc_max_scratch(void) { return kScratchBytes; }

extern "C" int mlxq_qmatmul_noalloc(const void* x, int64_t M, const uint32_t* wq, const void* scales,
                                    const void* biases, const void* bias_vec, int64_t N, int64_t K, int group_size,
                                    int bits, void* y, void* stream) {
  clear_error();
  size_t need = 0;
  int rc = check_shape(M, N, K, group_size, bits);
  if (rc) return rc;
  need = fused_workspace_bytes(M, N, K, group_size, bits);
  if (need > kScratchBytes)
    return fail(MLXQ_ERR_WORKSPACE, "qmatmul_noalloc: this shape needs " + std::to_string(need) +
                                        " bytes of scratch; the library's fixed scratch holds " +
                                        std::to_string(kScratchBytes) + " (use mlxq_qmatmul with a workspace)");
  void* ws = nullptr;
  if (need) {
    rc = scratch_ptr(&ws);
    if (rc) return rc;
  }
  // the same kernels as mlxq_qmatmul with a workspace of exactly `need`
  // bytes; every partial they read back is written earlier in the same
  // call, so the scratch needs no clearing
  return qmatmul_dispatch(x, M, wq, scales, biases, bias_vec, N, K, group_size, bits, y, ws, need, MLXQ_ALGO_AUTO,
                          false, stream);
}
