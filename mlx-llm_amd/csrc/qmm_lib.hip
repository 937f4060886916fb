// Prefill quantized matmul as dequantize + the library's bf16 GEMM, for
// large M on gfx950.
//
// Reference: QuantizedLinear::forward (src/primitives/quant.rs:56-70) ->
// mlx_rs::ops::quantized_matmul at prefill shapes (MLX's qmm kernels).
//
// At M >= 512-2048 (shape-dependent) the matmul is MFMA-bound and the weight
// traffic is small against it: dequantizing the whole weight once into the
// caller's workspace (N x K bf16, HBM-bound: 2.5 bytes per Q4 code moved)
// and running hipBLASLt's bf16 GEMM on it is faster than the fused LDS
// dequant kernel (qmm.hip), whose dequantization sits on the matrix cores'
// critical path.  The dequantized values are the fused kernel's: bf16(s q +
// b) rounded to nearest even from the same f32 expression, i.e. what MLX's
// qmm places in threadgroup memory; accumulation is f32 in both.
//
// hipBLASLt is driven column-major: y^T [N x M] = W [K x N]^T . x^T [K x M]
// with W = the row-major [N, K] weight read as a column-major K x N matrix
// (op T), x the row-major [M, K] activations read as K x M (op N), y^T the
// row-major [M, N] output as an N x M column-major matrix; the dense bias is
// the GEMM's bias epilogue (one value per row of y^T).  One plan (descriptors
// and the heuristic's first algorithm that fits the workspace) is cached per
// device and shape.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "common.hpp"
#include "qmatmul.hpp"

namespace mlxq {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr size_t kLtWorkspace = size_t(32) << 20;  // hipBLASLt's workspace, carved from the caller's
constexpr int kMaxDev = 64;

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(a);  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

// Units of 8 codes (Q4: one dword, Q8: two) -> 16 bytes of bf16(s * q + b),
// all of a unit in one group (groups are 32..128 codes and rows whole
// groups).  A workgroup covers 1024 consecutive units, thread t units t +
// 256 j: every load and every 16-byte store of a wave is contiguous.
template <int BITS>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(const uint32_t* __restrict__ wq,
                                                           const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ b, u32x4* __restrict__ out,
                                                           int64_t units, int gshift) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 1024 + threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int64_t u = base + 256 * j;
    if (u >= units) break;
    const int64_t g = (u * 8) >> gshift;
    const float sc = bf16_bits_to_f32(s[g]), zz = bf16_bits_to_f32(b[g]);
    uint32_t o[4];
    if constexpr (BITS == 4) {
      const uint32_t q = wq[u];
#pragma unroll
      for (int i = 0; i < 4; i++)
        o[i] = pack2(sc * static_cast<float>((q >> (8 * i)) & 0xFu) + zz,
                     sc * static_cast<float>((q >> (8 * i + 4)) & 0xFu) + zz);
    } else {
      const uint2 q = reinterpret_cast<const uint2*>(wq)[u];
      o[0] = pack2(sc * static_cast<float>(q.x & 0xFFu) + zz, sc * static_cast<float>((q.x >> 8) & 0xFFu) + zz);
      o[1] = pack2(sc * static_cast<float>((q.x >> 16) & 0xFFu) + zz, sc * static_cast<float>(q.x >> 24) + zz);
      o[2] = pack2(sc * static_cast<float>(q.y & 0xFFu) + zz, sc * static_cast<float>((q.y >> 8) & 0xFFu) + zz);
      o[3] = pack2(sc * static_cast<float>((q.y >> 16) & 0xFFu) + zz, sc * static_cast<float>(q.y >> 24) + zz);
    }
    out[u] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
  bool ok = false;
};

std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDev] = {};
std::map<std::tuple<int, int64_t, int64_t, int64_t, bool, int>, LtPlan> g_plans;

int lt_fail(const char* what, hipblasStatus_t st) {
  return fail(MLXQ_ERR_UNSUPPORTED, std::string("qmatmul (library GEMM): ") + what + " failed (status " +
                                         std::to_string(static_cast<int>(st)) + ")");
}

// The cached plan of (device, M, N, K, bias); built on first use (the
// descriptors and the heuristic query allocate nothing on the device).
int get_plan(int dev, int64_t M, int64_t N, int64_t K, bool bias, const LtPlan** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  const int pick = overrides().qmm_lib_algo;  // MLXQ_QMM_LIB_ALGO: the heuristic's i-th algorithm (tuning)
  auto key = std::make_tuple(dev, M, N, K, bias, pick);
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return it->second.ok ? MLXQ_OK : fail(MLXQ_ERR_UNSUPPORTED, "qmatmul (library GEMM): no algorithm for this shape");
  }
  hipblasStatus_t st;
  if (!g_handle[dev]) {
    st = hipblasLtCreate(&g_handle[dev]);
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail("hipblasLtCreate", st);
  }
  LtPlan& p = g_plans[key];
  *out = &p;
  st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail("MatmulDescCreate", st);
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN));
  if (bias) {
    const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bt = HIP_R_16BF;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
  }
  if ((st = hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, N, K)) != HIPBLAS_STATUS_SUCCESS ||
      (st = hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, M, K)) != HIPBLAS_STATUS_SUCCESS ||
      (st = hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, N, M, N)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail("MatrixLayoutCreate", st);
  hipblasLtMatmulPreference_t pref = nullptr;
  st = hipblasLtMatmulPreferenceCreate(&pref);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail("MatmulPreferenceCreate", st);
  const uint64_t maxws = kLtWorkspace;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &maxws, sizeof(maxws));
  hipblasLtMatmulHeuristicResult_t res[16];
  int n = 0;
  st = hipblasLtMatmulAlgoGetHeuristic(g_handle[dev], p.desc, p.a, p.b, p.c, p.c, pref, 16, res, &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail("MatmulAlgoGetHeuristic", st);
  for (int i = 0, valid = 0; i < n; i++) {
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kLtWorkspace && valid++ >= pick) {
      p.algo = res[i].algo;
      p.ws = res[i].workspaceSize;
      p.ok = true;
      break;
    }
  }
  return p.ok ? MLXQ_OK : fail(MLXQ_ERR_UNSUPPORTED, "qmatmul (library GEMM): no algorithm for this shape");
}

size_t weight_bytes(int64_t N, int64_t K) { return (static_cast<size_t>(N) * K * 2 + 255) & ~size_t(255); }

}  // namespace

size_t qmm_lib_workspace_bytes(int64_t N, int64_t K) { return weight_bytes(N, K) + kLtWorkspace; }

int launch_qmm_lib(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (!workspace || workspace_bytes < qmm_lib_workspace_bytes(N, K))
    return fail(MLXQ_ERR_WORKSPACE, "qmatmul (library GEMM): workspace of " +
                                        std::to_string(qmm_lib_workspace_bytes(N, K)) + " bytes required, got " +
                                        std::to_string(workspace_bytes));
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(MLXQ_ERR_WORKSPACE, "qmatmul (library GEMM): workspace must be 256-byte aligned");
  if ((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(b)) & 1u)
    return fail(MLXQ_ERR_INVALID, "qmatmul (library GEMM): scales/biases must be 2-byte aligned");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MLXQ_ERR_UNSUPPORTED, "qmatmul (library GEMM): shape not supported");
  int dev = 0;
  hipError_t he = hipGetDevice(&dev);
  if (he != hipSuccess || dev < 0 || dev >= kMaxDev)
    return fail(MLXQ_ERR_DEVICE, "qmatmul (library GEMM): no current device");
  const LtPlan* p = nullptr;
  if (!route_query_active())
    if (int rc = get_plan(dev, M, N, K, bias != nullptr, &p)) return rc;

  uint16_t* wd = static_cast<uint16_t*>(workspace);
  void* ltws = static_cast<char*>(workspace) + weight_bytes(N, K);
  const int64_t units = N * K / 8;
  const int gshift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
  const dim3 grid(static_cast<unsigned>(ceil_div(units, 1024)));
  if (bits == 4)
    MLXQ_LAUNCH(dequant_bf16_kernel<4>, grid, dim3(256), 0, st, wq, s, b, reinterpret_cast<u32x4*>(wd), units,
                       gshift);
  else
    MLXQ_LAUNCH(dequant_bf16_kernel<8>, grid, dim3(256), 0, st, wq, s, b, reinterpret_cast<u32x4*>(wd), units,
                       gshift);
  if (int rc = check_launch("qmm_lib dequant")) return rc;
  if (route_query_active()) {  // no handle, no plan: the GEMM's place in the route only
    route_query_note("hipBLASLt GEMM");
    return MLXQ_OK;
  }

  const float alpha = 1.f, beta = 0.f;
  hipblasStatus_t ls;
  {
    // the bias pointer lives in the shared descriptor: set and enqueue
    // under the lock (the enqueue reads it)
    std::unique_lock<std::mutex> lk(g_mu, std::defer_lock);
    if (bias) {
      lk.lock();
      const void* bp = bias;
      hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp));
    }
    ls = hipblasLtMatmul(g_handle[dev], p->desc, &alpha, wd, p->a, x, p->b, &beta, y, p->c, y, p->c, &p->algo, ltws,
                         p->ws, st);
  }
  if (ls != HIPBLAS_STATUS_SUCCESS) return lt_fail("hipblasLtMatmul", ls);
  return MLXQ_OK;
}

}  // namespace mlxq
