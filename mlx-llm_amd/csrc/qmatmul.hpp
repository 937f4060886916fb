// Internal interface between the qmatmul dispatcher and its kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

namespace mlxq {

// qmv launch geometry: workgroups of 16*sub weight rows over the whole K.
struct QmvPlan {
  int64_t row_tiles;
  int sub;
  int unroll;
  bool wide;  // 16-byte-per-lane chunk loader (else 8-byte group loader)
  size_t workspace_bytes() const { return 0; }
};

constexpr int64_t kQmvMaxM = 32;

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits);
int launch_qmv(const QmvPlan& p, const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s,
               const uint16_t* b, const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
               hipStream_t st);

// qmv_row: decode GEMV (M <= 4), whole rows per wave, 1 KB loads (qmv_row.hip).
bool qmv_row_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits);
int launch_qmv_row(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   hipStream_t st);

// qmv_dot: vector-ALU decode GEMV for M <= kQmvDotMaxM (no MFMA padding).
constexpr int64_t kQmvDotMaxM = 4;
bool qmv_dot_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits);
size_t qmv_dot_lds_bytes(int64_t M, int64_t K, int bits, int sub);
int launch_qmv_dot(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   hipStream_t st);

// Fused decode GEMV: up to 3 projections of the same activations (optionally
// RMS-normalized or GQA head-repeated while staged), each with an optional
// residual added to its bf16 output; or gate/up with the SwiGLU epilogue.
struct QmvProj {
  const uint32_t* wq;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* bias;  // [N] or null
  const uint16_t* res;   // [M, N] residual or null
  uint16_t* y;           // [M, N]
  int64_t N;
};
struct QmvFused {
  const uint16_t* x;
  int64_t M, K, x_stride;
  const uint16_t* norm_w;  // [K] or null
  float eps;
  int rep_hd, rep;         // rep > 1: activation k reads source (k / (rep_hd*rep)) * rep_hd + k % rep_hd
  int nproj;
  QmvProj proj[3];
  bool swiglu;             // proj[0] = gate, proj[1] = up; y = silu(gate) * up into proj[0].y
  int group_size, bits;
};
int launch_qmv_dot_fused(const QmvFused& f, hipStream_t st);
// the same fused forms on the whole-row kernel (qmv_row.hip): M = 1, K*bits/8
// of 1, 2 or 4 KB
bool qmv_row_fused_eligible(const QmvFused& f);
int launch_qmv_row_fused(const QmvFused& f, hipStream_t st);

// qmv_mfma: matrix-core GEMV for M <= kQmvMaxM with the streaming structure
// of qmv_dot; plain and residual / multi-projection forms (no norm, SwiGLU or
// head repeat: those return MLXQ_ERR_UNSUPPORTED).
bool qmv_mfma_eligible(int64_t M, int64_t K, int group_size, int bits);
int launch_qmv_mfma(const QmvFused& f, hipStream_t st);

// qmv_tile: matrix-core GEMV for batched decode (M <= kQmvMaxM) with the
// activations shared through LDS and an optional split of K across
// workgroups (f32 partials in the caller's workspace, added by a second
// kernel).
// Returns MLXQ_ERR_UNSUPPORTED, without launching or setting an error, when
// the shape would need a split the workspace cannot hold.
bool qmv_tile_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits);
// the fused forms (head repeat, residual, up to 3 projections) on the
// whole-K tile form: 5 <= M <= 32, K one workgroup slice, no norm or SwiGLU
bool qmv_tile_fused_eligible(const QmvFused& f);
int launch_qmv_tile_fused(const QmvFused& f, hipStream_t st);
// SwiGLU of gate/up (no norm) on the streaming tile form, 5 <= M <= 32
bool qmv_tile_swiglu_eligible(const QmvFused& f);
int launch_qmv_tile_swiglu(const QmvFused& f, hipStream_t st);
size_t qmv_tile_workspace_bytes(int64_t M, int64_t N);
bool qmv_tile_preferred(int64_t M, int64_t N, int64_t K, int bits);
bool qmv_dot_preferred(int64_t M, int64_t N, int64_t K, int bits);  // M <= 4: vector-ALU kernel
// Short prefills (33..256 rows) of large matrices on the streaming form with
// 64 activation rows per workgroup (down-like ones with four K splits).
bool qmv_stream64_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits);
size_t qmv_stream64_workspace_bytes(int64_t M, int64_t N, int64_t K);
int launch_qmv_stream64(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                        const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                        void* workspace, size_t workspace_bytes, hipStream_t st);

// The decode chain's down projection with the residual add and the next
// RMSNorm in the second kernel of a split-K launch: instead of y, sum_out =
// bf16(res + bf16(sum + bias)) and y_norm = rms_norm(sum_out) (one workgroup
// per row).  applied: the launch took it (split K); else y was written.
struct AddNormEpilogue {
  const uint16_t* res;
  const uint16_t* norm_w;
  float eps;
  uint16_t* sum_out;
  uint16_t* y_norm;
  bool applied;
};
int launch_qmv_tile(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                    const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                    void* workspace, size_t workspace_bytes, hipStream_t st, AddNormEpilogue* ep = nullptr);

int launch_split_add_norm(const float* part, const uint16_t* bias, int64_t M, int64_t N, int splits,
                          const AddNormEpilogue& ep, hipStream_t st);
// y = bf16(sum over the splits of part[split][M][N], in split order, + bias):
// the second kernel of every split-K launch.
int launch_split_reduce(const float* part, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int splits,
                        hipStream_t st);

// qmm: the prefill GEMM (bf16 MFMA on weights dequantized in registers),
// any M; K % 512 == 0 and K % (8 * group_size) == 0 (qmm_eligible).  Shapes
// whose tiles leave most CUs idle split K (qmm_split_k slices, f32 partials
// in the workspace); without a workspace large enough the call runs unsplit.
constexpr int kQmmMaxSplits = 8;
bool qmm_eligible(int64_t K, int group_size);
int qmm_split_k(int64_t M, int64_t N, int64_t K, int group_size);
size_t qmm_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size);
// prefill as dequantize into the workspace + hipBLASLt bf16 GEMM (qmm_lib.hip)
size_t qmm_lib_workspace_bytes(int64_t N, int64_t K);
int launch_qmm_lib(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   void* workspace, size_t workspace_bytes, hipStream_t st);
int launch_qmm(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y, void* workspace,
               size_t workspace_bytes, hipStream_t st);

}  // namespace mlxq
