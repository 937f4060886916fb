// Internal interface between the qmatmul dispatcher and its kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

namespace mlxq {

// Workspace layout shared by every qmv shape: a fixed ticket area (one u32
// per 64-row tile, always left zero) followed by f32 split-K partials.  The
// ticket area never moves, so partials of one shape cannot land on the
// tickets of another.
constexpr size_t kTicketBytes = 64 * 1024;
constexpr int64_t kMaxRowTiles = kTicketBytes / sizeof(uint32_t);  // N <= 1,048,576

// qmv launch geometry: row tiles of 64 weight rows x K-splits.
struct QmvPlan {
  int64_t row_tiles;
  int64_t splits;
  int64_t groups_per_split;
  int unroll;
  size_t partial_bytes;  // f32 [splits, M, N] when splits > 1
  size_t workspace_bytes() const { return splits > 1 ? kTicketBytes + partial_bytes : 0; }
};

constexpr int64_t kQmvMaxM = 32;

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits);
int launch_qmv(const QmvPlan& p, const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s,
               const uint16_t* b, const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
               void* workspace, hipStream_t st);

// qmm: LDS-dequant bf16 MFMA GEMM, any M, K % 64 == 0.  No workspace.
int launch_qmm(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y, hipStream_t st);

}  // namespace mlxq
