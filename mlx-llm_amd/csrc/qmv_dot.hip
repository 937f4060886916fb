// Host side of the vector-ALU decode GEMV (kernel: qmv_dot_kernel.hpp):
// eligibility, launch configuration, and the plain (F = 0) instantiation.
// The fused forms are instantiated in qmv_dot_norm.hip, qmv_dot_swiglu.hip
// and qmv_dot_repeat.hip so the four compile in parallel.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "qmatmul.hpp"
#include "qmv_dot_kernel.hpp"

namespace mlxq {
namespace dot {

template int dispatch<0>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);

namespace {

// Pieces (8 activations) per thread in the prologue: whole segments.
int prologue_pieces(int64_t M, int64_t K, int bits, int wv) {
  const int64_t segp = 64 * 8 / bits / 4 / 8;
  int64_t pt = ceil_div(M * K / 8, 64 * wv);
  pt = ceil_div(std::max<int64_t>(pt, segp), segp) * segp;
  return static_cast<int>(pt);
}

size_t lds_bytes(int64_t M, int64_t K, int bits, int sub, int wv) {
  const int64_t kl = 64 * 8 / bits / 4;
  // staged activations, segment sums, the cross-wave reduction (which also
  // holds the RMSNorm partial sums before the contraction)
  return static_cast<size_t>(M * K * 2 + M * (K / kl) * 4 + wv * M * 16 * sub * 4);
}

int cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

int call(int f, int64_t M, int gs, int bits, const Cfg& c, const Params& a, hipStream_t st, int* q) {
  if (f == 0) return dispatch<0>(M, gs, bits, c, a, st, q);
  if (f == kNorm) return dispatch<kNorm>(M, gs, bits, c, a, st, q);
  if (f == kRepeat) return dispatch<kRepeat>(M, gs, bits, c, a, st, q);
  return dispatch<kNorm | kSwiGLU>(M, gs, bits, c, a, st, q);
}

}  // namespace
}  // namespace dot

using namespace dot;

size_t qmv_dot_lds_bytes(int64_t M, int64_t K, int bits, int sub) { return lds_bytes(M, K, bits, sub, kMaxWaves); }

bool qmv_dot_eligible(int64_t M, int64_t N, int64_t K, int group_size, int bits) {
  if (M < 1 || M > kQmvDotMaxM) return false;
  if ((K * bits / 8) % 64 || K * bits / 8 < 64 * kRound) return false;  // whole 64-byte chunks, >= one round per row
  const int64_t gb = static_cast<int64_t>(group_size) * bits / 8;
  const int64_t ngr = kRound * (gb >= 64 ? 1 : 64 / gb) / (gb > 64 ? gb / 64 : 1);  // groups per round
  if ((K / group_size) % std::min<int64_t>(ngr, 8)) return false;  // aligned vector loads of round params
  (void)N;
  // activations staged through registers (<= 8 pieces per thread) and LDS
  return prologue_pieces(M, K, bits, kMaxWaves) <= 8 && lds_bytes(M, K, bits, 2, kMaxWaves) <= 160 * 1024;
}

int launch_qmv_dot_fused(const QmvFused& f, hipStream_t st) {
  const int64_t M = f.M, K = f.K;
  if (f.nproj < 1 || f.nproj > kMaxSegs || (f.swiglu && f.nproj != 2))
    return fail(MLXQ_ERR_INVALID, "qmv_dot: bad projection count");
  for (int i = 0; i < f.nproj; i++)
    if (!qmv_dot_eligible(M, f.proj[i].N, K, f.group_size, f.bits))
      return fail(MLXQ_ERR_UNSUPPORTED, "qmv_dot: shape not supported by the decode kernel");
  if (f.swiglu && f.proj[0].N != f.proj[1].N) return fail(MLXQ_ERR_SHAPE, "qmv_dot: gate and up differ in N");
  if (f.rep > 1 && (f.rep_hd <= 0 || f.rep_hd % 8 || K % (static_cast<int64_t>(f.rep_hd) * f.rep)))
    return fail(MLXQ_ERR_SHAPE, "qmv_dot: head repeat does not tile K");
  if (f.swiglu && !f.norm_w) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_dot: SwiGLU form expects a normalized input");
  if (f.rep > 1 && f.norm_w) return fail(MLXQ_ERR_UNSUPPORTED, "qmv_dot: norm and head repeat together");
  const int form = f.swiglu ? (kNorm | kSwiGLU) : f.norm_w ? kNorm : f.rep > 1 ? kRepeat : 0;

  Params a{};
  a.x = f.x;
  a.norm_w = f.norm_w;
  a.eps = f.eps;
  a.K = static_cast<int>(K);
  a.x_stride = static_cast<int>(f.x_stride);
  a.rep = f.rep > 1 ? f.rep : 1;
  a.rep_hd8 = f.rep > 1 ? f.rep_hd / 8 : 1;
  a.rcp_hd8 = 1.0f / static_cast<float>(a.rep_hd8);
  a.rcp_grp = 1.0f / static_cast<float>(a.rep_hd8 * a.rep);
  a.nseg = f.nproj;
  for (int i = 0; i < f.nproj; i++) {
    const QmvProj& P = f.proj[i];
    a.seg[i] = Seg{P.wq, P.s, P.b, P.bias, P.res, P.y, static_cast<int>(P.N), 0};
  }

  // Pick rows per workgroup (16 or 32) and waves per workgroup (4 or 8) so
  // that the whole grid is resident at once (no second, partly filled pass
  // of workgroups), preferring the most waves in flight.  SwiGLU streams 16
  // rows of gate and up in one workgroup, half of its waves on each.
  static const int cus = cu_count();
  const int64_t chunks = K * f.bits / 8 / 64;
  Cfg best;
  int64_t best_pass = -1, best_waves = 0;
  const int forced_sub = overrides().dot_sub, forced_wv = overrides().dot_wv;
  for (int sub = 1; sub <= 2; sub++)
    for (int wv = 4; wv <= 8; wv += 4) {
      if (f.swiglu && sub != 1) continue;
      if (!f.swiglu && ((forced_sub && sub != forced_sub) || (forced_wv && wv != forced_wv))) continue;
      Cfg c;
      c.sub = sub;
      c.wv = wv;
      c.pt = prologue_pieces(M, K, f.bits, wv);
      c.lds = lds_bytes(M, K, f.bits, sub, wv);
      if (c.pt > 8 || c.lds > 160 * 1024) continue;
      for (int i = 0; i < (f.swiglu ? 1 : f.nproj); i++) c.tiles += ceil_div(f.proj[i].N, 16 * sub);
      int nb = 0;
      if (int rc = call(form, M, f.group_size, f.bits, c, a, st, &nb)) return rc;
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
  // each wave owns a contiguous range of whole rounds of chunks
  const int rc = round_chunks(f.bits, f.group_size, best.sub);
  const int kw = f.swiglu ? best.wv / 2 : best.wv;  // waves sharing one row tile's K
  a.cw = static_cast<int>(ceil_div(ceil_div(chunks, kw), rc) * rc);
  const int rows = 16 * best.sub;
  int64_t end = 0;
  for (int i = 0; i < f.nproj; i++) {
    if (!(f.swiglu && i)) end += ceil_div(f.proj[i].N, rows);
    a.seg[i].tile_end = static_cast<int>(end);
  }
  return call(form, M, f.group_size, f.bits, best, a, st, nullptr);
}

int launch_qmv_dot(const uint16_t* x, int64_t M, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, int64_t N, int64_t K, int group_size, int bits, uint16_t* y,
                   hipStream_t st) {
  QmvFused f{};
  f.x = x;
  f.M = M;
  f.K = K;
  f.x_stride = K;
  f.nproj = 1;
  f.proj[0] = QmvProj{wq, s, b, bias, nullptr, y, N};
  f.group_size = group_size;
  f.bits = bits;
  return launch_qmv_dot_fused(f, st);
}

}  // namespace mlxq
