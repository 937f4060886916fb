// RMSNorm + SwiGLU-fused form of the vector-ALU decode GEMV (kernel:
// qmv_dot_kernel.hpp): gate and up projections in one launch.
#include "qmv_dot_kernel.hpp"

namespace mlxq {
namespace dot {
template int dispatch<kNorm | kSwiGLU>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);
}  // namespace dot
}  // namespace mlxq
