// GQA head-repeat form of the vector-ALU decode GEMV (kernel: qmv_dot_kernel.hpp).
#include "qmv_dot_kernel.hpp"

namespace mlxq {
namespace dot {
template int dispatch<kRepeat>(int64_t, int, int, const Cfg&, const Params&, hipStream_t, int*);
}  // namespace dot
}  // namespace mlxq
