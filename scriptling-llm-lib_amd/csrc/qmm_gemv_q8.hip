// GEMV launch chain for one weight format (see qmm_gemv_kernel.hpp).
#include "qmm_gemv_kernel.hpp"

namespace sllm {
namespace gemv {
template sllm_status launch_mt<SLLM_Q8_0>(int, int, int, const SegTable &, const float *, int, int, int, int, int, int,
                                     size_t, hipStream_t);
}  // namespace gemv
}  // namespace sllm
