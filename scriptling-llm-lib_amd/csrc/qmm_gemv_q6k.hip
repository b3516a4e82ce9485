// GEMV launch chain for one weight format (see qmm_gemv_kernel.hpp): single /
// multi-weight launches and paired gate / up launches.
#include "qmm_gemv_kernel.hpp"

namespace sllm {
namespace gemv {
template sllm_status launch_mt<SLLM_Q6K_STREAM, false>(int, int, int, const SegTable &, const float *, int, int, int, int,
                                            int, int, size_t, hipStream_t);
template sllm_status launch_mt<SLLM_Q6K_STREAM, true>(int, int, int, const SegTable &, const float *, int, int, int, int,
                                           int, int, size_t, hipStream_t);
}  // namespace gemv
}  // namespace sllm
