// Instantiations of the int8-activation GEMV for Q4 weights.
#include "vh_gemv_dispatch.hpp"

namespace vh {
hipError_t launch_gemv_int_q4(int pro, int epi, int M, int R, const GemvArgs &a, hipStream_t s) {
    return dispatch_int<WT_Q4>(pro, epi, M, R, a, s);
}
}  // namespace vh
