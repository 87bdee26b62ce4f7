// Instantiations of the f32-activation GEMV (F32 / F16 / BF16 weights, and Q8 with m > 8) and the
// shape-based tile choice shared by all GEMV launches.
#include "vh_gemv_dispatch.hpp"

namespace vh {

hipError_t launch_gemv_flt(int wt, int pro, int epi, int M, int R, const GemvArgs &a, hipStream_t s) {
    switch (wt) {
        case WT_F32: return dispatch_flt<WT_F32>(pro, epi, M, R, a, s);
        case WT_F16: return dispatch_flt<WT_F16>(pro, epi, M, R, a, s);
        case WT_BF16: return dispatch_flt<WT_BF16>(pro, epi, M, R, a, s);
        case WT_Q8: return dispatch_flt<WT_Q8>(pro, epi, M, R, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(int wt, bool int_path, int pro, int epi, const GemvArgs &a, hipStream_t s) {
    if (a.m <= 0) return hipSuccess;
    // Rows per wave: enough waves to cover the 256 CUs with at least one block each, with R x IT = 4
    // 16-byte loads in flight per lane either way.
    int R = a.rows >= 4096 ? 4 : a.rows >= 2048 ? 2 : 1;
    if (epi == EPI_SWIGLU && R == 1) R = 2;
    if (int_path) {
        const int M = a.m <= 1 ? 1 : a.m <= 2 ? 2 : a.m <= 4 ? 4 : a.m <= 8 ? 8 : 0;
        if (!M) return hipErrorInvalidValue;
        if (wt == WT_Q8) return launch_gemv_int_q8(pro, epi, M, R, a, s);
        if (wt == WT_Q4) return launch_gemv_int_q4(pro, epi, M, R, a, s);
        return hipErrorInvalidValue;
    }
    const int M = a.m <= 1 ? 1 : a.m <= 4 ? 4 : 0;
    if (!M) return hipErrorInvalidValue;
    return launch_gemv_flt(wt, pro, epi, M, R, a, s);
}

}  // namespace vh
