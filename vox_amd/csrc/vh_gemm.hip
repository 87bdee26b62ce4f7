// Instantiations of the f32 MFMA GEMM (multi-row passes) and the attention-partials merge.
#include "vh_gemm.hpp"
#include "vh_launch.hpp"

namespace vh {

template <int WT, int EPI>
static hipError_t gemm_run(const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s) {
    const dim3 grid((g.n + kGemmBN - 1) / kGemmBN, (g.m + kGemmBM - 1) / kGemmBM);
    return launch(k_gemm_f32<WT, EPI>, grid, dim3(256), 0, s, w, scale, A, g);
}

template <int WT>
static hipError_t gemm_epi(int epi, const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s) {
    switch (epi) {
        case EPI_STORE: return gemm_run<WT, EPI_STORE>(w, scale, A, g, s);
        case EPI_ACC: return gemm_run<WT, EPI_ACC>(w, scale, A, g, s);
        case EPI_SWIGLU: return gemm_run<WT, EPI_SWIGLU>(w, scale, A, g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(int wt, int epi, const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s) {
    if (g.m <= 0) return hipSuccess;
    if (g.K % 8 || g.n <= 0) return hipErrorInvalidValue;
    if (epi == EPI_SWIGLU && g.n % 2) return hipErrorInvalidValue;
    switch (wt) {
        case WT_F32: return gemm_epi<WT_F32>(epi, w, scale, A, g, s);
        case WT_F16: return gemm_epi<WT_F16>(epi, w, scale, A, g, s);
        case WT_BF16: return gemm_epi<WT_BF16>(epi, w, scale, A, g, s);
        case WT_Q8: return g.K % 32 ? hipErrorInvalidValue : gemm_epi<WT_Q8>(epi, w, scale, A, g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_merge(const AttnPartials &P, float *ao, int m, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (P.hd > 128) return hipErrorInvalidValue;
    return launch(k_attn_merge, dim3(P.heads, m), dim3(P.hd), 0, s, P, ao);
}

}  // namespace vh
