// Launchers of the CosyVoice2 LM sampling step and the speech-token embedding.
#include "vh_launch.hpp"
#include "vh_lm.hpp"

namespace vh {

hipError_t launch_lm_sample(const float *logits, int n, const LmCfgDev *cfg, LmState *st, int32_t *decoded, float *logp_out,
                            int64_t logp_stride, bool append, hipStream_t s) {
    if (n < 2 || n > kLmMaxN) return hipErrorInvalidValue;
    return launch(k_lm_sample, dim3(1), dim3(kLmThreads), 0, s, logits, int32_t(n), cfg, st, decoded, logp_out,
                  logp_stride, int32_t(append));
}

hipError_t launch_pred_embed(const PredEmbedArgs &a, hipStream_t s) {
    if (a.m <= 0 || a.hd <= 0 || (a.w && (a.cols <= 0 || !a.codes || !a.x || !a.err || (a.type == WT_Q8 || a.type == WT_Q4) && a.cols % 32)))
        return hipErrorInvalidValue;
    return launch(k_pred_embed, dim3(1), dim3(256), 0, s, a);
}

hipError_t launch_mat_gather(const uint8_t *w, const void *scale, int type, int s16, int64_t cols, const int32_t *ids,
                             int64_t n, float *out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n > INT32_MAX || cols <= 0 || (type == WT_Q8 || type == WT_Q4) && cols % 32) return hipErrorInvalidValue;
    return launch(k_mat_gather, dim3(unsigned(n)), dim3(256), 0, s, w, scale, int32_t(type), int32_t(s16), cols, ids, out);
}

hipError_t launch_lm_embed(const LmEmbedArgs &a, hipStream_t s) {
    if (a.hd <= 0 || a.cols <= 0 || (a.type == WT_Q8 || a.type == WT_Q4) && a.cols % 32) return hipErrorInvalidValue;
    return launch(k_lm_embed, dim3(1), dim3(256), 0, s, a);
}

}  // namespace vh
