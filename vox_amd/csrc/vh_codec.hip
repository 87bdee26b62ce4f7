// Launchers of the Qwen3-TTS codec decoder kernels.
#include <algorithm>

#include "vh_codec.hpp"
#include "vh_launch.hpp"

namespace vh {

static dim3 blocks_of(int64_t n) { return dim3(unsigned((n + 255) / 256)); }

hipError_t launch_hist_shift(float *dst, const float *old, const float *x, int64_t ldx, int T, int ctx, int C, hipStream_t s) {
    if (ctx <= 0) return hipSuccess;
    if (T <= 0 || C <= 0 || dst == old) return hipErrorInvalidValue;
    return launch(k_hist_shift, blocks_of(int64_t(ctx) * C), dim3(256), 0, s, dst, old, x, ldx, int32_t(T), int32_t(ctx), int32_t(C));
}

hipError_t launch_dwconv_causal(const float *x, const float *hist, const float *w, const float *b, float *y, int T, int C, int K,
                                hipStream_t s, float *hist_next) {
    if (T <= 0) return hipSuccess;
    if (C <= 0 || K <= 0 || !w || !b || (K > 1 && !hist) || (hist_next && hist_next == hist)) return hipErrorInvalidValue;
    const int64_t n = std::max<int64_t>(int64_t(T), hist_next ? int64_t(K - 1) : 0) * C;
    return launch(k_dwconv_causal, blocks_of(n), dim3(256), 0, s, x, hist, w, b, y, int32_t(T), int32_t(C), int32_t(K), hist_next);
}

hipError_t launch_ola(const float *tmp, const float *tail_old, float *tail_new, const float *bias, float *y, int T, int stride,
                      int K, int co, hipStream_t s, float *snake_y, const float *snake_a, const float *snake_ib) {
    if (T <= 0) return hipSuccess;
    if (stride <= 0 || K < stride || K > 2 * stride || co <= 0 || !bias || (K > stride && (!tail_old || !tail_new || tail_old == tail_new)))
        return hipErrorInvalidValue;
    if (snake_y && (!snake_a || !snake_ib || snake_y == y)) return hipErrorInvalidValue;
    return launch(k_ola, blocks_of((int64_t(T) * stride + K - stride) * co), dim3(256), 0, s, tmp, tail_old, tail_new, bias, y,
                  int32_t(T), int32_t(stride), int32_t(K), int32_t(co), snake_y, snake_a, snake_ib);
}

hipError_t launch_convt_gather(const float *z, const float *bias, float *y, int T, int To, int stride, int K, int pad, int co,
                               hipStream_t s) {
    if (T <= 0 || To <= 0) return hipSuccess;
    if (stride <= 0 || K <= 0 || pad < 0 || co <= 0 || !z || !y) return hipErrorInvalidValue;
    return launch(k_convt_gather, blocks_of(int64_t(To) * co), dim3(256), 0, s, z, bias, y, int32_t(T), int32_t(To),
                  int32_t(stride), int32_t(K), int32_t(pad), int32_t(co));
}

hipError_t launch_codec_rope_ring(float *qkv, int ld, int F, int heads, int kvh, int hd, const float *rope, float *ring_k,
                                  float *ring_v, int R, const int64_t *pos, hipStream_t s) {
    if (F <= 0) return hipSuccess;
    if (hd <= 0 || hd % 2 || heads <= 0 || kvh <= 0 || ld < (heads + 2 * kvh) * hd || R < F || !pos) return hipErrorInvalidValue;
    return launch(k_codec_rope_ring, dim3(unsigned(F)), dim3(256), 0, s, qkv, int32_t(ld), int32_t(heads), int32_t(kvh),
                  int32_t(hd), rope, ring_k, ring_v, int32_t(R), pos);
}

hipError_t launch_codec_attn(const float *qkv, int ld, const float *ring_k, const float *ring_v, int R, int F, int heads, int kvh,
                             int hd, const int64_t *pos, int W, float scale, float *ao, hipStream_t s) {
    if (F <= 0) return hipSuccess;
    // the ring holds the window of every row of the call: R >= W + F - 1
    if (hd <= 0 || hd > 128 || hd % 4 || heads <= 0 || kvh <= 0 || heads % kvh || W <= 0 || W > 1024 || R < W + F - 1 || !pos)
        return hipErrorInvalidValue;
    return launch(k_codec_attn, dim3(unsigned(F), unsigned(heads)), dim3(64), 0, s, qkv, int32_t(ld), ring_k, ring_v, int32_t(R),
                  int32_t(heads), int32_t(kvh), int32_t(hd), pos, int32_t(W), scale, ao);
}

hipError_t launch_scale_acc(float *h, const float *t, const float *sc, int64_t rows, int H, hipStream_t s) {
    const int64_t n = rows * H;
    if (n <= 0) return hipSuccess;
    if (!sc) return hipErrorInvalidValue;
    return launch(k_scale_acc, blocks_of(n), dim3(256), 0, s, h, t, sc, n, int32_t(H));
}

hipError_t launch_clamp1(float *y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    return launch(k_clamp1, blocks_of(n), dim3(256), 0, s, y, n);
}

}  // namespace vh
