// Launchers of the F5-TTS DiT step kernels (AdaLN modulation, attention, input columns).
#include "vh_f5.hpp"
#include "vh_launch.hpp"

namespace vh {

hipError_t launch_norm_rows(const NormArgs &a0, hipStream_t s) {
    NormArgs a = a0;
    a.status = status_word();
    if (a.R <= 0) return hipSuccess;
    if (a.D <= 0 || a.D % 4 || !a.x || (!a.y && !a.y16) || a.lo_off % 4 || !a.sc || (!a.affine && !a.sh) || !(a.eps > 0.0))
        return hipErrorInvalidValue;
    if (a.D <= 4 * 256) return launch(k_f5_modulate<4, true>, dim3(unsigned((a.R + 3) / 4)), dim3(256), 0, s, a);
    return launch(k_f5_modulate<kNormRegChunks, false>, dim3(unsigned((a.R + 3) / 4)), dim3(256), 0, s, a);
}

hipError_t launch_f5_modulate(const float *x, int64_t R, int D, const float *sc, const float *sh, float *y, _Float16 *y16,
                              int64_t lo_off, hipStream_t s) {
    if (R > INT32_MAX) return hipErrorInvalidValue;
    NormArgs a{};
    a.x = x; a.y = y; a.y16 = y16; a.lo_off = lo_off; a.sc = sc; a.sh = sh;
    a.eps = 1e-6;  // the modulation adds the double 1e-6 (f5.cpp:608-625)
    a.R = int32_t(R); a.D = D;
    return launch_norm_rows(a, s);
}

hipError_t launch_layernorm_rows(const float *x, int64_t R, int D, const float *w, const float *b, float *y, hipStream_t s) {
    if (R > INT32_MAX || !y) return hipErrorInvalidValue;
    NormArgs a{};
    a.x = x; a.y = y; a.sc = w; a.sh = b;
    a.eps = double(1e-6f);  // LayerNorm's float eps 1e-6f, widened (kernels.cpp:721)
    a.R = int32_t(R); a.D = D; a.affine = 1;
    return launch_norm_rows(a, s);
}

hipError_t launch_dwconv(const float *x, const float *w, const float *b, float *y, int64_t R, int C, int K, int seq, hipStream_t s) {
    if (R <= 0) return hipSuccess;
    if (C <= 0 || K <= 0 || K % 2 == 0 || seq <= 0 || R % seq || !w) return hipErrorInvalidValue;
    const int64_t n = R * C;
    return launch(k_dwconv, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, w, b, y, R, int32_t(C), int32_t(K), int32_t(seq));
}

hipError_t launch_f5_fill_x(const float *x, int N, int mel, float *cat, int W, int B, hipStream_t s) {
    const int64_t n = int64_t(B) * N * mel;
    if (n <= 0) return hipSuccess;
    return launch(k_f5_fill_x, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, int32_t(N), int32_t(mel), cat, int32_t(W),
                  int32_t(B));
}

hipError_t launch_f5_attn(const _Float16 *qkv16, int64_t lo_off, float *out, _Float16 *out16, int64_t out_lo, int B, int N,
                          int heads, int hd, int ldvt, int ldo, float scale, hipStream_t s) {
    if (B <= 0 || N <= 0) return hipSuccess;
    if (hd != kF5Hd || heads <= 0 || ldvt < N || ldvt % 64 || lo_off % 8 || ldo % 4 || (!out && !out16)) return hipErrorInvalidValue;
    if ((int64_t(N) + 64) * 2 * heads * hd * 2 > INT32_MAX) return hipErrorInvalidValue;  // the q / k buffer offsets
    F5AttnArgs a{qkv16, lo_off, out, int32_t(N), int32_t(ldo), int32_t(heads * hd), int32_t(ldvt), scale, out16, out_lo};
    // 4 query waves (64 rows) per block; when that leaves fewer blocks than CUs, 2 query waves (32 rows) times 2 key
    // halves
    if (int64_t((N + 63) / 64) * heads * B >= 256)
        return launch(k_f5_attn<4, 1>, dim3(unsigned((N + 63) / 64), unsigned(heads), unsigned(B)), dim3(256), 0, s, a);
    return launch(k_f5_attn<2, 2>, dim3(unsigned((N + 31) / 32), unsigned(heads), unsigned(B)), dim3(256), 0, s, a);
}

}  // namespace vh
