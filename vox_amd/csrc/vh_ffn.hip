// vh_ffn.hip — launchers of the fused decode FFN (k_ffn_int), the down-panel repack and the accumulator fold.
#include <cstdlib>

#include "vh_ffn.hpp"
#include "vh_launch.hpp"

namespace vh {

// Blocks per 32-column group (each takes H / parts of the down rows). VOXHIP_FFN_PARTS overrides it (tuning).
int ffn_parts() {
    static const int p = [] {
        const char *e = std::getenv("VOXHIP_FFN_PARTS");
        const int v = e ? std::atoi(e) : 1;
        return v == 2 || v == 4 ? v : 1;
    }();
    return p;
}

namespace {
template <int WT, int GIT>
hipError_t ffn_by_dl(int dl, const FfnArgs &a, dim3 grid, hipStream_t s) {
    switch (dl) {
        case 1: return launch(k_ffn_int<WT, GIT, 1>, grid, dim3(kFfnThreads), 0, s, a);
        case 2: return launch(k_ffn_int<WT, GIT, 2>, grid, dim3(kFfnThreads), 0, s, a);
        case 4: return launch(k_ffn_int<WT, GIT, 4>, grid, dim3(kFfnThreads), 0, s, a);
        case 8: return launch(k_ffn_int<WT, GIT, 8>, grid, dim3(kFfnThreads), 0, s, a);
        default: return hipErrorInvalidValue;
    }
}
template <int WT>
hipError_t ffn_by_git(int git, int dl, const FfnArgs &a, dim3 grid, hipStream_t s) {
    switch (git) {
        case 1: return ffn_by_dl<WT, 1>(dl, a, grid, s);
        case 2: return ffn_by_dl<WT, 2>(dl, a, grid, s);
        default: return hipErrorInvalidValue;
    }
}
int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p *= 2;
    return p;
}
}  // namespace

bool ffn_shape_ok(int wt, int H, int I) {
    // I <= 32768: at most 1024 groups add into one accumulator row (the fixed-point terms' range)
    return (wt == WT_Q8 || wt == WT_Q4 || wt == WT_Q4H) && H > 0 && I > 0 && H % 32 == 0 && I % 32 == 0 && H <= kFfnMaxH &&
           I <= 32 * 1024;
}

hipError_t launch_ffn(int wt, const FfnArgs &a0, hipStream_t s) {
    FfnArgs a = a0;
    a.status = status_word();
    if (!ffn_shape_ok(wt, a.H, a.I) || !a.gu || !a.gu_s || !a.dp || !a.dp_s || !a.x || !a.gamma || !a.acc)
        return hipErrorInvalidValue;
    if (a.parts != 1 && a.parts != 2 && a.parts != 4) return hipErrorInvalidValue;
    const bool q8 = wt == WT_Q8;
    const int nchunk = a.H / (q8 ? 16 : 32), cpr = q8 ? 2 : 1;
    const int git = pow2_at_least((nchunk + 63) / 64);
    const int dl = pow2_at_least((a.H / a.parts * cpr + kFfnThreads - 1) / kFfnThreads);
    const int G = a.I / 32;
    const dim3 grid(unsigned((G + 7) / 8 * 8 * a.parts));
    switch (wt) {
        case WT_Q8: return ffn_by_git<WT_Q8>(git, dl, a, grid, s);
        case WT_Q4: return ffn_by_git<WT_Q4>(git, dl, a, grid, s);
        case WT_Q4H: return ffn_by_git<WT_Q4H>(git, dl, a, grid, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_panel_pack(int wt, const uint8_t *w, const void *scale, int H, int I, uint8_t *pw, void *ps, hipStream_t s) {
    if (!ffn_shape_ok(wt, H, I)) return hipErrorInvalidValue;
    const int64_t n = int64_t(H) * (I / 32);
    const dim3 grid(unsigned((n + 255) / 256)), block(256);
    switch (wt) {
        case WT_Q8: return launch(k_panel_pack<WT_Q8>, grid, block, 0, s, w, scale, H, I, pw, ps);
        case WT_Q4: return launch(k_panel_pack<WT_Q4>, grid, block, 0, s, w, scale, H, I, pw, ps);
        case WT_Q4H: return launch(k_panel_pack<WT_Q4H>, grid, block, 0, s, w, scale, H, I, pw, ps);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_acc_fold(float *h, int64_t *acc, int H, hipStream_t s) {
    if (H <= 0 || !h || !acc) return hipErrorInvalidValue;
    return launch(k_acc_fold, dim3(unsigned((H + 255) / 256)), dim3(256), 0, s, h, acc, H);
}

}  // namespace vh
