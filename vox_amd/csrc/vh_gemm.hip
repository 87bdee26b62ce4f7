// Instantiations of the f32 MFMA GEMM (multi-row passes, DiT linears, grouped convolutions) and the
// attention-partials merge.
#include <atomic>
#include <algorithm>

#include "vh_gemm.hpp"
#include "vh_launch.hpp"

namespace vh {

template <int WT, int EPI, int ASRC, int T>
static hipError_t gemm_run(const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, int groups, hipStream_t s) {
    constexpr int B = 32 * T;
    const dim3 grid((g.n + B - 1) / B, (g.m + B - 1) / B, groups);
    return launch(k_gemm_f32<WT, EPI, ASRC, T, T>, grid, dim3(256), 0, s, w, scale, A, g);
}

// F32 weights: the three-product split-f16 kernel (z: groups of a grouped conv, or K slices when g.kchunk is set).
template <int EPI, int ASRC>
static hipError_t x3_run(const uint8_t *w, const float *A, const GemmArgs &g, int z, hipStream_t s) {
    const dim3 grid((g.n + 63) / 64, (g.m + 63) / 64, z);
    return launch(k_gemm_x3<EPI, ASRC>, grid, dim3(256), 0, s, w, A, g);
}

// F32 weights: the split kernel, or k_gemm_f32 (f32 matrix cores, one product) when the weights are too large for
// its scaled f16 halves (g.f32_wide).
template <int EPI, int ASRC>
static hipError_t f32w_run(const uint8_t *w, const float *A, const GemmArgs &g, int z, hipStream_t s) {
    if (g.f32_wide) return gemm_run<WT_F32, EPI, ASRC, 2>(w, nullptr, A, g, z, s);
    return x3_run<EPI, ASRC>(w, A, g, z, s);
}

template <int WT, int EPI, int TM, int TN>
static hipError_t gemm_run_h16(const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s) {
    constexpr int BM = 32 * TM, BN = 32 * TN;
    const dim3 grid((g.n + BN - 1) / BN, (g.m + BM - 1) / BM, g.kchunk ? (g.K + g.kchunk - 1) / g.kchunk : 1);
    // K steps of 64 throughout, A rows 16-byte aligned, and a tile's byte offsets within 32 bits: the buffered pipeline
    if (TM == 2 && TN == 2 && g.K % 64 == 0 && g.kchunk % 64 == 0 && g.lda % 4 == 0 && int64_t(64) * g.lda * 4 <= INT32_MAX &&
        int64_t(64) * g.K * 2 <= INT32_MAX)
        return launch(k_gemm_h16b<WT, EPI>, grid, dim3(256), 0, s, w, scale, A, g);
    return launch(k_gemm_h16<WT, EPI, TM, TN, 64>, grid, dim3(256), 0, s, w, scale, A, g);
}

// Split K for a grid of 64 x 64 tiles too small to fill the CUs with a long K (prefill down projections, small
// matrices): up to 8 slices of K (32 for grids under 64 tiles), each a multiple of 64 columns, summed in order by the
// reduce pass. Slices are
// added until the launch has about kSplitTargetBlocks blocks (two per CU: measured faster than one per CU on the
// 512-row prefill shapes even with the larger reduce).
constexpr int64_t kSplitTargetBlocks = 512;
constexpr int64_t kSplitMaxSmall = 32;
constexpr int64_t kSplitTargetOneRow = 1024;
// The K slices for a split of g (64 x 64 tiles): 0 when the tiles already fill the CUs, K is short or the workspace
// is too small; else the slice count, with *kchunk the slice width (a multiple of 64). A grid of fewer than 192
// tiles gets enough slices for about kSplitTargetBlocks blocks, at most 8, or at most kSplitMaxSmall for grids of
// under 64 tiles (few-row passes over large weights, such as a streaming codec frame's convolutions, whose tiles
// would otherwise each stream megabytes of weights) when their partials fit the workspace.
static int split_plan(const GemmArgs &g, int *kchunk) {
    const int64_t blocks = int64_t((g.n + 63) / 64) * ((g.m + 63) / 64);
    // one row tile: every tile streams its own columns of the weights, so such grids take slices up to about
    // kSplitTargetOneRow blocks (a streaming codec frame's transposed convolutions and pointwise products)
    const bool one_row = g.m <= 64 && blocks < kSplitTargetOneRow / 2;
    if (!g.ws || (blocks >= 192 && !one_row) || g.K < 512) return 0;
    const int64_t target = one_row ? kSplitTargetOneRow : kSplitTargetBlocks;
    const int64_t want = (target + blocks - 1) / blocks;
    auto plan = [&](int64_t cap) {
        int splits = int(std::min<int64_t>(cap, want));
        *kchunk = ((g.K + splits - 1) / splits + 63) / 64 * 64;
        splits = (g.K + *kchunk - 1) / *kchunk;
        return splits < 2 || int64_t(splits) * g.m * g.n > g.ws_cap ? 0 : splits;
    };
    if (want > 8)
        if (const int splits = plan(kSplitMaxSmall)) return splits;
    return plan(8);
}
template <int EPI>
static hipError_t splitk_reduce(const GemmArgs &g, int splits, hipStream_t s) {
    const int nout = EPI == EPI_SWIGLU ? g.n / 2 : g.n;
    const int64_t total = int64_t(g.m) * nout;
    return launch(k_gemm_splitk_reduce<EPI>, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, g, int32_t(splits));
}
template <int WT, int EPI>
static hipError_t gemm_splitk(const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s, bool *done) {
    *done = false;
    if constexpr (EPI != EPI_STORE && EPI != EPI_ACC && EPI != EPI_GATED_ACC && EPI != EPI_SWIGLU && EPI != EPI_ACC_SNAKE &&
                  EPI != EPI_GELU_ERF) {
        return hipSuccess;
    } else {
        GemmArgs gs = g;
        const int splits = split_plan(g, &gs.kchunk);
        if (!splits) return hipSuccess;
        hipError_t e = gemm_run_h16<WT, EPI_STORE, 2, 2>(w, scale, A, gs, s);
        if (e != hipSuccess) return e;
        *done = true;
        return splitk_reduce<EPI>(g, splits, s);
    }
}

// 64 x 64 block tiles: measured faster than 128 x 128 and 128 x 64 on the DiT and prefill shapes, because more
// blocks per CU hide the global latency of each K step (split K when even these leave the CUs idle). F16 and Q8
// weights take the split-f16 matrix cores.
template <int WT, int EPI>
static hipError_t gemm_tile(const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s) {
    if constexpr (WT == WT_F16 || WT == WT_Q8) {
        bool split = false;
        hipError_t e = gemm_splitk<WT, EPI>(w, scale, A, g, s, &split);
        if (e != hipSuccess || split) return e;
        return gemm_run_h16<WT, EPI, 2, 2>(w, scale, A, g, s);
    } else {
        if constexpr (EPI == EPI_STORE || EPI == EPI_ACC || EPI == EPI_GATED_ACC || EPI == EPI_SWIGLU || EPI == EPI_ACC_SNAKE ||
                      EPI == EPI_GELU_ERF) {
            GemmArgs gs = g;  // the same K slices (few-row passes over f32 / bf16 weights)
            const int splits = split_plan(g, &gs.kchunk);
            if (splits) {
                hipError_t e = WT == WT_F32 ? f32w_run<EPI_STORE, ASRC_ROWS>(w, A, gs, splits, s)
                                            : gemm_run<WT, EPI_STORE, ASRC_ROWS, 2>(w, scale, A, gs, splits, s);
                return e != hipSuccess ? e : splitk_reduce<EPI>(g, splits, s);
            }
        }
        if constexpr (WT == WT_F32) return f32w_run<EPI, ASRC_ROWS>(w, A, g, 1, s);
        return gemm_run<WT, EPI, ASRC_ROWS, 2>(w, scale, A, g, 1, s);
    }
}


static bool rope_h16_ok(const GemmArgs &g) {
    return g.h16 && g.hd > 0 && g.hd % 2 == 0 && g.seq > 0 && g.rope_cols % (2 * g.hd) == 0 && g.m % g.seq == 0 &&
           g.n == g.rope_cols + g.rope_cols / 2 && g.ldvt >= g.seq && g.ldvt % 8 == 0 && g.lo_off % 8 == 0;
}

template <int WT>
static hipError_t gemm_epi(int epi, const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s) {
    switch (epi) {
        case EPI_STORE: return gemm_tile<WT, EPI_STORE>(w, scale, A, g, s);
        case EPI_ACC: return gemm_tile<WT, EPI_ACC>(w, scale, A, g, s);
        case EPI_SWIGLU: return gemm_tile<WT, EPI_SWIGLU>(w, scale, A, g, s);
        case EPI_GATED_ACC: return g.gate ? gemm_tile<WT, EPI_GATED_ACC>(w, scale, A, g, s) : hipErrorInvalidValue;
        case EPI_GELU: return gemm_tile<WT, EPI_GELU>(w, scale, A, g, s);
        case EPI_GELU_ERF: return gemm_tile<WT, EPI_GELU_ERF>(w, scale, A, g, s);
        case EPI_ACC_SNAKE:
            return g.snake_a && g.snake_ib && g.snake_y ? gemm_tile<WT, EPI_ACC_SNAKE>(w, scale, A, g, s) : hipErrorInvalidValue;
        case EPI_ROPE:
            if (!g.rope || g.hd <= 0 || g.hd % 2 || g.seq <= 0 || g.rope_cols % (2 * g.hd)) return hipErrorInvalidValue;
            return gemm_tile<WT, EPI_ROPE>(w, scale, A, g, s);
        case EPI_ROPE_H16:
            return rope_h16_ok(g) ? gemm_tile<WT, EPI_ROPE_H16>(w, scale, A, g, s) : hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(int wt, int epi, const uint8_t *w, const float *scale, const float *A, const GemmArgs &g0, hipStream_t s) {
    GemmArgs g = g0;
    g.status = status_word();
    if (g.m <= 0) return hipSuccess;
    if (g.K % 8 || g.n <= 0 || g.lda % 4) return hipErrorInvalidValue;
    if ((epi == EPI_SWIGLU || epi == EPI_ROPE) && g.n % 2) return hipErrorInvalidValue;
    switch (wt) {
        case WT_F32: return gemm_epi<WT_F32>(epi, w, scale, A, g, s);
        case WT_F16: return gemm_epi<WT_F16>(epi, w, scale, A, g, s);
        case WT_BF16: return gemm_epi<WT_BF16>(epi, w, scale, A, g, s);
        case WT_Q8: return g.K % 32 ? hipErrorInvalidValue : gemm_epi<WT_Q8>(epi, w, scale, A, g, s);
        default: return hipErrorInvalidValue;
    }
}

// 64 x 64 tiles, K steps of 64: measured faster on the DiT shapes than 64 x 128 tiles or K steps of 128.
// Tiles by how many 64 x 64 tiles the product has (measured on the flow estimator's and the DiT's shapes): below 256
// the 32 x 32 tiles (the 1024 x 256 projections: 4.4 against 8.0 us, and faster than splitting K), below 512 with
// K <= 512 the 32 x 64 ones (1024 x 1536, K 256: 7.0 against 8.4 us), else 64 x 64 (2000 x 1024, K 1024: 19.0
// against 21-25 us for the smaller tiles). Below 256 tiles with K >= 2048 (the 512-row prefill's down projection,
// K 4864) the 64 x 64 tiles split K instead, as the f32-activation GEMM does. Q8: the int8 values as f16 in w, the
// block scales in q8_scale.
template <int EPI, int TM, int TN, bool Q8, int WN = 2>
static hipError_t gemm_hh_tiles(const _Float16 *w, const float *q8_scale, const GemmArgs &g, hipStream_t s) {
    const dim3 grid(unsigned((g.n + 16 * TN * WN - 1) / (16 * TN * WN)), unsigned((g.m + 32 * TM - 1) / (32 * TM)),
                    unsigned(g.kchunk ? (g.K + g.kchunk - 1) / g.kchunk : 1));
    return launch(k_gemm_hh<EPI, TM, TN, 64, Q8, WN>, grid, dim3(128 * WN), 0, s, w, q8_scale, g);
}
// A tile forced by voxhip_bench_gemm_hh (0: the policy below): 1 32 x 32, 2 32 x 64, 3 64 x 64, 4 64 x 128 (8
// waves), as rows of A x rows of W.
static std::atomic<int> g_hh_tile{0};
void set_gemm_hh_tile(int tile) { g_hh_tile.store(tile); }
template <int EPI, bool Q8>
static hipError_t gemm_hh_forced(int tile, const _Float16 *w, const float *q8_scale, const GemmArgs &g, hipStream_t s) {
    switch (tile) {
        case 1: return gemm_hh_tiles<EPI, 1, 1, Q8>(w, q8_scale, g, s);
        case 2: return gemm_hh_tiles<EPI, 1, 2, Q8>(w, q8_scale, g, s);
        case 3: return gemm_hh_tiles<EPI, 2, 2, Q8>(w, q8_scale, g, s);
        case 4: return gemm_hh_tiles<EPI, 2, 2, Q8, 4>(w, q8_scale, g, s);
        default: return hipErrorInvalidValue;
    }
}
template <int EPI, bool Q8>
static hipError_t gemm_hh_run(const _Float16 *w, const float *q8_scale, const GemmArgs &g, hipStream_t s) {
    if (const int tile = g_hh_tile.load()) return gemm_hh_forced<EPI, Q8>(tile, w, q8_scale, g, s);
    const int64_t blocks = int64_t((g.n + 63) / 64) * ((g.m + 63) / 64);
    if constexpr (EPI == EPI_STORE || EPI == EPI_ACC || EPI == EPI_GATED_ACC || EPI == EPI_SWIGLU) {
        GemmArgs gs = g;
        const int splits = blocks < 256 && g.K >= 2048 ? split_plan(g, &gs.kchunk) : 0;
        if (splits) {
            hipError_t e = gemm_hh_tiles<EPI_STORE, 2, 2, Q8>(w, q8_scale, gs, s);
            return e != hipSuccess ? e : splitk_reduce<EPI>(g, splits, s);
        }
    }
    if (blocks < 256) return gemm_hh_tiles<EPI, 1, 1, Q8>(w, q8_scale, g, s);
    if (blocks < 512 && g.K <= 512) return gemm_hh_tiles<EPI, 1, 2, Q8>(w, q8_scale, g, s);
    // f16 weights: 64 x 128 tiles of 8 waves while they still make 256 blocks (the DiT's 2000 x 3072 x 1024 q|k|v
    // 36.5 against 42.2 us, 2000 x 1024 x 2048 27.9 against 31.2 us, 1000 x 2048 x 1024 16.7 against 19.0 us; at 128
    // blocks they lose, 1000 x 1024 x 2048 24.9 against 21.6 us; the q8 prefill shapes measured slower, 37.2 against
    // 36.1 us for 512 x 9728 x 896)
    if constexpr (!Q8)
        if (int64_t((g.n + 127) / 128) * ((g.m + 63) / 64) >= 256) return gemm_hh_tiles<EPI, 2, 2, Q8, 4>(w, q8_scale, g, s);
    return gemm_hh_tiles<EPI, 2, 2, Q8>(w, q8_scale, g, s);
}
template <int EPI>
static hipError_t gemm_hh_wt(const _Float16 *w, const float *q8_scale, const GemmArgs &g, hipStream_t s) {
    return q8_scale ? gemm_hh_run<EPI, true>(w, q8_scale, g, s) : gemm_hh_run<EPI, false>(w, nullptr, g, s);
}

static bool hh_args_ok(const _Float16 *w, const float *q8_scale, const GemmArgs &g) {
    return w && g.a16 && g.n > 0 && g.K > 0 && g.K % 64 == 0 && g.lda >= g.K && g.lda % 8 == 0 && g.a_lo % 8 == 0 &&
           int64_t(64) * g.lda * 2 <= INT32_MAX && int64_t(64) * g.K * 2 <= INT32_MAX &&
           (!q8_scale || int64_t(64) * (g.K / 32) * 4 <= INT32_MAX);
}

hipError_t launch_gemm_hh_acc_rms(const _Float16 *w, const float *q8_scale, const GemmArgs &g0, const float *gamma, float eps,
                                  _Float16 *out16, int64_t ldo, int64_t lo_off, hipStream_t s, bool *normed) {
    GemmArgs g = g0;
    g.status = status_word();
    *normed = false;
    if (g.m <= 0) return hipSuccess;
    if (!hh_args_ok(w, q8_scale, g) || !g.y) return hipErrorInvalidValue;
    const int64_t blocks = int64_t((g.n + 63) / 64) * ((g.m + 63) / 64);
    GemmArgs gs = g;
    const int splits = blocks < 256 && g.K >= 2048 ? split_plan(g, &gs.kchunk) : 0;
    // the row pass holds 8 columns per thread; without a split the ACC epilogue already wrote y
    if (!splits || splits > 8 || g.n > 8 * 256 || !gamma || !out16 || ldo < g.n || lo_off % 8)
        return launch_gemm_hh(EPI_ACC, w, q8_scale, g, s);
    hipError_t e = q8_scale ? gemm_hh_tiles<EPI_STORE, 2, 2, true>(w, q8_scale, gs, s)
                            : gemm_hh_tiles<EPI_STORE, 2, 2, false>(w, nullptr, gs, s);
    if (e != hipSuccess) return e;
    const dim3 grid(unsigned(g.m));
    if (g.n <= 4 * 256) e = launch(k_splitk_acc_rms_h16<4>, grid, dim3(256), 0, s, g, int32_t(splits), gamma, eps, out16, ldo, lo_off);
    else e = launch(k_splitk_acc_rms_h16<8>, grid, dim3(256), 0, s, g, int32_t(splits), gamma, eps, out16, ldo, lo_off);
    if (e == hipSuccess) *normed = true;
    return e;
}

hipError_t launch_gemm_hh(int epi, const _Float16 *w, const float *q8_scale, const GemmArgs &g0, hipStream_t s) {
    GemmArgs g = g0;
    g.status = status_word();
    if (g.m <= 0) return hipSuccess;
    if (!hh_args_ok(w, q8_scale, g)) return hipErrorInvalidValue;
    if ((epi == EPI_SWIGLU || epi == EPI_SWIGLU_H16) && g.n % 2) return hipErrorInvalidValue;
    const bool y_ok = g.y != nullptr;
    switch (epi) {
        case EPI_STORE: return y_ok ? gemm_hh_wt<EPI_STORE>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_ACC: return y_ok ? gemm_hh_wt<EPI_ACC>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_GATED_ACC: return y_ok && g.gate ? gemm_hh_wt<EPI_GATED_ACC>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_GELU: return y_ok ? gemm_hh_wt<EPI_GELU>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_SWIGLU: return y_ok && g.ldy >= g.n / 2 ? gemm_hh_wt<EPI_SWIGLU>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_GELU_H16: return g.h16 && g.ldy >= g.n ? gemm_hh_wt<EPI_GELU_H16>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_SWIGLU_H16:
            return g.h16 && g.ldy >= g.n / 2 ? gemm_hh_wt<EPI_SWIGLU_H16>(w, q8_scale, g, s) : hipErrorInvalidValue;
        case EPI_ROPE_H16: return rope_h16_ok(g) ? gemm_hh_wt<EPI_ROPE_H16>(w, q8_scale, g, s) : hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_conv_gemm(int epi, const float *w, const float *A, const GemmArgs &g0, int groups, hipStream_t s) {
    GemmArgs g = g0;
    g.status = status_word();
    if (g.m <= 0) return hipSuccess;
    // K: ksize * cig, rounded up to a multiple of 8 with zero weights (the A loader reads zeros there)
    if (g.cig <= 0 || g.cig % 4 || g.ksize <= 0 || g.ksize % 2 == 0 || g.K < g.ksize * g.cig || g.K >= g.ksize * g.cig + 8 ||
        g.K % 8 || g.seq <= 0 || g.lda % 4 || groups <= 0 || g.n <= 0)
        return hipErrorInvalidValue;
    const uint8_t *wb = reinterpret_cast<const uint8_t *>(w);
    if (groups == 1 && (epi == EPI_STORE || epi == EPI_ACC)) {  // one group: K slices in place of groups when idle
        GemmArgs gs = g;
        const int splits = split_plan(g, &gs.kchunk);
        if (splits) {
            hipError_t e = f32w_run<EPI_STORE, ASRC_CONV>(wb, A, gs, splits, s);
            if (e != hipSuccess) return e;
            return epi == EPI_STORE ? splitk_reduce<EPI_STORE>(g, splits, s) : splitk_reduce<EPI_ACC>(g, splits, s);
        }
    }
    if (epi == EPI_MISH) return f32w_run<EPI_MISH, ASRC_CONV>(wb, A, g, groups, s);
    if (epi == EPI_MISH_ACC) return f32w_run<EPI_MISH_ACC, ASRC_CONV>(wb, A, g, groups, s);
    if (epi == EPI_STORE) return f32w_run<EPI_STORE, ASRC_CONV>(wb, A, g, groups, s);
    if (epi == EPI_ACC) return f32w_run<EPI_ACC, ASRC_CONV>(wb, A, g, groups, s);
    return hipErrorInvalidValue;
}

// The codec's streaming convolution: y = W im2col([hist; x]) + bias (qwen3.cpp:102-121), or Snake of it (EPI_SNAKE),
// F32 / F16 / BF16 weights [cout][K cin] on the MFMA GEMMs (f32 weights: three f16 products), split K when the
// 64 x 64 tiles leave the CUs idle.
template <int WT, int EPI>
static hipError_t stream_conv(const uint8_t *w, const float *scale, const float *x, const GemmArgs &g, hipStream_t s) {
    GemmArgs gs = g;
    const int splits = split_plan(g, &gs.kchunk);
    if (splits) {
        hipError_t e = WT == WT_F32 ? f32w_run<EPI_STORE, ASRC_STREAM>(w, x, gs, splits, s)
                                    : gemm_run<WT, EPI_STORE, ASRC_STREAM, 2>(w, scale, x, gs, splits, s);
        return e != hipSuccess ? e : splitk_reduce<EPI>(g, splits, s);
    }
    if constexpr (WT == WT_F32) return f32w_run<EPI, ASRC_STREAM>(w, x, g, 1, s);
    return gemm_run<WT, EPI, ASRC_STREAM, 2>(w, scale, x, g, 1, s);
}
template <int EPI>
static hipError_t stream_conv_wt(int wt, const uint8_t *w, const float *scale, const float *x, const GemmArgs &g, hipStream_t s) {
    switch (wt) {
        case WT_F32: return stream_conv<WT_F32, EPI>(w, scale, x, g, s);
        case WT_F16: return stream_conv<WT_F16, EPI>(w, scale, x, g, s);
        case WT_BF16: return stream_conv<WT_BF16, EPI>(w, scale, x, g, s);
        default: return hipErrorInvalidValue;
    }
}
hipError_t launch_stream_conv(int wt, int epi, const uint8_t *w, const float *scale, const float *x, const GemmArgs &g0,
                              hipStream_t s) {
    GemmArgs g = g0;
    g.status = status_word();
    if (g.m <= 0) return hipSuccess;
    if (g.cig <= 0 || g.cig % 4 || g.ksize <= 0 || g.dil <= 0 || g.K != g.ksize * g.cig || g.K % 8 || g.lda % 4 || g.n <= 0 ||
        g.ctx != (g.ksize - 1) * g.dil || (g.ctx && !g.hist) || !g.y ||
        (g.hist_next && (!g.ctx || g.hist_next == g.hist)))
        return hipErrorInvalidValue;
    if (epi == EPI_STORE) return stream_conv_wt<EPI_STORE>(wt, w, scale, x, g, s);
    if (epi == EPI_SNAKE) return g.snake_a && g.snake_ib ? stream_conv_wt<EPI_SNAKE>(wt, w, scale, x, g, s) : hipErrorInvalidValue;
    return hipErrorInvalidValue;
}

hipError_t launch_attn_merge(const AttnPartials &P, float *ao, int m, hipStream_t s) {
    if (m <= 0) return hipSuccess;
    if (P.hd > 128) return hipErrorInvalidValue;
    return launch(k_attn_merge, dim3(P.heads, m), dim3(P.hd), 0, s, P, ao);
}

}  // namespace vh
