// vh_gemv_dispatch.hpp — template dispatch from runtime (prologue, epilogue, M, R, IT) to GEMV instantiations.
// Included by the vh_gemv_*.hip translation units, each instantiating one weight family (VH_GEMV_WT) on one
// activation path (VH_GEMV_INT).
#pragma once
#include "vh_gemv.hpp"
#include "vh_launch.hpp"

namespace vh {

template <int WT, int M, int R, int IT, int PRO, int EPI, bool INT, bool STAGE, bool ACC>
hipError_t gemv_run_staged(const GemvArgs &a, hipStream_t s) {
    constexpr int NT = EPI == EPI_SWIGLU_Q ? 1024 : kGemvThreads;
    const int per_block = (NT / 64) * R;
    const dim3 grid((a.rows + per_block - 1) / per_block), block(NT);
    if constexpr (INT) {
        // xq [M][K] int8, xs [M][K/32] f32, red [M][4], xsum [M][K/32] int32 (Q4), EPI_SWIGLU_Q's outputs [M][32] f32
        const size_t smem = size_t(M) * a.K + size_t(M) * (a.K / 32) * 4 + size_t(M) * 16 + (WT == WT_Q8 ? 0 : size_t(M) * (a.K / 32) * 4) +
                            (EPI == EPI_SWIGLU_Q ? size_t(M) * 32 * 4 : 0);
        if (EPI == EPI_SWIGLU_Q && (a.rows % 64 || !a.yq || !a.yqs || !a.yqsum)) return hipErrorInvalidValue;
        hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_gemv_int<WT, M, R, IT, PRO, EPI, STAGE, ACC, NT>), smem);
        if (e != hipSuccess) return e;
        return launch(k_gemv_int<WT, M, R, IT, PRO, EPI, STAGE, ACC, NT>, grid, block, smem, s, a.w, a.scale, a.x, a.rows, a.K, a);
    } else if constexpr (ACC || EPI == EPI_SWIGLU_Q) {
        return hipErrorInvalidValue;  // pending FFN sums come with int-path layers only
    } else {
        const size_t smem = size_t(M) * a.K * 4 + size_t(M) * 16;
        hipError_t e = ensure_smem(reinterpret_cast<const void *>(&k_gemv_flt<WT, M, R, IT, PRO, EPI, STAGE>), smem);
        if (e != hipSuccess) return e;
        return launch(k_gemv_flt<WT, M, R, IT, PRO, EPI, STAGE>, grid, block, smem, s, a.w, a.scale, a.x, a.rows, a.K, a);
    }
}

// Staged prologue (inputs loaded ahead of the weight stream) when they fit the staging registers. ACC: the row's
// pending FFN sums, staged with one input slot per thread.
template <int WT, int M, int R, int IT, int PRO, int EPI, bool INT, bool ACC>
hipError_t gemv_run(const GemvArgs &a, hipStream_t s) {
    if constexpr (ACC) {
        if (a.K / 8 > kGemvThreads || a.m != 1) return hipErrorInvalidValue;
        return gemv_run_staged<WT, M, R, IT, PRO, EPI, INT, true, true>(a, s);
    } else {
        if constexpr (PRO != PRO_Q) {
            if (pro_stageable<M, PRO>(a.K)) return gemv_run_staged<WT, M, R, IT, PRO, EPI, INT, true, false>(a, s);
        } else {  // the deeper staging of the quantized rows only where the shallow one does not hold them
            if (int64_t(M) * a.K / 16 > int64_t(kQStageChunksLo) * kGemvThreads || int64_t(M) * (a.K / 32) > int64_t(kQStageScalesLo) * kGemvThreads)
                return gemv_run_staged<WT, M, R, IT, PRO, EPI, INT, true, false>(a, s);
        }
        return gemv_run_staged<WT, M, R, IT, PRO, EPI, INT, false, false>(a, s);
    }
}

// The (R, IT) tiles instantiated; gemv_tile() (vh_gemv_tile.cpp) picks only these.
template <int WT, int M, int PRO, int EPI, bool INT, bool ACC = false>
hipError_t gemv_by_tile(int R, int IT, const GemvArgs &a, hipStream_t s) {
#define VH_TILE(r, it) \
    if (R == r && IT == it) return gemv_run<WT, M, r, it, PRO, EPI, INT, ACC>(a, s);
    if constexpr (PRO == PRO_Q) {  // pre-quantized rows: larger tiles, fewer copies of the rows per launch
        if constexpr (EPI == EPI_SWIGLU_Q) {
            VH_TILE(4, 1)
        } else if constexpr (EPI == EPI_SWIGLU) {
            VH_TILE(2, 1) VH_TILE(4, 1) VH_TILE(8, 1)
        } else {
            VH_TILE(2, 1) VH_TILE(4, 1) VH_TILE(8, 1) VH_TILE(2, 2) VH_TILE(2, 3)
        }
    } else if constexpr (M == 1) {
        if constexpr (EPI == EPI_SWIGLU) {
            VH_TILE(2, 1) VH_TILE(4, 1) VH_TILE(6, 1) VH_TILE(8, 1) VH_TILE(12, 1) VH_TILE(2, 2) VH_TILE(2, 3)
        } else {
            VH_TILE(1, 1) VH_TILE(2, 1) VH_TILE(3, 1) VH_TILE(4, 1) VH_TILE(6, 1) VH_TILE(8, 1)
            VH_TILE(1, 2) VH_TILE(1, 3) VH_TILE(1, 4) VH_TILE(1, 5) VH_TILE(1, 6)
        }
    } else {
        if constexpr (EPI == EPI_SWIGLU) {
            VH_TILE(2, 1)
        } else {
            VH_TILE(1, 1) VH_TILE(2, 1) VH_TILE(1, 2)
        }
    }
#undef VH_TILE
    return hipErrorInvalidValue;
}

template <int WT, int PRO, int EPI, bool INT>
hipError_t gemv_by_m(int M, int R, int IT, const GemvArgs &a, hipStream_t s) {
    if constexpr (PRO == PRO_Q) {
        if constexpr (!INT) return hipErrorInvalidValue;
        else if (M == 4) return gemv_by_tile<WT, 4, PRO, EPI, INT>(R, IT, a, s);
        else if (M == 8) return gemv_by_tile<WT, 8, PRO, EPI, INT>(R, IT, a, s);
        else return hipErrorInvalidValue;
    }
    switch (M) {
        case 1:
            // one row after a fused FFN: q|k|v (RMS + store) and o (attention merge + residual) add its pending sums
            if constexpr (INT && ((PRO == PRO_RMS && EPI == EPI_STORE) || (PRO == PRO_ATTN && EPI == EPI_ACC)))
                if (a.acc) return gemv_by_tile<WT, 1, PRO, EPI, INT, true>(R, IT, a, s);
            if (a.acc) return hipErrorInvalidValue;
            return gemv_by_tile<WT, 1, PRO, EPI, INT>(R, IT, a, s);
        case 2: if constexpr (INT) return gemv_by_tile<WT, 2, PRO, EPI, INT>(R, IT, a, s); else return hipErrorInvalidValue;
        case 4: return gemv_by_tile<WT, 4, PRO, EPI, INT>(R, IT, a, s);
        case 8: if constexpr (INT) return gemv_by_tile<WT, 8, PRO, EPI, INT>(R, IT, a, s); else return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

// (prologue, epilogue) pairs the backend uses: RMS+store (q|k|v, head), ATTN+acc (o: attention merge and
// residual), RMS+swiglu (gate|up), X+acc (down: residual), X+store (in_proj, plain matmul).
template <int WT, bool INT>
hipError_t gemv_dispatch(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s) {
    if (pro == PRO_RMS && epi == EPI_STORE) return gemv_by_m<WT, PRO_RMS, EPI_STORE, INT>(M, R, IT, a, s);
    if (pro == PRO_ATTN && epi == EPI_ACC) return gemv_by_m<WT, PRO_ATTN, EPI_ACC, INT>(M, R, IT, a, s);
    if (pro == PRO_RMS && epi == EPI_SWIGLU) return gemv_by_m<WT, PRO_RMS, EPI_SWIGLU, INT>(M, R, IT, a, s);
    if (pro == PRO_X && epi == EPI_ACC) return gemv_by_m<WT, PRO_X, EPI_ACC, INT>(M, R, IT, a, s);
    if (pro == PRO_X && epi == EPI_STORE) return gemv_by_m<WT, PRO_X, EPI_STORE, INT>(M, R, IT, a, s);
    if constexpr (INT) {  // the same passes on rows quantized beforehand
        if (pro == PRO_Q && epi == EPI_STORE) return gemv_by_m<WT, PRO_Q, EPI_STORE, INT>(M, R, IT, a, s);
        if (pro == PRO_Q && epi == EPI_ACC) return gemv_by_m<WT, PRO_Q, EPI_ACC, INT>(M, R, IT, a, s);
        if (pro == PRO_Q && epi == EPI_SWIGLU) return gemv_by_m<WT, PRO_Q, EPI_SWIGLU, INT>(M, R, IT, a, s);
        if (pro == PRO_Q && epi == EPI_SWIGLU_Q) return gemv_by_m<WT, PRO_Q, EPI_SWIGLU_Q, INT>(M, R, IT, a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace vh

// One translation unit per (weight type, activation path): defines its launch entry point.
#if defined(VH_GEMV_WT) && defined(VH_GEMV_INT) && defined(VH_GEMV_ENTRY)
namespace vh {
hipError_t VH_GEMV_ENTRY(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s) {
    return gemv_dispatch<VH_GEMV_WT, VH_GEMV_INT>(pro, epi, M, R, IT, a, s);
}
}  // namespace vh
#endif
