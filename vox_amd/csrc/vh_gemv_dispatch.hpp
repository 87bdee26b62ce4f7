// vh_gemv_dispatch.hpp — template dispatch from runtime (prologue, epilogue, M, R) to GEMV instantiations.
// Included by the vh_gemv_*.hip translation units, each instantiating one weight family.
#pragma once
#include "vh_gemv.hpp"
#include "vh_launch.hpp"

namespace vh {

template <int WT, int M, int R, int IT, int PRO, int EPI>
hipError_t run_int(const GemvArgs &a, hipStream_t s) {
    const void *k = reinterpret_cast<const void *>(&k_gemv_int<WT, M, R, IT, PRO, EPI>);
    const size_t smem = size_t(M) * a.K + size_t(M) * (a.K / 32) * 4 + 16;
    hipError_t e = ensure_smem(k, smem);
    if (e != hipSuccess) return e;
    const int per_block = (kGemvThreads / 64) * R;
    return launch(k_gemv_int<WT, M, R, IT, PRO, EPI>, dim3((a.rows + per_block - 1) / per_block), dim3(kGemvThreads), smem, s, a);
}

template <int WT, int M, int R, int IT, int PRO, int EPI>
hipError_t run_flt(const GemvArgs &a, hipStream_t s) {
    const void *k = reinterpret_cast<const void *>(&k_gemv_flt<WT, M, R, IT, PRO, EPI>);
    const size_t smem = size_t(M) * a.K * 4 + 16;
    hipError_t e = ensure_smem(k, smem);
    if (e != hipSuccess) return e;
    const int per_block = (kGemvThreads / 64) * R;
    return launch(k_gemv_flt<WT, M, R, IT, PRO, EPI>, dim3((a.rows + per_block - 1) / per_block), dim3(kGemvThreads), smem, s, a);
}

template <int WT, int M, int R, int IT, int PRO, int EPI, bool INT>
hipError_t run_any(const GemvArgs &a, hipStream_t s) {
    if constexpr (INT) return run_int<WT, M, R, IT, PRO, EPI>(a, s);
    else return run_flt<WT, M, R, IT, PRO, EPI>(a, s);
}

template <int WT, int M, int PRO, int EPI, bool INT>
hipError_t by_r(int R, const GemvArgs &a, hipStream_t s) {
    if (R == 4) return run_any<WT, M, 4, 1, PRO, EPI, INT>(a, s);
    if (R == 2) return run_any<WT, M, 2, 2, PRO, EPI, INT>(a, s);
    if constexpr (EPI != EPI_SWIGLU) return run_any<WT, M, 1, 4, PRO, EPI, INT>(a, s);
    return hipErrorInvalidValue;
}

template <int WT, int PRO, int EPI, bool INT>
hipError_t by_m(int M, int R, const GemvArgs &a, hipStream_t s) {
    switch (M) {
        case 1: return by_r<WT, 1, PRO, EPI, INT>(R, a, s);
        case 2: if constexpr (INT) return by_r<WT, 2, PRO, EPI, INT>(R, a, s); else return hipErrorInvalidValue;
        case 4: return by_r<WT, 4, PRO, EPI, INT>(R, a, s);
        case 8: if constexpr (INT) return by_r<WT, 8, PRO, EPI, INT>(R, a, s); else return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

// (prologue, epilogue) pairs the backend uses: RMS+store (qkv, head), X+acc (o, down: residual),
// RMS+swiglu (gate|up), X+store (in_proj, plain matmul).
template <int WT, bool INT>
hipError_t by_pe(int pro, int epi, int M, int R, const GemvArgs &a, hipStream_t s) {
    if (pro == PRO_RMS && epi == EPI_STORE) return by_m<WT, PRO_RMS, EPI_STORE, INT>(M, R, a, s);
    if (pro == PRO_X && epi == EPI_ACC) return by_m<WT, PRO_X, EPI_ACC, INT>(M, R, a, s);
    if (pro == PRO_RMS && epi == EPI_SWIGLU) return by_m<WT, PRO_RMS, EPI_SWIGLU, INT>(M, R, a, s);
    if (pro == PRO_X && epi == EPI_STORE) return by_m<WT, PRO_X, EPI_STORE, INT>(M, R, a, s);
    return hipErrorInvalidValue;
}

template <int WT>
hipError_t dispatch_int(int pro, int epi, int M, int R, const GemvArgs &a, hipStream_t s) {
    return by_pe<WT, true>(pro, epi, M, R, a, s);
}
template <int WT>
hipError_t dispatch_flt(int pro, int epi, int M, int R, const GemvArgs &a, hipStream_t s) {
    return by_pe<WT, false>(pro, epi, M, R, a, s);
}

}  // namespace vh
