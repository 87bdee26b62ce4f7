// GEMV launch: picks the activation path's row block M and the (R, IT) tile from the matrix shape, then calls the
// translation unit that instantiates the weight family.
#include <cstdlib>

#include "vh_gemv.hpp"
#include "vh_launch.hpp"

namespace vh {

hipError_t launch_gemv_int_q8(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);
hipError_t launch_gemv_int_q4(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);
hipError_t launch_gemv_int_q4h(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);
hipError_t launch_gemv_flt_q8(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);
hipError_t launch_gemv_flt_f32(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);
hipError_t launch_gemv_flt_f16(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);
hipError_t launch_gemv_flt_bf16(int pro, int epi, int M, int R, int IT, const GemvArgs &a, hipStream_t s);

// Waves one launch aims for: 256 CUs x 4 waves, so a decode GEMV is one round of blocks in which every lane
// issues all of its weight loads before the activation prologue. VOXHIP_GEMV_WAVES overrides it (tuning).
static int target_waves() {
    static const int w = [] {
        const char *e = std::getenv("VOXHIP_GEMV_WAVES");
        const int v = e ? std::atoi(e) : 0;
        return v >= 64 ? v : 1024;
    }();
    return w;
}

// Pre-quantized rows (PRO_Q): each block copies the M quantized rows into LDS, so larger tiles (up to 8 rows per
// wave) copy them fewer times, as long as the launch keeps one block per CU. (The same tiles with the fused prologue
// measured slower than quantizing once: 2.58 against 2.00 ms for the 1.7B q4 step at 8 sessions.)
static int q_rmax() {  // VOXHIP_GEMVQ_RMAX caps the rows per wave of these tiles (2 or 4; tuning)
    static const int r = [] {
        const char *e = std::getenv("VOXHIP_GEMVQ_RMAX");
        const int v = e ? std::atoi(e) : 0;
        return v == 2 || v == 4 ? v : 8;
    }();
    return r;
}
// Rows per wave: 2, and 4 for the SwiGLU pass while that still makes 256 blocks. Measured on configs[2] at 8 rows
// (1.7B q4, graph step 1.747 / 1.672 / 1.653 ms with at most 8 / 4 / 2 rows a wave): gate|up 12.7 / 10.1 / 11.1 us,
// q|k|v, o and down fastest at 2 (a block's copy of the rows serves fewer weight rows, but more blocks share the
// stream).
static void gemv_tile_q(int rows, int nchunk, bool swiglu, int *R, int *IT) {
    int r = 2;
    if (swiglu && q_rmax() >= 4 && int64_t(rows) / (4 * 4) >= 256) r = 4;
    *R = r;
    // one pass of chunks where the tile allows it: every weight load of a wave in flight at once (K 6144 q4: 3)
    *IT = swiglu || r != 2 || nchunk <= 64 ? 1 : nchunk <= 128 ? 2 : 3;
}

void gemv_tile(int rows, int nchunk, int M, bool swiglu, int *R, int *IT) {
    if (M > 1) {  // tiles (1,1) (2,1) (1,2); swiglu (2,1)
        *IT = !swiglu && nchunk > 64 ? 2 : 1;
        *R = swiglu ? 2 : (*IT == 1 && rows >= 2048) ? 2 : 1;
        return;
    }
    int it = (nchunk + 63) / 64;
    it = it < 1 ? 1 : it > 6 ? 6 : it;
    if (it > 1) {  // (1,2) .. (1,6): one pass of chunks up to K = 384 16-byte chunks (q8 K 6144); swiglu (2,2) (2,3)
        *R = swiglu ? 2 : 1;
        *IT = swiglu && it > 3 ? 3 : it;
        return;
    }
    // the fewest rows per wave that keep the launch at one round of target_waves() waves; SwiGLU up to 12 (the 1.7B
    // talker's 12,288 gate|up rows at 12 a wave: one 256-thread block per CU, 0.655-0.659 -> 0.651-0.653 ms a step)
    const int need = (rows + target_waves() - 1) / target_waves();
    static const int kR[] = {1, 2, 3, 4, 6, 8}, kRs[] = {2, 4, 6, 8, 12};
    const int *set = swiglu ? kRs : kR;
    const int n = swiglu ? 5 : 6;
    int r = set[n - 1];
    for (int i = 0; i < n; ++i)
        if (set[i] >= need) { r = set[i]; break; }
    *R = r;
    *IT = 1;
}

hipError_t launch_gemv(int wt, bool int_path, int pro, int epi, const GemvArgs &a, hipStream_t s) {
    if (a.m <= 0) return hipSuccess;
    const int epc = int_path ? ((wt == WT_Q4 || wt == WT_Q4H) ? 32 : 16) : (wt == WT_F32 ? 4 : wt == WT_Q8 ? 16 : 8);
    const int nchunk = a.K / epc;
    int M, R, IT;
    if (int_path) {
        M = a.m <= 1 ? 1 : a.m <= 2 ? 2 : a.m <= 4 ? 4 : a.m <= 8 ? 8 : 0;
    } else {
        M = a.m <= 1 ? 1 : a.m <= 4 ? 4 : 0;
    }
    if (!M) return hipErrorInvalidValue;
    if (pro == PRO_Q) {
        if (!int_path || M < 4 || !a.q || !a.qs || !a.qsum) return hipErrorInvalidValue;
        gemv_tile_q(a.rows, nchunk, epi == EPI_SWIGLU, &R, &IT);
        if (epi == EPI_SWIGLU_Q) R = 4, IT = 1;  // 16 waves of 4 rows: one block per 32 SwiGLU outputs
    } else {
        gemv_tile(a.rows, nchunk, M, epi == EPI_SWIGLU, &R, &IT);
    }
    if (int_path) {
        if (wt == WT_Q8) return launch_gemv_int_q8(pro, epi, M, R, IT, a, s);
        if (wt == WT_Q4) return launch_gemv_int_q4(pro, epi, M, R, IT, a, s);
        if (wt == WT_Q4H) return launch_gemv_int_q4h(pro, epi, M, R, IT, a, s);
        return hipErrorInvalidValue;
    }
    switch (wt) {
        case WT_F32: return launch_gemv_flt_f32(pro, epi, M, R, IT, a, s);
        case WT_F16: return launch_gemv_flt_f16(pro, epi, M, R, IT, a, s);
        case WT_BF16: return launch_gemv_flt_bf16(pro, epi, M, R, IT, a, s);
        case WT_Q8: return launch_gemv_flt_q8(pro, epi, M, R, IT, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_quant_rows(int pro, const GemvArgs &a, int8_t *q, float *qs, int32_t *qsum, hipStream_t s) {
    if (a.m <= 0) return hipSuccess;
    if (a.K <= 0 || a.K % 32 || !q || !qs || !qsum) return hipErrorInvalidValue;
    const dim3 grid(unsigned(a.m)), block(kGemvThreads);
    switch (pro) {
        case PRO_X: return launch(k_quant_rows<PRO_X>, grid, block, 0, s, a, q, qs, qsum);
        case PRO_RMS: return launch(k_quant_rows<PRO_RMS>, grid, block, 0, s, a, q, qs, qsum);
        case PRO_ATTN: return launch(k_quant_rows<PRO_ATTN>, grid, block, 0, s, a, q, qs, qsum);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace vh
