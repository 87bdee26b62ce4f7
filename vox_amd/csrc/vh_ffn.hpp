// vh_ffn.hpp — the decode FFN of one row as one kernel (gfx950).
//
// h += down(silu(gate(RMSNorm(h))) * up(RMSNorm(h))) for one row, the reference's kernels.cpp:833-839 with the
// q8 / q4 matmul of kernels.cpp:653-705. As two GEMVs this is two dependent launches, and on this hardware every
// dependent launch costs about as much as its data movement. Here the down product is split by its INPUT columns
// instead: block group g computes the 32 SwiGLU outputs 32g .. 32g+31 (64 interleaved gate|up rows), quantizes them
// per 32-block exactly as the reference quantizes the down product's input (they are one quantization block), and
// multiplies them with its 32-column panel of the down weights. Every group contributes one block term
// float(dot) * (ws * xs) to each down row; those terms are added by 64-bit integer atomics in fixed point (units of
// 2^-32), so the sum is exact and the same in any order, and the next launch reads it (GemvArgs::acc). The order
// in which the reference adds the block terms in float is not kept (a few ulps of the down output), as in the GEMV.
//
// Per block: the staged input row, the 64 gate|up rows and its panel share are all issued before the prologue
// (RMSNorm + int8 quantization into LDS) runs; then gate|up dots (as k_gemv_int), SwiGLU into LDS, the 32-value
// quantization (every wave on its own, no second barrier), the down block dots, and the atomics.
#pragma once
#include "vh_gemv.hpp"

namespace vh {

constexpr int kFfnThreads = 512;  // 8 waves: a block streams its ~100 KB with twice the loads in flight of 4 waves
constexpr int kFfnMaxH = 2048;    // hidden sizes up to 2048: at most 2 gate|up chunks and 8 panel chunks per lane

template <int WT>
struct FfnFmt {
    static constexpr int EPC = WT == WT_Q8 ? 16 : 32;  // weight elements per 16-byte chunk
    static constexpr int PRB = WT == WT_Q8 ? 32 : 16;  // bytes of one down row in a 32-column panel
    static constexpr int CPR = PRB / 16;               // 16-byte chunks per panel row (lanes per down row)
};

VH_DEV float scale_at(const float *s, int64_t i, bool f16) {
    return f16 ? float(reinterpret_cast<const _Float16 *>(s)[i]) : s[i];
}

// GIT: 16-byte chunks in flight per gate|up row and lane (H <= 1024 GIT EPC); DL: panel chunks per thread.
// The launcher checks H <= kFfnMaxH, H % 32 == 0 and I % 32 == 0.
template <int WT, int GIT, int DL>
__global__ __launch_bounds__(kFfnThreads) void k_ffn_int(FfnArgs a) {
    using F = FfnFmt<WT>;
    constexpr int NW = kFfnThreads / 64, GR = 64 / NW;  // gate|up rows per wave
    constexpr bool S16 = WT == WT_Q4H;
    __shared__ __align__(16) int8_t xq[kFfnMaxH];  // the normed row quantized
    __shared__ float xs[kFfnMaxH / 32];            // its block scales
    __shared__ int xsum[kFfnMaxH / 32];            // Q4: the blocks' sums of quantized inputs
    __shared__ float red[NW];
    __shared__ float hv[32];                   // the group's SwiGLU outputs
    const int H = a.H, nb = H / 32, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // blocks of one group are 8 apart in the grid, so they share an XCD (the dispatcher deals blocks round-robin)
    const int G = a.I / 32, P = a.parts;
    const int g = (blockIdx.x / (8 * P)) * 8 + blockIdx.x % 8, p = (blockIdx.x / 8) % P;
    if (g >= G) return;  // the whole block leaves before any barrier
    const int HP = H / P, nchunk = H / F::EPC;

    // --- the input slot and gamma first (loads return in issue order), then every weight this block streams
    const int spr = H / 8;
    const int sl = int(threadIdx.x) < spr ? int(threadIdx.x) : 0;
    float xv[8], gv[8];
    load8(a.x + sl * 8, xv);
    load8(a.gamma + sl * 8, gv);
    __builtin_amdgcn_sched_barrier(0);
    const int64_t grb = row_bytes<WT>(H);
    const int gr0 = 64 * g + wave * GR;  // this wave's first gate|up row
    u32x4 gw[GIT][GR];
    float gs[GIT][GR];
#pragma unroll
    for (int j = 0; j < GIT; ++j) {
        const int c = 64 * j + lane;
        const bool ok = c < nchunk;
        const int cc = ok ? c : 0;
#pragma unroll
        for (int r = 0; r < GR; ++r) {
            const int row = gr0 + r;
            const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(a.gu + int64_t(row) * grb) + cc);
            const float sc = scale_at(a.gu_s, int64_t(row) * nb + (WT == WT_Q8 ? (cc >> 1) : cc), S16);
            gw[j][r] = ok ? t : u32x4{0u, 0u, 0u, 0u};
            gs[j][r] = ok ? sc : 0.f;
        }
    }
    // panel share: rows p*HP .. p*HP+HP-1 of group g's panel, CPR chunks per row, chunk ci = i * 512 + thread
    const int nd = HP * F::CPR;
    const uint8_t *pan = a.dp + (int64_t(g) * H + int64_t(p) * HP) * F::PRB;
    u32x4 dw[DL];
    float ds[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        const int ci = i * kFfnThreads + int(threadIdx.x);
        const bool ok = ci < nd;
        const int cc = ok ? ci : 0;
        const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(pan) + cc);
        const float sc = scale_at(a.dp_s, int64_t(g) * H + int64_t(p) * HP + cc / F::CPR, S16);
        dw[i] = ok ? t : u32x4{0u, 0u, 0u, 0u};
        ds[i] = ok ? sc : 0.f;
    }
    // the biases this thread adds, loaded now and used as loaded at the end (a load inside the atomics loop would
    // make each atomic wait for everything issued before it); without a bias, element 0 of x, never used
    const float *gbp = a.gu_b ? a.gu_b : a.x, *dbp = a.d_b ? a.d_b : a.x;
    const float gbias = gbp[a.gu_b ? gr0 + (lane < GR ? lane : 0) : 0];
    float dbias[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        const int ci = i * kFfnThreads + int(threadIdx.x);
        dbias[i] = dbp[a.d_b && ci < nd ? p * HP + ci / F::CPR : 0];
    }

    // --- prologue: RMSNorm of the row (kernels.cpp:707-712), quantized per 32-block into LDS (kernels.cpp:515-523)
    {
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) q = fmaf(xv[j], xv[j], q);
        q = int(threadIdx.x) < spr ? q : 0.f;
        q = wave_sum(q);
        if (lane == 0) red[wave] = q;
        __syncthreads();
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) t += red[w];
        const float inv = 1.0f / sqrtf(t / float(H) + a.eps);
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = gv[j] * (xv[j] * inv);
        // every 4-lane group is one 32-block; threads past the row quantize a copy of slot 0 and store nothing
        uint32_t q2[2];
        float sc;
        quant_slot(v, q2, &sc);
        const int bs = WT == WT_Q8 ? 0 : block_qsum(q2);
        if (int(threadIdx.x) < spr) {
            *reinterpret_cast<uint2 *>(xq + sl * 8) = make_uint2(q2[0], q2[1]);
            if ((sl & 3) == 0) {
                xs[sl >> 2] = sc;
                if (WT != WT_Q8) xsum[sl >> 2] = bs;
            }
        }
    }
    __syncthreads();

    // --- gate|up dots (the k_gemv_int arithmetic, one input row)
    float acc[GR];
#pragma unroll
    for (int r = 0; r < GR; ++r) acc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < GIT; ++j) {
        const int c = 64 * j + lane;
        const int cc = c < nchunk ? c : 0;
        if (WT == WT_Q8) {
            const u32x4 x4 = *reinterpret_cast<const u32x4 *>(xq + cc * 16);
            const float xsv = xs[cc >> 1];
#pragma unroll
            for (int r = 0; r < GR; ++r) {
                int d = __builtin_amdgcn_sdot4(int(gw[j][r].x), int(x4.x), 0, false);
                d = __builtin_amdgcn_sdot4(int(gw[j][r].y), int(x4.y), d, false);
                d = __builtin_amdgcn_sdot4(int(gw[j][r].z), int(x4.z), d, false);
                d = __builtin_amdgcn_sdot4(int(gw[j][r].w), int(x4.w), d, false);
                d += dpp<kDppXor1>(d);
                acc[r] += (lane & 1) ? 0.f : float(d) * (gs[j][r] * xsv);
            }
        } else {
            const u32x4 xl = *reinterpret_cast<const u32x4 *>(xq + cc * 32);
            const u32x4 xh = *reinterpret_cast<const u32x4 *>(xq + cc * 32 + 16);
            const float xsv = xs[cc];
            const int sx = xsum[cc];
            const uint32_t m4 = 0x0F0F0F0Fu;
#pragma unroll
            for (int r = 0; r < GR; ++r) {
                const u32x4 w = gw[j][r];
                int d = __builtin_amdgcn_sdot4(int(w.x & m4), int(xl.x), 0, false);
                d = __builtin_amdgcn_sdot4(int(w.y & m4), int(xl.y), d, false);
                d = __builtin_amdgcn_sdot4(int(w.z & m4), int(xl.z), d, false);
                d = __builtin_amdgcn_sdot4(int(w.w & m4), int(xl.w), d, false);
                d = __builtin_amdgcn_sdot4(int((w.x >> 4) & m4), int(xh.x), d, false);
                d = __builtin_amdgcn_sdot4(int((w.y >> 4) & m4), int(xh.y), d, false);
                d = __builtin_amdgcn_sdot4(int((w.z >> 4) & m4), int(xh.z), d, false);
                d = __builtin_amdgcn_sdot4(int((w.w >> 4) & m4), int(xh.w), d, false);
                d -= 8 * sx;
                acc[r] += float(d) * (gs[j][r] * xsv);
            }
        }
    }
    // row totals into lanes 0..GR-1, bias, SwiGLU of the (gate, up) pairs (kernels.cpp:836)
    float out = 0.f;
    if constexpr ((GR & (GR - 1)) == 0 && GR > 1) {  // wave_sum's totals, by one reduce-scatter
        out = wave_sums_scatter<GR>(acc, lane);
    } else {
#pragma unroll
        for (int r = 0; r < GR; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == r) out = s;
        }
    }
    const float v = out + (a.gu_b ? gbias : 0.f);
    const float other = __shfl_xor(v, 1, 64);
    if (lane < GR && (lane & 1) == 0) hv[(wave * GR + lane) >> 1] = silu(v) * other;
    __syncthreads();

    // --- the group's 32 SwiGLU outputs quantized as one block (each wave on its own copy)
    float hq[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) hq[j] = hv[(lane & 3) * 8 + j];
    uint32_t q2[2];
    float hsc;
    quant_slot(hq, q2, &hsc);
    uint32_t qw[8];  // the 32 quantized values, bytes 4k..4k+3 in qw[k]
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        qw[2 * k] = uint32_t(__builtin_amdgcn_readlane(int(q2[0]), k));
        qw[2 * k + 1] = uint32_t(__builtin_amdgcn_readlane(int(q2[1]), k));
    }
    const int hsum = WT == WT_Q8 ? 0 : block_qsum(q2);

    // --- down block dots of the panel share, added to the accumulators in fixed point: every term first, then the
    // atomics back to back (an atomic issued between them would make the next term's wait include it)
    int64_t *accp = a.acc + int64_t(g % kAccCopies) * H;
    int64_t terms[DL];
    bool bad = false;  // a term outside the fixed-point range
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        const int ci = i * kFfnThreads + int(threadIdx.x);
        float f;
        if (WT == WT_Q8) {  // two lanes per row: even lane bytes 0..15, odd lane 16..31
            const bool hi = ci & 1;
            const uint32_t x0 = hi ? qw[4] : qw[0], x1 = hi ? qw[5] : qw[1], x2 = hi ? qw[6] : qw[2], x3 = hi ? qw[7] : qw[3];
            int d = __builtin_amdgcn_sdot4(int(dw[i].x), int(x0), 0, false);
            d = __builtin_amdgcn_sdot4(int(dw[i].y), int(x1), d, false);
            d = __builtin_amdgcn_sdot4(int(dw[i].z), int(x2), d, false);
            d = __builtin_amdgcn_sdot4(int(dw[i].w), int(x3), d, false);
            d += dpp<kDppXor1>(d);
            f = float(d) * (ds[i] * hsc);
        } else {  // one lane per row: element t in the low nibble of byte t, t + 16 in its high nibble
            const uint32_t m4 = 0x0F0F0F0Fu;
            const u32x4 w = dw[i];
            int d = __builtin_amdgcn_sdot4(int(w.x & m4), int(qw[0]), 0, false);
            d = __builtin_amdgcn_sdot4(int(w.y & m4), int(qw[1]), d, false);
            d = __builtin_amdgcn_sdot4(int(w.z & m4), int(qw[2]), d, false);
            d = __builtin_amdgcn_sdot4(int(w.w & m4), int(qw[3]), d, false);
            d = __builtin_amdgcn_sdot4(int((w.x >> 4) & m4), int(qw[4]), d, false);
            d = __builtin_amdgcn_sdot4(int((w.y >> 4) & m4), int(qw[5]), d, false);
            d = __builtin_amdgcn_sdot4(int((w.z >> 4) & m4), int(qw[6]), d, false);
            d = __builtin_amdgcn_sdot4(int((w.w >> 4) & m4), int(qw[7]), d, false);
            d -= 8 * hsum;
            f = float(d) * (ds[i] * hsc);
        }
        terms[i] = fix_of(f, bad) + ((g == 0 && a.d_b) ? fix_of(dbias[i], bad) : 0);
    }
    raise_status(a.status, bad, kStatusFixRange);
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        const int ci = i * kFfnThreads + int(threadIdx.x);
        if (ci < nd && (F::CPR == 1 || (ci & 1) == 0))
            __hip_atomic_fetch_add(accp + p * HP + ci / F::CPR, terms[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Down weights [H][I] (row bytes of I) and scales [H][I/32] into panels [I/32][H][32 columns] and [I/32][H]:
// thread (g, r) moves row r's block g.
template <int WT>
__global__ void k_panel_pack(const uint8_t *__restrict__ w, const void *__restrict__ s, int H, int I, uint8_t *__restrict__ pw,
                             void *__restrict__ ps) {
    using F = FfnFmt<WT>;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x, nb = I / 32;
    if (i >= int64_t(H) * nb) return;
    const int64_t g = i / H, r = i % H;
    const uint8_t *src = w + r * row_bytes<WT>(I) + g * F::PRB;
    uint8_t *dst = pw + (g * H + r) * F::PRB;
#pragma unroll
    for (int c = 0; c < F::CPR; ++c) reinterpret_cast<u32x4 *>(dst)[c] = reinterpret_cast<const u32x4 *>(src)[c];
    if (WT == WT_Q4H) reinterpret_cast<_Float16 *>(ps)[g * H + r] = reinterpret_cast<const _Float16 *>(s)[r * nb + g];
    else reinterpret_cast<float *>(ps)[g * H + r] = reinterpret_cast<const float *>(s)[r * nb + g];
}

// h += the pending FFN sums; the accumulators back to zero.
__global__ void k_acc_fold(float *__restrict__ h, int64_t *__restrict__ acc, int H) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    int64_t c[kAccCopies];
#pragma unroll
    for (int k = 0; k < kAccCopies; ++k) c[k] = acc[int64_t(k) * H + i];
    h[i] = h[i] + acc_value(c);
#pragma unroll
    for (int k = 0; k < kAccCopies; ++k) acc[int64_t(k) * H + i] = 0;
}

}  // namespace vh
