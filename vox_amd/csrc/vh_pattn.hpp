// vh_pattn.hpp — causal attention of a prefill pass on the matrix cores.
//
// transformer_forward's attention (kernels.cpp:812-826) for m consecutive rows of one sequence: row r at position
// pos0 + r takes softmax(q . k_j * scale) over keys j = 0 .. pos0 + r of the f16 cache (which already holds the
// pass's own keys, appended by k_qk_post) and returns the weighted sum of the values. The decode kernel (k_attn)
// gives every row its own blocks and re-reads the keys per row; here a block takes 64 rows of one query head and
// streams each 64-key tile of its kv head once for all of them.
//
// grid (ceil(m / 64), heads), block 256: wave w holds rows 16 w .. 16 w + 15. Per key tile: S = Q K^T and O += P V
// on v_mfma_f32_16x16x32_f16. The keys and values are f16 in the cache, so exact in the MFMA; q and the softmax
// weights P are f32, split into two f16 halves x = hi + lo with both halves multiplied (products exact in the f32
// accumulator), which keeps them to about 2^-22. An online softmax (running max and sum per row) replaces the
// reference's whole-row max, which changes only the rounding. The next tile's keys and values are loaded during
// the current tile's MFMAs.
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

typedef _Float16 ph16x8 __attribute__((ext_vector_type(8)));
typedef float pf32x4 __attribute__((ext_vector_type(4)));

template <int HD>
__global__ __launch_bounds__(256) void k_prefill_attn(PrefillAttnArgs a) {
    constexpr int NC = HD / 32;               // 32-deep chunks of the head dim
    constexpr int ND = HD / 16;               // 16-wide output tiles
    constexpr int KQ = 64 * HD / 8 / 256;     // 8-half chunks of a key / value tile per thread
    constexpr int LDK = HD + 8, LDP = 64 + 8;  // LDS strides in halves
    __shared__ __align__(16) _Float16 Ks[64][LDK];  // [key][d]
    __shared__ __align__(16) _Float16 Vt[HD][LDP];  // [d][key]
    __shared__ __align__(16) _Float16 Ph[4][16][LDP], Pl[4][16][LDP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.x * 64, h = blockIdx.y, g = h / (a.heads / a.kv_heads);
    const int64_t qd = int64_t(a.heads) * HD;
    const int64_t plane = (int64_t(a.layer) * a.kv_heads + g) * a.cap * HD;
    const _Float16 *K = a.k + plane, *V = a.v + plane;
    // A operand of S: lane holds q[r0 + 16 wave + lr][32 c + 8 lg + e] as hi / lo halves
    ph16x8 qh[NC], ql[NC];
    {
        const int qr = r0 + 16 * wave + lr;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            pf32x4 x0 = {0.f, 0.f, 0.f, 0.f}, x1 = {0.f, 0.f, 0.f, 0.f};
            if (qr < a.m) {
                const float *src = a.q + qr * qd + int64_t(h) * HD + 32 * c + 8 * lg;
                x0 = *reinterpret_cast<const pf32x4 *>(src);
                x1 = *reinterpret_cast<const pf32x4 *>(src + 4);
            }
            bool bad = false;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 hi, lo;
                bad |= split_f16(e < 4 ? x0[e] : x1[e - 4], hi, lo);
                qh[c][e] = hi;
                ql[c][e] = lo;
            }
            raise_status(a.status, bad, kStatusF16Range);
        }
    }
    float mrow[4], lrow[4];
    pf32x4 o[ND];
#pragma unroll
    for (int i = 0; i < 4; ++i) { mrow[i] = -INFINITY; lrow[i] = 0.f; }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o[dt] = pf32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t pos0 = a.rows[0].pos;
    const int64_t last_row = r0 + 63 < a.m - 1 ? r0 + 63 : a.m - 1;
    const int64_t kend = pos0 + last_row + 1;  // keys [0, kend) reach some row of this block
    // this block's key tiles: all of them, or the z-th of gridDim.z contiguous runs
    const int64_t ntile = (kend + 63) / 64, per = (ntile + gridDim.z - 1) / gridDim.z;
    const int64_t kt_begin = int64_t(blockIdx.z) * per * 64;
    const int64_t kt_end = (int64_t(blockIdx.z) + 1) * per * 64 < kend ? (int64_t(blockIdx.z) + 1) * per * 64 : kend;
    u32x4 kr[KQ], vr[KQ];
    auto fetch = [&](int64_t kt) {
#pragma unroll
        for (int q = 0; q < KQ; ++q) {
            const int idx = tid + 256 * q, key = idx / (HD / 8), d8 = (idx % (HD / 8)) * 8;
            kr[q] = vr[q] = u32x4{0u, 0u, 0u, 0u};
            if (kt + key < kend) {
                kr[q] = *reinterpret_cast<const u32x4 *>(K + (kt + key) * HD + d8);
                vr[q] = *reinterpret_cast<const u32x4 *>(V + (kt + key) * HD + d8);
            }
        }
    };
    if (kt_begin < kt_end) fetch(kt_begin);
    for (int64_t kt = kt_begin; kt < kt_end; kt += 64) {
#pragma unroll
        for (int q = 0; q < KQ; ++q) {
            const int idx = tid + 256 * q, key = idx / (HD / 8), d8 = (idx % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(&Ks[key][d8]) = kr[q];
            const ph16x8 vv = __builtin_bit_cast(ph16x8, vr[q]);
#pragma unroll
            for (int e = 0; e < 8; ++e) Vt[d8 + e][key] = vv[e];
        }
        __syncthreads();
        if (kt + 64 < kt_end) fetch(kt + 64);
        pf32x4 s[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const ph16x8 b = *reinterpret_cast<const ph16x8 *>(&Ks[16 * j + lr][32 * c + 8 * lg]);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[c], b, s[j], 0, 0, 0);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[c], b, s[j], 0, 0, 0);
            }
        }
        // lane holds S[4 lg + i][16 j + lr]; row 4 lg + i of the wave sits at position pos0 + r0 + 16 wave + 4 lg + i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t pos = pos0 + r0 + 16 * wave + 4 * lg + i;
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t key = kt + 16 * j + lr;
                const float v = key <= pos && key < kend ? s[j][i] * a.scale : -INFINITY;
                s[j][i] = v;
                mx = fmaxf(mx, v);
            }
            mx = fmaxf(mx, dpp<kDppXor1>(mx));
            mx = fmaxf(mx, dpp<kDppXor2>(mx));
            mx = fmaxf(mx, dpp<kDppRowHalfMirror>(mx));
            mx = fmaxf(mx, dpp<kDppRowMirror>(mx));
            const float mnew = fmaxf(mrow[i], mx);
            const bool any = mnew != -INFINITY;  // some key so far (always, for a row of the pass)
            const float alpha = any ? expf(mrow[i] - mnew) : 1.f;
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = any ? expf(s[j][i] - mnew) : 0.f;
                sum += p;
                const _Float16 hi = _Float16(p);
                Ph[wave][4 * lg + i][16 * j + lr] = hi;
                Pl[wave][4 * lg + i][16 * j + lr] = _Float16(p - float(hi));
            }
            sum += dpp<kDppXor1>(sum);
            sum += dpp<kDppXor2>(sum);
            sum += dpp<kDppRowHalfMirror>(sum);
            sum += dpp<kDppRowMirror>(sum);
            lrow[i] = lrow[i] * alpha + sum;
            mrow[i] = mnew;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) o[dt][i] *= alpha;
        }
        __syncthreads();
        // O += P V: A lane holds P[lr][32 c + 8 lg + e]; B lane holds V[32 c + 8 lg + e][16 dt + lr] (= Vt rows)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const ph16x8 pah = *reinterpret_cast<const ph16x8 *>(&Ph[wave][lr][32 * c + 8 * lg]);
            const ph16x8 pal = *reinterpret_cast<const ph16x8 *>(&Pl[wave][lr][32 * c + 8 * lg]);
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                const ph16x8 b = *reinterpret_cast<const ph16x8 *>(&Vt[16 * dt + lr][32 * c + 8 * lg]);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, b, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pal, b, o[dt], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    if (gridDim.z > 1) {  // this run's partials: max, sum and the unnormalized output per row (slot z)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = r0 + 16 * wave + 4 * lg + i;
            if (row >= a.m) continue;
            const int64_t pidx = (int64_t(row) * a.heads + h) * kAttnMaxSplits + blockIdx.z;
            if (lr == 0) {
                a.part.pm[pidx] = mrow[i];
                a.part.pl[pidx] = lrow[i];
            }
            if (mrow[i] != -INFINITY)  // the merge reads no output of a run without keys for the row
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) a.part.po[pidx * HD + 16 * dt + lr] = o[dt][i];
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = r0 + 16 * wave + 4 * lg + i;
        if (row >= a.m) continue;
        const float inv = 1.0f / lrow[i];
        const int64_t off = row * qd + int64_t(h) * HD;
        if (a.out16) {  // f16 halves for the o projection's split-f16 product
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                const float x = o[dt][i] * inv;
                const _Float16 hi = _Float16(x);
                a.out16[off + 16 * dt + lr] = hi;
                a.out16[a.lo_off + off + 16 * dt + lr] = _Float16(x - float(hi));
            }
        } else {
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) a.out[off + 16 * dt + lr] = o[dt][i] * inv;
        }
    }
}

// The runs of a key-split prefill attention merged per (row, head): M = the runs' largest max, the sums and
// outputs scaled by exp(max - M) and added in run order, then out = O (1 / L) as f32 or as f16 halves (hi at out16,
// lo at out16 + lo_off). grid (ceil(heads HD / 256), m), block 256: thread t of a block takes element t % HD of
// head (256 blockIdx.x + t) / HD; every run's values are loaded before any is used.
template <int HD>
__global__ __launch_bounds__(256) void k_pattn_merge(PrefillAttnArgs a) {
    const int t = int(blockIdx.x) * 256 + int(threadIdx.x), h = t / HD, i = blockIdx.y, e = t % HD;
    if (h >= a.heads) return;
    const int64_t base = (int64_t(i) * a.heads + h) * kAttnMaxSplits;
    float pm[kAttnMaxSplits], pl[kAttnMaxSplits], po[kAttnMaxSplits];
    // every run's partial output is loaded with its max and sum (the choice depends only on the run count), so the
    // loads share one round trip; a run without keys for the row left no output, and its value is skipped below
#pragma unroll
    for (int z = 0; z < kAttnMaxSplits; ++z) {
        const bool in = z < a.splits;
        pm[z] = in ? a.part.pm[base + z] : -INFINITY;
        pl[z] = in ? a.part.pl[base + z] : 0.f;
        po[z] = in ? a.part.po[(base + z) * HD + e] : 0.f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int z = 0; z < kAttnMaxSplits; ++z) mx = fmaxf(mx, pm[z]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int z = 0; z < kAttnMaxSplits; ++z) {
        if (pm[z] == -INFINITY) continue;
        const float w = expf(pm[z] - mx);
        L = fmaf(w, pl[z], L);
        O = fmaf(w, po[z], O);
    }
    const float x = O * (1.0f / L);
    const int64_t off = int64_t(i) * a.heads * HD + int64_t(h) * HD + e;
    if (a.out16) {
        const _Float16 hi = _Float16(x);
        a.out16[off] = hi;
        a.out16[a.lo_off + off] = _Float16(x - float(hi));
    } else {
        a.out[off] = x;
    }
}

}  // namespace vh
