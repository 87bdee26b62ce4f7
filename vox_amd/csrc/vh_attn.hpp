// vh_attn.hpp — decode/prefill attention on an f16 KV cache (gfx950, wave64).
//
// Semantics follow transformer_forward (kernels.cpp:797-828): per-head RMSNorm of q and k (q_norm/k_norm),
// rotate-half RoPE with a host-built cos/sin table (the table rows are computed like rope_apply,
// kernels.cpp:740-757: angle float(inv_freq[i] * float(pos)), cosf/sinf), the new key/value appended at the
// row's position, then causal GQA softmax attention with scale 1/sqrt(hd) over keys 0..pos.
//
// The cache lives in HBM as f16 [layer][kv_head][cap][head_dim] per sequence (K and V separate), so one
// kv head's keys are contiguous. Attention is split-K ("flash-decode"): block (split, kv_head, row) runs an
// online softmax over its key range for all G = heads/kv_heads query heads that share the kv head, and
// k_attn_combine merges the splits in a fixed order (deterministic).
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {


// grid (heads + kv_heads, m), block 64. Thread t handles the rotate-half pair (t, t + hd/2).
__global__ __launch_bounds__(64) void k_qk_post(QkArgs a) {
    const int hh = blockIdx.x, i = blockIdx.y, t = threadIdx.x;
    const int hd = a.hd, half = hd / 2, qd = a.heads * hd, kd = a.kv_heads * hd;
    const RowRef rr = a.rows[i];
    const bool is_q = hh < a.heads;
    const int g = hh - a.heads;
    const float *src = a.qkv + int64_t(i) * a.ldqkv + (is_q ? hh * hd : qd + g * hd);
    const float *nw = is_q ? a.qn : a.kn;
    const bool on = t < half;
    float x0 = on ? src[t] : 0.f, x1 = on ? src[t + half] : 0.f;
    if (nw) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / float(hd) + a.eps);
        if (on) { x0 = nw[t] * (x0 * inv); x1 = nw[t + half] * (x1 * inv); }
    }
    if (!on) return;
    const float c = a.rope[(rr.pos * half + t) * 2], s = a.rope[(rr.pos * half + t) * 2 + 1];
    const float r0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    const float r1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
    if (is_q) {
        float *dst = a.q + int64_t(i) * qd + hh * hd;
        dst[t] = r0;
        dst[t + half] = r1;
    } else {
        const int64_t off = ((int64_t(a.layer) * a.kv_heads + g) * rr.cap + rr.pos) * hd;
        rr.k[off + t] = _Float16(r0);
        rr.k[off + t + half] = _Float16(r1);
        const float *vs = a.qkv + int64_t(i) * a.ldqkv + qd + kd + g * hd;
        rr.v[off + t] = _Float16(vs[t]);
        rr.v[off + t + half] = _Float16(vs[t + half]);
    }
}


// Keys per split for n visible keys: at least one block step, at most kAttnSplits splits.
VH_DEV int split_len(int64_t n, int kpb) {
    int64_t c = (n + kAttnSplits - 1) / kAttnSplits;
    c = (c + kpb - 1) / kpb * kpb;
    return int(c);
}

// grid (kAttnSplits, kv_heads, m), block 256. Each lane holds 8 consecutive elements of one key row;
// LPK = HD/8 lanes share a key, a wave covers 64/LPK keys per step.
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_partial(AttnArgs a) {
    constexpr int LPK = HD / 8, KPW = 64 / LPK, NGRP = 4 * KPW;
    extern __shared__ __align__(16) float st[];  // [NGRP][G] m, [NGRP][G] l, [NGRP][G][HD] o
    const int s = blockIdx.x, g = blockIdx.y, i = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane % LPK, kg = lane / LPK;
    const RowRef rr = a.rows[i];
    const int64_t n = rr.pos + 1;
    const int C = split_len(n, NGRP);
    const int64_t k0 = int64_t(s) * C, k1 = k0 + C < n ? k0 + C : n;
    const int qd = a.heads * HD;
    const int64_t pbase = (int64_t(i) * a.heads + g * G) * kAttnSplits + s;
    if (k0 >= n) return;  // unused split: k_attn_combine never reads it

    float qh[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) qh[h][e] = a.q[int64_t(i) * qd + (g * G + h) * HD + sub * 8 + e];
    float mh[G], lh[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mh[h] = -INFINITY; lh[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    }
    const int64_t cbase = (int64_t(a.layer) * a.kv_heads + g) * rr.cap * HD;
    const _Float16 *K = rr.k + cbase, *V = rr.v + cbase;
    for (int64_t j = k0 + wave * KPW + kg; j < k1; j += NGRP) {
        const f16x8 kv = *reinterpret_cast<const f16x8 *>(K + j * HD + sub * 8);
        const f16x8 vv = *reinterpret_cast<const f16x8 *>(V + j * HD + sub * 8);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(qh[h][e], float(kv[e]), d);
            d = group_sum<LPK>(d);
            const float sc = a.scale * d;
            const float mnew = fmaxf(mh[h], sc);
            const float corr = expf(mh[h] - mnew), p = expf(sc - mnew);
            lh[h] = lh[h] * corr + p;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = acc[h][e] * corr + p * float(vv[e]);
            mh[h] = mnew;
        }
    }
    float *sm = st, *sl = st + NGRP * G, *so = st + 2 * NGRP * G;
    const int grp = wave * KPW + kg;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (sub == 0) { sm[grp * G + h] = mh[h]; sl[grp * G + h] = lh[h]; }
#pragma unroll
        for (int e = 0; e < 8; ++e) so[(grp * G + h) * HD + sub * 8 + e] = acc[h][e];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < G * HD; t += 256) {
        const int h = t / HD, e = t % HD;
        float M = -INFINITY;
        for (int q = 0; q < NGRP; ++q) M = fmaxf(M, sm[q * G + h]);
        float L = 0.f, O = 0.f;
        for (int q = 0; q < NGRP; ++q) {
            const float w = sm[q * G + h] == -INFINITY ? 0.f : expf(sm[q * G + h] - M);
            L += w * sl[q * G + h];
            O += w * so[(q * G + h) * HD + e];
        }
        const int64_t pidx = pbase + int64_t(h) * kAttnSplits;
        a.po[pidx * HD + e] = O;
        if (e == 0) { a.pm[pidx] = M; a.pl[pidx] = L; }
    }
}

// grid (heads, m), block HD: merges the used splits of k_attn_partial in split order.
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(AttnArgs a) {
    constexpr int LPK = HD / 8, NGRP = 4 * (64 / LPK);
    const int h = blockIdx.x, i = blockIdx.y, e = threadIdx.x;
    const int64_t n = a.rows[i].pos + 1;
    const int C = split_len(n, NGRP);
    const int used = int((n + C - 1) / C);
    const int64_t base = (int64_t(i) * a.heads + h) * kAttnSplits;
    float M = -INFINITY;
    for (int s = 0; s < used; ++s) M = fmaxf(M, a.pm[base + s]);
    float L = 0.f, O = 0.f;
    for (int s = 0; s < used; ++s) {
        const float w = expf(a.pm[base + s] - M);
        L += w * a.pl[base + s];
        O += w * a.po[(base + s) * HD + e];
    }
    a.out[int64_t(i) * a.heads * HD + h * HD + e] = O / L;
}

}  // namespace vh
