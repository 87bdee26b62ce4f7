// vh_attn.hpp — decode/prefill attention on an f16 KV cache (gfx950, wave64).
//
// Semantics follow transformer_forward (kernels.cpp:797-828): per-head RMSNorm of q and k (q_norm/k_norm),
// rotate-half RoPE with a host-built cos/sin table (rows computed like rope_apply, kernels.cpp:740-757:
// angle float(inv_freq[i] * float(pos)), cosf/sinf), the new key/value appended at the row's position, then
// causal GQA softmax attention with scale 1/sqrt(hd) over keys 0..pos (kernels.cpp:812-826).
//
// The cache lives in HBM as f16 [layer][kv_head][cap][head_dim] per sequence (K and V separate), so one kv head's
// keys are contiguous. Attention is split-K: block (split, kv_head, row) runs an online softmax over its key range
// for the G = heads / kv_heads query heads sharing the kv head and writes unnormalized partials (max, denominator,
// weighted value sum). The consumer (the o-projection GEMV's prologue) merges the splits in split order.
//
// FUSED (decode, and rows of distinct sequences): the kernel also does k_qk_post's work for its row. Every split
// block normalizes and rotates its G query heads itself; the last split, whose range holds the new key at `pos`,
// writes the new key/value to the cache and uses them from LDS, so no block reads a cache entry written by
// another block of the same launch. Not FUSED (prefill of one sequence): k_qk_post has already written q and the
// pass's keys, and every key is read from the cache.
#pragma once
#include <type_traits>

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
    // Every input that does not depend on the row reference (the q|k|v values, the norm weights, the v values) is
    // loaded with it, then the RoPE row it names: two round trips. Lanes past half read element 0 and drop it.
    const int tt = on ? t : 0;
    const float *nwp = nw ? nw : src;
    const float *vs = a.qkv + int64_t(i) * a.ldqkv + qd + kd + (is_q ? 0 : g * hd);
    const float lx0 = src[tt], lx1 = src[tt + half];
    const float lw0 = nwp[tt], lw1 = nwp[tt + half];
    const float v0 = vs[tt], v1 = vs[tt + half];
    const float c = a.rope[(rr.pos * half + tt) * 2], s = a.rope[(rr.pos * half + tt) * 2 + 1];
    float x0 = on ? lx0 : 0.f, x1 = on ? lx1 : 0.f;
    if (nw) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / float(hd) + a.eps);
        x0 = lw0 * (x0 * inv);
        x1 = lw1 * (x1 * inv);
    }
    if (!on) return;
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
        rr.v[off + t] = _Float16(v0);
        rr.v[off + t + half] = _Float16(v1);
    }
}

// k_qk_post for head_dim 2 HALF (64 or 128) with several heads per block: grid (ceil((heads + kv_heads) / (256 /
// HALF)), m), block 256. The HALF lanes of a head are consecutive lanes of one wave, so its norm sums over them
// (group_sum<HALF>, the same sum of the same squares as k_qk_post's wave sum, whose other lanes add zeros, in the
// same tree order); every lane holds one rotate-half pair, so no lane is idle.
template <int HALF>
__global__ __launch_bounds__(256) void k_qk_post_wide(QkArgs a) {
    constexpr int HD = 2 * HALF;
    const int t = int(threadIdx.x), hh = int(blockIdx.x) * (256 / HALF) + t / HALF, i = blockIdx.y, p = t % HALF;
    const int nh = a.heads + a.kv_heads;
    const int hc = hh < nh ? hh : nh - 1;  // lanes past the last head compute a copy of it and store nothing
    const int qd = a.heads * HD, kd = a.kv_heads * HD;
    const RowRef rr = a.rows[i];
    const bool is_q = hc < a.heads;
    const int g = hc - a.heads;
    const float *src = a.qkv + int64_t(i) * a.ldqkv + (is_q ? hc * HD : qd + g * HD);
    const float *nw = is_q ? a.qn : a.kn;
    const float *nwp = nw ? nw : src;
    const float *vs = a.qkv + int64_t(i) * a.ldqkv + qd + kd + (is_q ? 0 : g * HD);
    float x0 = src[p], x1 = src[p + HALF];
    const float lw0 = nwp[p], lw1 = nwp[p + HALF];
    const float v0 = vs[p], v1 = vs[p + HALF];
    const float c = a.rope[(rr.pos * HALF + p) * 2], sn = a.rope[(rr.pos * HALF + p) * 2 + 1];
    if (nw) {  // a head's lanes share the branch (the head's kind decides nw)
        const float ss = group_sum<HALF>(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / float(HD) + a.eps);
        x0 = lw0 * (x0 * inv);
        x1 = lw1 * (x1 * inv);
    }
    if (hh >= nh) return;
    const float r0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
    const float r1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, sn));
    if (is_q) {
        float *dst = a.q + int64_t(i) * qd + hc * HD;
        dst[p] = r0;
        dst[p + HALF] = r1;
    } else {
        const int64_t off = ((int64_t(a.layer) * a.kv_heads + g) * rr.cap + rr.pos) * HD;
        rr.k[off + p] = _Float16(r0);
        rr.k[off + p + HALF] = _Float16(r1);
        rr.v[off + p] = _Float16(v0);
        rr.v[off + p + HALF] = _Float16(v1);
    }
}

// Attention for the head sizes the split-K and MFMA kernels are not built for (any even hd <= 128): grid (heads, m),
// block 256. Lane l of each wave holds dims l and l + 64; wave w takes keys w, w + 4, ... of the row's cache with an
// online softmax (score = scale * q.k, as kernels.cpp:818-819), and the four waves are merged through LDS.
__global__ __launch_bounds__(256) void k_attn_rows(AttnRowsArgs a) {
    const int h = blockIdx.x, i = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int hd = a.hd, qd = a.heads * hd, g = h / (a.heads / a.kv_heads);
    const RowRef rr = a.rows[i];
    const float *q = a.q + int64_t(i) * qd + h * hd;
    const int d0 = lane, d1 = lane + 64;
    const bool on0 = d0 < hd, on1 = d1 < hd;
    const float q0 = on0 ? q[d0] : 0.f, q1 = on1 ? q[d1] : 0.f;
    const int64_t plane = ((int64_t(a.layer) * a.kv_heads + g) * rr.cap) * hd;
    const _Float16 *K = rr.k + plane, *V = rr.v + plane;
    const int64_t n = rr.pos + 1;
    float mx = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
    for (int64_t j = w; j < n; j += 4) {
        const _Float16 *kr = K + j * hd, *vr = V + j * hd;
        const float k0 = on0 ? float(kr[d0]) : 0.f, k1 = on1 ? float(kr[d1]) : 0.f;
        const float v0 = on0 ? float(vr[d0]) : 0.f, v1 = on1 ? float(vr[d1]) : 0.f;
        const float sc = a.scale * wave_sum(q0 * k0 + q1 * k1);
        const float mn = fmaxf(mx, sc), corr = expf(mx - mn), p = expf(sc - mn);
        o0 = o0 * corr + p * v0;
        o1 = o1 * corr + p * v1;
        l = l * corr + p;
        mx = mn;
    }
    __shared__ float sm_m[4], sm_l[4], sm_o[4][128];
    if (lane == 0) { sm_m[w] = mx; sm_l[w] = l; }
    sm_o[w][d0] = o0;
    sm_o[w][d1] = o1;
    __syncthreads();
    const float M = fmaxf(fmaxf(sm_m[0], sm_m[1]), fmaxf(sm_m[2], sm_m[3]));  // wave 0 holds key 0: finite
    float e[4], L = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) { e[u] = expf(sm_m[u] - M); L += sm_l[u] * e[u]; }
    for (int d = threadIdx.x; d < hd; d += 256) {
        float O = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) O += sm_o[u][d] * e[u];
        a.out[int64_t(i) * qd + h * hd + d] = O / L;
    }
}

// One rotate-half pair of a head: optional RMSNorm over the head (the HALF lanes of a group hold its pairs),
// then RoPE. Rounding as rope_apply: products and the difference/sum each rounded (no contraction).
// Eight f16 of a KV cache through the global address space: the cache pointers of the row table are generic, and a
// flat load would make every later wait count for all outstanding loads (flat also counts as an LDS access).
VH_DEV f16x8 ld_cache8(const _Float16 *p) {
    return *(const __attribute__((address_space(1))) f16x8 *)(p);
}

// norm: whether the head has a norm; w0, w1: its weights at p and p + HALF (loaded by the caller).
template <int HALF>
VH_DEV void norm_rope(float &x0, float &x1, bool norm, float w0, float w1, float eps, float c, float s) {
    if (norm) {
        const float ss = group_sum<HALF>(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / float(2 * HALF) + eps);
        x0 = w0 * (x0 * inv);
        x1 = w1 * (x1 * inv);
    }
    const float r0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    const float r1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x0, s));
    x0 = r0;
    x1 = r1;
}

template <int HD, int G>
struct AttnSmem {
    static constexpr int LPK = HD / 8, KPW = 64 / LPK, NGRP = 4 * KPW;
    float q[G][HD];
    float knew[HD], vnew[HD];  // the new key (f16-rounded) and value, last split of a fused row
    float m[NGRP][G], l[NGRP][G], w[NGRP][G];
    float o[NGRP][G][HD];
};

// grid (kAttnMaxSplits, kv_heads x group / G, m), block 256. A block takes G of the group's query heads (all of
// them, or a subgroup when there are few kv heads, so that more blocks share the work). Each lane holds 8 consecutive elements of one key row;
// LPK = HD / 8 lanes share a key, a wave covers 64 / LPK keys per step, a block NGRP keys. Split s takes the keys
// j = s + S (grp + NGRP u). Row 0's cache bases, the q|k|v input and the RoPE rows are leading scalar arguments
// (preloaded with the dispatch): the first batch's loads go out before the row's position arrives and are masked by
// it afterwards, so the cache fetch does not wait for the row view. The first batch is kAttnSpecKeys keys in a
// launch of one row and U groups (S NGRP U keys) in a launch of several, whose blocks have less to hide the
// dependent round trip behind; later keys load per batch of U.
// ONE_ROW (launches of one row, m == 1): only row 0's path is compiled, so the compiler's wait counts follow one
// static load sequence. LONG (one row at a position past kAttnSpecKeys): the first batch is U groups, as for
// several rows, since the keys past kAttnSpecKeys are there to be read.
template <int HD, int G, bool FUSED, bool ONE_ROW = false, bool LONG = false>
__global__ __launch_bounds__(256) void k_attn(const _Float16 *kc0, const _Float16 *vc0, const float *qkv,
                                              const float *rope_rows, int32_t cap0, int32_t layer, AttnArgs a) {
    using Sm = AttnSmem<HD, G>;
    constexpr int LPK = Sm::LPK, KPW = Sm::KPW, NGRP = Sm::NGRP, HALF = HD / 2, S = kAttnMaxSplits;
    constexpr int U = G <= 2 ? 8 : G <= 4 ? 4 : 2;
    // groups in the first batch: U1S (kAttnSpecKeys keys) for one row, U for several or for one row far enough in
    constexpr int U1S = kAttnSpecKeys / (S * NGRP) < U ? kAttnSpecKeys / (S * NGRP) : U;
    constexpr int U1 = ONE_ROW && !LONG ? U1S : U;
    constexpr int NQ = (G * HALF + 255) / 256;  // q rotate-half pairs per thread
    extern __shared__ __align__(16) uint8_t attn_smem[];
    Sm &sm = *reinterpret_cast<Sm *>(attn_smem);
    const int s = blockIdx.x, i = blockIdx.z, tid = threadIdx.x;
    // blockIdx.y = kv head x (group / G) + query-head subgroup: this block's query heads are h0 .. h0 + G - 1
    const int hsplit = a.group / G, g = blockIdx.y / hsplit, hs = blockIdx.y % hsplit, h0 = g * a.group + hs * G;
    const int lane = tid & 63, wave = tid >> 6, sub = lane % LPK, grp = wave * KPW + lane / LPK;
    const AttnPartials &P = a.part;
    const int qd = P.heads * HD, kd = a.kv_heads * HD;
    const float *row = qkv + int64_t(i) * a.ldqkv;
    const int64_t plane = (int64_t(layer) * a.kv_heads + g) * HD;  // x cap: offset of this kv head's plane

    // Every small input first (q/k/v of the row, its RoPE row, the q/k norm weights, the row view), then the
    // speculative cache loads: loads return in issue order, so the q/k work below waits only for the small ones and
    // runs while the keys are in flight.
    float qx0[NQ], qx1[NQ], qc[NQ], qsn[NQ], qg0[NQ], qg1[NQ];
    float kx0 = 0.f, kx1 = 0.f, vx0 = 0.f, vx1 = 0.f, kc = 0.f, ksn = 0.f, kg0 = 0.f, kg1 = 0.f;
    const bool kv_lane = tid >= 192 && tid - 192 < HALF;  // last wave: the new key/value of a fused row
    if (FUSED) {
        // branch-free: lanes without a pair load pair 0 and never use it, so every wave issues the same loads
        const float *cs = rope_rows + int64_t(i) * HD;
        const float *qn = a.qn ? a.qn : cs, *kn = a.kn ? a.kn : cs;  // without norms: loaded from cs, never used
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int t = tid + 256 * k, tq = t < G * HALF ? t : 0, h = tq / HALF, p = tq % HALF;
            qx0[k] = row[(h0 + h) * HD + p];
            qx1[k] = row[(h0 + h) * HD + p + HALF];
            qc[k] = cs[2 * p];
            qsn[k] = cs[2 * p + 1];
            qg0[k] = qn[p];
            qg1[k] = qn[p + HALF];
        }
        const int p = kv_lane ? tid - 192 : 0;
        kx0 = row[qd + g * HD + p];
        kx1 = row[qd + g * HD + p + HALF];
        vx0 = row[qd + kd + g * HD + p];
        vx1 = row[qd + kd + g * HD + p + HALF];
        kc = cs[2 * p];
        ksn = cs[2 * p + 1];
        kg0 = kn[p];
        kg1 = kn[p + HALF];
    }
    const RowRef rr = P.rows[i];

    // row 0 (every decode step): cache bases from the arguments, speculative loads of the first keys
    f16x8 kb[U], vb[U];
    if (ONE_ROW || i == 0) {
        const _Float16 *K = kc0 + plane * cap0, *V = vc0 + plane * cap0;
#pragma unroll
        for (int u = 0; u < U1; ++u) {
            const int64_t j = s + int64_t(S) * (grp + NGRP * u);
            const int64_t jc = j < cap0 ? j : 0;  // stay inside the cache; masked below
            kb[u] = ld_cache8(K + jc * HD + sub * 8);
            vb[u] = ld_cache8(V + jc * HD + sub * 8);
        }
    }
    // the new value's f16 bits (the last split's kv lanes use them), converted only after the cache loads are issued
    __builtin_amdgcn_sched_barrier(0);
    const _Float16 v0h = _Float16(vx0), v1h = _Float16(vx1);

    const int64_t n = rr.pos + 1;
    const int64_t pb = (int64_t(i) * P.heads + h0) * kAttnMaxSplits + s;  // + h * kAttnMaxSplits
    if (s >= n) {  // no keys in this split
        for (int t = tid; t < G * HD; t += 256) {
            const int h = t / HD, e = t % HD;
            const int64_t pidx = pb + int64_t(h) * kAttnMaxSplits;
            P.po[pidx * HD + e] = 0.f;
            if (e == 0) { P.pm[pidx] = -INFINITY; P.pl[pidx] = 0.f; }
        }
        return;
    }
    const bool last = FUSED && rr.pos % S == s;  // this split holds the new key at pos
    const _Float16 *K = rr.k + plane * rr.cap, *V = rr.v + plane * rr.cap;
    // keys read from the cache: j < kend, except the new key of a fused row (processed from LDS below)
    const int64_t kend = last ? n - 1 : n;
    if (!ONE_ROW && i != 0) {  // other rows: their speculative batch waits for the row view
#pragma unroll
        for (int u = 0; u < U1; ++u) {
            const int64_t j = s + int64_t(S) * (grp + NGRP * u);
            const int64_t jc = j < rr.cap ? j : 0;
            kb[u] = ld_cache8(K + jc * HD + sub * 8);
            vb[u] = ld_cache8(V + jc * HD + sub * 8);
        }
    }

    if (FUSED) {
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int t = tid + 256 * k, h = t / HALF, p = t % HALF;
            if (t < G * HALF) {
                norm_rope<HALF>(qx0[k], qx1[k], a.qn != nullptr, qg0[k], qg1[k], a.eps, qc[k], qsn[k]);
                sm.q[h][p] = qx0[k];
                sm.q[h][p + HALF] = qx1[k];
            }
        }
        if (last && kv_lane) {
            const int p = tid - 192;
            norm_rope<HALF>(kx0, kx1, a.kn != nullptr, kg0, kg1, a.eps, kc, ksn);
            const _Float16 k0h = _Float16(kx0), k1h = _Float16(kx1);
            if (hs == 0) {  // one block of the kv head appends the new key/value
                const int64_t off = rr.pos * HD;
                typedef __attribute__((address_space(1))) _Float16 gf16;  // a global store, as ld_cache8's loads
                gf16 *Kw = (gf16 *)(rr.k + plane * rr.cap), *Vw = (gf16 *)(rr.v + plane * rr.cap);
                Kw[off + p] = k0h;
                Kw[off + p + HALF] = k1h;
                Vw[off + p] = v0h;
                Vw[off + p + HALF] = v1h;
            }
            sm.knew[p] = float(k0h);
            sm.knew[p + HALF] = float(k1h);
            sm.vnew[p] = float(v0h);
            sm.vnew[p + HALF] = float(v1h);
        }
    } else {
        for (int t = tid; t < G * HD; t += 256) {
            const int h = t / HD, e = t % HD;
            sm.q[h][e] = a.q[int64_t(i) * qd + (h0 + h) * HD + e];
        }
    }
    __syncthreads();

    float qh[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) qh[h][e] = sm.q[h][sub * 8 + e];
    float mh[G], lh[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mh[h] = -INFINITY;
        lh[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    }
    // Online softmax update with a batch of NU keys (invalid ones masked); all LPK lanes of a group call it
    // together. The NU x G dot products and their group sums are independent, so their latencies overlap.
    auto consume = [&](auto nu_tag, const f16x8 *kq, const f16x8 *vq, const bool *valid) {
        constexpr int NU = decltype(nu_tag)::value;
        float sc[NU][G];
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qh[h][e], float(kq[u][e]), d);
                sc[u][h] = d;
            }
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int h = 0; h < G; ++h) sc[u][h] = valid[u] ? a.scale * group_sum<LPK>(sc[u][h]) : -INFINITY;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float mnew = mh[h];
#pragma unroll
            for (int u = 0; u < NU; ++u) mnew = fmaxf(mnew, sc[u][h]);
            if (mnew == -INFINITY) continue;  // no key in this group yet
            const float corr = expf(mh[h] - mnew);
            float l = lh[h] * corr, o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = acc[h][e] * corr;
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const float p = valid[u] ? expf(sc[u][h] - mnew) : 0.f;
                l += p;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = fmaf(p, float(vq[u][e]), o[e]);
            }
            lh[h] = l;
            mh[h] = mnew;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = o[e];
        }
    };
    // Keys are consumed (one online-softmax update per batch) in the batches of a one-row launch: groups [0, U1S),
    // then [U1S + k U, U1S + (k + 1) U). Launches of several rows load U groups first, one round trip for up to
    // S NGRP U keys, and consume the same batches, so one and several rows sum in the same order.
    int64_t jb0 = s + int64_t(S) * (grp + NGRP * U1S);  // first group of the next batch to load
    {
        bool valid[U1];
#pragma unroll
        for (int u = 0; u < U1; ++u) {
            valid[u] = s + int64_t(S) * (grp + NGRP * u) < kend;
            if (!valid[u]) kb[u] = vb[u] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};  // masked: finite zeros, weight 0
        }
        consume(std::integral_constant<int, U1S>(), kb, vb, valid);
        if constexpr (U1 > U1S) {
            // groups [U1S, U) are in registers: the head of batch [U1S, U1S + U). Without keys past them in this
            // block (block-uniform) that batch is those groups alone (masked groups leave the softmax state as it
            // is); otherwise its other U1S groups are loaded now.
            if (s + int64_t(S) * NGRP * U < kend) {
                bool v2[U];
#pragma unroll
                for (int u = 0; u < U - U1S; ++u) {
                    kb[u] = kb[u + U1S];
                    vb[u] = vb[u + U1S];
                    v2[u] = valid[u + U1S];
                }
#pragma unroll
                for (int u = U - U1S; u < U; ++u) {
                    const int64_t j = jb0 + int64_t(S) * NGRP * u;
                    v2[u] = j < kend;
                    if (v2[u]) {
                        kb[u] = ld_cache8(K + j * HD + sub * 8);
                        vb[u] = ld_cache8(V + j * HD + sub * 8);
                    } else {
                        kb[u] = vb[u] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
                    }
                }
                consume(std::integral_constant<int, U>(), kb, vb, v2);
            } else {
                consume(std::integral_constant<int, U - U1S>(), kb + U1S, vb + U1S, valid + U1S);
            }
            jb0 += int64_t(S) * NGRP * U;
        }
    }
    for (int64_t jb = jb0; jb < kend; jb += int64_t(S) * NGRP * U) {
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = jb + int64_t(S) * NGRP * u;
            valid[u] = j < kend;
            if (valid[u]) {
                kb[u] = ld_cache8(K + j * HD + sub * 8);
                vb[u] = ld_cache8(V + j * HD + sub * 8);
            } else {
                kb[u] = vb[u] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
        consume(std::integral_constant<int, U>(), kb, vb, valid);
    }
    if (last && grp == 0) {  // the new key at pos, from LDS (f16-rounded like the cache)
        f16x8 kn1[1], vn1[1];
#pragma unroll
        for (int e = 0; e < 8; ++e) { kn1[0][e] = _Float16(sm.knew[sub * 8 + e]); vn1[0][e] = _Float16(sm.vnew[sub * 8 + e]); }
        const bool v1[1] = {true};
        consume(std::integral_constant<int, 1>(), kn1, vn1, v1);
    }

    // merge the NGRP key groups in LDS, in group order
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (sub == 0) { sm.m[grp][h] = mh[h]; sm.l[grp][h] = lh[h]; }
#pragma unroll
        for (int e = 0; e < 8; ++e) sm.o[grp][h][sub * 8 + e] = acc[h][e];
    }
    __syncthreads();
    for (int t = tid; t < NGRP * G; t += 256) {
        const int q = t / G, h = t % G;
        float M = -INFINITY;
        for (int r = 0; r < NGRP; ++r) M = fmaxf(M, sm.m[r][h]);
        sm.w[q][h] = sm.m[q][h] == -INFINITY ? 0.f : expf(sm.m[q][h] - M);
    }
    __syncthreads();
    for (int t = tid; t < G * HD; t += 256) {
        const int h = t / HD, e = t % HD;
        float O = 0.f;
        for (int r = 0; r < NGRP; ++r) O = fmaf(sm.w[r][h], sm.o[r][h][e], O);
        const int64_t pidx = pb + int64_t(h) * kAttnMaxSplits;
        P.po[pidx * HD + e] = O;
        if (e == 0) {
            float M = -INFINITY, L = 0.f;
            for (int r = 0; r < NGRP; ++r) M = fmaxf(M, sm.m[r][h]);
            for (int r = 0; r < NGRP; ++r) L = fmaf(sm.w[r][h], sm.l[r][h], L);
            P.pm[pidx] = M;
            P.pl[pidx] = L;
        }
    }
}

}  // namespace vh
