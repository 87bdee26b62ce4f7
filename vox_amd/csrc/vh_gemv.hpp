// vh_gemv.hpp — weight-streaming GEMV kernels for gfx950 (decode, m <= 8 rows).
//
// y[i][r] (+)= sum_k W[r][k] * x[i][k] (+ bias[r]) for i < m, the device counterpart of matmul()
// (kernels.cpp:653-705). The weights are the HBM stream: each lane issues 16-byte non-temporal loads, 64
// consecutive lanes cover 1 KiB of one row, and every wave keeps R rows x IT such chunks in flight. The tile
// (R, IT) is picked so one launch is one round of blocks over the 256 CUs, and the weight loads are issued
// before the activation prologue, which does not depend on them.
//
// Two arithmetic families, as the reference dispatcher chooses them:
//  - k_gemv_int: Q8 (m <= 8) and Q4. The input is quantized per 32-block to int8 in LDS exactly as
//    kernels.cpp:515-523; block dots are exact int32 (v_dot4_i32_i8), then float(dot) * (ws * xs).
//  - k_gemv_flt: F32 / F16 / BF16 and Q8 with m > 8: f32 activations in LDS, weights widened
//    (Q8: float(q) * scale as kernels.cpp:665-674), f32 FMA accumulation.
// Prologues (one global round trip each, every block computing its own copy of the input):
//  PRO_X     x as given;
//  PRO_RMS   RMSNorm(x, gamma, eps) first (kernels.cpp:707-712);
//  PRO_ATTN  x = merge of the split-K attention partials of each head (the softmax-weighted sum over keys of
//            kernels.cpp:818-826, finished here instead of in a separate kernel).
// Epilogues: store, accumulate (the residual add of kernels.cpp:831/:839), or SwiGLU over interleaved
// (gate, up) row pairs (kernels.cpp:836).
#pragma once
#include <type_traits>

#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

template <int WT>
VH_DEV int64_t row_bytes(int K) {
    return WT == WT_F32 ? int64_t(K) * 4 : WT == WT_Q8 ? int64_t(K) : (WT == WT_Q4 || WT == WT_Q4H) ? int64_t(K) / 2 : int64_t(K) * 2;
}

// ---------------------------------------------------------------------------------------------- prologue
// The prologue produces the f32 input rows v[mm][K] (mm < a.m; rows a.m..M-1 are zeros) in 8-element slots: slot s
// of row mm holds elements 8s..8s+7, a 32-block is 4 consecutive slots handled by 4 consecutive lanes.
// `sink(mm, s, v)` receives each slot with all 4 lanes of its block active.
//
// The partner lane of step S of wave_sum's tree: xor 1, xor 2, mirror in 8 (lane ^ 7), mirror in 16 (lane ^ 15),
// then the rows: lane ^ 16, lane ^ 32.
template <int S>
VH_DEV float tree_partner(float x) {
    if constexpr (S == 0) return dpp<kDppXor1>(x);
    else if constexpr (S == 1) return dpp<kDppXor2>(x);
    else if constexpr (S == 2) return dpp<kDppRowHalfMirror>(x);
    else if constexpr (S == 3) return dpp<kDppRowMirror>(x);
    else if constexpr (S == 4) return __shfl_xor(x, 16, kWave);
    else return __shfl_xor(x, 32, kWave);
}

// N = 2^n values per lane (all 64 lanes active), each summed over the wave; returns the total of value `lane` to
// lane < N. A reduce-scatter on wave_sum's tree: at step s (partner as tree_partner<s>) a lane keeps half of its
// values and adds its partner's copies of them, so each total is the same sum, in the same order, as wave_sum's,
// with N - 1 partner exchanges instead of 6 N. The half a lane keeps at step s is bit h_s of
//   (b0 ^ b2, b1 ^ b2, b2 ^ b3, b3, b4, b5)   (b_i: bit i of the lane),
// which flips between the step's partners and is the same for the partners of every later step, so both lanes of
// every exchange hold the same values. After n steps the lane's value is number sum_s h_s 2^(n-1-s); steps n..5
// add whole totals (wave_sum's remaining steps) and a last exchange moves value j to lane j.
template <int N>
VH_DEV float wave_sums_scatter(float (&v)[N], int lane) {
    constexpr int n = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : N == 16 ? 4 : N == 32 ? 5 : 6;
    static_assert((1 << n) == N && N <= 64, "a power of two up to 64");
    const int b0 = lane & 1, b1 = (lane >> 1) & 1, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
    const bool h[6] = {(b0 ^ b2) != 0, (b1 ^ b2) != 0, (b2 ^ b3) != 0, b3 != 0, ((lane >> 4) & 1) != 0, ((lane >> 5) & 1) != 0};
    auto step = [&](auto s_tag) {
        constexpr int S = decltype(s_tag)::value;
        if constexpr (S < n) {
            constexpr int H = N >> (S + 1);  // values kept after this step
#pragma unroll
            for (int t = 0; t < H; ++t) {
                const float keep = h[S] ? v[t + H] : v[t], give = h[S] ? v[t] : v[t + H];
                v[t] = keep + tree_partner<S>(give);
            }
        } else {
            v[0] = v[0] + tree_partner<S>(v[0]);
        }
    };
    step(std::integral_constant<int, 0>());
    step(std::integral_constant<int, 1>());
    step(std::integral_constant<int, 2>());
    step(std::integral_constant<int, 3>());
    step(std::integral_constant<int, 4>());
    step(std::integral_constant<int, 5>());
    // the lane holding value j = lane: h_s = bit n-1-s of j for s < n, 0 after; solve for the lane bits
    int hj[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < n; ++s) hj[s] = (lane >> (n - 1 - s)) & 1;
    const int c3 = hj[3], c2 = hj[2] ^ c3, c1 = hj[1] ^ c2, c0 = hj[0] ^ c2;
    return __shfl(v[0], c0 | (c1 << 1) | (c2 << 2) | (c3 << 3) | (hj[4] << 4) | (hj[5] << 5), kWave);
}

// When its global inputs fit in registers (slot s = threadIdx.x + 256 k, k < KS), pro_stage() loads them BEFORE the
// kernel issues its weight stream. Vector loads return in issue order, so the prologue then waits for its own
// inputs only and the weights arrive while it computes. Larger inputs are read inside prologue(), after the weights.
template <int M, int PRO>
struct ProStage {
    static constexpr int KS = PRO == PRO_ATTN ? 1 : 4;
    float x[KS][8];  // PRO_X, PRO_RMS: input slots
    float g[KS][8];  // PRO_RMS: gamma slots
    float pm[kAttnMaxSplits], pl[kAttnMaxSplits];
    f32x4 o0[kAttnMaxSplits], o1[kAttnMaxSplits];  // PRO_ATTN: the slot's split partials
};

VH_DEV void load8(const float *p, float (&v)[8]) {
    const f32x4 t0 = *reinterpret_cast<const f32x4 *>(p), t1 = *reinterpret_cast<const f32x4 *>(p + 4);
    v[0] = t0.x; v[1] = t0.y; v[2] = t0.z; v[3] = t0.w; v[4] = t1.x; v[5] = t1.y; v[6] = t1.z; v[7] = t1.w;
}

// Partials of one slot (row mm, elements e0..e0+7 of head e0 / hd) for all kAttnMaxSplits splits.
template <class PM, class PO>
VH_DEV void load_partials(const AttnPartials &P, int mm, int sl, PM &pm, PM &pl, PO &o0, PO &o1) {
    const int e0 = sl * 8, h = e0 / P.hd, d0 = e0 % P.hd;
    const int64_t base = (int64_t(mm) * P.heads + h) * kAttnMaxSplits;
#pragma unroll
    for (int q = 0; q < kAttnMaxSplits; ++q) {
        pm[q] = P.pm[base + q];
        pl[q] = P.pl[base + q];
        o0[q] = *reinterpret_cast<const f32x4 *>(P.po + (base + q) * P.hd + d0);
        o1[q] = *reinterpret_cast<const f32x4 *>(P.po + (base + q) * P.hd + d0 + 4);
    }
}

// Merge of all kAttnMaxSplits partials (empty splits have max -inf and weigh 0): softmax-weighted value sum.
template <class PM, class PO>
VH_DEV void merge_partials(const PM &pm, const PM &pl, const PO &o0, const PO &o1, float (&v)[8]) {
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < kAttnMaxSplits; ++q) mx = fmaxf(mx, pm[q]);
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = 0.f;
#pragma unroll
    for (int q = 0; q < kAttnMaxSplits; ++q) {
        const float w = pm[q] == -INFINITY ? 0.f : expf(pm[q] - mx);
        L = fmaf(w, pl[q], L);
        v[0] = fmaf(w, o0[q].x, v[0]); v[1] = fmaf(w, o0[q].y, v[1]); v[2] = fmaf(w, o0[q].z, v[2]); v[3] = fmaf(w, o0[q].w, v[3]);
        v[4] = fmaf(w, o1[q].x, v[4]); v[5] = fmaf(w, o1[q].y, v[5]); v[6] = fmaf(w, o1[q].z, v[6]); v[7] = fmaf(w, o1[q].w, v[7]);
    }
    const float il = 1.0f / L;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= il;
}

// Whether a prologue's inputs fit the staging registers (the host instantiates STAGE accordingly).
template <int M, int PRO>
__host__ __device__ inline bool pro_stageable(int K) {
    return M * (K / 8) <= ProStage<M, PRO>::KS * kGemvThreads;
}

template <int M, int PRO>
VH_DEV void pro_stage(const GemvArgs &a, const float *x, int K, ProStage<M, PRO> &st) {
    constexpr int KS = ProStage<M, PRO>::KS;
    const int spr = K / 8, nslot = M * spr;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        // branch-free: slots past the end read slot 0 and are never used, so the load count is static
        const int s = threadIdx.x + k * kGemvThreads;
        const bool in = s < nslot;
        const int mm = in ? s / spr : 0, sl = in ? s % spr : 0;
        const bool on = in && mm < a.m;
        if (PRO == PRO_ATTN) {
            load_partials(a.attn, on ? mm : 0, sl, st.pm, st.pl, st.o0, st.o1);
        } else {
            // raw values only: masking them here would make the compiler wait for them before the weight stream
            load8(x + int64_t(on ? mm : 0) * a.ldx + sl * 8, st.x[k]);
            if (PRO == PRO_RMS) load8(a.gamma + sl * 8, st.g[k]);
        }
    }
}

template <int M, int PRO, bool STAGE, class Sink>
VH_DEV void prologue(const GemvArgs &a, const float *x, int K, float *red, const ProStage<M, PRO> &st, Sink &&sink) {
    constexpr int KS = ProStage<M, PRO>::KS;
    const int spr = K / 8, nslot = M * spr;
    // Runs f(k, s) over this thread's slots s = threadIdx.x + 256 k; unrolled when staged, so st.x[k] is static.
    auto for_slots = [&](auto &&f) {
        if constexpr (STAGE) {
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const int s = threadIdx.x + k * kGemvThreads;
                if (s < nslot) f(k, s);
            }
        } else {
            for (int s = threadIdx.x; s < nslot; s += kGemvThreads) f(-1, s);
        }
    };
    // slot k of this thread (k < 0: not staged, read it from global memory)
    auto get_x = [&](int k, int mm, int sl, float (&v)[8]) {
        if (k >= 0) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = mm < a.m ? st.x[k][j] : 0.f;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = 0.f;
            if (mm < a.m) load8(x + int64_t(mm) * a.ldx + sl * 8, v);
        }
    };
    auto emit = [&](int mm, int sl, float (&v)[8]) {
        if (PRO != PRO_X && a.xnorm && blockIdx.x == 0 && mm < a.m)
#pragma unroll
            for (int j = 0; j < 8; ++j) a.xnorm[int64_t(mm) * K + sl * 8 + j] = v[j];
        sink(mm, sl, v);
    };
    if (PRO == PRO_RMS) {
        float ss[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) ss[mm] = 0.f;
        // pass 1: sum of squares of every row (kernels.cpp:709-710)
        for_slots([&](int k, int s) {
            const int mm = s / spr, sl = s % spr;
            float t[8];
            get_x(k, mm, sl, t);
            float q = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) q = fmaf(t[j], t[j], q);
#pragma unroll
            for (int r = 0; r < M; ++r)
                if (r == mm) ss[r] += q;
        });
        if constexpr (M > 1) {  // wave_sum's totals by one reduce-scatter: lane mm holds row mm's
            const int lane = threadIdx.x & 63;
            const float tot = wave_sums_scatter<M>(ss, lane);
            if (lane < M) red[lane * 4 + (threadIdx.x >> 6)] = tot;
        } else {
            ss[0] = wave_sum(ss[0]);
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss[0];
        }
        __syncthreads();
        float inv[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const float t = red[mm * 4] + red[mm * 4 + 1] + red[mm * 4 + 2] + red[mm * 4 + 3];
            inv[mm] = 1.0f / sqrtf(t / float(K) + a.eps);
        }
        // pass 2: w * (x * inv) (kernels.cpp:711)
        for_slots([&](int k, int s) {
            const int mm = s / spr, sl = s % spr;
            float t[8], gg[8];
            get_x(k, mm, sl, t);
            if (k >= 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) gg[j] = st.g[k][j];
            } else {
                load8(a.gamma + sl * 8, gg);
            }
            float iv = 0.f;
#pragma unroll
            for (int r = 0; r < M; ++r)
                if (r == mm) iv = inv[r];
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = mm < a.m ? gg[j] * (t[j] * iv) : 0.f;
            emit(mm, sl, o);
        });
        return;
    }
    for_slots([&](int k, int s) {
        const int mm = s / spr, sl = s % spr;
        float v[8];
        if (PRO == PRO_ATTN) {
            if (mm >= a.m) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = 0.f;
            } else if (k >= 0) {
                merge_partials(st.pm, st.pl, st.o0, st.o1, v);
            } else {
                float pm[kAttnMaxSplits], pl[kAttnMaxSplits];
                f32x4 o0[kAttnMaxSplits], o1[kAttnMaxSplits];
                load_partials(a.attn, mm, sl, pm, pl, o0, o1);
                merge_partials(pm, pl, o0, o1, v);
            }
        } else {
            get_x(k, mm, sl, v);
        }
        emit(mm, sl, v);
    });
}

// Quantizes one 8-element slot of a 32-block held by 4 consecutive lanes (kernels.cpp:515-523): the block max
// is exact under any reduction order; sc = max/127, inv = 1/sc, q = rint(v * inv).
VH_DEV void quant_slot(const float (&v)[8], uint32_t *q2, float *sc_out) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float t = fabsf(v[j]);
        mx = mx < t ? t : mx;
    }
    mx = fmaxf(mx, dpp<kDppXor1>(mx));
    mx = fmaxf(mx, dpp<kDppXor2>(mx));
    const float sc = mx / 127.0f, inv = sc > 0.f ? 1.0f / sc : 0.0f;
    *sc_out = sc;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int qi = int(__builtin_rintf(__fmul_rn(v[j], inv)));
        w[j >> 2] |= uint32_t(uint8_t(int8_t(qi))) << (8 * (j & 3));
    }
    q2[0] = w[0];
    q2[1] = w[1];
}

// Sum of the 32 quantized inputs of a block held by 4 consecutive lanes (all 4 active), each lane's 8 in q2.
VH_DEV int block_qsum(const uint32_t (&q2)[2]) {
    int bs = __builtin_amdgcn_sdot4(int(q2[0]), 0x01010101, 0, false);
    bs = __builtin_amdgcn_sdot4(int(q2[1]), 0x01010101, bs, false);
    bs += dpp<kDppXor1>(bs);
    return bs + dpp<kDppXor2>(bs);
}

// The int path's prologue for a pass of several input rows, run once (one block per row) instead of in every block
// of the GEMV: row blockIdx.x of x as given, of RMSNorm(x), or of the attention merge, quantized per 32-block by
// quant_slot exactly as the fused prologue does, into q [m][K], qs [m][K/32] and qsum [m][K/32] (the GEMV then
// takes PRO_Q). xnorm, when set, receives the f32 rows as the fused prologue writes them.
template <int PRO>
__global__ __launch_bounds__(kGemvThreads) void k_quant_rows(GemvArgs a, int8_t *__restrict__ q, float *__restrict__ qs,
                                                          int32_t *__restrict__ qsum) {
    __shared__ float red[4];
    const int mm = blockIdx.x, K = a.K, nb = K / 32;
    GemvArgs b = a;  // row mm as a one-row prologue
    b.m = 1;
    b.xnorm = nullptr;
    const float *x = a.x ? a.x + int64_t(mm) * a.ldx : nullptr;
    if (PRO == PRO_ATTN) {
        const int64_t hs = int64_t(mm) * a.attn.heads * kAttnMaxSplits;
        b.attn.pm += hs;
        b.attn.pl += hs;
        b.attn.po += hs * a.attn.hd;
    }
    float *xn = (PRO != PRO_X && a.xnorm) ? a.xnorm + int64_t(mm) * K : nullptr;
    ProStage<1, PRO> st;
    auto sink = [&](int, int sl, const float (&v)[8]) {
        if (xn)
#pragma unroll
            for (int j = 0; j < 8; ++j) xn[sl * 8 + j] = v[j];
        uint32_t q2[2];
        float sc;
        quant_slot(v, q2, &sc);
        *reinterpret_cast<uint2 *>(q + int64_t(mm) * K + sl * 8) = make_uint2(q2[0], q2[1]);
        const int bs = block_qsum(q2);
        if ((sl & 3) == 0) {
            qs[mm * nb + (sl >> 2)] = sc;
            qsum[mm * nb + (sl >> 2)] = bs;
        }
    };
    // every input load issued first and kept in registers for both passes of the RMSNorm (one round trip), when the
    // row fits the staging slots; the same arithmetic either way
    if (pro_stageable<1, PRO>(K)) {
        pro_stage<1, PRO>(b, x, K, st);
        prologue<1, PRO, true>(b, x, K, red, st, sink);
    } else {
        prologue<1, PRO, false>(b, x, K, red, st, sink);
    }
}

// Fixed-point form of the FFN's down product: units of 2^-32, summed exactly (and so in any order) by integer
// atomics. A term may span +-2^18 (2^50 units): with at most 1024 groups plus the bias, any sum of terms, and the
// sum of the kAccCopies planes, stays below 2^61 units, inside int64. A term outside that range, infinite or NaN
// cannot be represented: it is clamped, so every sum stays defined, and `bad` is set, so the call fails
// (kStatusFixRange) and the caller computes the FFN another way instead of using a masked value.
constexpr float kFixOne = 4294967296.0f;
VH_DEV int64_t fix_of(float v, bool &bad) {
    const float lim = 1125899906842624.0f;  // 2^50 units = 2^18
    const float t = __builtin_rintf(v * kFixOne);
    const bool in = fabsf(t) <= lim;  // false for infinities and NaN
    bad |= !in;
    return int64_t(in ? t : (t > 0.f ? lim : -lim));
}
// The pending value of element i: the kAccCopies partial sums added as integers, then one rounding to float.
VH_DEV float acc_value(const int64_t (&c)[kAccCopies]) {
    int64_t t = 0;
#pragma unroll
    for (int k = 0; k < kAccCopies; ++k) t += c[k];
    return float(t) * (1.0f / kFixOne);
}

// What the epilogue reads besides the totals, loaded with the prologue's inputs at kernel start (the epilogue would
// otherwise wait one more global round trip at the end): the row's bias, and for EPI_ACC the residual, the row scale
// and, with ACC, the rows' pending FFN sums. Lane r*M + mm holds row0 + r, input row mm.
template <int M, int R, int EPI, bool ACC>
struct EpiPre {
    float y = 0.f, b = 0.f, ys = 1.f;  // residual, bias, row scale (b and ys as loaded: used only where set)
    int64_t c[kAccCopies];
};
template <int M, int R, int EPI, bool ACC>
VH_DEV void epi_prefetch(const GemvArgs &a, int rows, int lane, int row0, EpiPre<M, R, EPI, ACC> &e) {
    const int r = lane / M, mm = lane % M, row = row0 + r;
    const bool ok = lane < R * M && row < rows && mm < a.m;
    // Every load is issued, from element 0 of a valid array when unused, so the count in flight stays static; the
    // values are used as loaded only in the epilogue (a select here would wait for them before the weight stream).
    const float *bp = a.bias ? a.bias : a.y;
    e.b = bp[ok && a.bias ? row : 0];
    if constexpr (EPI == EPI_ACC) {
        const float *src = a.res ? a.res : a.y;
        e.y = src[ok ? int64_t(mm) * a.ldy + row : 0];
        const float *sp = a.yscale ? a.yscale : a.y;
        e.ys = sp[ok && a.yscale ? row : 0];
        if constexpr (ACC)
#pragma unroll
            for (int k = 0; k < kAccCopies; ++k) e.c[k] = a.acc[k * a.acc_ld + (ok ? row : 0)];
    }
}

// Epilogue: lane r*M + mm holds the total of (row0 + r, input row mm). SwiGLU pairs rows (2u, 2u+1) =
// (gate u, up u); the partner value is fetched with all lanes active, then only valid lanes store.
template <int M, int R, int EPI, bool ACC>
VH_DEV void store_out(const GemvArgs &a, int rows, float out, int lane, int row0, const EpiPre<M, R, EPI, ACC> &e) {
    const int r = lane / M, mm = lane % M, row = row0 + r;
    const bool ok = lane < R * M && row < rows && mm < a.m;
    const float v = out + ((ok && a.bias) ? e.b : 0.f);
    if (EPI == EPI_SWIGLU) {
        const float other = __shfl_xor(v, M, kWave);  // lane of row r ^ 1, same input row
        if (ok && (r & 1) == 0) a.y[int64_t(mm) * a.ldy + row / 2] = silu(v) * other;
    } else if (ok) {
        if (EPI == EPI_STORE) {
            a.y[int64_t(mm) * a.ldy + row] = v;
        } else {
            float base = e.y;
            if constexpr (ACC) {  // the FFN's residual add first, then this product's (one row: mm == 0)
                base = base + acc_value(e.c);
#pragma unroll
                for (int k = 0; k < kAccCopies; ++k) a.acc[k * a.acc_ld + row] = 0;
            }
            a.y[int64_t(mm) * a.ldy + row] = base + (a.yscale ? v * e.ys : v);
        }
    }
}

template <int R, int M>
VH_DEV void reduce_store_prep(float (&acc)[R][M], float &out, int lane) {
    constexpr int N = R * M, P = N <= 2 ? 2 : N <= 4 ? 4 : N <= 8 ? 8 : N <= 16 ? 16 : N <= 32 ? 32 : 64;
    if constexpr (N > 1 && N <= 64) {  // lane r M + mm gets the total of acc[r][mm]; values N .. P - 1 are zero pads
        float v[P];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int mm = 0; mm < M; ++mm) v[r * M + mm] = acc[r][mm];
#pragma unroll
        for (int k = N; k < P; ++k) v[k] = 0.f;
        out = wave_sums_scatter<P>(v, lane);
        if (lane >= N) out = 0.f;
    } else {
        out = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int mm = 0; mm < M; ++mm) {
                const float s = wave_sum(acc[r][mm]);
                if (lane == r * M + mm) out = s;
            }
    }
}

// ------------------------------------------------------------------------------------------ int8 path
// PRO_Q staging per thread: 16-byte chunks of the quantized rows and block scales / sums; STAGE picks the deeper set
// (8 rows of K 6144), otherwise the shallow one (8 rows of K 2048), so no lane issues loads it does not use.
constexpr int kQStageChunks = 12, kQStageScales = 6, kQStageChunksLo = 4, kQStageScalesLo = 2;
// ACC (one row): the input or the residual carries pending FFN sums (GemvArgs::acc).
// NT: threads per block (more than kGemvThreads only for pre-quantized rows: EPI_SWIGLU_Q takes 1024, so that one
// block holds the 64 interleaved gate|up rows of 32 SwiGLU outputs, one quantization block of the next pass).
template <int WT, int M, int R, int IT, int PRO, int EPI, bool STAGE, bool ACC = false, int NT = kGemvThreads>
// The weight stream's operands come first so they are preloaded into SGPRs with the dispatch (kernarg preload).
__global__ __launch_bounds__(NT) void k_gemv_int(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                 const float *x, int32_t rows, int32_t K, GemvArgs a) {
    static_assert(WT == WT_Q8 || WT == WT_Q4 || WT == WT_Q4H, "int path is Q8/Q4");
    static_assert(!ACC || (M == 1 && STAGE && (PRO == PRO_RMS || EPI == EPI_ACC)), "pending sums: one staged row");
    static_assert(NT == kGemvThreads || PRO == PRO_Q, "wider blocks take pre-quantized rows");
    static_assert(EPI != EPI_SWIGLU_Q || (PRO == PRO_Q && (NT / 64) * R == 64), "a block holds one output block");
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K / 32;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);                 // [M][K]
    float *xs = reinterpret_cast<float *>(smem + M * K);           // [M][nb]
    float *red = xs + M * nb;                                      // [M][4]
    int *xsum = reinterpret_cast<int *>(red + M * 4);              // Q4: [M][nb] sums of the quantized blocks
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * (NT / 64) + wave) * R;
    constexpr int EPC = WT == WT_Q8 ? 16 : 32;  // weight elements per 16-byte chunk
    const int nchunk = K / EPC;
    const int64_t rb = row_bytes<WT>(K);

    u32x4 wv[IT][R];
    float sv[IT][R];
    auto load = [&](int c0) {
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int c = c0 + 64 * j + lane;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = row0 + r;
                // branch-free: out-of-range lanes read row 0 and drop it, so the load count is static
                const bool ok = c < nchunk && row < rows;
                const int rowc = ok ? row : 0, cc = ok ? c : 0;
                const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + int64_t(rowc) * rb) + cc);
                const int64_t si = int64_t(rowc) * nb + (WT == WT_Q8 ? (cc >> 1) : cc);
                const float sc = WT == WT_Q4H ? float(reinterpret_cast<const _Float16 *>(scale)[si]) : scale[si];
                wv[j][r] = ok ? t : u32x4{0u, 0u, 0u, 0u};
                sv[j][r] = ok ? sc : 0.f;
            }
        }
    };
    constexpr int PS = PRO == PRO_Q ? PRO_X : PRO;  // PRO_Q stages its rows below instead
    ProStage<M, PS> st;
    EpiPre<M, R, EPI, ACC> ep;
    int64_t xa[kAccCopies][8];  // ACC + PRO_RMS: the pending sums of this thread's slot (K <= 8 * kGemvThreads)
    if constexpr (STAGE && PRO != PRO_Q) pro_stage<M, PS>(a, x, K, st);  // the prologue's inputs first: loads return in issue order
    // PRO_Q: the quantized rows, their scales and block sums are loaded into registers ahead of the weight stream
    // too (16-byte chunk i = threadIdx.x + 256 u), so the copy into LDS waits for one round trip that overlaps the
    // weights' instead of one per chunk after them; rows past a.m read row 0 and are stored as zeros
    constexpr int QC = PRO != PRO_Q ? 1 : ((STAGE ? kQStageChunks : kQStageChunksLo) * kGemvThreads + NT - 1) / NT;
    constexpr int QSC = PRO != PRO_Q ? 1 : ((STAGE ? kQStageScales : kQStageScalesLo) * kGemvThreads + NT - 1) / NT;
    u32x4 qv[QC];
    float qsv[QSC];
    int qzv[QSC];
    const int qn16 = M * K / 16, qns = M * nb;
    const bool qstaged = PRO == PRO_Q && qn16 <= QC * NT && qns <= QSC * NT;
    if constexpr (PRO == PRO_Q) {
        if (qstaged) {
#pragma unroll
            for (int u = 0; u < QC; ++u) {
                const int i = int(threadIdx.x) + u * NT;
                qv[u] = reinterpret_cast<const u32x4 *>(a.q)[i < qn16 && i * 16 / K < a.m ? i : 0];
            }
#pragma unroll
            for (int u = 0; u < QSC; ++u) {
                const int i = int(threadIdx.x) + u * NT;
                const int ii = i < qns && i / nb < a.m ? i : 0;
                qsv[u] = a.qs[ii];
                qzv[u] = WT != WT_Q8 ? a.qsum[ii] : 0;
            }
        }
    }
    if constexpr (ACC && PRO == PRO_RMS) {
        const int sl = int(threadIdx.x) < K / 8 ? int(threadIdx.x) : 0;
#pragma unroll
        for (int k = 0; k < kAccCopies; ++k)
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const i64x2 t = *reinterpret_cast<const i64x2 *>(a.acc + k * a.acc_ld + sl * 8 + j);
                xa[k][j] = t.x;
                xa[k][j + 1] = t.y;
            }
    }
    epi_prefetch(a, rows, lane, row0, ep);
    __builtin_amdgcn_sched_barrier(0);                                  // keep the weight stream behind them
    load(0);
    if constexpr (ACC && PRO == PRO_RMS) {  // x + the FFN's pending residual sums, as the reference's residual add
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int64_t c[kAccCopies];
#pragma unroll
            for (int k = 0; k < kAccCopies; ++k) c[k] = xa[k][j];
            st.x[0][j] = st.x[0][j] + acc_value(c);
        }
    }

    if constexpr (PRO == PRO_Q) {  // the rows come quantized: copy them (rows past a.m as zeros)
        if (qstaged) {
#pragma unroll
            for (int u = 0; u < QC; ++u) {
                const int i = int(threadIdx.x) + u * NT;
                if (i < qn16) reinterpret_cast<u32x4 *>(xq)[i] = i * 16 / K < a.m ? qv[u] : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < QSC; ++u) {
                const int i = int(threadIdx.x) + u * NT;
                if (i < qns) {
                    const bool on = i / nb < a.m;
                    xs[i] = on ? qsv[u] : 0.f;
                    if (WT != WT_Q8) xsum[i] = on ? qzv[u] : 0;
                }
            }
        } else {
            for (int i = threadIdx.x; i < qn16; i += NT)
                reinterpret_cast<u32x4 *>(xq)[i] = i * 16 / K < a.m ? reinterpret_cast<const u32x4 *>(a.q)[i] : u32x4{0u, 0u, 0u, 0u};
            for (int i = threadIdx.x; i < qns; i += NT) {
                const bool on = i / nb < a.m;
                xs[i] = on ? a.qs[i] : 0.f;
                if (WT != WT_Q8) xsum[i] = on ? a.qsum[i] : 0;
            }
        }
    } else {
        prologue<M, PRO, STAGE>(a, x, K, red, st, [&](int mm, int sl, const float (&v)[8]) {
            uint32_t q2[2];
            float sc;
            quant_slot(v, q2, &sc);
            *reinterpret_cast<uint2 *>(xq + mm * K + sl * 8) = make_uint2(q2[0], q2[1]);
            if ((sl & 3) == 0) xs[mm * nb + (sl >> 2)] = sc;
            if (WT != WT_Q8) {  // the block's sum of quantized inputs, for the (u - 8) offset of the Q4 weights
                const int bs = block_qsum(q2);
                if ((sl & 3) == 0) xsum[mm * nb + (sl >> 2)] = bs;
            }
        });
    }
    __syncthreads();

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;

    for (int c0 = 0; c0 < nchunk; c0 += 64 * IT) {
        if (c0 > 0) load(c0);
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int c = c0 + 64 * j + lane;
            const int cc = c < nchunk ? c : 0;  // invalid lanes hold zero weights; keep LDS reads in range
#pragma unroll
            for (int mm = 0; mm < M; ++mm) {
                if (WT == WT_Q8) {
                    const u32x4 xv = *reinterpret_cast<const u32x4 *>(xq + mm * K + cc * 16);
                    const float xsv = xs[mm * nb + (cc >> 1)];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        int d = __builtin_amdgcn_sdot4(int(wv[j][r].x), int(xv.x), 0, false);
                        d = __builtin_amdgcn_sdot4(int(wv[j][r].y), int(xv.y), d, false);
                        d = __builtin_amdgcn_sdot4(int(wv[j][r].z), int(xv.z), d, false);
                        d = __builtin_amdgcn_sdot4(int(wv[j][r].w), int(xv.w), d, false);
                        d += dpp<kDppXor1>(d);  // the two 16-byte halves of one 32-block: exact block dot
                        const float f = (lane & 1) ? 0.f : float(d) * (sv[j][r] * xsv);
                        acc[r][mm] += f;
                    }
                } else {
                    const u32x4 xl = *reinterpret_cast<const u32x4 *>(xq + mm * K + cc * 32);
                    const u32x4 xh = *reinterpret_cast<const u32x4 *>(xq + mm * K + cc * 32 + 16);
                    const float xsv = xs[mm * nb + cc];
                    const int sx = xsum[mm * nb + cc];  // sum of the block's 32 quantized inputs
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const u32x4 w = wv[j][r];
                        const uint32_t m4 = 0x0F0F0F0Fu;
                        // byte t of the block: element t in the low nibble, element t + 16 in the high nibble
                        int d = __builtin_amdgcn_sdot4(int(w.x & m4), int(xl.x), 0, false);
                        d = __builtin_amdgcn_sdot4(int(w.y & m4), int(xl.y), d, false);
                        d = __builtin_amdgcn_sdot4(int(w.z & m4), int(xl.z), d, false);
                        d = __builtin_amdgcn_sdot4(int(w.w & m4), int(xl.w), d, false);
                        d = __builtin_amdgcn_sdot4(int((w.x >> 4) & m4), int(xh.x), d, false);
                        d = __builtin_amdgcn_sdot4(int((w.y >> 4) & m4), int(xh.y), d, false);
                        d = __builtin_amdgcn_sdot4(int((w.z >> 4) & m4), int(xh.z), d, false);
                        d = __builtin_amdgcn_sdot4(int((w.w >> 4) & m4), int(xh.w), d, false);
                        d -= 8 * sx;  // weights are (u - 8)
                        acc[r][mm] += float(d) * (sv[j][r] * xsv);
                    }
                }
            }
        }
    }
    float out;
    reduce_store_prep<R, M>(acc, out, lane);
    if constexpr (EPI == EPI_SWIGLU_Q) {
        // The block's 32 SwiGLU outputs u0 .. u0 + 31 of each input row (store_out's arithmetic) into LDS, then one
        // wave quantizes them as k_quant_rows<PRO_X> would for the next pass: the same quant_slot on the same
        // 32-block (4 lanes of 8), so the int8 rows, scales and block sums are bit-identical.
        float *sw = reinterpret_cast<float *>(smem + M * K + M * nb * 4 + M * 16 + (WT == WT_Q8 ? 0 : M * nb * 4));  // [M][32]
        const int r = lane / M, mm = lane % M, row = row0 + r;
        const bool ok = lane < R * M && row < rows && mm < a.m;
        const float v = out + ((ok && a.bias) ? ep.b : 0.f);
        const float other = __shfl_xor(v, M, kWave);  // lane of row r ^ 1, same input row
        if (ok && (r & 1) == 0) sw[mm * 32 + (row - int(blockIdx.x) * 64) / 2] = silu(v) * other;
        __syncthreads();
        if (wave == 0) {
            const int qm = lane >> 2, sl = lane & 3, qmc = qm < M ? qm : 0;  // input row qm, 8-element slot sl
            float vv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) vv[e] = sw[qmc * 32 + sl * 8 + e];
            uint32_t q2[2];
            float sc;
            quant_slot(vv, q2, &sc);
            const int bs = block_qsum(q2);
            const int ko = rows / 2, nbo = ko / 32, ub = int(blockIdx.x);
            if (qm < a.m) {
                *reinterpret_cast<uint2 *>(a.yq + int64_t(qm) * ko + ub * 32 + sl * 8) = make_uint2(q2[0], q2[1]);
                if (sl == 0) {
                    a.yqs[qm * nbo + ub] = sc;
                    a.yqsum[qm * nbo + ub] = bs;
                }
            }
        }
    } else {
        store_out<M, R, EPI, ACC>(a, rows, out, lane, row0, ep);
    }
}

// ------------------------------------------------------------------------------------------ f32 path
template <int WT, int M, int R, int IT, int PRO, int EPI, bool STAGE>
// The weight stream's operands come first so they are preloaded into SGPRs with the dispatch (kernarg preload).
__global__ __launch_bounds__(kGemvThreads) void k_gemv_flt(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                       const float *x, int32_t rows, int32_t K, GemvArgs a) {
    static_assert(WT != WT_Q4 && WT != WT_Q4H, "Q4 always uses the int path");
    extern __shared__ __align__(16) uint8_t smem[];
    float *xf = reinterpret_cast<float *>(smem);  // [M][K]
    float *red = xf + M * K;                      // [M][4]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * (kGemvThreads / 64) + wave) * R;
    constexpr int EPC = WT == WT_F32 ? 4 : WT == WT_Q8 ? 16 : 8;
    const int nchunk = K / EPC;
    const int64_t rb = row_bytes<WT>(K);
    const int nb = K / 32;

    u32x4 wv[IT][R];
    float sv[IT][R];
    auto load = [&](int c0) {
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int c = c0 + 64 * j + lane;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = row0 + r;
                const bool ok = c < nchunk && row < rows;
                const int rowc = ok ? row : 0, cc = ok ? c : 0;
                const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + int64_t(rowc) * rb) + cc);
                wv[j][r] = ok ? t : u32x4{0u, 0u, 0u, 0u};
                if (WT == WT_Q8) {
                    const float sc = scale[int64_t(rowc) * nb + (cc >> 1)];
                    sv[j][r] = ok ? sc : 0.f;
                } else {
                    sv[j][r] = 0.f;
                }
            }
        }
    };
    ProStage<M, PRO> st;
    EpiPre<M, R, EPI, false> ep;
    if constexpr (STAGE) pro_stage<M, PRO>(a, x, K, st);
    epi_prefetch(a, rows, lane, row0, ep);
    __builtin_amdgcn_sched_barrier(0);
    load(0);

    prologue<M, PRO, STAGE>(a, x, K, red, st, [&](int mm, int sl, const float (&v)[8]) {
        *reinterpret_cast<f32x4 *>(xf + mm * K + sl * 8) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4 *>(xf + mm * K + sl * 8 + 4) = f32x4{v[4], v[5], v[6], v[7]};
    });
    __syncthreads();

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) acc[r][mm] = 0.f;

    for (int c0 = 0; c0 < nchunk; c0 += 64 * IT) {
        if (c0 > 0) load(c0);
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int c = c0 + 64 * j + lane;
            const int cc = c < nchunk ? c : 0;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float w[EPC];
                const u32x4 u = wv[j][r];
                const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
                if (WT == WT_F32) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = __uint_as_float(uw[e]);
                } else if (WT == WT_F16) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint16_t h = uint16_t(uw[e >> 1] >> (16 * (e & 1)));
                        w[e] = float(__builtin_bit_cast(_Float16, h));
                    }
                } else if (WT == WT_BF16) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) w[e] = bf16_to_f32(uint16_t(uw[e >> 1] >> (16 * (e & 1))));
                } else {
#pragma unroll
                    for (int e = 0; e < 16; ++e) w[e] = float(int8_t(uw[e >> 2] >> (8 * (e & 3)))) * sv[j][r];
                }
#pragma unroll
                for (int mm = 0; mm < M; ++mm) {
                    const float *xv = xf + mm * K + cc * EPC;
                    float s = acc[r][mm];
#pragma unroll
                    for (int e = 0; e < EPC; ++e) s = fmaf(w[e], xv[e], s);
                    acc[r][mm] = s;
                }
            }
        }
    }
    float out;
    reduce_store_prep<R, M>(acc, out, lane);
    store_out<M, R, EPI, false>(a, rows, out, lane, row0, ep);
}

}  // namespace vh
