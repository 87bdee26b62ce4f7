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
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

template <int WT>
VH_DEV int64_t row_bytes(int K) {
    return WT == WT_F32 ? int64_t(K) * 4 : WT == WT_Q8 ? int64_t(K) : WT == WT_Q4 ? int64_t(K) / 2 : int64_t(K) * 2;
}

// ---------------------------------------------------------------------------------------------- prologue
// Produces the f32 input rows v[mm][K] (mm < a.m; rows a.m..M-1 are zeros) in 8-element slots: slot s of row mm
// holds elements 8s..8s+7, a 32-block is 4 consecutive slots handled by 4 consecutive lanes. `sink(mm, s, v)`
// receives each slot; it runs with all 4 lanes of a block active. Every input is read from global memory once:
// PRO_RMS keeps its slots in registers between the sum of squares and the scaling when they fit (KS per thread).
template <int M, int PRO, class Sink>
VH_DEV void prologue(const GemvArgs &a, const float *x, int K, float *red, Sink &&sink) {
    const int spr = K / 8;  // slots per row
    const int nslot = M * spr;
    auto load_x = [&](int mm, int sl, float (&v)[8]) {
        const float *xr = x + int64_t(mm) * a.ldx + sl * 8;
        const f32x4 t0 = *reinterpret_cast<const f32x4 *>(xr), t1 = *reinterpret_cast<const f32x4 *>(xr + 4);
        v[0] = t0.x; v[1] = t0.y; v[2] = t0.z; v[3] = t0.w; v[4] = t1.x; v[5] = t1.y; v[6] = t1.z; v[7] = t1.w;
    };
    auto emit = [&](int mm, int sl, float (&v)[8]) {
        if (PRO != PRO_X && a.xnorm && blockIdx.x == 0 && mm < a.m)
#pragma unroll
            for (int j = 0; j < 8; ++j) a.xnorm[int64_t(mm) * K + sl * 8 + j] = v[j];
        sink(mm, sl, v);
    };
    if (PRO == PRO_RMS) {
        constexpr int KS = 4;
        const bool in_regs = nslot <= KS * kGemvThreads;
        float v[KS][8], gm[KS][8];
        float ss[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) ss[mm] = 0.f;
        // pass 1: sum of squares of every row (kernels.cpp:709-710), slots kept when they fit
        for (int k = 0, s = threadIdx.x; s < nslot; ++k, s += kGemvThreads) {
            const int mm = s / spr, sl = s % spr;
            float t[8];
            if (mm < a.m) load_x(mm, sl, t);
            else
#pragma unroll
                for (int j = 0; j < 8; ++j) t[j] = 0.f;
            float q = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) q = fmaf(t[j], t[j], q);
#pragma unroll
            for (int r = 0; r < M; ++r)
                if (r == mm) ss[r] += q;
            if (in_regs) {
#pragma unroll
                for (int kk = 0; kk < KS; ++kk)
                    if (kk == k) {
                        const f32x4 g0 = *reinterpret_cast<const f32x4 *>(a.gamma + sl * 8),
                                    g1 = *reinterpret_cast<const f32x4 *>(a.gamma + sl * 8 + 4);
#pragma unroll
                        for (int j = 0; j < 8; ++j) v[kk][j] = t[j];
                        gm[kk][0] = g0.x; gm[kk][1] = g0.y; gm[kk][2] = g0.z; gm[kk][3] = g0.w;
                        gm[kk][4] = g1.x; gm[kk][5] = g1.y; gm[kk][6] = g1.z; gm[kk][7] = g1.w;
                    }
            }
        }
#pragma unroll
        for (int mm = 0; mm < M; ++mm) ss[mm] = wave_sum(ss[mm]);
        if ((threadIdx.x & 63) == 0)
#pragma unroll
            for (int mm = 0; mm < M; ++mm) red[mm * 4 + (threadIdx.x >> 6)] = ss[mm];
        __syncthreads();
        float inv[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const float t = red[mm * 4] + red[mm * 4 + 1] + red[mm * 4 + 2] + red[mm * 4 + 3];
            inv[mm] = 1.0f / sqrtf(t / float(K) + a.eps);
        }
        // pass 2: w * (x * inv) (kernels.cpp:711)
        for (int k = 0, s = threadIdx.x; s < nslot; ++k, s += kGemvThreads) {
            const int mm = s / spr, sl = s % spr;
            float t[8], gg[8];
            if (in_regs) {
#pragma unroll
                for (int kk = 0; kk < KS; ++kk)
                    if (kk == k)
#pragma unroll
                        for (int j = 0; j < 8; ++j) { t[j] = v[kk][j]; gg[j] = gm[kk][j]; }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) t[j] = 0.f;
                if (mm < a.m) load_x(mm, sl, t);
                const f32x4 g0 = *reinterpret_cast<const f32x4 *>(a.gamma + sl * 8),
                            g1 = *reinterpret_cast<const f32x4 *>(a.gamma + sl * 8 + 4);
                gg[0] = g0.x; gg[1] = g0.y; gg[2] = g0.z; gg[3] = g0.w; gg[4] = g1.x; gg[5] = g1.y; gg[6] = g1.z; gg[7] = g1.w;
            }
            float iv = 0.f;
#pragma unroll
            for (int r = 0; r < M; ++r)
                if (r == mm) iv = inv[r];
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = mm < a.m ? gg[j] * (t[j] * iv) : 0.f;
            emit(mm, sl, o);
        }
        return;
    }
    for (int s = threadIdx.x; s < nslot; s += kGemvThreads) {
        const int mm = s / spr, sl = s % spr;
        float v[8];
        if (mm >= a.m) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = 0.f;
        } else if (PRO == PRO_ATTN) {
            // merge of all kAttnMaxSplits partials (empty splits have max -inf and weigh 0)
            const AttnPartials &P = a.attn;
            const int e0 = sl * 8, h = e0 / P.hd, d0 = e0 % P.hd;
            const int64_t base = (int64_t(mm) * P.heads + h) * kAttnMaxSplits;
            float pm[kAttnMaxSplits], pl[kAttnMaxSplits];
            f32x4 o0[kAttnMaxSplits], o1[kAttnMaxSplits];
#pragma unroll
            for (int q = 0; q < kAttnMaxSplits; ++q) {
                pm[q] = P.pm[base + q];
                pl[q] = P.pl[base + q];
                o0[q] = *reinterpret_cast<const f32x4 *>(P.po + (base + q) * P.hd + d0);
                o1[q] = *reinterpret_cast<const f32x4 *>(P.po + (base + q) * P.hd + d0 + 4);
            }
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
        } else {
            load_x(mm, sl, v);
        }
        emit(mm, sl, v);
    }
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

// Epilogue: lane r*M + mm holds the total of (row0 + r, input row mm). SwiGLU pairs rows (2u, 2u+1) =
// (gate u, up u); the partner value is fetched with all lanes active, then only valid lanes store.
template <int M, int R, int EPI>
VH_DEV void store_out(const GemvArgs &a, int rows, float out, int lane, int row0) {
    const int r = lane / M, mm = lane % M, row = row0 + r;
    const bool ok = lane < R * M && row < rows && mm < a.m;
    const float v = out + ((ok && a.bias) ? a.bias[row] : 0.f);
    if (EPI == EPI_SWIGLU) {
        const float other = __shfl_xor(v, M, kWave);  // lane of row r ^ 1, same input row
        if (ok && (r & 1) == 0) a.y[int64_t(mm) * a.ldy + row / 2] = silu(v) * other;
    } else if (ok) {
        if (EPI == EPI_STORE) a.y[int64_t(mm) * a.ldy + row] = v;
        else a.y[int64_t(mm) * a.ldy + row] += v;
    }
}

template <int R, int M>
VH_DEV void reduce_store_prep(float (&acc)[R][M], float &out, int lane) {
    out = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const float s = wave_sum(acc[r][mm]);
            if (lane == r * M + mm) out = s;
        }
}

// ------------------------------------------------------------------------------------------ int8 path
template <int WT, int M, int R, int IT, int PRO, int EPI>
// The weight stream's operands come first so they are preloaded into SGPRs with the dispatch (kernarg preload).
__global__ __launch_bounds__(kGemvThreads) void k_gemv_int(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                       const float *x, int32_t rows, int32_t K, GemvArgs a) {
    static_assert(WT == WT_Q8 || WT == WT_Q4, "int path is Q8/Q4");
    extern __shared__ __align__(16) uint8_t smem[];
    const int nb = K / 32;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);                 // [M][K]
    float *xs = reinterpret_cast<float *>(smem + M * K);           // [M][nb]
    float *red = xs + M * nb;                                      // [M][4]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * (kGemvThreads / 64) + wave) * R;
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
                const bool ok = c < nchunk && row < rows;
                const u32x4 *p = reinterpret_cast<const u32x4 *>(w + int64_t(row) * rb) + c;
                wv[j][r] = ok ? __builtin_nontemporal_load(p) : u32x4{0u, 0u, 0u, 0u};
                const int blk = WT == WT_Q8 ? (c >> 1) : c;
                sv[j][r] = ok ? scale[int64_t(row) * nb + blk] : 0.f;
            }
        }
    };
    load(0);

    prologue<M, PRO>(a, x, K, red, [&](int mm, int sl, const float (&v)[8]) {
        uint32_t q2[2];
        float sc;
        quant_slot(v, q2, &sc);
        *reinterpret_cast<uint2 *>(xq + mm * K + sl * 8) = make_uint2(q2[0], q2[1]);
        if ((sl & 3) == 0) xs[mm * nb + (sl >> 2)] = sc;
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
                    int sx = __builtin_amdgcn_sdot4(0x01010101, int(xl.x), 0, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xl.y), sx, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xl.z), sx, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xl.w), sx, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xh.x), sx, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xh.y), sx, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xh.z), sx, false);
                    sx = __builtin_amdgcn_sdot4(0x01010101, int(xh.w), sx, false);
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
    store_out<M, R, EPI>(a, rows, out, lane, row0);
}

// ------------------------------------------------------------------------------------------ f32 path
template <int WT, int M, int R, int IT, int PRO, int EPI>
// The weight stream's operands come first so they are preloaded into SGPRs with the dispatch (kernarg preload).
__global__ __launch_bounds__(kGemvThreads) void k_gemv_flt(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                       const float *x, int32_t rows, int32_t K, GemvArgs a) {
    static_assert(WT != WT_Q4, "Q4 always uses the int path");
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
                const u32x4 *p = reinterpret_cast<const u32x4 *>(w + int64_t(row) * rb) + c;
                wv[j][r] = ok ? __builtin_nontemporal_load(p) : u32x4{0u, 0u, 0u, 0u};
                sv[j][r] = (WT == WT_Q8 && ok) ? scale[int64_t(row) * nb + (c >> 1)] : 0.f;
            }
        }
    };
    load(0);

    prologue<M, PRO>(a, x, K, red, [&](int mm, int sl, const float (&v)[8]) {
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
    store_out<M, R, EPI>(a, rows, out, lane, row0);
}

}  // namespace vh
