// vh_f5.hpp — F5-TTS DiT step kernels besides the GEMMs: AdaLN modulation, non-causal softmax attention on the
// matrix cores, and the x columns of the step input.
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

typedef float f32x4a __attribute__((ext_vector_type(4)));

// LayerNorm without parameters + modulation (f5.cpp:608-625) of one row per block (256 threads): mean and
// variance in double, inv = float(1 / sqrt(var + 1e-6)), y = (x - float(mean)) * inv * (1 + scale) + shift.
// With y16 set, y goes out as f16 halves instead (hi at y16, lo at y16 + lo_off) for a split-f16 GEMM.
__global__ __launch_bounds__(256) void k_f5_modulate(const float *__restrict__ x, int32_t D, const float *__restrict__ sc,
                                                     const float *__restrict__ sh, float *__restrict__ y,
                                                     _Float16 *__restrict__ y16, int64_t lo_off) {
    __shared__ double red[4];
    const float *xr = x + int64_t(blockIdx.x) * D;
    float *yr = y + int64_t(blockIdx.x) * D;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    auto bsum = [&](double v) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
        __syncthreads();
        if (lane == 0) red[w] = v;
        __syncthreads();
        return (red[0] + red[1]) + (red[2] + red[3]);
    };
    double s = 0.0;
    for (int i = t; i < D; i += 256) s += double(xr[i]);
    const double mean = bsum(s) / D;
    double v = 0.0;
    for (int i = t; i < D; i += 256) {
        const double dd = double(xr[i]) - mean;
        v += dd * dd;
    }
    const double var = bsum(v) / D;
    const float inv = float(1.0 / sqrt(var + 1e-6)), fm = float(mean);
    if (y16) {
        _Float16 *hr = y16 + int64_t(blockIdx.x) * D;
        for (int i = t; i < D; i += 256) {
            const float r = (xr[i] - fm) * inv * (1.0f + sc[i]) + sh[i];
            const _Float16 hi = _Float16(r);
            hr[i] = hi;
            hr[lo_off + i] = _Float16(r - float(hi));
        }
        return;
    }
    for (int i = t; i < D; i += 256) yr[i] = (xr[i] - fm) * inv * (1.0f + sc[i]) + sh[i];
}

// cat[b][t][0..mel) = x[t][0..mel) for every batch b (the x columns of the DiT input, gpu.hpp:85-88).
__global__ __launch_bounds__(256) void k_f5_fill_x(const float *__restrict__ x, int32_t N, int32_t mel, float *__restrict__ cat,
                                                   int32_t W, int32_t B) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(B) * N * mel) return;
    const int64_t r = i / mel, c = i % mel;
    cat[r * W + c] = x[(r % N) * mel + c];
}

// Non-causal softmax attention of one head over N keys (f5.cpp:626-650): S = (q . k) * scale, softmax per row,
// O = P V, for head_dim 64. grid (ceil(N / 64), heads, B), block 256: each wave takes 16 query rows; key tiles of
// 64 go through LDS; an online softmax (running max and sum per row, O rescaled) replaces the reference's
// whole-row max, which changes only the rounding.
// Both products run on the f16 matrix cores (v_mfma_f32_16x16x32_f16) with every f32 operand as two f16 halves,
// x = hi + lo, and three products per pair (hi.hi + hi.lo + lo.hi; the dropped lo.lo term is below 2^-22 relative):
// each product is exact in the f32 accumulator, so S and P V keep f32-level accuracy. q, k and v arrive already
// split (the q|k|v GEMM's EPI_ROPE_H16 epilogue: q | k rows and v transposed to [d][key]), so key and value tiles
// are plain 16-byte loads; the softmax weights are split here. The next tile's loads are in flight during the
// current tile's MFMAs.
struct F5AttnArgs {
    const _Float16 *h16;  // hi plane; the lo plane is lo_off halves further
    int64_t lo_off;
    float *out;           // [B N][ldo], head h at column h * 64
    int32_t N, ldo, inner, ldvt;
    float scale;
    _Float16 *out16;      // when set: the output as f16 halves, hi at out16, lo at out16 + out_lo (rows of ldo)
    int64_t out_lo;
};
constexpr int kF5Hd = kF5HeadDim;
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
constexpr int kF5Ld = 64 + 8;  // LDS row stride in halves
VH_DEV h16x8 ld16(const _Float16 *p) { return *reinterpret_cast<const h16x8 *>(p); }
VH_DEV f32x4a mfma3(h16x8 ah, h16x8 al, h16x8 bh, h16x8 bl, f32x4a c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, c, 0, 0, 0);
}
__global__ __launch_bounds__(256) void k_f5_attn(F5AttnArgs a) {
    __shared__ __align__(16) _Float16 Kh[64][kF5Ld], Kl[64][kF5Ld];  // [key][d]
    __shared__ __align__(16) _Float16 Vh[64][kF5Ld], Vl[64][kF5Ld];  // [d][key]
    __shared__ __align__(16) float Ps[4][16][68];                     // per wave [row][key]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int q0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z, heads = gridDim.y;
    const int64_t ldqk = 2 * int64_t(a.inner), rb = int64_t(b) * a.N;
    const _Float16 *QK = a.h16;                                                  // q | k rows
    const _Float16 *VT = a.h16 + int64_t(gridDim.z) * a.N * ldqk + (int64_t(b) * heads + h) * kF5Hd * a.ldvt;  // [d][key]
    // A operand of S: lane holds q[16 wave + lr][32 c + 8 lg + e]
    h16x8 qh[2], ql[2];
    {
        const int qr = q0 + 16 * wave + lr;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            qh[c] = ql[c] = h16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (qr < a.N) {
                const _Float16 *p = QK + (rb + qr) * ldqk + h * kF5Hd + 32 * c + 8 * lg;
                qh[c] = ld16(p);
                ql[c] = ld16(p + a.lo_off);
            }
        }
    }
    float mrow[4], lrow[4];
    f32x4a o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { mrow[i] = -INFINITY; lrow[i] = 0.f; o[i] = f32x4a{0.f, 0.f, 0.f, 0.f}; }
    // per thread and tile: 2 chunks of 8 halves of K (hi, lo) and of v^T (hi, lo)
    h16x8 kr[2][2], vr[2][2];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int idx = tid + 256 * q, r = idx >> 3, c8 = (idx & 7) * 8;  // r: key (K) or d (v^T); c8: d or key
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) {
                kr[q][hl] = vr[q][hl] = h16x8{0, 0, 0, 0, 0, 0, 0, 0};
                const int64_t off = hl ? a.lo_off : 0;
                if (kt + r < a.N) kr[q][hl] = ld16(QK + off + (rb + kt + r) * ldqk + a.inner + h * kF5Hd + c8);
                if (kt + c8 < a.N) vr[q][hl] = ld16(VT + off + int64_t(r) * a.ldvt + kt + c8);
            }
        }
    };
    fetch(0);
    for (int kt = 0; kt < a.N; kt += 64) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int idx = tid + 256 * q, r = idx >> 3, c8 = (idx & 7) * 8;
            *reinterpret_cast<h16x8 *>(&Kh[r][c8]) = kr[q][0];
            *reinterpret_cast<h16x8 *>(&Kl[r][c8]) = kr[q][1];
            *reinterpret_cast<h16x8 *>(&Vh[r][c8]) = vr[q][0];
            *reinterpret_cast<h16x8 *>(&Vl[r][c8]) = vr[q][1];
        }
        __syncthreads();
        if (kt + 64 < a.N) fetch(kt + 64);
        // S tiles: B operand lane holds K[16 j + lr][32 c + 8 lg + e]
        f32x4a s[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j] = f32x4a{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 2; ++c)
                s[j] = mfma3(qh[c], ql[c], ld16(&Kh[16 * j + lr][32 * c + 8 * lg]), ld16(&Kl[16 * j + lr][32 * c + 8 * lg]), s[j]);
        }
        // lane holds S[4 lg + i][16 j + lr]: the 16 lanes of a DPP row share the rows
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v = kt + 16 * j + lr < a.N ? s[j][i] * a.scale : -INFINITY;
                s[j][i] = v;
                mx = fmaxf(mx, v);
            }
            mx = fmaxf(mx, dpp<kDppXor1>(mx));
            mx = fmaxf(mx, dpp<kDppXor2>(mx));
            mx = fmaxf(mx, dpp<kDppRowHalfMirror>(mx));
            mx = fmaxf(mx, dpp<kDppRowMirror>(mx));
            const float mnew = fmaxf(mrow[i], mx);
            const float alpha = expf(mrow[i] - mnew);  // 0 on the first tile (mrow = -inf)
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = expf(s[j][i] - mnew);
                sum += p;
                Ps[wave][4 * lg + i][16 * j + lr] = p;
            }
            sum += dpp<kDppXor1>(sum);
            sum += dpp<kDppXor2>(sum);
            sum += dpp<kDppRowHalfMirror>(sum);
            sum += dpp<kDppRowMirror>(sum);
            lrow[i] = lrow[i] * alpha + sum;
            mrow[i] = mnew;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt][i] *= alpha;
        }
        __syncthreads();
        // O += P V: A lane holds P[lr][32 c + 8 lg + e] (split here); B lane holds V[32 c + 8 lg + e][16 dt + lr]
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const f32x4a p0 = *reinterpret_cast<const f32x4a *>(&Ps[wave][lr][32 * c + 8 * lg]);
            const f32x4a p1 = *reinterpret_cast<const f32x4a *>(&Ps[wave][lr][32 * c + 8 * lg + 4]);
            h16x8 pah, pal;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = e < 4 ? p0[e] : p1[e - 4];
                const _Float16 hi = _Float16(x);
                pah[e] = hi;
                pal[e] = _Float16(x - float(hi));
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
                o[dt] = mfma3(pah, pal, ld16(&Vh[16 * dt + lr][32 * c + 8 * lg]), ld16(&Vl[16 * dt + lr][32 * c + 8 * lg]), o[dt]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qr = q0 + 16 * wave + 4 * lg + i;
        if (qr >= a.N) continue;
        const float inv = 1.0f / lrow[i];
        const int64_t off = (rb + qr) * a.ldo + int64_t(h) * kF5Hd;
        if (a.out16) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const float r = o[dt][i] * inv;
                const _Float16 hi = _Float16(r);
                a.out16[off + 16 * dt + lr] = hi;
                a.out16[a.out_lo + off + 16 * dt + lr] = _Float16(r - float(hi));
            }
        } else {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) a.out[off + 16 * dt + lr] = o[dt][i] * inv;
        }
    }
}

}  // namespace vh
