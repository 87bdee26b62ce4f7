// vh_f5.hpp — F5-TTS DiT step kernels besides the GEMMs: AdaLN modulation, non-causal softmax attention on the
// matrix cores, and the x columns of the step input.
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

typedef float f32x4a __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4a __attribute__((ext_vector_type(4)));

// mish as nn.hpp:103-107 (the CosyVoice2 / Chatterbox estimator's): x tanh(softplus(x)) with tanh(log(1 + e)) =
// n / (n + 2), n = e (e + 2), and x itself above 20.
VH_DEV float mish_nn_f(float x) {
    if (x > 20.f) return x;
    const float e = expf(x), n = e * (e + 2.0f);
    return x * (n / (n + 2.0f));
}

// Row LayerNorm (NormArgs), one wave per row (4 rows per 256-thread block): mean and variance in double (two passes
// over the row, which stays in L1), inv = float(1 / sqrt(var + eps)). The forms: AdaLN modulation without
// parameters (f5.cpp:608-625, eps 1e-6), y = (x - float(mean)) * inv * (1 + scale) + shift; LayerNorm with weight
// and bias (kernels.cpp:714-723 and nn.cpp:248-265, which compute alike), y = (x - float(mean)) * inv * w + b; then
// mish and a per-channel bias when asked (the estimator's CausalBlock1D and its time bias, cosyvoice.cpp:155-178).
// D % 4 == 0.
// NC chunks of 4 columns per lane stay in registers between the passes (NC = 8: rows up to 2048 values, longer rows
// are read again); PRE (rows of at most 4 x 256 = 1024 values): the row's parameters (scale, shift, time bias) are
// loaded with the row, before the statistics, instead of one more round trip after them; the arithmetic is the same.
constexpr int kNormRegChunks = 8;
template <int NC, bool PRE>
__global__ __launch_bounds__(256) void k_f5_modulate(NormArgs a) {
    static_assert(!PRE || NC <= 4, "parameters in registers only for short rows");
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.R) return;
    const int D = a.D;
    const float *xr = a.x + int64_t(row) * D;
    auto wsum = [&](double v) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
        return v;
    };
    // the row is read once: chunk c of this lane is columns 4 lane + 256 c .. + 3; the first NC chunks stay in
    // registers (fully unrolled loops), columns beyond 256 NC are read again from memory
    f32x4a reg[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = 4 * lane + 256 * c;
        reg[c] = i < D ? *reinterpret_cast<const f32x4a *>(xr + i) : f32x4a{0.f, 0.f, 0.f, 0.f};
    }
    // PRE: the parameters of this lane's chunks (shift / time bias read from the scale row when absent, never used)
    f32x4a pcs[PRE ? NC : 1], psh[PRE ? NC : 1], ptb[PRE ? NC : 1];
    if constexpr (PRE) {
        const float *shp = a.sh ? a.sh : a.sc, *tbp = a.tb ? a.tb : a.sc;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = 4 * lane + 256 * c < D ? 4 * lane + 256 * c : 0;
            pcs[c] = *reinterpret_cast<const f32x4a *>(a.sc + i);
            psh[c] = *reinterpret_cast<const f32x4a *>(shp + i);
            ptb[c] = *reinterpret_cast<const f32x4a *>(tbp + i);
        }
    }
    const int tail0 = 256 * NC;
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < NC; ++c)
        s += double(reg[c][0]) + double(reg[c][1]) + double(reg[c][2]) + double(reg[c][3]);  // zeros past D
    for (int i = tail0 + 4 * lane; i < D; i += 256) {
        const f32x4a v = *reinterpret_cast<const f32x4a *>(xr + i);
        s += double(v[0]) + double(v[1]) + double(v[2]) + double(v[3]);
    }
    const double mean = wsum(s) / D;
    double q = 0.0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (4 * lane + 256 * c >= D) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const double dd = double(reg[c][e]) - mean;
            q += dd * dd;
        }
    }
    for (int i = tail0 + 4 * lane; i < D; i += 256) {
        const f32x4a v = *reinterpret_cast<const f32x4a *>(xr + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const double dd = double(v[e]) - mean;
            q += dd * dd;
        }
    }
    const double var = wsum(q) / D;
    const float inv = float(1.0 / sqrt(var + a.eps)), fm = float(mean);
    auto emit = [&](int i, const f32x4a &v, const f32x4a &cs, const f32x4a &t, const f32x4a &b) {
        f32x4a r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (v[e] - fm) * inv * (a.affine ? cs[e] : 1.0f + cs[e]) + (a.sh ? t[e] : 0.f);
        if (a.mish) {
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = mish_nn_f(r[e]);
        }
        if (a.tb) {
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] += b[e];
        }
        if (a.y16) {
            f16x4a hi, lo;
            bool bad = false;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 h, l;
                bad |= split_f16(r[e], h, l);
                hi[e] = h;
                lo[e] = l;
            }
            raise_status(a.status, bad, kStatusF16Range);
            _Float16 *hr = a.y16 + int64_t(row) * D + i;
            *reinterpret_cast<f16x4a *>(hr) = hi;
            *reinterpret_cast<f16x4a *>(hr + a.lo_off) = lo;
        } else {
            *reinterpret_cast<f32x4a *>(a.y + int64_t(row) * D + i) = r;
        }
    };
    auto emit_load = [&](int i, const f32x4a &v) {  // the parameters read here, after the statistics
        const f32x4a cs = *reinterpret_cast<const f32x4a *>(a.sc + i);
        const f32x4a t = a.sh ? *reinterpret_cast<const f32x4a *>(a.sh + i) : f32x4a{0.f, 0.f, 0.f, 0.f};
        const f32x4a b = a.tb ? *reinterpret_cast<const f32x4a *>(a.tb + i) : f32x4a{0.f, 0.f, 0.f, 0.f};
        emit(i, v, cs, t, b);
    };
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (4 * lane + 256 * c >= D) continue;
        if constexpr (PRE) emit(4 * lane + 256 * c, reg[c], pcs[c], psh[c], ptb[c]);
        else emit_load(4 * lane + 256 * c, reg[c]);
    }
    for (int i = tail0 + 4 * lane; i < D; i += 256) emit_load(i, *reinterpret_cast<const f32x4a *>(xr + i));
}

// Depthwise "same" Conv1d (f5_ops.cpp:106-147 with groups = channels: the Vocos blocks' dwconv, f5.cpp:341) over
// batches of seq rows: y[t][c] = b[c] + sum_k w[c][k] x[t + k - K/2][c], zeros outside the batch, k in order. One
// thread per output, consecutive threads on consecutive channels.
__global__ __launch_bounds__(256) void k_dwconv(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ b,
                                                float *__restrict__ y, int64_t R, int32_t C, int32_t K, int32_t seq) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= R * C) return;
    const int64_t r = i / C;
    const int c = int(i % C), t = int(r % seq);
    const int64_t r0 = r - t;
    float acc = b ? b[c] : 0.f;
    for (int k = 0; k < K; ++k) {
        const int tt = t + k - K / 2;
        if (tt >= 0 && tt < seq) acc += w[int64_t(c) * K + k] * x[(r0 + tt) * C + c];
    }
    y[i] = acc;
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
// O = P V, for head_dim 64. grid (ceil(N / (16 W)), heads, B), block 64 W: each of the W waves takes 16 query rows
// (W = 2 doubles the blocks of a short sequence, the flow estimator's, at the cost of staging each key tile for half
// as many rows); key tiles of 64 go through LDS; an online softmax (running max and sum per row, O rescaled) replaces the reference's
// whole-row max, which changes only the rounding; exp(x) is taken as 2^(x log2 e) on v_exp_f32.
// Both products run on the f16 matrix cores (v_mfma_f32_16x16x32_f16) with every f32 operand as two f16 halves,
// x = hi + lo, and three products per pair (hi.hi + hi.lo + lo.hi; the dropped lo.lo term is below 2^-22 relative):
// each product is exact in the f32 accumulator, so S and P V keep f32-level accuracy. q, k and v arrive already
// split (the q|k|v GEMM's EPI_ROPE_H16 epilogue: q | k rows and v transposed to [d][key], its key columns padded
// with zeros to a multiple of 64), so key and value tiles are plain 16-byte loads.
// The products are taken transposed, S^T = K Q^T and O^T = V^T P^T, so that a lane holds one query row (lane % 16)
// throughout: its S^T values (keys 16 j + 4 (lane / 16) + i) are already the B operand of P^T once the 32 keys
// of a chunk are numbered in the order the lanes hold them (V^T's A operand read in that same order), P never
// leaves registers, and the row's max, sum and rescale need only two cross-row shuffles each.
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
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
constexpr int kF5Ld = 64 + 8;  // LDS row stride in halves
VH_DEV h16x8 ld16(const _Float16 *p) { return *reinterpret_cast<const h16x8 *>(p); }
VH_DEV h16x8 ld8x2(const _Float16 *p, const _Float16 *q) {  // halves p[0..3], q[0..3]
    const h16x4 x = *reinterpret_cast<const h16x4 *>(p), y = *reinterpret_cast<const h16x4 *>(q);
    return h16x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}
VH_DEV f32x4a mfma3(h16x8 ah, h16x8 al, h16x8 bh, h16x8 bl, f32x4a c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, c, 0, 0, 0);
}
template <int W, int KS>
__global__ __launch_bounds__(64 * W * KS) void k_f5_attn(F5AttnArgs a) {
    constexpr int RS = 8 * W, RPT = 64 / RS;  // tile rows of a key half's threads: rows r + RS q, q < RPT
    __shared__ __align__(16) _Float16 Kh[KS][64][kF5Ld], Kl[KS][64][kF5Ld];  // [half][key][d]
    __shared__ __align__(16) _Float16 Vh[KS][64][kF5Ld], Vl[KS][64][kF5Ld];  // [half][d][key]
    // waves: query group qw (16 rows each), key half kh (KS = 2: the halves take alternate key tiles and are merged
    // at the end, doubling the waves of a short sequence without staging a tile twice)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int qw = KS == 1 ? wave : wave % W, kh = KS == 1 ? 0 : wave / W, ht = KS == 1 ? tid : tid % (64 * W);
    // a contiguous run of (batch, head) pairs per XCD, so each head's keys and values stay in one L2
    const int qt = gridDim.x, heads = gridDim.y;
    const int t = xcd_tile(int(blockIdx.x) + qt * (int(blockIdx.y) + heads * int(blockIdx.z)), qt * heads * int(gridDim.z));
    const int q0 = (t % qt) * (16 * W), h = (t / qt) % heads, b = t / (qt * heads);
    const int64_t ldqk = 2 * int64_t(a.inner);
    // this batch's q and k rows of head h as buffers ending at row N (rows past it read as zeros)
    const _Float16 *qb = a.h16 + int64_t(b) * a.N * ldqk + h * kF5Hd, *kb = qb + a.inner;
    const int32_t rows_bytes = int32_t(((a.N - 1) * ldqk + kF5Hd) * 2);
    const __amdgpu_buffer_rsrc_t rqh = buf_rsrc(qb, rows_bytes), rql = buf_rsrc(qb + a.lo_off, rows_bytes);
    const __amdgpu_buffer_rsrc_t rkh = buf_rsrc(kb, rows_bytes), rkl = buf_rsrc(kb + a.lo_off, rows_bytes);
    const _Float16 *VT = a.h16 + int64_t(gridDim.z) * a.N * ldqk + (int64_t(b) * heads + h) * kF5Hd * a.ldvt;  // [d][key]
    // B operand of S^T: lane holds q[q0 + 16 wave + lr][32 c + 8 lg + e]
    h16x8 qh[2], ql[2];
    {
        const int32_t off = int32_t(((q0 + 16 * qw + lr) * ldqk + 8 * lg) * 2);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            qh[c] = __builtin_bit_cast(h16x8, buf_ld16(rqh, off + 64 * c, 0));
            ql[c] = __builtin_bit_cast(h16x8, buf_ld16(rql, off + 64 * c, 0));
        }
    }
    const float sl = a.scale * 1.4426950408889634f;  // scores in log2 units
    float mrow = -INFINITY, lrow = 0.f;  // of query row lr
    f32x4a o[4];  // O^T: lane holds O[row lr][16 dt + 4 lg + i]
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x4a{0.f, 0.f, 0.f, 0.f};
    // per thread and tile: keys / d rows r + RS q, columns c8 .. c8 + 7, of K and v^T (hi, lo)
    const int r = ht >> 3, c8 = (ht & 7) * 8;
    int32_t ko[RPT];
    const _Float16 *vp[RPT];
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
        ko[q] = int32_t(((r + RS * q) * ldqk + c8) * 2);
        vp[q] = VT + int64_t(r + RS * q) * a.ldvt + c8;
    }
    u32x4 kr[2 * RPT], vr[2 * RPT];
    auto fetch = [&](int kt) {
        // the key row goes in the vector offset, which the buffer's range check covers
        const int32_t ro = int32_t(kt * ldqk * 2);
#pragma unroll
        for (int q = 0; q < RPT; ++q) {
            kr[q] = buf_ld16(rkh, ko[q] + ro, 0);
            kr[RPT + q] = buf_ld16(rkl, ko[q] + ro, 0);
            vr[q] = *reinterpret_cast<const u32x4 *>(vp[q] + kt);
            vr[RPT + q] = *reinterpret_cast<const u32x4 *>(vp[q] + a.lo_off + kt);
        }
    };
    const int niter = ((a.N + 63) / 64 + KS - 1) / KS;  // the same count in both halves: barriers stay uniform
    fetch(min(64 * kh, a.ldvt - 64));
    for (int it = 0; it < niter; ++it) {
        const int kt = 64 * (it * KS + kh);
#pragma unroll
        for (int q = 0; q < RPT; ++q) {
            *reinterpret_cast<u32x4 *>(&Kh[kh][r + RS * q][c8]) = kr[q];
            *reinterpret_cast<u32x4 *>(&Kl[kh][r + RS * q][c8]) = kr[RPT + q];
            *reinterpret_cast<u32x4 *>(&Vh[kh][r + RS * q][c8]) = vr[q];
            *reinterpret_cast<u32x4 *>(&Vl[kh][r + RS * q][c8]) = vr[RPT + q];
        }
        __syncthreads();
        fetch(min(kt + 64 * KS, a.ldvt - 64));  // unconditional (the last tile again at the end): exact wait counts
        if (KS == 1 || kt < a.N) {  // a half whose tile lies past the keys only keeps the barriers
        // S^T tiles: A operand lane holds K[16 j + lr][32 c + 8 lg + e]; lane gets S^T[16 j + 4 lg + i][lr]
        f32x4a s[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j] = f32x4a{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 2; ++c)
                s[j] = mfma3(ld16(&Kh[kh][16 * j + lr][32 * c + 8 * lg]), ld16(&Kl[kh][16 * j + lr][32 * c + 8 * lg]), qh[c],
                             ql[c], s[j]);
        }
        float mx = -INFINITY;
        if (kt + 64 <= a.N) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s[j][i] *= sl;
                    mx = fmaxf(mx, s[j][i]);
                }
        } else {  // the last, partial tile: keys past N drop out
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s[j][i] = kt + 16 * j + 4 * lg + i < a.N ? s[j][i] * sl : -INFINITY;
                    mx = fmaxf(mx, s[j][i]);
                }
        }
        // the row's keys sit in lanes lr, lr + 16, lr + 32, lr + 48
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float mnew = fmaxf(mrow, mx);
        const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);  // 0 on the first tile (mrow = -inf)
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[j][i] = __builtin_amdgcn_exp2f(s[j][i] - mnew);
                sum += s[j][i];
            }
        sum += __shfl_xor(sum, 16, kWave);
        sum += __shfl_xor(sum, 32, kWave);
        lrow = lrow * alpha + sum;
        mrow = mnew;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        // O^T += V^T P^T over the 32 keys of chunk c, numbered as the lanes hold them: index 8 lg + e is key
        // 32 c + 4 lg + e (e < 4) or 32 c + 16 + 4 lg + (e - 4); A operand lane holds V^T[16 dt + lr][those keys]
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            uint32_t hw[4], lw[4];  // elements 2u, 2u + 1 of P's hi and lo halves
#pragma unroll
            for (int u = 0; u < 4; ++u)
                split_f16x2(s[2 * c + (u >> 1)][2 * (u & 1)], s[2 * c + (u >> 1)][2 * (u & 1) + 1], hw[u], lw[u]);
            const h16x8 ph = __builtin_bit_cast(h16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
            const h16x8 pl = __builtin_bit_cast(h16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int d = 16 * dt + lr, k0 = 32 * c + 4 * lg;
                o[dt] = mfma3(ld8x2(&Vh[kh][d][k0], &Vh[kh][d][k0 + 16]), ld8x2(&Vl[kh][d][k0], &Vl[kh][d][k0 + 16]), ph,
                              pl, o[dt]);
            }
        }
        }
        __syncthreads();
    }
    if constexpr (KS == 2) {  // merge the second half's (max, sum, O) into the first's through LDS
        float *mg = reinterpret_cast<float *>(&Kh[0][0][0]) + (qw * 64 + lane) * 18;
        if (kh == 1) {
            mg[0] = mrow;
            mg[1] = lrow;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) mg[2 + 4 * dt + i] = o[dt][i];
        }
        __syncthreads();
        if (kh == 1) return;
        const float m1 = mg[0], l1 = mg[1], mn = fmaxf(mrow, m1);
        const float a0 = __builtin_amdgcn_exp2f(mrow - mn), a1 = __builtin_amdgcn_exp2f(m1 - mn);
        lrow = lrow * a0 + l1 * a1;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[dt][i] = o[dt][i] * a0 + mg[2 + 4 * dt + i] * a1;
    }
    const int qr = q0 + 16 * qw + lr;
    if (qr >= a.N) return;
    const float inv = 1.0f / lrow;
    const int64_t off = (int64_t(b) * a.N + qr) * a.ldo + int64_t(h) * kF5Hd + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        const f32x4a y = o[dt] * inv;
        if (a.out16) {
            h16x4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                hi[i] = _Float16(y[i]);
                lo[i] = _Float16(y[i] - float(hi[i]));
            }
            *reinterpret_cast<h16x4 *>(a.out16 + off + 16 * dt) = hi;
            *reinterpret_cast<h16x4 *>(a.out16 + a.out_lo + off + 16 * dt) = lo;
        } else {
            *reinterpret_cast<f32x4a *>(a.out + off + 16 * dt) = y;
        }
    }
}

}  // namespace vh
