// vh_gemm.hpp — f32 GEMM on the matrix cores for multi-row passes: LLM prefill (matmul's f32 paths above 8 rows /
// 4 rows), the F5 DiT linears and its grouped position convolutions.
//
// C[i][r] = sum_k A[i][k] * W[r][k] (+ bias[r]), then an epilogue. The device counterpart of matmul's f32 paths
// for m > 8 (Q8 dequantized as float(q) * scale, kernels.cpp:661-679) and for F32 / F16 / BF16 weights
// (kernels.cpp:337-412), and of Conv1d::forward's per-group im2col matmul (f5_ops.cpp:128-146). The products are
// the reference's (weights widened exactly to f32, f32 activations); only the summation order differs
// (v_mfma_f32_16x16x4_f32 accumulates in f32).
//
// Block: 256 threads = 4 waves as 2 x 2; each wave owns a (16 TM) x (16 TN) piece of C as TM x TN MFMA 16x16x4
// tiles, so the block tile is (32 TM) rows of A x (32 TN) rows of W. K steps of 32 are staged through LDS (W
// widened on the way in); the next step's global loads are issued before the current step's MFMAs.
// MFMA lane layouts (checked on gfx950): A 16x4 -> lane l holds A[l % 16][l / 16]; B 4x16 -> lane l holds
// B[l / 16][l % 16]; D 16x16 -> lane l holds D[4 (l / 16) + i][l % 16], i < 4.
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4v __attribute__((ext_vector_type(4)));

constexpr int kGemmBK = 32, kGemmLd = kGemmBK + 4;  // LDS row stride (bank spread)

template <int WT>
VH_DEV int64_t gemm_row_bytes(int K) {
    return WT == WT_F32 ? int64_t(K) * 4 : WT == WT_Q8 ? int64_t(K) : int64_t(K) * 2;
}

VH_DEV float gelu_tanh_f(float x) {  // f5.cpp:93-96
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}
VH_DEV float gelu_erf_f(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }  // kernels.hpp:106
VH_DEV float mish_f(float x) {  // f5.cpp:97-100
    const float sp = x > 20.f ? x : log1pf(expf(x));
    return x * tanhf(sp);
}

// Four consecutive A elements of row `row`, columns k..k+3 (zeros outside the matrix / the convolution window).
template <int ASRC>
VH_DEV f32x4v gemm_load_a(const float *__restrict__ A, const GemmArgs &g, int row, int k, int grp) {
    f32x4v v = {0.f, 0.f, 0.f, 0.f};
    if (row >= g.m || k >= g.K) return v;
    if (ASRC == ASRC_ROWS) return *reinterpret_cast<const f32x4v *>(A + int64_t(row) * g.lda + k);
    if (ASRC == ASRC_STREAM) {
        const int kt = k / g.cig, i = k % g.cig, r = row + kt * g.dil;
        if (r < g.ctx) return *reinterpret_cast<const f32x4v *>(g.hist + int64_t(r) * g.cig + i);
        return *reinterpret_cast<const f32x4v *>(A + int64_t(r - g.ctx) * g.lda + i);
    }
    const int s = row / g.seq, t = row % g.seq, kt = k / g.cig, i = k % g.cig;
    const int tt = t + kt - (g.causal ? g.ksize - 1 : g.ksize / 2);
    if (kt >= g.ksize || tt < 0 || tt >= g.seq) return v;  // kt >= ksize: the zero padding of a weight row
    return *reinterpret_cast<const f32x4v *>(A + (int64_t(s) * g.seq + tt) * g.lda + int64_t(grp) * g.cig + i);
}

// ASRC_STREAM with g.hist_next: this block's share of the next call's history, the last ctx rows of [hist; x]
// (k_hist_shift's rows), split evenly over every block of the launch (x, y and the K slices of z).
VH_DEV void stream_hist_next(const float *__restrict__ x, const GemmArgs &g) {
    const int64_t total = int64_t(g.ctx) * g.cig;
    const int64_t nb = int64_t(gridDim.x) * gridDim.y * gridDim.z;
    const int64_t b = (int64_t(blockIdx.z) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    const int64_t per = (total + nb - 1) / nb, i0 = b * per, i1 = min(total, i0 + per);
    for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
        const int j = int(i / g.cig), c = int(i % g.cig), r = j + g.m;  // row r of [hist; x]
        g.hist_next[i] = r < g.ctx ? g.hist[int64_t(r) * g.cig + c] : x[int64_t(r - g.ctx) * g.lda + c];
    }
}

// Eight consecutive W elements of row `row`, columns k..k+7, widened to f32.
template <int WT>
VH_DEV void gemm_load_w(const uint8_t *__restrict__ w, const float *__restrict__ scale, const GemmArgs &g, int row, int k,
                        float (&v)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
    if (row >= g.n || k >= g.K) return;
    const uint8_t *p = w + int64_t(row) * gemm_row_bytes<WT>(g.K);
    if (WT == WT_Q8) {
        const uint2 u = *reinterpret_cast<const uint2 *>(p + k);
        const float s = scale[int64_t(row) * (g.K / 32) + k / 32];
        const uint32_t uw[2] = {u.x, u.y};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = float(int8_t(uw[e >> 2] >> (8 * (e & 3)))) * s;
    } else if (WT == WT_F32) {
        const f32x4v a = *reinterpret_cast<const f32x4v *>(p + int64_t(k) * 4);
        const f32x4v b = *reinterpret_cast<const f32x4v *>(p + int64_t(k) * 4 + 16);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const u32x4 u = *reinterpret_cast<const u32x4 *>(p + int64_t(k) * 2);
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t h = uint16_t(uw[e >> 1] >> (16 * (e & 1)));
            v[e] = WT == WT_F16 ? float(__builtin_bit_cast(_Float16, h)) : bf16_to_f32(h);
        }
    }
}

// Epilogue of a wave's TM x TN accumulator tiles: lane holds C[row0 + 4 (lane / 16) + v][col], col = col0 + lane % 16.
template <int EPI, int TM, int TN>
VH_DEV void gemm_epilogue(const f32x4v (&acc)[TM][TN], const GemmArgs &g, int m0, int n0, int wm, int wn, int lane) {
    bool bad = false;  // an f16-halves output beyond the f16 range
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * 16 * TN + j * 16 + (lane & 15);
            const float bz = (g.bias && col < g.n) ? g.bias[col] : 0.f;
            const float gt = (EPI == EPI_GATED_ACC && col < g.n) ? g.gate[col] : 0.f;
            if (EPI == EPI_ROPE_H16 && n0 + wn * 16 * TN + j * 16 >= g.rope_cols && g.rope_cols % 16 == 0 && g.seq % 4 == 0) {
                // a tile of v columns: this lane's 4 rows are 4 consecutive keys of one batch (seq % 4 == 0), so
                // they go to v^T as one 8-byte store per plane instead of four strided 2-byte ones
                const int row0 = m0 + wm * 16 * TM + i * 16 + 4 * (lane >> 4);
                if (row0 < g.m && col < g.n) {
                    const int cv = col - g.rope_cols, b = row0 / g.seq, n = row0 % g.seq;
                    const int64_t idx = int64_t(g.m) * g.rope_cols +
                                        ((int64_t(b) * (g.rope_cols / 2 / g.hd) + cv / g.hd) * g.hd + cv % g.hd) * g.ldvt + n;
                    f16x4v hi, lo;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        _Float16 h, l;
                        bad |= split_f16(acc[i][j][v] + bz, h, l);
                        hi[v] = h;
                        lo[v] = l;
                    }
                    *reinterpret_cast<f16x4v *>(g.h16 + idx) = hi;
                    *reinterpret_cast<f16x4v *>(g.h16 + g.lo_off + idx) = lo;
                }
                continue;
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = m0 + wm * 16 * TM + i * 16 + 4 * (lane >> 4) + v;
                const float c = acc[i][j][v] + bz;
                const bool in = row < g.m && col < g.n;
                float *dst = g.y + int64_t(row) * g.ldy + col;
                if (EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_H16) {
                    const float up = __shfl_xor(c, 1, kWave);  // column col ^ 1 of the same row
                    if (in && (col & 1) == 0) {
                        const float r = silu(c) * up;
                        if (EPI == EPI_SWIGLU) {
                            g.y[int64_t(row) * g.ldy + col / 2] = r;
                        } else {
                            _Float16 hi, lo;
                            bad |= split_f16(r, hi, lo);
                            const int64_t idx = int64_t(row) * g.ldy + col / 2;
                            g.h16[idx] = hi;
                            g.h16[g.lo_off + idx] = lo;
                        }
                    }
                } else if (EPI == EPI_ROPE || EPI == EPI_ROPE_H16) {
                    const float o = __shfl_xor(c, 1, kWave);  // the pair partner (2j <-> 2j + 1)
                    float r = c;
                    if (col < g.rope_cols && g.rope) {
                        const int inner = g.rope_cols / 2, d = col % g.hd, head = (col % inner) / g.hd;
                        const int rhd = g.rope_hd ? g.rope_hd : g.hd;  // the padding dims (d >= rhd) stay zero
                        if (d < rhd && (g.rope_heads <= 0 || head < g.rope_heads)) {
                            const float *cs = g.rope + ((int64_t(row % g.seq) * (rhd / 2) + d / 2) * 2);
                            const float cc = cs[0], sn = cs[1];
                            r = (col & 1) ? c * cc + o * sn : c * cc - o * sn;
                        }
                    }
                    if (EPI == EPI_ROPE) {
                        if (in) *dst = r;
                    } else if (in) {
                        _Float16 hi, lo;
                        bad |= split_f16(r, hi, lo);
                        int64_t idx;
                        if (col < g.rope_cols) {
                            idx = int64_t(row) * g.rope_cols + col;
                        } else {  // v, transposed: [batch][head][d][key]
                            const int cv = col - g.rope_cols, b = row / g.seq, n = row % g.seq;
                            const int64_t vbase = int64_t(g.m) * g.rope_cols;
                            idx = vbase + ((int64_t(b) * (g.rope_cols / 2 / g.hd) + cv / g.hd) * g.hd + cv % g.hd) * g.ldvt + n;
                        }
                        g.h16[idx] = hi;
                        g.h16[g.lo_off + idx] = lo;
                    }
                } else if (in) {
                    if (EPI == EPI_STORE) *dst = c;
                    else if (EPI == EPI_ACC) *dst += c;
                    else if (EPI == EPI_GATED_ACC) *dst += gt * c;
                    else if (EPI == EPI_GELU) *dst = gelu_tanh_f(c);
                    else if (EPI == EPI_GELU_ERF) *dst = gelu_erf_f(c);
                    else if (EPI == EPI_GELU_H16) {
                        const float r = g.gelu_erf ? gelu_erf_f(c) : gelu_tanh_f(c);
                        _Float16 hi, lo;
                        bad |= split_f16(r, hi, lo);
                        const int64_t idx = int64_t(row) * g.ldy + col;
                        g.h16[idx] = hi;
                        g.h16[g.lo_off + idx] = lo;
                    }
                    else if (EPI == EPI_SNAKE) {
                        const float sn = sinf(c * g.snake_a[col]);
                        *dst = c + g.snake_ib[col] * sn * sn;
                    }
                    else if (EPI == EPI_ACC_SNAKE) {
                        const float v = *dst + c, sn = sinf(v * g.snake_a[col]);
                        *dst = v;
                        g.snake_y[int64_t(row) * g.ldy + col] = v + g.snake_ib[col] * sn * sn;
                    }
                    else if (EPI == EPI_MISH) *dst = mish_f(c);
                    else if (EPI == EPI_MISH_ACC) *dst += mish_f(c);
                }
            }
        }
    raise_status(g.status, bad, kStatusF16Range);
}

// Split K: a block's TM x TN accumulator tiles as partial sums into slice blockIdx.z of ws ([m][n] per slice), no
// bias or epilogue (k_gemm_splitk_reduce applies them).
template <int TM, int TN>
VH_DEV void gemm_store_partial(const f32x4v (&acc)[TM][TN], const GemmArgs &g, int m0, int n0, int wm, int wn, int lane) {
    float *ws = g.ws + int64_t(blockIdx.z) * g.m * g.n;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * 16 * TN + j * 16 + (lane & 15);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = m0 + wm * 16 * TM + i * 16 + 4 * (lane >> 4) + v;
                if (row < g.m && col < g.n) ws[int64_t(row) * g.n + col] = acc[i][j][v];
            }
        }
}

// Epilogues: EPI_STORE y = c + bias; EPI_ACC y += c + bias; EPI_SWIGLU W rows are (gate u, up u) pairs, y[u] =
// silu(gate) * up; EPI_GATED_ACC y += gate[col] * (c + bias); EPI_GELU y = gelu_tanh(c + bias); EPI_MISH
// y = mish(c + bias); EPI_MISH_ACC y += mish(c + bias); EPI_GELU_ERF y = gelu_erf(c + bias); EPI_ROPE y = c + bias
// with the pairs of q | k rotated;
// EPI_ROPE_H16 and EPI_GELU_H16 write their results as f16 halves (hi, lo) for a following split-f16 product.
// ASRC_CONV: W (F32) and y columns are those of group blockIdx.z.
template <int WT, int EPI, int ASRC, int TM, int TN>
__global__ __launch_bounds__(256) void k_gemm_f32(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                  const float *__restrict__ A, GemmArgs g) {
    static_assert(WT == WT_F32 || WT == WT_F16 || WT == WT_BF16 || WT == WT_Q8, "f32-activation weight types");
    static_assert(ASRC != ASRC_CONV || WT == WT_F32, "grouped convolution weights are f32");
    constexpr int BM = 32 * TM, BN = 32 * TN;
    constexpr int AQ = BM * kGemmBK / 4 / 256;  // f32x4 A loads per thread and K step
    constexpr int WQ = BN * kGemmBK / 8 / 256;  // 8-element W loads per thread and K step
    __shared__ __align__(16) float As[BM][kGemmLd];
    __shared__ __align__(16) float Bs[BN][kGemmLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int K = g.K;
    // blockIdx.z: the K slice of a split (kchunk set, one group), else the convolution group
    const int grp = g.kchunk ? 0 : int(blockIdx.z);
    const int kbeg = g.kchunk ? int(blockIdx.z) * g.kchunk : 0, kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    if (ASRC == ASRC_CONV) {
        w += int64_t(grp) * g.n * K * 4;
        g.y += int64_t(grp) * g.n;
        if (g.bias) g.bias += int64_t(grp) * g.n;
    }
    f32x4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    f32x4v ra[AQ];
    float rw[WQ][8];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int idx = tid + 256 * q;
            ra[q] = gemm_load_a<ASRC>(A, g, m0 + (idx >> 3), k0 + (idx & 7) * 4, grp);
        }
#pragma unroll
        for (int q = 0; q < WQ; ++q) {
            const int idx = tid + 256 * q;
            gemm_load_w<WT>(w, scale, g, n0 + (idx >> 2), k0 + (idx & 3) * 8, rw[q]);
        }
    };
    if (ASRC == ASRC_STREAM && g.hist_next) stream_hist_next(A, g);  // the history moves on in the same launch
    fetch(kbeg);
    for (int k0 = kbeg; k0 < kend; k0 += kGemmBK) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int idx = tid + 256 * q;
            *reinterpret_cast<f32x4v *>(&As[idx >> 3][(idx & 7) * 4]) = ra[q];
        }
#pragma unroll
        for (int q = 0; q < WQ; ++q) {
            const int idx = tid + 256 * q, r = idx >> 2, kq = (idx & 3) * 8;
            *reinterpret_cast<f32x4v *>(&Bs[r][kq]) = f32x4v{rw[q][0], rw[q][1], rw[q][2], rw[q][3]};
            *reinterpret_cast<f32x4v *>(&Bs[r][kq + 4]) = f32x4v{rw[q][4], rw[q][5], rw[q][6], rw[q][7]};
        }
        __syncthreads();
        if (k0 + kGemmBK < kend) fetch(k0 + kGemmBK);  // in flight during the MFMAs below
#pragma unroll
        for (int kk = 0; kk < kGemmBK; kk += 4) {
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = As[wm * 16 * TM + i * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = Bs[wn * 16 * TN + j * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    if (g.kchunk) return gemm_store_partial<TM, TN>(acc, g, m0, n0, wm, wn, lane);
    gemm_epilogue<EPI, TM, TN>(acc, g, m0, n0, wm, wn, lane);
}


// F32 weights and f32 activations on the f16 matrix cores: both operands split at staging into f16 halves, x = hi + lo,
// and three products per pair (hi.hi + hi.lo + lo.hi; the dropped lo.lo term is below 2^-22 relative), each exact in
// the f32 accumulator. The weights are scaled by 2^10 before the split, so that the lo half of weights down to about
// 1e-4 stays a normal f16, and the sum is scaled back (exactly) before the epilogue. Any A source of k_gemm_f32 (rows,
// grouped conv, causal conv, streaming conv), split K, its tiles (64 x 64, K steps of 32) and epilogues; activations
// below 65504 in magnitude (f16 range) and weights below 64. The convolutions' f32 products run at the f16 rate.
template <int EPI, int ASRC>
__global__ __launch_bounds__(256) void k_gemm_x3(const uint8_t *__restrict__ w, const float *__restrict__ A, GemmArgs g) {
    constexpr int BM = 64, BN = 64, BK = 32, LD = BK + 8;
    constexpr float kWs = 1024.0f, kWsInv = 1.0f / 1024.0f;
    __shared__ __align__(16) _Float16 Ah[BM][LD], Al[BM][LD], Bh[BN][LD], Bl[BN][LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN, K = g.K;
    const int grp = g.kchunk ? 0 : int(blockIdx.z);
    const int kbeg = g.kchunk ? int(blockIdx.z) * g.kchunk : 0, kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    if (ASRC == ASRC_CONV) {
        w += int64_t(grp) * g.n * K * 4;
        g.y += int64_t(grp) * g.n;
        if (g.bias) g.bias += int64_t(grp) * g.n;
    }
    f32x4v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // per thread and K step: A rows tid / 8 and tid / 8 + 32, columns (tid % 8) 4 .. + 3; W row tid / 4, columns
    // (tid % 4) 8 .. + 7
    f32x4v ra[2];
    float rw[8];
    const int ar = tid >> 3, ac = (tid & 7) * 4, wr = tid >> 2, wc = (tid & 3) * 8;
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int k = k0 + ac;
            ra[q] = k < kend ? gemm_load_a<ASRC>(A, g, m0 + ar + 32 * q, k, grp) : f32x4v{0.f, 0.f, 0.f, 0.f};
        }
        if (k0 + wc < kend) {
            gemm_load_w<WT_F32>(w, nullptr, g, n0 + wr, k0 + wc, rw);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) rw[e] = 0.f;
        }
    };
    if (ASRC == ASRC_STREAM && g.hist_next) stream_hist_next(A, g);  // the history moves on in the same launch
    fetch(kbeg);
    bool bad = false;  // an activation beyond the f16 range
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            f16x4v hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 h, l;
                bad |= split_f16(ra[q][e], h, l);
                hi[e] = h;
                lo[e] = l;
            }
            *reinterpret_cast<f16x4v *>(&Ah[ar + 32 * q][ac]) = hi;
            *reinterpret_cast<f16x4v *>(&Al[ar + 32 * q][ac]) = lo;
        }
        {
            f16x8v hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 h, l;
                bad |= split_f16(rw[e] * kWs, h, l);  // |w| >= 64 (the callers route such weights to k_gemm_f32)
                hi[e] = h;
                lo[e] = l;
            }
            *reinterpret_cast<f16x8v *>(&Bh[wr][wc]) = hi;
            *reinterpret_cast<f16x8v *>(&Bl[wr][wc]) = lo;
        }
        __syncthreads();
        if (k0 + BK < kend) fetch(k0 + BK);  // in flight during the products below
        f16x8v ah[2], al[2], bh[2], bl[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = wm * 32 + i * 16 + (lane & 15), c = 8 * (lane >> 4);
            ah[i] = *reinterpret_cast<const f16x8v *>(&Ah[r][c]);
            al[i] = *reinterpret_cast<const f16x8v *>(&Al[r][c]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = wn * 32 + j * 16 + (lane & 15), c = 8 * (lane >> 4);
            bh[j] = *reinterpret_cast<const f16x8v *>(&Bh[r][c]);
            bl[j] = *reinterpret_cast<const f16x8v *>(&Bl[r][c]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
            }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] *= kWsInv;
    raise_status(g.status, bad, kStatusF16Range);
    if (g.kchunk) return gemm_store_partial<2, 2>(acc, g, m0, n0, wm, wn, lane);
    gemm_epilogue<EPI, 2, 2>(acc, g, m0, n0, wm, wn, lane);
}

// F16 or Q8 weights on the f16 matrix cores with the f32 activations split in two halves: a = hi + lo with
// hi = f16(a), lo = f16(a - hi), so W a = W hi + W lo. F16 weights and the int8 values of Q8 weights are exact in
// f16 and every f16 x f16 product is exact in the f32 accumulator, so the result keeps the activations to about
// 2^-22 relative (v_mfma_f32_16x16x32_f16, two per tile and 32-deep K step). Q8: one 32-deep step is one scale
// block, so its two MFMAs start from zero and the block sum is scaled by the row's block scale into the
// accumulator: s (q . a) for the reference's (float(q) s) . a, equal up to rounding. Activations must stay below
// 65504 in magnitude (f16 range). Tiles and epilogues as k_gemm_f32, K steps of BK (32 or 64) staged through LDS
// with the next step's global loads in flight. MFMA lane layouts (checked on gfx950): A 16x32 -> lane l holds
// A[l % 16][8 (l / 16) + e]; B 32x16 -> lane l holds B[8 (l / 16) + e][l % 16]; D as the f32 MFMA.
template <int WT, int EPI, int TM, int TN, int BK>
__global__ __launch_bounds__(256) void k_gemm_h16(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                  const float *__restrict__ A, GemmArgs g) {
    static_assert(WT == WT_F16 || WT == WT_Q8, "f16 or q8 weights");
    constexpr int BM = 32 * TM, BN = 32 * TN, LD = BK + 8;  // LDS row stride in halves
    constexpr int AQ = BM * BK / 4 / 256;  // f32x4 A loads per thread and K step
    constexpr int WQ = BN * BK / 8 / 256;  // 8-element W loads per thread and K step
    constexpr int CPR = BK / 4, WPR = BK / 8;  // f32x4 / 8-element chunks per row
    constexpr int NB = BK / 32;                // scale blocks per K step (Q8)
    __shared__ __align__(16) _Float16 Ah[BM][LD];
    __shared__ __align__(16) _Float16 Al[BM][LD];
    __shared__ __align__(16) _Float16 Bs[BN][LD];
    __shared__ float Ss[WT == WT_Q8 ? BN : 1][NB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int K = g.K;  // the row length of A and W; this block sums columns [kbeg, kend)
    const int kbeg = g.kchunk ? int(blockIdx.z) * g.kchunk : 0, kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    f32x4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    f32x4v ra[AQ];
    u32x4 rw[WQ];  // F16: 8 halves; Q8: 8 int8 in .x .y
    float rs = 0.f;
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int idx = tid + 256 * q, row = m0 + idx / CPR, k = k0 + (idx % CPR) * 4;
            ra[q] = f32x4v{0.f, 0.f, 0.f, 0.f};
            if (row < g.m && k < kend) ra[q] = *reinterpret_cast<const f32x4v *>(A + int64_t(row) * g.lda + k);
        }
#pragma unroll
        for (int q = 0; q < WQ; ++q) {
            const int idx = tid + 256 * q, row = n0 + idx / WPR, k = k0 + (idx % WPR) * 8;
            rw[q] = u32x4{0u, 0u, 0u, 0u};
            if (row < g.n && k < kend) {
                if (WT == WT_F16) {
                    rw[q] = *reinterpret_cast<const u32x4 *>(w + (int64_t(row) * K + k) * 2);
                } else {
                    const uint2 u = *reinterpret_cast<const uint2 *>(w + int64_t(row) * K + k);
                    rw[q].x = u.x; rw[q].y = u.y;
                }
            }
        }
        if (WT == WT_Q8 && tid < BN * NB) {
            const int row = n0 + tid / NB, kb = k0 / 32 + tid % NB;
            rs = (row < g.n && kb < kend / 32) ? scale[int64_t(row) * (K / 32) + kb] : 0.f;
        }
    };
    fetch(kbeg);
    bool bad = false;  // an activation beyond the f16 range
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int idx = tid + 256 * q, r = idx / CPR, c = (idx % CPR) * 4;
            f16x4v hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 h, l;
                bad |= split_f16(ra[q][e], h, l);
                hi[e] = h;
                lo[e] = l;
            }
            *reinterpret_cast<f16x4v *>(&Ah[r][c]) = hi;
            *reinterpret_cast<f16x4v *>(&Al[r][c]) = lo;
        }
#pragma unroll
        for (int q = 0; q < WQ; ++q) {
            const int idx = tid + 256 * q;
            if (WT == WT_F16) {
                *reinterpret_cast<u32x4 *>(&Bs[idx / WPR][(idx % WPR) * 8]) = rw[q];
            } else {
                f16x8v hv;
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = _Float16(int8_t((e < 4 ? rw[q].x : rw[q].y) >> (8 * (e & 3))));
                *reinterpret_cast<f16x8v *>(&Bs[idx / WPR][(idx % WPR) * 8]) = hv;
            }
        }
        if (WT == WT_Q8 && tid < BN * NB) Ss[tid / NB][tid % NB] = rs;
        __syncthreads();
        if (k0 + BK < kend) fetch(k0 + BK);  // in flight during the MFMAs below
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            f16x8v ah[TM], al[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int r = wm * 16 * TM + i * 16 + (lane & 15);
                ah[i] = *reinterpret_cast<const f16x8v *>(&Ah[r][kk + 8 * (lane >> 4)]);
                al[i] = *reinterpret_cast<const f16x8v *>(&Al[r][kk + 8 * (lane >> 4)]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const f16x8v *>(&Bs[wn * 16 * TN + j * 16 + (lane & 15)][kk + 8 * (lane >> 4)]);
            if (WT == WT_F16) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], acc[i][j], 0, 0, 0);
                    }
            } else {
                float sc[TN];  // the block scale of this lane's W row (its C column)
#pragma unroll
                for (int j = 0; j < TN; ++j) sc[j] = Ss[wn * 16 * TN + j * 16 + (lane & 15)][kk / 32];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        f32x4v t = {0.f, 0.f, 0.f, 0.f};
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], t, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], t, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[i][j][v] = fmaf(t[v], sc[j], acc[i][j][v]);
                    }
            }
        }
        __syncthreads();
    }
    raise_status(g.status, bad, kStatusF16Range);
    if (g.kchunk) return gemm_store_partial<TM, TN>(acc, g, m0, n0, wm, wn, lane);
    gemm_epilogue<EPI, TM, TN>(acc, g, m0, n0, wm, wn, lane);
}

// k_gemm_h16 for K (and the split-K chunk) a multiple of 64, with k_gemm_hh's load pipeline: buffer loads cut at
// the tile's last row of A and of W (rows past m or n read as zeros, no per-load bounds check, the K offset in the
// scalar operand), two K steps in flight in alternating register sets, unconditional fetches (steps past the end
// re-read the last one) so the wait counts are exact. A arrives as f32 and is split into hi / lo at staging; Q8
// weights are widened to f16 at staging and their block scales staged beside them. 64 x 64 tiles, K steps of 64,
// S register sets in flight (2: three or four measured slower on the prefill shapes).
template <int WT, int EPI, int S = 2>
__global__ __launch_bounds__(256) void k_gemm_h16b(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                   const float *__restrict__ A, GemmArgs g) {
    static_assert(WT == WT_F16 || WT == WT_Q8, "f16 or q8 weights");
    constexpr int BK = 64, LD = BK + 8, WQ = WT == WT_F16 ? 2 : 1;
    __shared__ __align__(16) _Float16 Ah[64][LD], Al[64][LD], Bs[64][LD];
    __shared__ float Ss[WT == WT_Q8 ? 64 : 1][2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    int tm, tn;  // A f32 (4 bytes an element) against W f16 (2) or q8 (1)
    gemm_tile(gridDim.x, gridDim.y, int64_t(g.n) * (WT == WT_F16 ? 2 : 1) > int64_t(g.m) * 4, tm, tn);
    const int m0 = tm * 64, n0 = tn * 64, K = g.K, nb = K / 32;
    const int kbeg = g.kchunk ? int(blockIdx.z) * g.kchunk : 0, kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    const int mr = min(64, g.m - m0), nr = min(64, g.n - n0);
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(A + int64_t(m0) * g.lda, int32_t(mr * g.lda * 4));
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(w + int64_t(n0) * K * (WT == WT_F16 ? 2 : 1), nr * K * (WT == WT_F16 ? 2 : 1));
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(WT == WT_Q8 ? scale + int64_t(n0) * nb : scale, WT == WT_Q8 ? nr * nb * 4 : 0);
    // A: rows ar + 16 q, columns ac .. ac + 3 (f32); W: F16 rows wr + 32 q, columns wc .. wc + 7; Q8 row wr, wc .. wc + 15
    const int ar = tid >> 4, ac = (tid & 15) * 4;
    const int wr = WT == WT_F16 ? tid >> 3 : tid >> 2, wc = WT == WT_F16 ? (tid & 7) * 8 : (tid & 3) * 16;
    int va[4], vw[WQ];
#pragma unroll
    for (int q = 0; q < 4; ++q) va[q] = int32_t(((ar + 16 * q) * g.lda + ac) * 4);
#pragma unroll
    for (int q = 0; q < WQ; ++q) vw[q] = WT == WT_F16 ? ((wr + 32 * q) * K + wc) * 2 : wr * K + wc;
    const int vs = ((tid >> 1) * nb + (tid & 1)) * 4;  // Q8 scales: threads < 128 take row tid / 2, block tid % 2
    f32x4v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    u32x4 xa[S][4], xw[S][WQ];
    float xs[S];
    bool bad = false;  // an activation beyond the f16 range
    auto fetch = [&](u32x4(&a)[4], u32x4(&b)[WQ], float &sc, int k0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] = buf_ld16(ra, va[q], k0 * 4);
#pragma unroll
        for (int q = 0; q < WQ; ++q) b[q] = buf_ld16(rw, vw[q], WT == WT_F16 ? k0 * 2 : k0);
        if (WT == WT_Q8) sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vs, k0 / 32 * 4, 0));
    };
    auto stage = [&](const u32x4(&a)[4], const u32x4(&b)[WQ], float sc) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4v x = __builtin_bit_cast(f32x4v, a[q]);
            f16x4v hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 h, l;
                bad |= split_f16(x[e], h, l);
                hi[e] = h;
                lo[e] = l;
            }
            *reinterpret_cast<f16x4v *>(&Ah[ar + 16 * q][ac]) = hi;
            *reinterpret_cast<f16x4v *>(&Al[ar + 16 * q][ac]) = lo;
        }
        if (WT == WT_F16) {
#pragma unroll
            for (int q = 0; q < WQ; ++q) *reinterpret_cast<u32x4 *>(&Bs[wr + 32 * q][wc]) = b[q];
        } else {
            const uint32_t u[4] = {b[0].x, b[0].y, b[0].z, b[0].w};
            f16x8v h0, h1;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                h0[e] = _Float16(int8_t(u[e >> 2] >> (8 * (e & 3))));
                h1[e] = _Float16(int8_t(u[2 + (e >> 2)] >> (8 * (e & 3))));
            }
            *reinterpret_cast<f16x8v *>(&Bs[wr][wc]) = h0;
            *reinterpret_cast<f16x8v *>(&Bs[wr][wc + 8]) = h1;
            if (tid < 128) Ss[tid >> 1][tid & 1] = sc;
        }
    };
    auto mma = [&]() {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            f16x8v ah[2], al[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int rr = wm * 32 + i * 16 + (lane & 15);
                ah[i] = *reinterpret_cast<const f16x8v *>(&Ah[rr][kk + 8 * (lane >> 4)]);
                al[i] = *reinterpret_cast<const f16x8v *>(&Al[rr][kk + 8 * (lane >> 4)]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const f16x8v *>(&Bs[wn * 32 + j * 16 + (lane & 15)][kk + 8 * (lane >> 4)]);
            if (WT == WT_F16) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], acc[i][j], 0, 0, 0);
                    }
            } else {
                float sc[2];  // the block scale of this lane's W row (its C column)
#pragma unroll
                for (int j = 0; j < 2; ++j) sc[j] = Ss[wn * 32 + j * 16 + (lane & 15)][kk / 32];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        f32x4v tt = {0.f, 0.f, 0.f, 0.f};
                        tt = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], tt, 0, 0, 0);
                        tt = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], tt, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[i][j][v] = fmaf(tt[v], sc[j], acc[i][j][v]);
                    }
            }
        }
    };
    // S register sets, set i holding step s + i: one back edge, so set 0 is always the oldest in flight
    const int ns = (kend - kbeg) / BK, klast = kend - BK;
#pragma unroll
    for (int i = 0; i < S; ++i) {
        fetch(xa[i], xw[i], xs[i], min(kbeg + i * BK, klast));
        __builtin_amdgcn_sched_barrier(0);  // keep each set's loads behind the previous set's
    }
    int s = 0;
    for (; s + S <= ns; s += S) {
#pragma unroll
        for (int i = 0; i < S; ++i) {
            stage(xa[i], xw[i], xs[i]);
            __syncthreads();
            fetch(xa[i], xw[i], xs[i], min(kbeg + (s + i + S) * BK, klast));
            mma();
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < S - 1; ++i) {  // the last ns % S steps, in sets 0 ..
        if (s + i < ns) {
            stage(xa[i], xw[i], xs[i]);
            __syncthreads();
            mma();
            __syncthreads();
        }
    }
    raise_status(g.status, bad, kStatusF16Range);
    if (g.kchunk) return gemm_store_partial<2, 2>(acc, g, m0, n0, wm, wn, lane);
    gemm_epilogue<EPI, 2, 2>(acc, g, m0, n0, wm, wn, lane);
}

// The split-f16 GEMM of k_gemm_h16 when the producer has already split A: hi plane g.a16, lo plane g.a16 + g.a_lo
// (rows of g.lda halves), K a multiple of BK. Weights: F16, or (Q8) the int8 values of Q8 weights widened once to f16
// (exact) with their block scales `scale` [n][K / 32], applied per 32-deep block as k_gemm_h16 does (the block's
// two MFMAs start from zero, s (q . a) goes into the accumulator). Block tile 32 TM rows of A x 32 TN rows of W (4
// waves of 16 TM x 16 TN), K steps of BK through LDS as 16-byte copies (rows padded by 16 halves: fewer LDS bank
// conflicts than 8 on the DiT shapes), no conversion. The loads go through buffer resources cut at the block's last
// row of A and of W, so rows past m or n read as zeros without a per-load bounds check, and the K offset of a step
// is the scalar offset. Two K steps are in flight (two register sets alternate), so a load has two steps' MFMAs to
// arrive. g.kchunk: slice blockIdx.z of K (a multiple of BK) as partial sums into g.ws (k_gemm_splitk_reduce).
template <int EPI, int TM, int TN, int BK, bool Q8 = false, int WN = 2>
// The q8 instances hold the accumulators in VGPRs for the scale FMA; asking for 4 waves per SIMD (128 VGPRs, a
// register or two spilled) measured faster on the prefill shapes than the 3 their unconstrained 165 registers allow.
__global__ __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(Q8 ? 4 : 1))) void k_gemm_hh(const _Float16 *__restrict__ w, const float *__restrict__ scale, GemmArgs g) {
    // 2 x WN waves of 16 TM x 16 TN outputs each (WN = 2: 64 x 64 tiles for TM = TN = 2, 256 threads; WN = 4: 64 x 128,
    // 512 threads, so each block's A tile serves twice the columns)
    constexpr int NT = 128 * WN, LD = BK + 16, BM = 32 * TM, BN = 16 * TN * WN, CPR = BK / 8, RS = NT / CPR, AQ = BM / RS,
                  WQ = BN / RS;
    constexpr int SB = BK / 32;  // scale blocks per K step
    static_assert(AQ >= 1 && WQ >= 1 && BM % RS == 0 && BN % RS == 0, "tile rows per load pass");
    static_assert(!Q8 || BN * SB <= NT, "one scale per thread per K step");
    __shared__ __align__(16) _Float16 Ah[BM][LD], Al[BM][LD], Bs[BN][LD];
    __shared__ float Ss[Q8 ? BN : 1][SB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave / WN, wn = wave % WN;
    int tm, tn;  // A as two f16 planes (4 bytes an element) against W f16 (2)
    gemm_tile(gridDim.x, gridDim.y, g.n > 2 * g.m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN, K = g.K, nb = K / 32;
    const int kbeg = g.kchunk ? int(blockIdx.z) * g.kchunk : 0, kend = g.kchunk ? min(K, kbeg + g.kchunk) : K;
    const int mr = min(BM, g.m - m0), nr = min(BN, g.n - n0);
    const _Float16 *a0 = g.a16 + int64_t(m0) * g.lda;
    const __amdgpu_buffer_rsrc_t rah = buf_rsrc(a0, int32_t(mr * g.lda * 2));
    const __amdgpu_buffer_rsrc_t ral = buf_rsrc(a0 + g.a_lo, int32_t(mr * g.lda * 2));
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(w + int64_t(n0) * K, nr * K * 2);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(Q8 ? scale + int64_t(n0) * nb : scale, Q8 ? nr * nb * 4 : 0);
    // this thread's 8-half chunks of a tile: rows r + RS q, columns c8 .. c8 + 7
    const int r = tid / CPR, c8 = (tid % CPR) * 8;
    int va[AQ], vw[WQ];
#pragma unroll
    for (int q = 0; q < AQ; ++q) va[q] = int32_t(((r + RS * q) * g.lda + c8) * 2);
#pragma unroll
    for (int q = 0; q < WQ; ++q) vw[q] = ((r + RS * q) * K + c8) * 2;
    const int vs = ((tid / SB) * nb + tid % SB) * 4;  // Q8: threads < BN SB take row tid / SB, block tid % SB
    f32x4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    u32x4 xa0[2 * AQ], xw0[WQ], xa1[2 * AQ], xw1[WQ];
    float xs0 = 0.f, xs1 = 0.f;
    auto fetch = [&](u32x4(&a)[2 * AQ], u32x4(&b)[WQ], float &sc, int k0) {
        const int so = k0 * 2;
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            a[q] = buf_ld16(rah, va[q], so);
            a[AQ + q] = buf_ld16(ral, va[q], so);
        }
#pragma unroll
        for (int q = 0; q < WQ; ++q) b[q] = buf_ld16(rw, vw[q], so);
        if (Q8) sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vs, k0 / 32 * 4, 0));
    };
    auto stage = [&](const u32x4(&a)[2 * AQ], const u32x4(&b)[WQ], float sc) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            *reinterpret_cast<u32x4 *>(&Ah[r + RS * q][c8]) = a[q];
            *reinterpret_cast<u32x4 *>(&Al[r + RS * q][c8]) = a[AQ + q];
        }
#pragma unroll
        for (int q = 0; q < WQ; ++q) *reinterpret_cast<u32x4 *>(&Bs[r + RS * q][c8]) = b[q];
        if (Q8 && tid < BN * SB) Ss[tid / SB][tid % SB] = sc;
    };
    auto mma = [&]() {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            f16x8v ah[TM], al[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int rr = wm * 16 * TM + i * 16 + (lane & 15);
                ah[i] = *reinterpret_cast<const f16x8v *>(&Ah[rr][kk + 8 * (lane >> 4)]);
                al[i] = *reinterpret_cast<const f16x8v *>(&Al[rr][kk + 8 * (lane >> 4)]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const f16x8v *>(&Bs[wn * 16 * TN + j * 16 + (lane & 15)][kk + 8 * (lane >> 4)]);
            if (Q8) {
                float sc[TN];  // the block scale of this lane's W row (its C column)
#pragma unroll
                for (int j = 0; j < TN; ++j) sc[j] = Ss[wn * 16 * TN + j * 16 + (lane & 15)][kk / 32];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        f32x4v tt = {0.f, 0.f, 0.f, 0.f};
                        tt = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], tt, 0, 0, 0);
                        tt = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], tt, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[i][j][v] = fmaf(tt[v], sc[j], acc[i][j][v]);
                    }
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], acc[i][j], 0, 0, 0);
                    }
            }
        }
    };
    // Every fetch is unconditional (steps past the end re-read the last one), so the compiler's count of loads in
    // flight is exact: staging one set waits only for that set, the other stays in flight.
    const int ns = (kend - kbeg) / BK, klast = kend - BK;
    fetch(xa0, xw0, xs0, kbeg);
    __builtin_amdgcn_sched_barrier(0);  // keep the first set's loads ahead of the second's
    fetch(xa1, xw1, xs1, min(kbeg + BK, klast));
    for (int s = 0; s + 1 < ns; s += 2) {  // one back edge: the first set is always the older in flight
        stage(xa0, xw0, xs0);
        __syncthreads();
        fetch(xa0, xw0, xs0, min(kbeg + (s + 2) * BK, klast));
        mma();
        __syncthreads();
        stage(xa1, xw1, xs1);
        __syncthreads();
        fetch(xa1, xw1, xs1, min(kbeg + (s + 3) * BK, klast));
        mma();
        __syncthreads();
    }
    if (ns & 1) {  // the last step, in the first set
        stage(xa0, xw0, xs0);
        __syncthreads();
        mma();
    }
    if (g.kchunk) return gemm_store_partial<TM, TN>(acc, g, m0, n0, wm, wn, lane);
    gemm_epilogue<EPI, TM, TN>(acc, g, m0, n0, wm, wn, lane);
}

// The split-K partial slices ws[z][m][n], added in z order, then bias and the epilogue (STORE, ACC, GATED_ACC, SWIGLU,
// SNAKE, GELU_ERF, ACC_SNAKE: one thread per output element; SWIGLU outputs pair columns 2u, 2u + 1). grid
// ceil(m n' / 256).
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_splitk_reduce(GemmArgs g, int32_t splits) {
    const int nout = EPI == EPI_SWIGLU ? g.n / 2 : g.n;
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= int64_t(g.m) * nout) return;
    const int row = int(t / nout), c = int(t % nout);
    const int64_t slice = int64_t(g.m) * g.n;
    auto sum = [&](int col) {  // 8 slices' loads in flight at once (past `splits`, slice 0, left out), added in order
        float v = 0.f;
        for (int z0 = 0; z0 < splits; z0 += 8) {
            float t[8];
#pragma unroll
            for (int z = 0; z < 8; ++z) t[z] = g.ws[(z0 + z < splits ? z0 + z : 0) * slice + int64_t(row) * g.n + col];
#pragma unroll
            for (int z = 0; z < 8; ++z)
                if (z0 + z < splits) v += t[z];
        }
        return v + (g.bias ? g.bias[col] : 0.f);
    };
    float *dst = g.y + int64_t(row) * g.ldy + c;
    if (EPI == EPI_SWIGLU) *dst = silu(sum(2 * c)) * sum(2 * c + 1);
    else if (EPI == EPI_STORE) *dst = sum(c);
    else if (EPI == EPI_ACC) *dst += sum(c);
    else if (EPI == EPI_GATED_ACC) *dst += g.gate[c] * sum(c);
    else if (EPI == EPI_SNAKE) {
        const float v = sum(c), sn = sinf(v * g.snake_a[c]);
        *dst = v + g.snake_ib[c] * sn * sn;
    }
    else if (EPI == EPI_GELU_ERF) *dst = gelu_erf_f(sum(c));
    else if (EPI == EPI_ACC_SNAKE) {
        const float v = *dst + sum(c), sn = sinf(v * g.snake_a[c]);
        *dst = v;
        g.snake_y[int64_t(row) * g.ldy + c] = v + g.snake_ib[c] * sn * sn;
    }
}

// The split-K slices of an EPI_ACC product added into its rows, y[row][c] += (sum_z ws[z][row][c]) + bias[c], as
// k_gemm_splitk_reduce<EPI_ACC> does, then the RMSNorm (gamma, eps) of each updated row written as f16 halves (hi at
// out16, lo at out16 + lo_off, rows of ldo halves) with k_rmsnorm_rows_h16's arithmetic: the residual add and the
// next norm in one pass over the row. grid m, block 256, n <= 256 NV, splits <= 8.
template <int NV>
__global__ __launch_bounds__(256) void k_splitk_acc_rms_h16(GemmArgs g, int32_t splits, const float *gamma, float eps,
                                                           _Float16 *out16, int64_t ldo, int64_t lo_off) {
    __shared__ float red[4];
    const int row = int(blockIdx.x);
    const int64_t slice = int64_t(g.m) * g.n;
    float *yr = g.y + int64_t(row) * g.ldy;
    // every slice's value and the row's own first, so the loads are in flight together (slices past `splits`, at
    // most kMaxSplits, read slice 0 and are left out), then the sums in split order as the reduce kernel adds them
    constexpr int kMaxSplits = 8;
    float t[NV][kMaxSplits], hv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = min(int(threadIdx.x) + 256 * k, g.n - 1);
        hv[k] = yr[c];
#pragma unroll
        for (int z = 0; z < kMaxSplits; ++z) t[k][z] = g.ws[(z < splits ? z : 0) * slice + int64_t(row) * g.n + c];
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = int(threadIdx.x) + 256 * k;
        if (c < g.n) {
            float v = 0.f;
#pragma unroll
            for (int z = 0; z < kMaxSplits; ++z)
                if (z < splits) v += t[k][z];
            v = v + (g.bias ? g.bias[c] : 0.f);
            hv[k] = hv[k] + v;
            yr[c] = hv[k];
            ss = fmaf(hv[k], hv[k], ss);
        } else {
            hv[k] = 0.f;
        }
    }
    ss = block_sum<256>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(g.n) + eps);
    bool bad = false;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c = int(threadIdx.x) + 256 * k;
        if (c < g.n) {
            _Float16 hi, lo;
            bad |= split_f16(gamma[c] * (hv[k] * inv), hi, lo);
            out16[int64_t(row) * ldo + c] = hi;
            out16[lo_off + int64_t(row) * ldo + c] = lo;
        }
    }
    raise_status(g.status, bad, kStatusF16Range);
}

// Merge of the kAttnMaxSplits attention partials of m rows into ao [m][heads * hd] (the PRO_ATTN prologue of the
// GEMV, as its own pass before a GEMM). grid (heads, m), block hd.
__global__ __launch_bounds__(128) void k_attn_merge(AttnPartials P, float *ao) {
    const int h = blockIdx.x, i = blockIdx.y, e = threadIdx.x;
    const int64_t base = (int64_t(i) * P.heads + h) * kAttnMaxSplits;
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < kAttnMaxSplits; ++q) mx = fmaxf(mx, P.pm[base + q]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int q = 0; q < kAttnMaxSplits; ++q) {
        const float pmq = P.pm[base + q];
        const float wq = pmq == -INFINITY ? 0.f : expf(pmq - mx);
        L = fmaf(wq, P.pl[base + q], L);
        O = fmaf(wq, P.po[(base + q) * P.hd + e], O);
    }
    ao[int64_t(i) * P.heads * P.hd + h * P.hd + e] = O * (1.0f / L);
}

}  // namespace vh
