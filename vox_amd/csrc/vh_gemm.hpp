// vh_gemm.hpp — f32 GEMM on the matrix cores for multi-row passes (prefill, m > 4 on the f32-activation path).
//
// C[i][r] (+)= sum_k A[i][k] * W[r][k] (+ bias[r]): the device counterpart of matmul's f32 paths for m > 8 (Q8
// dequantized as float(q) * scale, kernels.cpp:661-679) and for F32 / F16 / BF16 weights (kernels.cpp:337-412).
// The products are the reference's (weights widened exactly to f32, f32 activations); only the summation order
// differs (v_mfma_f32_16x16x4_f32 accumulates in f32).
//
// Block: 256 threads = 4 waves as 2 x 2, tile 64 rows of A x 64 rows of W, K step 32 staged through LDS (W
// dequantized on the way in). Each wave owns a 32 x 32 piece of C as 2 x 2 MFMA 16x16x4 tiles. MFMA lane layouts
// (checked on gfx950): A 16x4 -> lane l holds A[l % 16][l / 16]; B 4x16 -> lane l holds B[l / 16][l % 16];
// D 16x16 -> lane l holds D[4 (l / 16) + i][l % 16], i < 4.
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 64, kGemmBN = 64, kGemmBK = 32, kGemmLd = kGemmBK + 4;  // LDS row stride (bank spread)

template <int WT>
VH_DEV int64_t gemm_row_bytes(int K) {
    return WT == WT_F32 ? int64_t(K) * 4 : WT == WT_Q8 ? int64_t(K) : int64_t(K) * 2;
}

// EPI_STORE: y = C + bias; EPI_ACC: y += C + bias; EPI_SWIGLU: W rows are (gate u, up u) pairs, y[u] = silu(gate) * up.
template <int WT, int EPI>
__global__ __launch_bounds__(256) void k_gemm_f32(const uint8_t *__restrict__ w, const float *__restrict__ scale,
                                                  const float *__restrict__ A, GemmArgs g) {
    static_assert(WT == WT_F32 || WT == WT_F16 || WT == WT_BF16 || WT == WT_Q8, "f32-activation weight types");
    __shared__ __align__(16) float As[kGemmBM][kGemmLd];
    __shared__ __align__(16) float Bs[kGemmBN][kGemmLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kGemmBM, n0 = blockIdx.x * kGemmBN;
    const int K = g.K, nb = K / 32;
    const int64_t rb = gemm_row_bytes<WT>(K);
    f32x4v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < K; k0 += kGemmBK) {
        // A tile: 64 rows x 32 k, two f32x4 per thread; rows past m and k past K read as zeros
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int idx = tid + 256 * q, r = idx >> 3, kq = (idx & 7) * 4;
            const int row = m0 + r, k = k0 + kq;
            f32x4v v = {0.f, 0.f, 0.f, 0.f};
            if (row < g.m && k < K) v = *reinterpret_cast<const f32x4v *>(A + int64_t(row) * g.lda + k);
            *reinterpret_cast<f32x4v *>(&As[r][kq]) = v;
        }
        // W tile: 64 rows x 32 k, widened to f32; 8 elements per thread
        {
            const int r = tid >> 2, kq = (tid & 3) * 8, row = n0 + r, k = k0 + kq;
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (row < g.n && k < K) {
                const uint8_t *p = w + int64_t(row) * rb;
                if (WT == WT_Q8) {
                    const uint2 u = *reinterpret_cast<const uint2 *>(p + k);
                    const float s = scale[int64_t(row) * nb + k / 32];
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
            *reinterpret_cast<f32x4v *>(&Bs[r][kq]) = f32x4v{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4v *>(&Bs[r][kq + 4]) = f32x4v{v[4], v[5], v[6], v[7]};
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGemmBK; kk += 4) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = As[wm * 32 + i * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = Bs[wn * 32 + j * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // epilogue: lane holds C[row0 + 4 (lane / 16) + v][col] of each tile, col = col0 + lane % 16
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 32 + j * 16 + (lane & 15);
            const float bz = (g.bias && col < g.n) ? g.bias[col] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + v;
                const float c = acc[i][j][v] + bz;
                if (EPI == EPI_SWIGLU) {
                    const float up = __shfl_xor(c, 1, kWave);  // column col ^ 1 of the same row
                    if (row < g.m && col < g.n && (col & 1) == 0) g.y[int64_t(row) * g.ldy + col / 2] = silu(c) * up;
                } else if (row < g.m && col < g.n) {
                    float *dst = g.y + int64_t(row) * g.ldy + col;
                    if (EPI == EPI_STORE) *dst = c;
                    else *dst += c;
                }
            }
        }
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
