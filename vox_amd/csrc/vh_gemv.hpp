// vh_gemv.hpp — weight-streaming GEMV kernels for gfx950 (decode, m <= 8 rows).
//
// y[i][r] (+)= sum_k W[r][k] * x[i][k] (+ bias[r]) for i < m, the device counterpart of matmul()
// (kernels.cpp:653-705). The weights are the HBM stream: each lane issues 16-byte non-temporal loads,
// 64 consecutive lanes cover 1 KiB of one row, and every wave keeps R rows x IT chunks of loads in
// flight. The first loads are issued before the activation prologue, since they do not depend on it.
//
// Two arithmetic families, as the reference dispatcher chooses them:
//  - k_gemv_int: Q8 (m <= 8) and Q4. x is quantized per 32-block to int8 in LDS exactly as
//    kernels.cpp:515-523; block dots are exact int32 (v_dot4_i32_i8), then float(dot) * (ws * xs).
//  - k_gemv_flt: F32 / F16 / BF16 and Q8 with m > 8: f32 activations in LDS, weights widened
//    (Q8: float(q) * scale as kernels.cpp:665-674), f32 FMA accumulation.
// Prologues: PRO_X reads x as is; PRO_RMS applies RMSNorm(x, gamma, eps) first (kernels.cpp:707-712),
// every block recomputing it (a 4 KiB L2-resident read), and block 0 stores the normed rows when asked.
// Epilogues: store, accumulate (the residual add of kernels.cpp:831/:839), or SwiGLU over interleaved
// (gate, up) row pairs (kernels.cpp:836).
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {


// RMSNorm scale of row mm (all threads get it): 1 / sqrt(sum(x^2)/K + eps).
template <int NT>
VH_DEV float rms_inv(const float *x, int K, float eps, float *red) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += NT) ss = fmaf(x[i], x[i], ss);
    ss = block_sum<NT>(ss, red);
    return 1.0f / sqrtf(ss / float(K) + eps);
}

// Bytes of one weight row.
template <int WT>
VH_DEV int64_t row_bytes(int K) {
    return WT == WT_F32 ? int64_t(K) * 4 : WT == WT_Q8 ? int64_t(K) : WT == WT_Q4 ? int64_t(K) / 2 : int64_t(K) * 2;
}

// Epilogue: lane r*M + mm holds the total of (row0 + r, input row mm). SwiGLU pairs rows (2u, 2u+1) =
// (gate u, up u); the partner value is fetched with all lanes active, then only valid lanes store.
template <int M, int R, int EPI>
VH_DEV void store_out(const GemvArgs &a, float out, int lane, int row0) {
    const int r = lane / M, mm = lane % M, row = row0 + r;
    const bool ok = lane < R * M && row < a.rows && mm < a.m;
    const float v = out + ((ok && a.bias) ? a.bias[row] : 0.f);
    if (EPI == EPI_SWIGLU) {
        const float other = __shfl_xor(v, M, kWave);  // lane of row r ^ 1, same input row
        if (ok && (r & 1) == 0) a.y[int64_t(mm) * a.ldy + row / 2] = silu(v) * other;
    } else if (ok) {
        if (EPI == EPI_STORE) a.y[int64_t(mm) * a.ldy + row] = v;
        else a.y[int64_t(mm) * a.ldy + row] += v;
    }
}

// ------------------------------------------------------------------------------------------ int8 path
template <int WT, int M, int R, int IT, int PRO, int EPI>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_int(GemvArgs a) {
    static_assert(WT == WT_Q8 || WT == WT_Q4, "int path is Q8/Q4");
    extern __shared__ __align__(16) uint8_t smem[];
    const int K = a.K, nb = K / 32;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);                 // [M][K]
    float *xs = reinterpret_cast<float *>(smem + M * K);           // [M][nb]
    float *red = xs + M * nb;                                      // [4]
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
                const bool ok = c < nchunk && row < a.rows;
                const u32x4 *p = reinterpret_cast<const u32x4 *>(a.w + int64_t(row) * rb) + c;
                wv[j][r] = ok ? __builtin_nontemporal_load(p) : u32x4{0u, 0u, 0u, 0u};
                const int blk = WT == WT_Q8 ? (c >> 1) : c;
                sv[j][r] = ok ? a.scale[int64_t(row) * nb + blk] : 0.f;
            }
        }
    };
    load(0);

    // ---- prologue: int8-quantize the m input rows into LDS
    for (int mm = 0; mm < M; ++mm) {
        const float *xr = a.x + int64_t(mm) * a.ldx;
        float inv = 1.f;
        if (PRO == PRO_RMS && mm < a.m) inv = rms_inv<kGemvThreads>(xr, K, a.eps, red);
        for (int b = threadIdx.x; b < nb; b += kGemvThreads) {
            float v[32];
            if (mm < a.m) {
#pragma unroll
                for (int j = 0; j < 32; j += 4) {
                    const f32x4 t = *reinterpret_cast<const f32x4 *>(xr + b * 32 + j);
                    v[j] = t.x; v[j + 1] = t.y; v[j + 2] = t.z; v[j + 3] = t.w;
                }
                if (PRO == PRO_RMS) {
#pragma unroll
                    for (int j = 0; j < 32; ++j) v[j] = a.gamma[b * 32 + j] * (v[j] * inv);
                    if (a.xnorm && blockIdx.x == 0)
#pragma unroll
                        for (int j = 0; j < 32; ++j) a.xnorm[int64_t(mm) * K + b * 32 + j] = v[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 32; ++j) v[j] = 0.f;
            }
            int8_t q[32];
            float sc;
            quant_block32(v, q, &sc);
            uint32_t *dst = reinterpret_cast<uint32_t *>(xq + mm * K + b * 32);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                dst[j] = uint32_t(uint8_t(q[4 * j])) | uint32_t(uint8_t(q[4 * j + 1])) << 8 |
                         uint32_t(uint8_t(q[4 * j + 2])) << 16 | uint32_t(uint8_t(q[4 * j + 3])) << 24;
            xs[mm * nb + b] = sc;
        }
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
                        d += __shfl_xor(d, 1, kWave);  // the two 16-byte halves of one 32-block: exact block dot
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

    // ---- reduce over the wave and write
    float out = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const float s = wave_sum(acc[r][mm]);
            if (lane == r * M + mm) out = s;
        }
    store_out<M, R, EPI>(a, out, lane, row0);
}

// ------------------------------------------------------------------------------------------ f32 path
template <int WT, int M, int R, int IT, int PRO, int EPI>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_flt(GemvArgs a) {
    static_assert(WT != WT_Q4, "Q4 always uses the int path");
    extern __shared__ __align__(16) uint8_t smem[];
    const int K = a.K;
    float *xf = reinterpret_cast<float *>(smem);  // [M][K]
    float *red = xf + M * K;                      // [4]
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
                const bool ok = c < nchunk && row < a.rows;
                const u32x4 *p = reinterpret_cast<const u32x4 *>(a.w + int64_t(row) * rb) + c;
                wv[j][r] = ok ? __builtin_nontemporal_load(p) : u32x4{0u, 0u, 0u, 0u};
                sv[j][r] = (WT == WT_Q8 && ok) ? a.scale[int64_t(row) * nb + (c >> 1)] : 0.f;
            }
        }
    };
    load(0);

    for (int mm = 0; mm < M; ++mm) {
        const float *xr = a.x + int64_t(mm) * a.ldx;
        float inv = 1.f;
        if (PRO == PRO_RMS && mm < a.m) inv = rms_inv<kGemvThreads>(xr, K, a.eps, red);
        for (int i = threadIdx.x; i < K; i += kGemvThreads) {
            float v = 0.f;
            if (mm < a.m) {
                v = xr[i];
                if (PRO == PRO_RMS) {
                    v = a.gamma[i] * (v * inv);
                    if (a.xnorm && blockIdx.x == 0) a.xnorm[int64_t(mm) * K + i] = v;
                }
            }
            xf[mm * K + i] = v;
        }
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

    float out = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const float s = wave_sum(acc[r][mm]);
            if (lane == r * M + mm) out = s;
        }
    store_out<M, R, EPI>(a, out, lane, row0);
}

}  // namespace vh
