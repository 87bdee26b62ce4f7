// vh_util.hpp — device quantizers of the reference formats, RMSNorm rows, synthetic data.
#pragma once
#include "vh_common.hpp"

namespace vh {

// quantize_q8 (kernels.cpp:918-929): per 32-block s = max|w| / 127, q = round-half-away(w / s). One thread per block.
__global__ void k_quant_q8(const float *w, int64_t nblocks, int8_t *q, float *scale) {
    const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *p = w + b * 32;
    float mx = 0.f;
    for (int j = 0; j < 32; ++j) { const float a = fabsf(p[j]); mx = mx < a ? a : mx; }
    const float s = mx / 127.0f;
    scale[b] = s;
    for (int j = 0; j < 32; ++j) q[b * 32 + j] = s > 0.f ? int8_t(int(roundf(p[j] / s))) : int8_t(0);
}

// quantize_q4 (kernels.cpp:606-645): scale search d = mx / -t for t = 7, 7.25 .. 9 by squared error (summed in
// double, kept as a float as kernels.cpp:616 declares it, so a stored error is rounded and later compared widened),
// then the least-squares scale when its double error is below that float. Packs byte j = (q[j] + 8) | (q[j + 16] + 8) << 4.
__global__ void k_quant_q4(const float *w, int64_t nblocks, uint8_t *q, float *scale) {
#pragma clang fp contract(off)
    const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *p = w + b * 32;
    float mx = 0.f;
    for (int j = 0; j < 32; ++j) if (fabsf(p[j]) > fabsf(mx)) mx = p[j];
    float best_d = mx / -8.0f, best_err = INFINITY;
    int8_t best_q[32];
    for (int j = 0; j < 32; ++j) best_q[j] = 0;
    if (mx != 0.0f)
        for (int k = 0; k <= 8; ++k) {
            const float d = mx / -(7.0f + 0.25f * float(k)), inv = 1.0f / d;
            int8_t qq[32];
            double err = 0;
            for (int j = 0; j < 32; ++j) {
                float c = floorf(p[j] * inv + 8.5f);
                c = c < 0.0f ? 0.0f : c;
                c = c > 15.0f ? 15.0f : c;
                qq[j] = int8_t(int(c) - 8);
                const double e = double(p[j]) - double(qq[j]) * double(d);
                err += e * e;
            }
            if (err < double(best_err)) {
                best_err = float(err); best_d = d;
                for (int j = 0; j < 32; ++j) best_q[j] = qq[j];
            }
        }
    if (mx != 0.0f) {
        double num = 0, den = 0;
        for (int j = 0; j < 32; ++j) { num += double(p[j]) * best_q[j]; den += double(best_q[j]) * best_q[j]; }
        if (den > 0) {
            const float d2 = float(num / den);
            double err = 0;
            for (int j = 0; j < 32; ++j) { const double e = double(p[j]) - double(best_q[j]) * double(d2); err += e * e; }
            if (err < double(best_err)) best_d = d2;
        }
    }
    scale[b] = best_d;
    for (int j = 0; j < 16; ++j) q[b * 16 + j] = uint8_t(uint8_t(best_q[j] + 8) | uint8_t((best_q[j + 16] + 8) << 4));
}

// Activation quantization (kernels.cpp:515-523), one thread per 32-block.
__global__ void k_quant_act(const float *x, int64_t nblocks, int8_t *xq, float *xs) {
    const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    float v[32];
    for (int j = 0; j < 32; ++j) v[j] = x[b * 32 + j];
    quant_block32(v, xq + b * 32, xs + b);
}

__global__ void k_to_f16(const float *x, int64_t n, _Float16 *y) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = _Float16(x[i]);
}
__global__ void k_to_bf16(const float *x, int64_t n, uint16_t *y) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = f32_to_bf16(x[i]);
}

// rmsnorm (kernels.cpp:707-712) of rows: out[i] = w * (x[i] * inv). grid (m), block 256.
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float *x, int64_t ldx, const float *w, int K, float eps,
                                                     float *out, int64_t ldo) {
    __shared__ float red[4];
    const float *xr = x + int64_t(blockIdx.x) * ldx;
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum<256>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(K) + eps);
    for (int i = threadIdx.x; i < K; i += 256) out[int64_t(blockIdx.x) * ldo + i] = w[i] * (xr[i] * inv);
}

// k_rmsnorm_rows with the normed rows written as f16 halves for a split-f16 product: x = hi + lo, hi = f16(x),
// lo = f16(x - hi); hi rows of ldo halves at out16, lo rows at out16 + lo_off.
// Rows of up to 8 x 256 values keep the row and the weights in registers, both loaded before the sum, so the
// weights' round trip overlaps the row's; the sums and products are those of the loop below.
__global__ __launch_bounds__(256) void k_rmsnorm_rows_h16(const float *x, int64_t ldx, const float *w, int K, float eps,
                                                         _Float16 *out16, int64_t ldo, int64_t lo_off, int32_t *status) {
    __shared__ float red[4];
    const float *xr = x + int64_t(blockIdx.x) * ldx;
    float ss = 0.f;
    bool bad = false;  // a normed value beyond the f16 range
    if (K <= 8 * 256) {
        float xv[8], wv[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int i = threadIdx.x + 256 * c;
            const int j = i < K ? i : 0;
            xv[c] = xr[j];
            wv[c] = w[j];
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
            if (threadIdx.x + 256 * c < K) ss = fmaf(xv[c], xv[c], ss);
        ss = block_sum<256>(ss, red);
        const float inv = 1.0f / sqrtf(ss / float(K) + eps);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int i = threadIdx.x + 256 * c;
            if (i >= K) continue;
            _Float16 hi, lo;
            bad |= split_f16(wv[c] * (xv[c] * inv), hi, lo);
            out16[int64_t(blockIdx.x) * ldo + i] = hi;
            out16[lo_off + int64_t(blockIdx.x) * ldo + i] = lo;
        }
        raise_status(status, bad, kStatusF16Range);
        return;
    }
    for (int i = threadIdx.x; i < K; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum<256>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(K) + eps);
    for (int i = threadIdx.x; i < K; i += 256) {
        _Float16 hi, lo;
        bad |= split_f16(w[i] * (xr[i] * inv), hi, lo);
        out16[int64_t(blockIdx.x) * ldo + i] = hi;
        out16[lo_off + int64_t(blockIdx.x) * ldo + i] = lo;
    }
    raise_status(status, bad, kStatusF16Range);
}

// int8 weight values widened to f16 (exact: |q| <= 127), 8 per thread; n a multiple of 8.
__global__ __launch_bounds__(256) void k_q8_to_f16(const int8_t *q, _Float16 *out, int64_t n) {
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= n) return;
    const uint2 u = *reinterpret_cast<const uint2 *>(q + i);
    _Float16 h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = _Float16(int8_t((e < 4 ? u.x : u.y) >> (8 * (e & 3))));
    *reinterpret_cast<uint4 *>(out + i) = *reinterpret_cast<const uint4 *>(h);
}

// Synthetic N(mean, std) data: Philox4x32-10 counter (pair p, stream, draw 0/1) under key (seed), Box-Muller.
VH_DEV void normal_pair(uint64_t seed, uint32_t stream, uint64_t p, float *z0, float *z1) {
    const float u1 = det_uniform(uint32_t(seed), uint32_t(seed >> 32), p, stream, 0);
    const float u2 = det_uniform(uint32_t(seed), uint32_t(seed >> 32), p, stream, 1);
    const float r = sqrtf(-2.0f * logf(1.0f - u1));
    const float a = 6.283185307179586f * u2;
    *z0 = r * cosf(a);
    *z1 = r * sinf(a);
}

__global__ void k_fill_normal(float *out, int64_t n, uint64_t seed, uint32_t stream, float mean, float std) {
    const int64_t p = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (2 * p >= n) return;
    float z0, z1;
    normal_pair(seed, stream, uint64_t(p), &z0, &z1);
    out[2 * p] = mean + std * z0;
    if (2 * p + 1 < n) out[2 * p + 1] = mean + std * z1;
}

// max |x| of n floats as the bits of a non-negative float in *out (zero on entry): non-negative floats order as
// their bits, and a NaN's |x| bits (0x7fc00000 and up) exceed every finite value's and infinity's. Grid-stride.
__global__ void k_absmax(const float *x, int64_t n, uint32_t *out) {
    uint32_t m = 0;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        m = max(m, __float_as_uint(x[i]) & 0x7fffffffu);
    if (m) atomicMax(out, m);
}

// Fills positions [0, len) of a [layers*kvh][cap][hd] f16 cache with N(mean, std).
__global__ void k_fill_cache(_Float16 *c, int64_t planes, int64_t cap, int64_t len, int hd, uint64_t seed,
                             uint32_t stream, float mean, float std) {
    const int64_t p = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // pair index over planes*len*hd/2
    const int64_t per_plane = len * hd / 2;
    if (p >= planes * per_plane) return;
    const int64_t plane = p / per_plane, r = p % per_plane;
    float z0, z1;
    normal_pair(seed, stream, uint64_t(p), &z0, &z1);
    _Float16 *dst = c + plane * cap * hd + 2 * r;
    dst[0] = _Float16(mean + std * z0);
    dst[1] = _Float16(mean + std * z1);
}

// Plain 16-byte copy (grid-stride): the STREAM reference of the benchmark and the calibration kernel of the
// HBM traffic counters (FETCH_SIZE / WRITE_SIZE read n * 16 bytes each for it).
__global__ __launch_bounds__(256) void k_copy16(const u32x4 *src, u32x4 *dst, int64_t n) {
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) dst[i] = __builtin_nontemporal_load(src + i);
}

// Self-test of split_f16x2 against the C++ form of split_f16 (hi = f16(x), lo = f16(x - float(hi))): thread t takes
// the pair of pseudo-random f32 bit patterns k = base + 2t, k + 1, every second pair confined to f32 exponents
// 96 .. 150 (|x| from 2^-31 to 2^23: f16 subnormals, normals and overflow); counts the pairs that differ, NaN inputs
// apart (their payloads may differ).
__global__ __launch_bounds__(256) void k_check_split(uint64_t base, uint64_t pairs, unsigned long long *bad) {
    const uint64_t t = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= pairs) return;
    const uint64_t k = base + 2 * t;
    uint32_t ua = uint32_t(k * 2654435761u) ^ uint32_t(k >> 7), ub = uint32_t((k + 1) * 40503u) ^ uint32_t(k >> 3);
    if (k & 2) {
        ua = (ua & 0x807FFFFFu) | ((96u + (ua >> 23) % 55u) << 23);
        ub = (ub & 0x807FFFFFu) | ((96u + (ub >> 23) % 55u) << 23);
    }
    const float a = __builtin_bit_cast(float, ua), b = __builtin_bit_cast(float, ub);
    if (a != a || b != b) return;
    uint32_t hp, lp;
    split_f16x2(a, b, hp, lp);
    _Float16 ha, la, hb, lb;
    (void)split_f16(a, ha, la);
    (void)split_f16(b, hb, lb);
    const uint32_t rh = uint32_t(__builtin_bit_cast(uint16_t, ha)) | (uint32_t(__builtin_bit_cast(uint16_t, hb)) << 16);
    const uint32_t rl = uint32_t(__builtin_bit_cast(uint16_t, la)) | (uint32_t(__builtin_bit_cast(uint16_t, lb)) << 16);
    if (rh != hp || rl != lp) atomicAdd(bad, 1ull);
}

// One wave that returns once the constant-rate real-time counter has advanced by `ticks`, or after `max_iter` sleeps
// of 64 x 8 cycles, whichever comes first (every launch ends). The decode benchmark's kernel-by-kernel pass puts it
// ahead of each step's launches, so the host has enqueued the whole step when the first of them runs, and they run
// back to back as in the graph instead of each waiting for the host's next launch.
__global__ __launch_bounds__(64) void k_hold(uint64_t ticks, int max_iter) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < max_iter; ++i) {
        if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(8);
    }
}

}  // namespace vh
