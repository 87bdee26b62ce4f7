// vh_common.hpp — device helpers shared by the gfx950 kernels (wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define VH_DEV __device__ __forceinline__

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

namespace vh {

constexpr int kWave = 64;

VH_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
VH_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
// Sum over groups of `width` consecutive lanes (width a power of two <= 64); every lane gets its group's sum.
template <int W>
VH_DEV float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Block-wide sum for blockDim.x == NT (multiple of 64). red must hold NT/64 floats. All threads get the sum.
template <int NT>
VH_DEV float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) s += red[i];
    return s;
}

VH_DEV float silu(float x) { return x / (1.0f + expf(-x)); }

VH_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
VH_DEV uint16_t f32_to_bf16(float f) {  // round to nearest even; NaN stays NaN
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x40u);
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// int8 activation quantization of one 32-block (kernels.cpp:515-523): sc = max|x| / 127,
// inv = sc > 0 ? 1/sc : 0, q = rint(x * inv) (round half to even, as lrintf). IEEE division.
VH_DEV void quant_block32(const float *v, int8_t *q, float *sc_out) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(v[j]);
        mx = mx < a ? a : mx;
    }
    const float sc = mx / 127.0f, inv = sc > 0.f ? 1.0f / sc : 0.0f;
    *sc_out = sc;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float p = __fmul_rn(v[j], inv);
        q[j] = int8_t(int(__builtin_rintf(p)));
    }
}

// Philox4x32-10 (sampling.hpp:16-33).
VH_DEV void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
        const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        if (r < 9) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    }
}
// DetRng::uniform (sampling.hpp:40-43)
VH_DEV float det_uniform(uint32_t key0, uint32_t key1, uint64_t frame, uint32_t cb, uint32_t draw) {
    uint32_t c[4] = {uint32_t(frame), uint32_t(frame >> 32), cb, draw};
    philox4x32_10(c, key0, key1);
    return float(c[0] >> 8) * (1.0f / 16777216.0f);
}

}  // namespace vh
