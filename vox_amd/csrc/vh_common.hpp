// vh_common.hpp — device helpers shared by the gfx950 kernels (wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vh_types.hpp"

#define VH_DEV __device__ __forceinline__

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef long long i64x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

namespace vh {

constexpr int kWave = 64;

// f32 -> the f16 halves of a split-f16 product, x = hi + lo to about 2^-22 relative. True when x is finite but
// outside the f16 range (|x| >= 65520 rounds hi to infinity), which the product cannot represent.
// Two values split as split_f16 does, packed (a in the low half): hi = f16(a), f16(b) by v_cvt_pk_f16_f32 (round to
// nearest even, as _Float16(x)); lo = f16(x - hi) by v_fma_mix{lo,hi}_f16, which reads hi as f16 and x as f32 and
// rounds once: x - hi is exact in f32, so that is f16(x - float(hi)). Three instructions instead of eight; checked
// bit for bit against the C++ form on 2^30 pairs across the f16 subnormal, normal and overflow ranges (NaN inputs
// aside, whose payloads may differ).
__device__ __forceinline__ void split_f16x2(float a, float b, uint32_t &hi, uint32_t &lo) {
    asm("v_cvt_pk_f16_f32 %0, %2, %3\n\t"
        "v_fma_mixlo_f16 %1, -%0, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %1, -%0, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(hi), "=&v"(lo)
        : "v"(a), "v"(b));
}
__device__ __forceinline__ bool split_f16(float x, _Float16 &hi, _Float16 &lo) {
    hi = _Float16(x);
    lo = _Float16(x - float(hi));
    return __builtin_isinf(float(hi)) && !__builtin_isinf(x);
}
// Sets `bit` in the status word when `bad` (a vector atomic; the common path is one predicated branch).
__device__ __forceinline__ void raise_status(int32_t *status, bool bad, int32_t bit) {
    if (__builtin_expect(bad, 0) && status) __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// MI355X hands the workgroups of a launch round-robin to its 8 XCDs (linear id % 8), and each XCD has its own L2.
// xcd_tile maps linear id L of T blocks to a tile index so that XCD x takes the contiguous tiles
// [x T / 8, (x + 1) T / 8): neighbouring tiles, which share operand rows, then meet in one L2 instead of every XCD
// streaming all of them. T % 8 != 0: identity.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_tile(int L, int T) { return T % kXcds ? L : (L % kXcds) * (T / kXcds) + L / kXcds; }
// Origin (tm, tn) of GEMM block (x, y) of an nt x mt tile grid through xcd_tile: row-major order (each XCD takes a
// band of A rows and streams all of W) unless w_band, column-major (a band of W rows per XCD, all of A). Each XCD
// then fetches A / 8 + W or A + W / 8 bytes; callers set w_band when W is the larger operand.
__device__ __forceinline__ void gemm_tile(int nt, int mt, bool w_band, int &tm, int &tn) {
    const int t = xcd_tile(int(blockIdx.y) * nt + int(blockIdx.x), nt * mt);
    tm = w_band ? t % mt : t / nt;
    tn = w_band ? t / mt : t % nt;
}

// Raw buffer loads: an access whose vector offset reaches `bytes` reads zeros, so tiles that overhang a matrix need
// no per-load bounds check. Only the vector offset is relied on for the range check: a scalar offset carries a
// uniform step that stays inside the row the vector offset selects.
constexpr int kBufFlags = 0x00020000;  // buffer resource word 3 for gfx9 raw buffers (32-bit data format)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, int32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, kBufFlags);
}
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, int32_t voff, int32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// Cross-lane steps on the DPP path (no LDS round trip): quad permutations and row mirrors within 16-lane rows.
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140 };
template <int CTRL>
VH_DEV int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
VH_DEV float dpp(float v) {
    return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(int, v)));
}
VH_DEV float readlane(float v, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); }

// Sum over groups of W consecutive lanes (W a power of two <= 64); every lane gets its group's sum. Within a
// 16-lane row the steps are xor 1, xor 2, mirror in 8, mirror in 16; rows are combined as (r0 + r1) + (r2 + r3).
template <int W>
VH_DEV float group_sum(float v) {
    if (W >= 2) v += dpp<kDppXor1>(v);
    if (W >= 4) v += dpp<kDppXor2>(v);
    if (W >= 8) v += dpp<kDppRowHalfMirror>(v);
    if (W >= 16) v += dpp<kDppRowMirror>(v);
    if (W == 32) {
        const float a = readlane(v, 0) + readlane(v, 16), b = readlane(v, 32) + readlane(v, 48);
        v = (threadIdx.x & 32) ? b : a;
    } else if (W == 64) {
        v = (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
    }
    return v;
}
VH_DEV float wave_sum(float v) { return group_sum<64>(v); }
VH_DEV float wave_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp<kDppRowMirror>(v));
    return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
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
