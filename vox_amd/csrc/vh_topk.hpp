// vh_topk.hpp — block-wide top-k selection of 64-bit keys (radix select + bitonic sort) and the cross-lane
// helpers it uses; shared by the logit sampler (k_sample) and the CosyVoice2 LM sampler (k_lm_sample).
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

// Order-preserving map of a float to uint32 (larger value -> larger key); -0 == +0; NaN lowest.
VH_DEV uint32_t ord_key(float f) {
    if (f == 0.f) f = 0.f;
    const uint32_t b = __float_as_uint(f);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
VH_DEV float ord_val(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

VH_DEV double readlane_d(double v, int j) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), j));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), j));
    return __longlong_as_double(int64_t(uint64_t(hi) << 32 | lo));
}
VH_DEV uint64_t readlane_u64(uint64_t v, int j) {
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), j));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), j));
    return uint64_t(hi) << 32 | lo;
}
// Value of lane (lane ^ m) for a 64-bit value: DPP within a 16-lane row for m <= 8, a swizzle for 16, a permute
// for 32 (m is a compile-time constant after unrolling).
VH_DEV int xor_lane(int x, int m) {
    const int lane = threadIdx.x & 63;
    switch (m) {
        case 1: return dpp<kDppXor1>(x);
        case 2: return dpp<kDppXor2>(x);
        case 4: {  // both DPP reads run with every lane active (a disabled source lane would read as 0)
            const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, false);  // row_shl:4 reads lane i + 4
            const int dn = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4 reads lane i - 4
            return (lane & 4) ? dn : up;
        }
        case 8: return __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);  // row_ror:8 = lane ^ 8 in the row
        case 16: return __builtin_amdgcn_ds_swizzle(x, 0x401F);  // bit mode: and 0x1F, xor 0x10
        default: return __shfl_xor(x, m, kWave);
    }
}
VH_DEV uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = uint32_t(xor_lane(int(uint32_t(v)), m));
    const uint32_t hi = uint32_t(xor_lane(int(uint32_t(v >> 32)), m));
    return uint64_t(hi) << 32 | lo;
}

// Orders one wave's LDS accesses around a cross-lane exchange (a write by one lane read by another): fences at
// wavefront scope and a code-motion barrier, so no access moves across it.
VH_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Dynamic LDS of k_sample in bytes for n logits: room for the sorted keys of the LDS path.
inline size_t sample_smem_bytes(int n) {
    size_t k2 = 64;
    while (k2 < size_t(n)) k2 <<= 1;
    return k2 * sizeof(uint64_t);
}

// LDS state of topk_sorted. Before the first call: hist all zero, prefix = bits = done = cnt = 0, followed by a
// __syncthreads(); topk_sorted leaves hist zero again (each radix pass clears the bins it reads).
struct TopkSmem {
    uint32_t hist[256];
    uint64_t prefix;
    int bits, kk, done, cnt;
};
VH_DEV void topk_reset(TopkSmem &S) {  // one thread; the caller synchronizes
    S.prefix = 0ull; S.bits = 0; S.done = 0; S.cnt = 0;
}

// The k largest of the block's 64-bit keys in descending order (0 marks "no key"; every key is distinct). The
// radix select finds the k-th key, 8 bits per pass: every thread adds its keys under the current prefix to an
// LDS histogram, wave 0 scans the 256 bins from the top (4 per lane, a prefix sum over lanes) and clears them.
// The selected keys are compacted (one LDS atomic per wave, lanes placed by ballot rank) into keys[0..K2),
// K2 = max(64, next power of two >= k), zero-padded, and bitonic-sorted: K2 == 64 in the registers of wave 0
// (lane j returns the j-th key in v; the function returns true), else in LDS (keys[0..k) sorted; returns false).
// Called by every thread of the block with the same k.
template <int E>
VH_DEV bool topk_sorted(const uint64_t (&key)[E], int per, int k, TopkSmem &S, uint64_t *keys, uint64_t &v) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (t == 0) S.kk = k;
    __syncthreads();
    for (int pass = 0; pass < 8; ++pass) {
        const uint64_t P = S.prefix;
        const int L = S.bits, shift = 56 - 8 * pass;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (key[e] && (L == 0 || (key[e] >> (64 - L)) == P)) atomicAdd(&S.hist[(key[e] >> shift) & 255u], 1u);
        __syncthreads();
        if (wave == 0) {
            int c[4], loc = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = int(S.hist[255 - 4 * lane - j]);
                loc += c[j];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) S.hist[255 - 4 * lane - j] = 0u;
            int incl = loc;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int x = __shfl_up(incl, o, kWave);
                if (lane >= o) incl += x;
            }
            const int kk = S.kk;
            const uint64_t bal = __ballot(incl >= kk);
            const int first = __ffsll((long long)bal) - 1;
            if (lane == first) {
                int before = incl - loc, digit = 0, cnt = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (before + c[j] >= kk) { digit = 255 - 4 * lane - j; cnt = c[j]; break; }
                    before += c[j];
                }
                S.prefix = (P << 8) | uint64_t(digit);
                S.bits = L + 8;
                S.kk = kk - before;
                S.done = cnt == kk - before;
            }
        }
        __syncthreads();
        if (S.done) break;
    }
    const uint64_t P = S.prefix;
    const int L = S.bits;
    int K2 = 64;
    while (K2 < k) K2 <<= 1;
    {
        uint64_t masks[E];
        int wave_total = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            masks[e] = e < per ? __ballot(key[e] && (key[e] >> (64 - L)) >= P) : 0ull;
            wave_total += __popcll(masks[e]);
        }
        int base = 0;
        if (wave_total) {
            if (lane == 0) base = atomicAdd(&S.cnt, wave_total);
            base = __builtin_amdgcn_readfirstlane(base);
        }
        const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if ((masks[e] >> lane) & 1ull) {
                const int p = base + __popcll(masks[e] & lt);
                if (p < K2) keys[p] = key[e];
            }
            base += __popcll(masks[e]);
        }
    }
    for (int i = k + t; i < K2; i += blockDim.x) keys[i] = 0ull;
    __syncthreads();
    if (K2 == 64) {
        if (wave == 0) {
            v = keys[lane];
#pragma unroll
            for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    const uint64_t o = shfl_xor_u64(v, stride);
                    const bool keep_max = ((lane & stride) == 0) == ((lane & size) == 0);
                    v = keep_max ? (o > v ? o : v) : (o < v ? o : v);
                }
        }
        return true;
    }
    for (int size = 2; size <= K2; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < K2; i += blockDim.x) {
                const int l = i ^ stride;
                if (l > i) {
                    const uint64_t x = keys[i], y = keys[l];
                    const bool desc = (i & size) == 0;
                    if (desc ? (x < y) : (x > y)) { keys[i] = y; keys[l] = x; }
                }
            }
            __syncthreads();
        }
    return false;
}

}  // namespace vh
