// vh_sample.hpp — sample_logits (sampling.hpp:61-119) as one 1024-thread block on the device.
//
// Order of operations as the reference and the engine's mask (engine.cpp:664-668):
//   mask [suppress_from, suppress_to) except eos, block eos -> repetition penalty (each seen token once)
//   -> greedy (T <= 0: first maximum) | top-k by (value desc, index asc) -> softmax in double over the
//   top-k at 1/T -> top-p minimal prefix -> inverse CDF with u = Philox(frame, codebook, draw).
// Exactness: the top-k set and its order are exact (64-bit keys (ordered value, ~index), radix select, bitonic
// sort); the probabilities are double; every sum runs sequentially in sorted order like the reference
// (one wave, values staged through lane reads). Only exp() may differ from glibc by an ulp of a double.
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

// Exclusive block scan of one int per thread (1024 threads). tmp: 16 ints.
VH_DEV int block_excl_scan(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    __syncthreads();
    if (lane == 63) tmp[w] = inc;
    __syncthreads();
    int before = 0, all = 0;
    for (int i = 0; i < kSampleThreads / 64; ++i) {
        if (i < w) before += tmp[i];
        all += tmp[i];
    }
    *total = all;
    return before + inc - v;
}

// out[0] = sampled index (or -1 when the request exceeds the kernel's limits).
__global__ __launch_bounds__(kSampleThreads) void k_sample(const SampleCfgDev *cfgp, const float *logits, int32_t n,
                                                           int32_t *out) {
    __shared__ uint32_t seen[kSampleMaxN / 32];
    __shared__ uint32_t hist[256];
    __shared__ int scan_tmp[16];
    __shared__ uint64_t sh_prefix;
    __shared__ int sh_bits, sh_kk, sh_done;
    __shared__ __align__(16) uint64_t sk[kSampleMaxK];  // selected keys; later the probabilities (double)
    __shared__ int32_t sidx[kSampleMaxK];
    __shared__ unsigned long long sh_best;
    const int t = threadIdx.x, lane = t & 63;
    const SampleCfgDev cfg = *cfgp;
    if (n <= 0 || n > kSampleMaxN) { if (t == 0) out[0] = -1; return; }
    constexpr int E = kSampleMaxN / kSampleThreads;
    const int per = (n + kSampleThreads - 1) / kSampleThreads;  // contiguous indices per thread (index order)

    for (int i = t; i < kSampleMaxN / 32; i += kSampleThreads) seen[i] = 0u;
    __syncthreads();
    if (cfg.rep != 1.0f && cfg.history)
        for (int i = t; i < cfg.n_history; i += kSampleThreads) {
            const int32_t h = cfg.history[i];
            if (h >= 0 && h < n) atomicOr(&seen[h >> 5], 1u << (h & 31));
        }
    __syncthreads();

    uint64_t key[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = t * per + e;
        key[e] = 0ull;
        if (e < per && idx < n) {
            float v = logits[idx];
            if (idx >= cfg.sup_from && idx < cfg.sup_to && idx != cfg.eos) v = -INFINITY;
            if (cfg.block_eos && idx == cfg.eos) v = -INFINITY;
            if (cfg.rep != 1.0f && (seen[idx >> 5] >> (idx & 31) & 1u)) v = v > 0.f ? v / cfg.rep : v * cfg.rep;
            key[e] = uint64_t(ord_key(v)) << 32 | uint64_t(0xFFFFFFFFu - uint32_t(idx));
        }
    }

    if (cfg.temperature <= 0.0f) {  // greedy: largest key = first maximum
        if (t == 0) sh_best = 0ull;
        __syncthreads();
        uint64_t b = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) b = key[e] > b ? key[e] : b;
        atomicMax(&sh_best, (unsigned long long)b);
        __syncthreads();
        if (t == 0) out[0] = int32_t(0xFFFFFFFFu - uint32_t(sh_best));
        return;
    }

    const int k = (cfg.top_k > 0 && cfg.top_k < n) ? cfg.top_k : n;
    if (k > kSampleMaxK) { if (t == 0) out[0] = -1; return; }

    // ---- radix select: the k-th largest key's prefix, 8 bits per pass, stopping once the prefix bucket
    // holds exactly the keys still needed.
    if (t == 0) { sh_prefix = 0ull; sh_bits = 0; sh_kk = k; sh_done = 0; }
    __syncthreads();
    for (int pass = 0; pass < 8; ++pass) {
        for (int i = t; i < 256; i += kSampleThreads) hist[i] = 0u;
        __syncthreads();
        const uint64_t P = sh_prefix;
        const int L = sh_bits, shift = 56 - 8 * pass;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (key[e] && (L == 0 || (key[e] >> (64 - L)) == P)) atomicAdd(&hist[(key[e] >> shift) & 255u], 1u);
        __syncthreads();
        if (t == 0) {
            int kk = sh_kk, cum = 0, digit = 0, cnt = 0;
            for (int d = 255; d >= 0; --d) {
                const int c = int(hist[d]);
                if (cum + c >= kk) { digit = d; cnt = c; break; }
                cum += c;
            }
            kk -= cum;
            sh_prefix = (P << 8) | uint64_t(digit);
            sh_bits = L + 8;
            sh_kk = kk;
            sh_done = cnt == kk;
        }
        __syncthreads();
        if (sh_done) break;
    }
    const uint64_t P = sh_prefix;
    const int L = sh_bits;
    auto selected = [&](uint64_t kv) { return kv != 0ull && (kv >> (64 - L)) >= P; };

    // ---- compact the k selected keys (any order), pad to a power of two, bitonic sort descending
    int mine = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) mine += selected(key[e]) ? 1 : 0;
    int total = 0;
    int off = block_excl_scan(mine, scan_tmp, &total);
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (selected(key[e]) && off < kSampleMaxK) sk[off++] = key[e];  // exactly k keys are selected
    int K2 = 1;
    while (K2 < k) K2 <<= 1;
    for (int i = k + t; i < K2; i += kSampleThreads) sk[i] = 0ull;
    __syncthreads();
    for (int size = 2; size <= K2; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < K2; i += kSampleThreads) {
                const int l = i ^ stride;
                if (l > i) {
                    const uint64_t x = sk[i], y = sk[l];
                    const bool desc = (i & size) == 0;
                    if (desc ? (x < y) : (x > y)) { sk[i] = y; sk[l] = x; }
                }
            }
            __syncthreads();
        }

    // ---- probabilities in double (sampling.hpp:91-99)
    const double inv_t = 1.0 / double(cfg.temperature);
    const double mx = double(ord_val(uint32_t(sk[0] >> 32)));
    double pv[kSampleMaxK / kSampleThreads];
#pragma unroll
    for (int r = 0; r < kSampleMaxK / kSampleThreads; ++r) {
        const int i = t + r * kSampleThreads;
        pv[r] = 0.0;
        if (i < k) {
            const uint64_t kv = sk[i];
            sidx[i] = int32_t(0xFFFFFFFFu - uint32_t(kv));
            pv[r] = exp((double(ord_val(uint32_t(kv >> 32))) - mx) * inv_t);
        }
    }
    __syncthreads();
    double *pr = reinterpret_cast<double *>(sk);
#pragma unroll
    for (int r = 0; r < kSampleMaxK / kSampleThreads; ++r) {
        const int i = t + r * kSampleThreads;
        if (i < k) pr[i] = pv[r];
    }
    __syncthreads();
    if (t >= 64) return;

    // ---- sequential sums in one wave, in sorted order
    double sum = 0.0;
    for (int base = 0; base < k; base += 64) {
        const double v = base + lane < k ? pr[base + lane] : 0.0;
        const int cnt = k - base < 64 ? k - base : 64;
        for (int j = 0; j < cnt; ++j) sum += readlane_d(v, j);
    }
    // each lane normalizes exactly the entries it reads below (index base + lane), so no cross-lane hazard
    for (int i = lane; i < k; i += 64) pr[i] = pr[i] / sum;
    int keep = k;
    if (cfg.top_p > 0.0f && cfg.top_p < 1.0f) {
        double c = 0.0;
        bool found = false;
        for (int base = 0; base < k && !found; base += 64) {
            const double v = base + lane < k ? pr[base + lane] : 0.0;
            const int cnt = k - base < 64 ? k - base : 64;
            for (int j = 0; j < cnt; ++j) {
                c += readlane_d(v, j);
                if (c >= double(cfg.top_p)) { keep = base + j + 1; found = true; break; }
            }
        }
    }
    double tot = 0.0;
    for (int base = 0; base < keep; base += 64) {
        const double v = base + lane < keep ? pr[base + lane] : 0.0;
        const int cnt = keep - base < 64 ? keep - base : 64;
        for (int j = 0; j < cnt; ++j) tot += readlane_d(v, j);
    }
    const float u = det_uniform(cfg.key0, cfg.key1, cfg.frame, cfg.cb, cfg.draw);
    const double target = double(u) * tot;
    double accp = 0.0;
    int pick = keep - 1;
    bool hit = false;
    for (int base = 0; base < keep && !hit; base += 64) {
        const double v = base + lane < keep ? pr[base + lane] : 0.0;
        const int cnt = keep - base < 64 ? keep - base : 64;
        for (int j = 0; j < cnt; ++j) {
            accp += readlane_d(v, j);
            if (target < accp) { pick = base + j; hit = true; break; }
        }
    }
    if (lane == 0) out[0] = sidx[pick];
}

}  // namespace vh
