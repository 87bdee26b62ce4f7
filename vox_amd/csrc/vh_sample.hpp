// vh_sample.hpp — sample_logits (sampling.hpp:61-119) as one 1024-thread block on the device.
//
// Order of operations as the reference and the engine's mask (engine.cpp:664-668):
//   mask [suppress_from, suppress_to) except eos, block eos -> repetition penalty (each seen token once)
//   -> greedy (T <= 0: first maximum) | top-k by (value desc, index asc) -> softmax in double over the
//   top-k at 1/T -> top-p minimal prefix -> inverse CDF with u = Philox(frame, codebook, draw).
// Exactness: the top-k set and its order are exact (64-bit keys (ordered value, ~index): a radix select finds
// the k-th key, the k selected keys are bitonic-sorted); the probabilities are double; every sum runs
// sequentially in sorted order like the reference (one wave, terms broadcast from LDS). Only exp() may
// differ from glibc by an ulp of a double.
//
// Cost shape for the talker head (n = 3072, k = 50; about 10 us): one radix pass per 8 key bits until the k-th
// key's bucket holds exactly the keys still needed (usually 2-3 passes; each pass is one LDS-atomic histogram and
// one wave scan of its 256 bins), then a register bitonic sort of 64 lanes in one wave (k > 64 sorts in LDS), then
// the double-precision sums, whose 64-term chains read the terms from LDS so that no register spills.
#pragma once
#include "vh_topk.hpp"

namespace vh {

// One block per row b: logits [b][n] with cfg[b] -> out[b] = sampled index (or -1 when n is outside
// 1..E kSampleThreads). E: logits per thread, the launcher's smallest power of two >= ceil(n / kSampleThreads), so
// the keys of small vocabularies stay in registers. Dynamic LDS: sample_smem_bytes(n).
template <int E>
__global__ __launch_bounds__(kSampleThreads) void k_sample(const SampleCfgDev *cfgs, const float *logits_all, int32_t n,
                                                           int32_t *outs) {
    const SampleCfgDev *cfgp = cfgs + blockIdx.x;
    const float *logits = logits_all + int64_t(blockIdx.x) * n;
    int32_t *out = outs + blockIdx.x;
    extern __shared__ __align__(16) uint64_t sample_keys[];
    __shared__ uint32_t seen[kSampleMaxN / 32];
    __shared__ TopkSmem S;
    __shared__ unsigned long long sh_best;
    __shared__ double sd[64];  // one chunk of the sequential sums
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (n <= 0 || n > E * kSampleThreads) { if (t == 0) out[0] = -1; return; }
    const int per = (n + kSampleThreads - 1) / kSampleThreads;
    // the logits and the configuration are independent loads: issue both before using either
    float lv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = e * kSampleThreads + t;
        lv[e] = (e < per && idx < n) ? logits[idx] : 0.f;
    }
    const SampleCfgDev cfg = *cfgp;

    if (t < 256) S.hist[t] = 0u;
    if (t == 0) { topk_reset(S); sh_best = 0ull; }
    const bool penalty = cfg.rep != 1.0f && cfg.history && cfg.n_history > 0;  // uniform
    if (penalty) {  // tokens seen in the history, each penalized once (sampling.hpp:65-73)
        for (int i = t; i < kSampleMaxN / 32; i += kSampleThreads) seen[i] = 0u;
        __syncthreads();
        for (int i = t; i < cfg.n_history; i += kSampleThreads) {
            // a global load (the history pointer comes from memory, so it would otherwise be a flat access, which
            // makes every later wait count conservative)
            const int32_t h = ((const __attribute__((address_space(1))) int32_t *)cfg.history)[i];
            if (h >= 0 && h < n) atomicOr(&seen[h >> 5], 1u << (h & 31));
        }
    }
    __syncthreads();

    // keys of indices e * 1024 + t (coalesced); 0 marks "no logit"
    uint64_t key[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int idx = e * kSampleThreads + t;
        key[e] = 0ull;
        if (e < per && idx < n) {
            float v = lv[e];
            if (idx >= cfg.sup_from && idx < cfg.sup_to && idx != cfg.eos) v = -INFINITY;
            if (cfg.block_eos && idx == cfg.eos) v = -INFINITY;
            if (penalty && (seen[idx >> 5] >> (idx & 31) & 1u)) v = v > 0.f ? v / cfg.rep : v * cfg.rep;
            key[e] = uint64_t(ord_key(v)) << 32 | uint64_t(0xFFFFFFFFu - uint32_t(idx));
        }
    }

    if (cfg.temperature <= 0.0f) {  // greedy: largest key = first maximum
        uint64_t b = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) b = key[e] > b ? key[e] : b;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t x = shfl_xor_u64(b, o);
            b = x > b ? x : b;
        }
        if (lane == 0) atomicMax(&sh_best, (unsigned long long)b);
        __syncthreads();
        if (t == 0) out[0] = int32_t(0xFFFFFFFFu - uint32_t(sh_best));
        return;
    }

    const int k = (cfg.top_k > 0 && cfg.top_k < n) ? cfg.top_k : n;
    uint64_t v = 0ull;  // small path: lane j of wave 0 holds the j-th largest key
    const bool small = topk_sorted<E>(key, per, k, S, sample_keys, v);
    if (wave != 0) return;

    // ---- probabilities in double (sampling.hpp:91-99), one wave; lanes compute the terms of a chunk of 64 in
    // parallel, the sums add them in sorted order like the reference's loops.
    auto key_of = [&](int base) -> uint64_t {  // this lane's key of the chunk starting at `base`
        if (small) return v;
        return base + lane < k ? sample_keys[base + lane] : 0ull;
    };
    const double inv_t = 1.0 / double(cfg.temperature);
    const double mx = double(ord_val(uint32_t((small ? readlane_u64(v, 0) : sample_keys[0]) >> 32)));
    auto weight = [&](uint64_t kv, int i) -> double {
        return i < k ? exp((double(ord_val(uint32_t(kv >> 32))) - mx) * inv_t) : 0.0;
    };
    // Sequential sums in sorted order over chunks of 64: the lanes put a chunk's terms in LDS and every lane adds
    // them in order from broadcast reads, continuing `run`; lane j keeps the running sum through term j of the
    // chunk. Only the chunk's cnt terms below k are added (past-the-end terms are +0.0 and would leave the sum of
    // non-negative terms unchanged); lanes from cnt on keep 0, and no reader looks at them.
    auto seq_chunk = [&](double x, double &run, int cnt) -> double {
        wave_lds_sync();
        sd[lane] = x;
        wave_lds_sync();
        double pre = 0.0;
#pragma unroll 8
        for (int j = 0; j < cnt; ++j) {
            run += sd[j];
            pre = lane == j ? run : pre;
        }
        return pre;
    };
    double sum = 0.0, w0 = 0.0;  // w0: this lane's term of the first chunk, reused by its prefix sums
    for (int base = 0; base < k; base += 64) {
        const double w = weight(key_of(base), base + lane);
        if (base == 0) w0 = w;
        (void)seq_chunk(w, sum, min(64, k - base));
    }
    // Running sums of the normalized terms, continued from `run`: lane j of the chunk gets the sum through term
    // base + j. These are the reference's top-p sum `c` and inverse-CDF sum `acc` (both start at 0 and add
    // probs[i] in order), and the top-p total is the running sum at the last kept term.
    auto prefix_chunk = [&](int base, double &run) -> double {
        return seq_chunk((base == 0 ? w0 : weight(key_of(base), base + lane)) / sum, run, min(64, k - base));
    };
    const bool use_p = cfg.top_p > 0.0f && cfg.top_p < 1.0f;
    int keep = k;
    double tot = 0.0, pre0 = 0.0, run0 = 0.0;  // chunk 0's running sums and the sum after it, reused below
    {
        double run = 0.0;
        for (int base = 0; base < k; base += 64) {
            const double pre = prefix_chunk(base, run);
            if (base == 0) { pre0 = pre; run0 = run; }
            const uint64_t m = use_p ? __ballot(base + lane < k && pre >= double(cfg.top_p)) : 0ull;
            if (m) {
                const int j = __ffsll((long long)m) - 1;
                keep = base + j + 1;
                tot = readlane_d(pre, j);
                break;
            }
            if (base + 64 >= k) tot = readlane_d(pre, k - 1 - base);
        }
    }
    const float u = det_uniform(cfg.key0, cfg.key1, cfg.frame, cfg.cb, cfg.draw);
    const double target = double(u) * tot;
    int pick = keep - 1;
    {
        double run = run0;
        for (int base = 0; base < keep; base += 64) {
            const double pre = base == 0 ? pre0 : prefix_chunk(base, run);
            const uint64_t m = __ballot(base + lane < keep && target < pre);
            if (m) { pick = base + __ffsll((long long)m) - 1; break; }
        }
    }
    const uint64_t kp = small ? readlane_u64(v, pick) : sample_keys[pick];
    if (lane == 0) out[0] = int32_t(0xFFFFFFFFu - uint32_t(kp));
}

}  // namespace vh
