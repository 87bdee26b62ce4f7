// vh_lm.hpp — one CosyVoice2 LM sampling step on the device, and the speech-token embedding that feeds the next
// decode step.
//
// k_lm_sample restates, in one 512-thread block:
//   lm_logp (cosyvoice.cpp:598-607): mx = max v, sum = sum exp(double(v - mx)), lse = mx + float(log(sum)),
//     logp = v - lse (v = head output + bias);
//   the trial loop of lm_generate (cosyvoice.cpp:674-683): u0, u1 = DetRng(seed).uniform(i, stream, 2 trial [+ 1]),
//     ras_sample, repeat while i < min_len and the token is an end token, fail after trial 101;
//   ras_sample (cosyvoice.cpp:617-664): pr = exp(double(logp - mx2)) / sum over all n; the top_k largest pr in
//     descending order (ties by index); keep while cum < top_p and count < top_k; pick by u0 * ksum; when the pick
//     occurs at least win_size * tau_r times in the last win_size decoded tokens, set its logp to -inf and draw
//     from the whole distribution without it in index order with u1.
// Order keys: the sort key is d = float(logp - mx2), the value pr is computed from. pr is a non-decreasing function
// of d, so (d desc, index asc) orders like (pr desc, index asc) except where two different d give the same double
// pr; that needs |d| < 1e-9 at d != 0 (two tokens of probability > 0.98) or pr in the subnormal range (never
// reached by the keep loop for top_p < 1), so the kept list and the pick are the reference's.
// Sums: the keep and pick sums run sequentially in sorted order like the reference; the softmax totals and the
// index-order running sum of the resampling draw are block reductions / a blocked scan (double), which round
// differently from a sequential sum by a few ulps of a double.
//
// Element layout: blocked, thread t holds indices [t * per, t * per + per), per = ceil(n / 512), so the
// index-order scan is a per-thread running sum after a block scan of the thread totals.
#pragma once
#include "vh_topk.hpp"

namespace vh {

constexpr int kLmThreads = 512, kLmWaves = kLmThreads / 64;
constexpr int kLmE = kLmMaxN / kLmThreads;  // elements per thread at the largest n

VH_DEV double shfl_xor_d(double v, int m) { return __longlong_as_double(int64_t(shfl_xor_u64(uint64_t(__double_as_longlong(v)), m))); }
// Butterfly sum: every lane gets the bitwise same total.
VH_DEV double wave_sum_d(double v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += shfl_xor_d(v, o);
    return v;
}
// Block reductions for kLmThreads threads; red holds kLmWaves entries. All threads return the same value.
VH_DEV float lm_block_max(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < kLmWaves; ++i) m = fmaxf(m, red[i]);
    return m;
}
VH_DEV double lm_block_sum(double v, double *red) {
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < kLmWaves; ++i) s += red[i];
    return s;
}
// Exclusive prefix of v over threads in thread order.
VH_DEV double lm_block_excl_scan(double v, double *red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double x = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += x;
    }
    double excl = __shfl_up(incl, 1, kWave);
    if (lane == 0) excl = 0.0;
    __syncthreads();
    if (lane == 63) red[w] = incl;
    __syncthreads();
    double off = 0.0;
    for (int i = 0; i < w; ++i) off += red[i];
    return off + excl;
}


// logits [n] (head + bias) -> one generation step. st: step i, decoded count, done; decoded [n_dec] history.
// logp_out (optional): the log-probabilities of lm_logp at logp_out + i * logp_stride. append: push a non-end
// token to decoded and advance the step (the generation loop); else only st->last is written.
__global__ __launch_bounds__(kLmThreads) void k_lm_sample(const float *__restrict__ logits, int32_t n,
                                                              const LmCfgDev *__restrict__ cfgp, LmState *st,
                                                              int32_t *decoded, float *logp_out, int64_t logp_stride,
                                                              int32_t append) {
    __shared__ __align__(16) uint64_t keys[kLmMaxK];
    __shared__ TopkSmem S;
    __shared__ float redf[kLmWaves];
    __shared__ double redd[kLmWaves];
    __shared__ double sq[kLmMaxK];             // sorted pr
    __shared__ int sidx[kLmMaxK], swin[kLmMaxK];  // sorted indices; decoded window
    __shared__ int sh_top, sh_resample, sh_found;
    __shared__ double sh_s2;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const LmState s0 = *st;
    const LmCfgDev cfg = *cfgp;
    if (s0.done) return;
    if (s0.step >= cfg.max_len) {  // past the last step of the loop
        if (t == 0) st->done = 1;
        return;
    }
    const int per = (n + kLmThreads - 1) / kLmThreads;
    const int i0 = t * per;
    float lp[kLmE];
#pragma unroll
    for (int e = 0; e < kLmE; ++e) lp[e] = (e < per && i0 + e < n) ? logits[i0 + e] : -INFINITY;
    if (t < 256) S.hist[t] = 0u;

    // ---- lm_logp
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < kLmE; ++e) mx = fmaxf(mx, lp[e]);
    mx = lm_block_max(mx, redf);
    double sum = 0.0;
#pragma unroll
    for (int e = 0; e < kLmE; ++e)
        if (e < per && i0 + e < n) sum += exp(double(lp[e] - mx));
    sum = lm_block_sum(sum, redd);
    const float lse = mx + float(log(sum));
#pragma unroll
    for (int e = 0; e < kLmE; ++e) lp[e] = lp[e] - lse;  // past-the-end entries stay -inf
    if (logp_out) {
        float *o = logp_out + int64_t(s0.step) * logp_stride;
#pragma unroll
        for (int e = 0; e < kLmE; ++e)
            if (e < per && i0 + e < n) o[i0 + e] = lp[e];
    }

    const int k = cfg.top_k < n ? cfg.top_k : n;
    const int from = s0.n_dec > cfg.win_size ? s0.n_dec - cfg.win_size : 0;
    const double rep_need = double(cfg.win_size) * double(cfg.tau_r);
    int result = -1, status = 0;
    for (int trial = 0;; ++trial) {
        const float u0 = det_uniform(cfg.key0, cfg.key1, uint64_t(s0.step), cfg.stream, uint32_t(2 * trial));
        const float u1 = det_uniform(cfg.key0, cfg.key1, uint64_t(s0.step), cfg.stream, uint32_t(2 * trial + 1));
        // ---- ras_sample: softmax over all n in double
        float mx2 = -INFINITY;
#pragma unroll
        for (int e = 0; e < kLmE; ++e) mx2 = fmaxf(mx2, lp[e]);
        mx2 = lm_block_max(mx2, redf);
        uint64_t key[kLmE];
        double sum2 = 0.0;
#pragma unroll
        for (int e = 0; e < kLmE; ++e) {
            const bool in = e < per && i0 + e < n;
            const float d = lp[e] - mx2;
            sum2 += in ? exp(double(d)) : 0.0;
            key[e] = in ? (uint64_t(ord_key(d)) << 32 | uint64_t(0xFFFFFFFFu - uint32_t(i0 + e))) : 0ull;
        }
        sum2 = lm_block_sum(sum2, redd);
        // pr of element e (ras_sample's normalized term)
        auto pr = [&](int e) -> double { return exp(double(lp[e] - mx2)) / sum2; };
        if (t == 0) topk_reset(S);
        __syncthreads();
        uint64_t v = 0ull;
        const bool small = topk_sorted<kLmE>(key, per, k, S, keys, v);
        // the sorted terms (pr, index) and the decoded window into LDS, then one thread runs the reference's
        // sequential keep / pick loops over them (k is small: the loop costs less than a parallel scan's sync)
        if (wave == 0) {
            for (int base = 0; base < k; base += 64) {
                const uint64_t kv = small ? v : (base + lane < k ? keys[base + lane] : 0ull);
                if (base + lane < k) {
                    sq[base + lane] = exp(double(ord_val(uint32_t(kv >> 32)))) / sum2;
                    sidx[base + lane] = int(0xFFFFFFFFu - uint32_t(kv));
                }
            }
            for (int j = lane; j < s0.n_dec - from; j += 64) swin[j] = decoded[from + j];
        }
        __syncthreads();
        if (t == 0) {
            int nkeep = 0;
            double cum = 0.0;
            while (nkeep < k && cum < double(cfg.top_p)) cum += sq[nkeep++];  // keep while cum < top_p, < top_k
            double ksum = 0.0;
            for (int j = 0; j < nkeep; ++j) ksum += sq[j];
            const double target = double(u0) * ksum;
            int top = sidx[nkeep - 1];
            double acc = 0.0;
            for (int j = 0; j < nkeep; ++j) {
                acc += sq[j];
                if (target < acc) { top = sidx[j]; break; }
            }
            int rep = 0;
            for (int j = 0; j < s0.n_dec - from; ++j) rep += swin[j] == top;
            sh_top = top;
            sh_resample = double(rep) >= rep_need;
            sh_found = 0x7FFFFFFF;
        }
        __syncthreads();
        const int top = sh_top;
        result = top;
        if (sh_resample) {
            // draw without top over the whole distribution in index order (u1): blocked running sums
            double p[kLmE];
            double loc = 0.0;
#pragma unroll
            for (int e = 0; e < kLmE; ++e) {
                p[e] = (e < per && i0 + e < n && i0 + e != top) ? pr(e) : 0.0;
                loc += p[e];
            }
            const double pre = lm_block_excl_scan(loc, redd);
            double a = pre;
            const int last_i = n - 1;
#pragma unroll
            for (int e = 0; e < kLmE; ++e)
                a += p[e];
            if (i0 <= last_i && last_i < i0 + per) sh_s2 = a;  // the running sum at the last index: s2
            __syncthreads();
            const double t2 = double(u1) * sh_s2;
            a = pre;
            int found = 0x7FFFFFFF;
#pragma unroll
            for (int e = 0; e < kLmE; ++e) {
                const int idx = i0 + e;
                if (e < per && idx < n && idx != top) {
                    a += p[e];
                    if (t2 < a && found == 0x7FFFFFFF) found = idx;
                }
            }
            if (found != 0x7FFFFFFF) atomicMin(&sh_found, found);
            // the pick's log-probability stays -inf for the next trials (ras_sample modifies logp)
#pragma unroll
            for (int e = 0; e < kLmE; ++e)
                if (i0 + e == top && e < per) lp[e] = -INFINITY;
            __syncthreads();
            result = sh_found != 0x7FFFFFFF ? sh_found : (top == n - 1 ? n - 2 : n - 1);
        }
        if (s0.step >= cfg.min_len || result < cfg.speech_tokens) break;
        if (trial >= cfg.max_trials) { status = 1; break; }
        __syncthreads();  // sh_* are rewritten by the next trial
    }
    if (t == 0) {
        st->last = result;
        if (status) {
            st->status = 1;
            st->done = 1;
        } else if (append) {
            if (result >= cfg.speech_tokens) {
                st->done = 1;
            } else {
                decoded[s0.n_dec] = result;
                st->n_dec = s0.n_dec + 1;
                st->step = s0.step + 1;
            }
        }
    }
}

// The embedding of the token the sampler just appended (mat_gather, kernels.cpp:468-471) into x [cols], and the
// decode row advanced to the next position: rows[0].pos + 1 with its RoPE row copied from the table. After the
// end of the generation the row goes to spare_pos instead (a cache slot the generation never uses), so the rest
// of the step writes nothing the generation keeps. Grid 1, block 256.
// Row r of an embedding of any weight type, widened as mat_gather does (kernels.cpp:432-471), into x [cols];
// the block's threads take the columns in turn.
VH_DEV void gather_row(const uint8_t *w, const void *scale, int type, int s16, int64_t cols, int64_t r, float *x) {
    const int64_t nb = cols / 32;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        float v;
        switch (type) {
            case WT_F32: v = reinterpret_cast<const float *>(w)[r * cols + c]; break;
            case WT_F16: v = float(reinterpret_cast<const _Float16 *>(w)[r * cols + c]); break;
            case WT_BF16: v = bf16_to_f32(reinterpret_cast<const uint16_t *>(w)[r * cols + c]); break;
            case WT_Q8: v = float(int8_t(w[r * cols + c])) * static_cast<const float *>(scale)[r * nb + c / 32]; break;
            default: {  // Q4: 16 bytes per 32-block, byte j = w[j] | w[j + 16] << 4, value (u - 8) * scale
                const int64_t b = c / 32, j = c % 32;
                const uint8_t u = w[r * (cols / 2) + b * 16 + (j & 15)];
                const int q = int(j < 16 ? (u & 15) : (u >> 4)) - 8;
                const float sc = s16 ? float(static_cast<const _Float16 *>(scale)[r * nb + b]) : static_cast<const float *>(scale)[r * nb + b];
                v = float(q) * sc;
            }
        }
        x[c] = v;
    }
}

// mat_gather (kernels.cpp:468-471) of n rows: block i widens row ids[i] of the matrix into out + i cols. The host
// checks every id against the row count before the launch. Grid n, block 256.
__global__ __launch_bounds__(256) void k_mat_gather(const uint8_t *w, const void *scale, int type, int s16, int64_t cols,
                                                    const int32_t *ids, float *out) {
    gather_row(w, scale, type, s16, cols, ids[blockIdx.x], out + int64_t(blockIdx.x) * cols);
}

// A pass of the code-predictor frame loop (gpu_vulkan.cpp:1004-1017): its rows at positions pos0 .. pos0 + m - 1
// with their RoPE rows from the table, and, after the first pass, the embedding row of the code just sampled
// (mat_gather of backend_qwen3.cpp:411). A code outside the embedding sets *err (check_id in the reference) and
// leaves x as it was. Grid 1, block 256.
__global__ __launch_bounds__(256) void k_pred_embed(PredEmbedArgs a) {
    for (int i = threadIdx.x; i < a.m; i += 256) {
        RowRef r = a.base;
        r.pos = a.base.pos + i;
        a.row[i] = r;
    }
    for (int j = threadIdx.x; j < a.m * a.hd; j += 256) a.rope_row[j] = a.rope[a.base.pos * a.hd + j];
    if (!a.w) return;
    const int64_t r = a.codes[a.code_idx];
    if (r < 0 || r >= a.rows) {
        if (threadIdx.x == 0) *a.err = 1;
        return;
    }
    gather_row(a.w, a.scale, a.type, a.s16, a.cols, r, a.x);
}

__global__ __launch_bounds__(256) void k_lm_embed(LmEmbedArgs a) {
    const LmState s = *a.st;
    const int64_t pos0 = a.row->pos;
    __syncthreads();
    const int64_t pos = s.done ? a.spare_pos : pos0 + 1;
    if (threadIdx.x == 0) a.row->pos = pos;
    for (int j = threadIdx.x; j < a.hd; j += 256) a.rope_row[j] = a.rope[pos * a.hd + j];
    if (s.done) return;
    const int64_t r = a.decoded[s.n_dec - 1];
    if (r < 0 || r >= a.rows) return;
    gather_row(a.w, a.scale, a.type, a.s16, a.cols, r, a.x);
}

}  // namespace vh
