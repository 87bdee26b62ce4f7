// vh_codec.hpp — Qwen3-TTS codec decoder kernels besides the GEMMs (qwen3.cpp:80-161, :366-481; the Vulkan shaders
// snake / hist / dwconv / ola / ringput / attnw of gpu_codec.cpp): streaming histories, the causal depthwise conv,
// the transposed conv's overlap-add with its tail (and the Snake of its output), the pre-transformer's RoPE + ring
// append and sliding-window attention over the ring, layer-scaled residual adds and the final clamp. The other Snakes
// are GEMM epilogues (EPI_SNAKE, EPI_ACC_SNAKE). Activations are time-major f32 rows.
#pragma once
#include "vh_common.hpp"
#include "vh_types.hpp"

namespace vh {

// A streaming history after a call of T rows: the last ctx rows of [old (ctx rows); x (T rows, stride ldx)] into
// dst (another buffer than old). qwen3.cpp:120, :136.
__global__ __launch_bounds__(256) void k_hist_shift(float *__restrict__ dst, const float *__restrict__ old,
                                                    const float *__restrict__ x, int64_t ldx, int32_t T, int32_t ctx,
                                                    int32_t C) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(ctx) * C) return;
    const int j = int(i / C), c = int(i % C), r = j + T;  // row r of the extended sequence
    dst[i] = r < ctx ? old[int64_t(r) * C + c] : x[int64_t(r - ctx) * ldx + c];
}

// dwconv_stream (qwen3.cpp:123-137): y[t][c] = b[c] + sum_k w[c][k] ext[t + k][c] over ext = [hist (K - 1 rows); x],
// taps in order. One thread per output.
// hist_next (may be null): also written, the next call's history (k_hist_shift's rows) by threads i < (K - 1) C.
__global__ __launch_bounds__(256) void k_dwconv_causal(const float *__restrict__ x, const float *__restrict__ hist,
                                                       const float *__restrict__ w, const float *__restrict__ b,
                                                       float *__restrict__ y, int32_t T, int32_t C, int32_t K,
                                                       float *__restrict__ hist_next) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (hist_next && i < int64_t(K - 1) * C) {
        const int j = int(i / C), c = int(i % C), r = j + T;  // row r of [hist; x]
        hist_next[i] = r < K - 1 ? hist[int64_t(r) * C + c] : x[int64_t(r - (K - 1)) * C + c];
    }
    if (i >= int64_t(T) * C) return;
    const int t = int(i / C), c = int(i % C), ctx = K - 1;
    float acc = b[c];
    for (int k = 0; k < K; ++k) {
        const int r = t + k;
        const float v = r < ctx ? hist[int64_t(r) * C + c] : x[int64_t(r - ctx) * C + c];
        acc += w[int64_t(c) * K + k] * v;
    }
    y[i] = acc;
}

// trans_stream's overlap-add (qwen3.cpp:139-161) from the GEMM output tmp [T][K co] (row k co + o of frame t): output
// row p (of T s + K - s) takes frame p / s at tap p % s and frame p / s - 1 at tap p % s + s (K <= 2 s), plus the old
// tail's row p; rows below T s go to y with the bias, the rest to the new tail (another buffer than the old one).
// sy, when set: Snake(y) (per-channel sa, sib) of those rows too, the first residual unit's input.
__global__ __launch_bounds__(256) void k_ola(const float *__restrict__ tmp, const float *__restrict__ tail_old,
                                             float *__restrict__ tail_new, const float *__restrict__ bias,
                                             float *__restrict__ y, int32_t T, int32_t s, int32_t K, int32_t co,
                                             float *__restrict__ sy, const float *__restrict__ sa, const float *__restrict__ sib) {
    const int tr = K - s;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= (int64_t(T) * s + tr) * co) return;
    const int64_t p = i / co;
    const int o = int(i % co);
    const int64_t t = p / s;
    const int k = int(p - t * s);
    float v = p < tr ? tail_old[p * co + o] : 0.f;
    if (t < T && k < K) v += tmp[(t * K + k) * co + o];
    if (t >= 1 && k + s < K) v += tmp[((t - 1) * K + k + s) * co + o];
    if (p < int64_t(T) * s) {
        const float yv = v + bias[o];
        y[p * co + o] = yv;
        if (sy) {
            const float sn = sinf(yv * sa[o]);
            sy[p * co + o] = yv + sib[o] * sn * sn;
        }
    } else {
        tail_new[(p - int64_t(T) * s) * co + o] = v;
    }
}

// nn::ConvT's overlap-add with padding (nn.cpp:217-245) in gather form, from the GEMM output z [T][K co] (row k co + o
// of input frame t): output row r of To takes z[t][r + pad - t s] for every frame t with 0 <= r + pad - t s < K, summed
// in increasing t (the order the reference adds them in), then the bias (or nothing). One thread per output element.
__global__ __launch_bounds__(256) void k_convt_gather(const float *__restrict__ z, const float *__restrict__ bias,
                                                      float *__restrict__ y, int32_t T, int32_t To, int32_t s, int32_t K,
                                                      int32_t pad, int32_t co) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(To) * co) return;
    const int64_t r = i / co;
    const int o = int(i - r * co);
    const int64_t q = r + pad;
    const int64_t lo_num = q - K + 1;
    const int64_t t_lo = lo_num <= 0 ? 0 : (lo_num + s - 1) / s;
    const int64_t t_hi = min(int64_t(T) - 1, q / s);
    float v = 0.f;
    for (int64_t t = t_lo; t <= t_hi; ++t) v += z[(t * K + (q - t * s)) * co + o];
    y[i] = bias ? v + bias[o] : v;
}

// The pre-transformer's q / k rotation (rope_apply, kernels.cpp:740-757: pairs (d, d + hd / 2)) with the host table
// rope [F][hd / 2][2] of positions pos0 + i, and the append of row i's keys and values to ring slot (pos0 + i) % R of
// the layer's f32 ring [R][kv_heads hd]. grid F, block 256; qkv rows [F][ld] = q | k | v; the call's first position
// pos0 is read from device memory (*pos), so a captured call replays at any position.
__global__ __launch_bounds__(256) void k_codec_rope_ring(float *__restrict__ qkv, int32_t ld, int32_t heads, int32_t kvh,
                                                         int32_t hd, const float *__restrict__ rope,
                                                         float *__restrict__ ring_k, float *__restrict__ ring_v,
                                                         int32_t R, const int64_t *__restrict__ pos) {
    const int i = blockIdx.x, half = hd / 2, qd = heads * hd, kd = kvh * hd;
    const int64_t pos0 = *pos;
    float *row = qkv + int64_t(i) * ld;
    const float *cs = rope + int64_t(i) * hd;
    const int64_t slot = (pos0 + i) % R;
    for (int e = threadIdx.x; e < (heads + kvh) * half; e += 256) {
        const int h = e / half, d = e % half;
        float *p = h < heads ? row + h * hd : row + qd + (h - heads) * hd;
        const float a = p[d], b = p[d + half], c = cs[2 * d], s = cs[2 * d + 1];
        const float r0 = a * c - b * s, r1 = b * c + a * s;
        if (h < heads) {
            p[d] = r0;
            p[d + half] = r1;
        } else {
            float *kr = ring_k + slot * kd + (h - heads) * hd;
            kr[d] = r0;
            kr[d + half] = r1;
        }
    }
    for (int e = threadIdx.x; e < kd; e += 256) ring_v[slot * kd + e] = row[qd + kd + e];
}

// Sliding-window attention of row i (position pos0 + i) and head h over the ring (kernels.cpp:809-828 with the window
// of :814): keys of positions (p - W, p], scores scale (q . k), softmax, sum p v. One wave per (row, head): lanes take
// keys for the scores (a key row read as float4s) and head dimensions for the output (the value rows read across the
// wave, eight positions in flight). Ring slots advance from the first one without a division per position.
// W <= 1024, hd <= 128, hd % 4 == 0.
__global__ __launch_bounds__(64) void k_codec_attn(const float *__restrict__ qkv, int32_t ld, const float *__restrict__ ring_k,
                                                   const float *__restrict__ ring_v, int32_t R, int32_t heads, int32_t kvh,
                                                   int32_t hd, const int64_t *__restrict__ pos, int32_t W, float scale,
                                                   float *__restrict__ ao) {
    __shared__ float p[1024];
    __shared__ __align__(16) float q[128];
    const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, kd = kvh * hd, off = (h / (heads / kvh)) * hd;
    const int64_t pos0 = *pos;
    const int64_t last = pos0 + i, first = last - W + 1 > 0 ? last - W + 1 : 0;
    const int n = int(last - first + 1), s0 = int(first % R);
    for (int d = lane; d < hd; d += 64) q[d] = qkv[int64_t(i) * ld + h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (int j = lane; j < n; j += 64) {
        int slot = s0 + j;
        if (slot >= R) slot -= R;
        const f32x4 *kr = reinterpret_cast<const f32x4 *>(ring_k + int64_t(slot) * kd + off);
        const f32x4 *qv = reinterpret_cast<const f32x4 *>(q);
        float dot = 0.f;
        for (int d4 = 0; d4 < hd / 4; ++d4) {
            const f32x4 a = kr[d4], b = qv[d4];
            dot += b[0] * a[0] + b[1] * a[1] + b[2] * a[2] + b[3] * a[3];
        }
        p[j] = scale * dot;
        mx = fmaxf(mx, p[j]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    float sum = 0.f;
    for (int j = lane; j < n; j += 64) {
        p[j] = expf(p[j] - mx);
        sum += p[j];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, kWave);
    __syncthreads();
    const float inv = 1.0f / sum;
    for (int d = lane; d < hd; d += 64) {
        const float *vb = ring_v + off + d;
        float acc = 0.f;
        int slot = s0;
#pragma unroll 8
        for (int j = 0; j < n; ++j) {
            acc += p[j] * vb[int64_t(slot) * kd];
            if (++slot == R) slot = 0;
        }
        ao[int64_t(i) * heads * hd + h * hd + d] = acc * inv;
    }
}

// h += s[e] t over rows of H (the layer scales of kernels.cpp:830, :838: the projection scaled, then added).
__global__ __launch_bounds__(256) void k_scale_acc(float *__restrict__ h, const float *__restrict__ t,
                                                   const float *__restrict__ s, int64_t n, int32_t H) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    h[i] += t[i] * s[int(i % H)];
}

// The final clamp to [-1, 1] (qwen3.cpp:478).
__global__ __launch_bounds__(256) void k_clamp1(float *__restrict__ y, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    y[i] = fminf(1.0f, fmaxf(-1.0f, y[i]));
}

}  // namespace vh
