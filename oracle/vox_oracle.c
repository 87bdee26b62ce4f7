/*
 * vox_oracle.c — CPU restatement of the reference hot path (see vox_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker, never the product. Built with
 * -ffp-contract=off; explicit fmaf() marks the places where the reference's
 * AVX2/FMA code paths fuse.
 */
#define _GNU_SOURCE
#include "vox_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ threads */
static int g_threads = 1;
void vo_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int vo_get_threads(void) { return g_threads; }

typedef void (*vo_range_fn)(void *ctx, int64_t r0, int64_t r1);
typedef struct { vo_range_fn fn; void *ctx; int64_t r0, r1; } vo_job;
static void *vo_job_run(void *p) { vo_job *j = (vo_job *)p; j->fn(j->ctx, j->r0, j->r1); return NULL; }

/* Splits [0, total) into contiguous ranges, one per thread. Each output row is computed by exactly one
 * thread with a fixed operation order, so results do not depend on the thread count (as kernels.cpp:681-685). */
static void vo_parallel_rows(int64_t total, vo_range_fn fn, void *ctx) {
    int nt = g_threads;
    if (nt <= 1 || total < 64) { fn(ctx, 0, total); return; }
    if (nt > 64) nt = 64;
    pthread_t th[64];
    vo_job jobs[64];
    const int64_t per = (total + nt - 1) / nt;
    int started = 0;
    for (int t = 0; t < nt; ++t) {
        int64_t a = (int64_t)t * per, b = a + per < total ? a + per : total;
        if (a >= b) break;
        jobs[t].fn = fn; jobs[t].ctx = ctx; jobs[t].r0 = a; jobs[t].r1 = b;
        if (t == 0) continue;
        if (pthread_create(&th[t], NULL, vo_job_run, &jobs[t]) != 0) { fn(ctx, a, b); jobs[t].fn = NULL; }
        started = t;
    }
    fn(ctx, jobs[0].r0, jobs[0].r1);
    for (int t = 1; t <= started; ++t) if (jobs[t].fn) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------ Philox / DetRng (sampling.hpp:16-50) */
void vo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        if (round < 9) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float vo_uniform(uint64_t seed, uint64_t frame, uint32_t codebook, uint32_t draw) {
    const uint32_t ctr[4] = {(uint32_t)frame, (uint32_t)(frame >> 32), codebook, draw};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t r[4];
    vo_philox4x32_10(ctr, key, r);
    return (float)(r[0] >> 8) * (1.0f / 16777216.0f);
}

void vo_noise(uint64_t seed, uint32_t stream, size_t n, float *out) {
    const double two_pi = 2.0 * 3.14159265358979323846;
    for (size_t p = 0; p < (n + 1) / 2; ++p) {
        const double u1 = (double)vo_uniform(seed, p, stream, 0), u2 = (double)vo_uniform(seed, p, stream, 1);
        const double r = sqrt(-2.0 * log(1.0 - u1));
        const double a = two_pi * u2;
        out[2 * p] = (float)(r * cos(a));
        if (2 * p + 1 < n) out[2 * p + 1] = (float)(r * sin(a));
    }
}

/* ------------------------------------------------------------------ sample_logits (sampling.hpp:61-119) */
static const float *g_sort_vals;
/* strict total order: larger value first, lower index on equal values (sampling.hpp:83-85) */
static int vo_better_cmp(const void *pa, const void *pb) {
    const int32_t a = *(const int32_t *)pa, b = *(const int32_t *)pb;
    const float va = g_sort_vals[a], vb = g_sort_vals[b];
    if (va > vb) return -1;
    if (vb > va) return 1;
    if (va == vb) return a < b ? -1 : (a > b ? 1 : 0);
    return a < b ? -1 : 1; /* NaN: keep index order (unordered in the reference) */
}

int32_t vo_sample_logits(float *l, int32_t n, float temperature, float top_p, int32_t top_k,
                         float repetition_penalty, const int32_t *history, int32_t n_history, float u) {
    if (n <= 0) return -1;
    if (history && repetition_penalty != 1.0f) {
        uint8_t *seen = (uint8_t *)calloc((size_t)n, 1);
        for (int32_t i = 0; i < n_history; ++i) {
            const int32_t t = history[i];
            if (t >= 0 && t < n && !seen[t]) {
                seen[t] = 1;
                l[t] = l[t] > 0 ? l[t] / repetition_penalty : l[t] * repetition_penalty;
            }
        }
        free(seen);
    }
    if (temperature <= 0.0f) { /* greedy: first maximum (std::max_element) */
        int32_t best = 0;
        for (int32_t i = 1; i < n; ++i) if (l[best] < l[i]) best = i;
        return best;
    }
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    for (int32_t i = 0; i < n; ++i) idx[i] = i;
    g_sort_vals = l;
    qsort(idx, (size_t)n, sizeof(int32_t), vo_better_cmp); /* sorted prefix == partial_sort prefix (total order) */
    const int32_t k = (top_k > 0 && top_k < n) ? top_k : n;
    double *probs = (double *)malloc(sizeof(double) * (size_t)k);
    const double inv_t = 1.0 / (double)temperature;
    const double mx = (double)l[idx[0]];
    double sum = 0;
    for (int32_t i = 0; i < k; ++i) { probs[i] = exp(((double)l[idx[i]] - mx) * inv_t); sum += probs[i]; }
    for (int32_t i = 0; i < k; ++i) probs[i] /= sum;
    int32_t keep = k;
    if (top_p > 0.0f && top_p < 1.0f) {
        double c = 0;
        for (int32_t i = 0; i < k; ++i) { c += probs[i]; if (c >= (double)top_p) { keep = i + 1; break; } }
    }
    double total = 0;
    for (int32_t i = 0; i < keep; ++i) total += probs[i];
    const double target = (double)u * total;
    double acc = 0;
    int32_t pick = idx[keep - 1];
    for (int32_t i = 0; i < keep; ++i) { acc += probs[i]; if (target < acc) { pick = idx[i]; break; } }
    free(probs);
    free(idx);
    return pick;
}

/* ------------------------------------------------------------------ RAS sampler (cosyvoice.cpp:617-664) */
static const double *g_sort_probs;
static int vo_prob_desc_cmp(const void *pa, const void *pb) {
    const int a = *(const int *)pa, b = *(const int *)pb;
    const double x = g_sort_probs[a], y = g_sort_probs[b];
    if (x > y) return -1;
    if (y > x) return 1;
    return a < b ? -1 : (a > b ? 1 : 0); /* equal: original order (std::stable_sort) */
}

int32_t vo_ras_sample(float *logp, int32_t n, const int32_t *decoded, int32_t n_decoded, float top_p, int32_t top_k,
                      int32_t win_size, float tau_r, float u0, float u1) {
    float mx = -INFINITY;
    for (int32_t i = 0; i < n; ++i) mx = mx < logp[i] ? logp[i] : mx; /* std::max(mx, v) */
    double *pr = (double *)malloc(sizeof(double) * (size_t)n);
    double sum = 0;
    for (int32_t i = 0; i < n; ++i) { pr[i] = exp((double)(logp[i] - mx)); sum += pr[i]; }
    for (int32_t i = 0; i < n; ++i) pr[i] /= sum;
    int *idx = (int *)malloc(sizeof(int) * (size_t)n);
    for (int32_t i = 0; i < n; ++i) idx[i] = i;
    g_sort_probs = pr;
    qsort(idx, (size_t)n, sizeof(int), vo_prob_desc_cmp);
    int32_t nkeep = 0;
    double cum = 0, ksum = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (cum < (double)top_p && nkeep < top_k) { cum += pr[idx[i]]; ++nkeep; }
        else break;
    }
    for (int32_t i = 0; i < nkeep; ++i) ksum += pr[idx[i]];
    int32_t top = idx[nkeep - 1];
    double acc = 0;
    const double target = (double)u0 * ksum;
    for (int32_t i = 0; i < nkeep; ++i) { acc += pr[idx[i]]; if (target < acc) { top = idx[i]; break; } }
    int rep = 0;
    const int32_t from = n_decoded > win_size ? n_decoded - win_size : 0;
    for (int32_t i = from; i < n_decoded; ++i) rep += decoded[i] == top;
    int32_t result = top;
    if ((double)rep >= (double)win_size * (double)tau_r) {
        logp[top] = -INFINITY;
        double s2 = 0;
        for (int32_t i = 0; i < n; ++i) s2 += i == top ? 0.0 : pr[i];
        const double t2 = (double)u1 * s2;
        double a2 = 0;
        int32_t last = top == 0 ? 1 : 0;
        result = -1;
        for (int32_t i = 0; i < n; ++i) {
            if (i == top) continue;
            last = i;
            a2 += pr[i];
            if (t2 < a2) { result = i; break; }
        }
        if (result < 0) result = last;
    }
    free(idx);
    free(pr);
    return result;
}

/* lm_logp (cosyvoice.cpp:598-607) after the head and bias */
void vo_lm_logp(float *v, int32_t n) {
    float mx = -INFINITY;
    for (int32_t i = 0; i < n; ++i) mx = mx < v[i] ? v[i] : mx;
    double sum = 0;
    for (int32_t i = 0; i < n; ++i) sum += exp((double)(v[i] - mx));
    const float lse = mx + (float)log(sum);
    for (int32_t i = 0; i < n; ++i) v[i] -= lse;
}

/* the trial loop of lm_generate (cosyvoice.cpp:674-683) */
int32_t vo_lm_step(float *logp, int32_t n, const int32_t *decoded, int32_t n_decoded, int64_t step, int32_t min_len,
                   int32_t speech_tokens, float top_p, int32_t top_k, int32_t win_size, float tau_r, uint64_t seed,
                   uint32_t piece) {
    const uint32_t stream = 0x43560000u + piece;
    for (int trial = 0;; ++trial) {
        const float u0 = vo_uniform(seed, (uint64_t)step, stream, (uint32_t)(2 * trial));
        const float u1 = vo_uniform(seed, (uint64_t)step, stream, (uint32_t)(2 * trial + 1));
        const int32_t top = vo_ras_sample(logp, n, decoded, n_decoded, top_p, top_k, win_size, tau_r, u0, u1);
        if (step >= min_len || top < speech_tokens) return top;
        if (trial > 100) return -2;
    }
}

/* ------------------------------------------------------------------ formats */
float vo_f16_to_f32(uint16_t h) { /* exact widening incl. subnormals (kernels.hpp:63-75) */
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (e == 0) {
        if (man == 0) bits = sign;
        else {
            int shift = 0;
            while (!(man & 0x400u)) { man <<= 1; ++shift; }
            bits = sign | (uint32_t)(113 - shift) << 23 | (man & 0x3FFu) << 13;
        }
    } else if (e == 31) bits = sign | 0x7F800000u | man << 13;
    else bits = sign | (e + 112) << 23 | man << 13;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t vo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) { /* result subnormal or zero: scale by 2^24 and round to integer (nearest even) */
        float a;
        memcpy(&a, &ax, 4);
        const float s = a * 16777216.0f; /* exact: a < 2^-14 */
        return (uint16_t)(sign | (uint16_t)lrintf(s));
    }
    const uint32_t mant = ax & 0x7FFFFFu, e = (ax >> 23) - 112;
    uint32_t r = e << 10 | mant >> 13;
    const uint32_t rest = mant & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float vo_bf16_to_f32(uint16_t h) {
    const uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* mat_row (kernels.cpp:432-466) */
void vo_mat_row(const vo_mat *W, int64_t r, float *out) {
    const int64_t c = W->cols;
    switch (W->type) {
        case VO_F32: memcpy(out, (const float *)W->data + r * c, sizeof(float) * (size_t)c); break;
        case VO_F16: { const uint16_t *p = (const uint16_t *)W->data + r * c; for (int64_t i = 0; i < c; ++i) out[i] = vo_f16_to_f32(p[i]); } break;
        case VO_BF16: { const uint16_t *p = (const uint16_t *)W->data + r * c; for (int64_t i = 0; i < c; ++i) out[i] = vo_bf16_to_f32(p[i]); } break;
        case VO_Q8: {
            const int8_t *p = (const int8_t *)W->data + r * c;
            const float *s = W->scale + r * (c / 32);
            for (int64_t i = 0; i < c; ++i) out[i] = (float)p[i] * s[i / 32];
        } break;
        case VO_Q4: {
            const uint8_t *p = (const uint8_t *)W->data + r * (c / 2);
            const float *s = W->scale + r * (c / 32);
            for (int64_t b = 0; b < c / 32; ++b)
                for (int j = 0; j < 16; ++j) {
                    const uint8_t v = p[b * 16 + j];
                    out[b * 32 + j] = (float)((int)(v & 15) - 8) * s[b];
                    out[b * 32 + 16 + j] = (float)((int)(v >> 4) - 8) * s[b];
                }
        } break;
        default: break;
    }
}

/* quantize_q8 (kernels.cpp:918-929): scale max|x|/127, q = lround(w / s), half away from zero */
void vo_quantize_q8(const float *w, int64_t rows, int64_t cols, int8_t *q, float *scale) {
    const int64_t nb = cols / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const float *p = w + r * cols + b * 32;
            float mx = 0;
            for (int j = 0; j < 32; ++j) { const float a = fabsf(p[j]); mx = mx < a ? a : mx; }
            const float s = mx / 127.0f;
            scale[r * nb + b] = s;
            for (int j = 0; j < 32; ++j) q[r * cols + b * 32 + j] = s > 0 ? (int8_t)lroundf(p[j] / s) : 0;
        }
}

/* quantize_q4 (kernels.cpp:606-645): scale search d = mx / -t, t = 7 .. 9 step 0.25, then least squares */
void vo_quantize_q4(const float *w, int64_t rows, int64_t cols, uint8_t *q, float *scale) {
    const int64_t nb = cols / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const float *p = w + r * cols + b * 32;
            float mx = 0; /* signed value of largest magnitude, first one wins */
            for (int j = 0; j < 32; ++j) if (fabsf(p[j]) > fabsf(mx)) mx = p[j];
            /* best_err is a float as at kernels.cpp:616: each candidate's double error is rounded when stored (:629),
               and the later comparisons (:629, :638) widen that float back to double */
            float best_d = mx / -8.0f, best_err = INFINITY;
            int8_t best_q[32];
            memset(best_q, 0, sizeof best_q);
            if (mx != 0.0f)
                for (int k = 0; k <= 8; ++k) {
                    const float d = mx / -(7.0f + 0.25f * (float)k), inv = 1.0f / d;
                    int8_t qq[32];
                    double err = 0;
                    for (int j = 0; j < 32; ++j) {
                        float c = floorf(p[j] * inv + 8.5f);
                        c = c < 0.0f ? 0.0f : c;
                        c = c > 15.0f ? 15.0f : c;
                        qq[j] = (int8_t)((int)c - 8);
                        const double e = (double)p[j] - (double)qq[j] * (double)d;
                        err += e * e;
                    }
                    if (err < (double)best_err) { best_err = (float)err; best_d = d; memcpy(best_q, qq, 32); }
                }
            if (mx != 0.0f) {
                double num = 0, den = 0;
                for (int j = 0; j < 32; ++j) { num += (double)p[j] * best_q[j]; den += (double)best_q[j] * best_q[j]; }
                if (den > 0) {
                    const float d2 = (float)(num / den);
                    double err = 0;
                    for (int j = 0; j < 32; ++j) { const double e = (double)p[j] - (double)best_q[j] * (double)d2; err += e * e; }
                    if (err < (double)best_err) best_d = d2;
                }
            }
            scale[r * nb + b] = best_d;
            uint8_t *o = q + r * (cols / 2) + b * 16;
            for (int j = 0; j < 16; ++j) o[j] = (uint8_t)((uint8_t)(best_q[j] + 8) | (uint8_t)((best_q[j + 16] + 8) << 4));
        }
}

/* activation quantization of matmul_q8 / matmul_q4 (kernels.cpp:515-523, :582-590) */
void vo_quantize_act(const float *x, int64_t n, int8_t *xq, float *xs) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *p = x + b * 32;
        float mx = 0;
        for (int j = 0; j < 32; ++j) { const float a = fabsf(p[j]); mx = mx < a ? a : mx; } /* std::max(mx, a) */
        const float sc = mx / 127.0f, inv = sc > 0 ? 1.0f / sc : 0.0f;
        xs[b] = sc;
        for (int j = 0; j < 32; ++j) xq[b * 32 + j] = (int8_t)lrintf(p[j] * inv);
    }
}

/* ------------------------------------------------------------------ integer dots */
/* AVX2 dot (kernels.cpp:485-501): lane l of the 8-lane accumulator takes the exact int sum of block elements
 * 4l..4l+3 and fuses it with (ws * xs); the lanes are summed as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
static float q8dot_avx2_order(const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int64_t nb) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < nb; ++b) {
        const float c = ws[b] * xs[b];
        for (int l = 0; l < 8; ++l) {
            int s = 0;
            for (int t = 0; t < 4; ++t) s += (int)wq[b * 32 + 4 * l + t] * (int)xq[b * 32 + 4 * l + t];
            acc[l] = fmaf((float)s, c, acc[l]);
        }
    }
    return ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
}

/* scalar dot (kernels.cpp:475-483): s += float(acc) * ws * xs, left to right */
static float q8dot_scalar_order(const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int64_t nb) {
    float s = 0;
    for (int64_t b = 0; b < nb; ++b) {
        int acc = 0;
        for (int j = 0; j < 32; ++j) acc += (int)wq[b * 32 + j] * (int)xq[b * 32 + j];
        s += (float)acc * ws[b] * xs[b];
    }
    return s;
}

static void q4_unpack_block(const uint8_t *src, int8_t *dst) { /* kernels.hpp:46, kernels.cpp:557-562 */
    for (int j = 0; j < 16; ++j) { dst[j] = (int8_t)((int)(src[j] & 15) - 8); dst[j + 16] = (int8_t)((int)(src[j] >> 4) - 8); }
}

typedef struct {
    const vo_mat *W;
    const int8_t *xq;
    const float *xs;
    int64_t m;
    float *y;
    int avx2;
} vo_int_ctx;

static void q8_rows(void *p, int64_t r0, int64_t r1) {
    const vo_int_ctx *c = (const vo_int_ctx *)p;
    const int64_t rows = c->W->rows, cols = c->W->cols, nb = cols / 32;
    for (int64_t r = r0; r < r1; ++r) {
        const int8_t *wr = (const int8_t *)c->W->data + r * cols;
        const float *ws = c->W->scale + r * nb;
        const float bz = c->W->bias ? c->W->bias[r] : 0.0f;
        for (int64_t i = 0; i < c->m; ++i) {
            const float d = c->avx2 ? q8dot_avx2_order(wr, ws, c->xq + i * cols, c->xs + i * nb, nb)
                                    : q8dot_scalar_order(wr, ws, c->xq + i * cols, c->xs + i * nb, nb);
            c->y[i * rows + r] = d + bz;
        }
    }
}

static void q4_rows(void *p, int64_t r0, int64_t r1) {
    const vo_int_ctx *c = (const vo_int_ctx *)p;
    const int64_t rows = c->W->rows, cols = c->W->cols, nb = cols / 32;
    int8_t *wr = (int8_t *)malloc((size_t)cols);
    for (int64_t r = r0; r < r1; ++r) {
        const uint8_t *src = (const uint8_t *)c->W->data + r * (cols / 2);
        for (int64_t b = 0; b < nb; ++b) q4_unpack_block(src + b * 16, wr + b * 32);
        const float *ws = c->W->scale + r * nb;
        const float bz = c->W->bias ? c->W->bias[r] : 0.0f;
        for (int64_t i = 0; i < c->m; ++i) {
            const float d = c->avx2 ? q8dot_avx2_order(wr, ws, c->xq + i * cols, c->xs + i * nb, nb)
                                    : q8dot_scalar_order(wr, ws, c->xq + i * cols, c->xs + i * nb, nb);
            c->y[i * rows + r] = d + bz;
        }
    }
    free(wr);
}

static void int_path(const vo_mat *W, const float *x, int64_t m, float *y, int avx2, vo_range_fn fn) {
    const int64_t cols = W->cols, nb = cols / 32;
    int8_t *xq = (int8_t *)malloc((size_t)(m * cols));
    float *xs = (float *)malloc(sizeof(float) * (size_t)(m * nb));
    for (int64_t i = 0; i < m; ++i) vo_quantize_act(x + i * cols, cols, xq + i * cols, xs + i * nb);
    vo_int_ctx c = {W, xq, xs, m, y, avx2};
    vo_parallel_rows(W->rows, fn, &c);
    free(xq);
    free(xs);
}

void vo_matmul_q8_int(const vo_mat *W, const float *x, int64_t m, float *y, int avx2) { int_path(W, x, m, y, avx2, q8_rows); }
void vo_matmul_q4_int(const vo_mat *W, const float *x, int64_t m, float *y, int avx2) { int_path(W, x, m, y, avx2, q4_rows); }

/* ------------------------------------------------------------------ f32 tiles (kernels.cpp:230-251) */
/* One output: 8 lanes over k (lane = k % 8), reduced as ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)), tail added in
 * order; every tile shape of rows_block gives this order per output. Whether a lane step fuses depends on how
 * the reference compiles the path (g++ 11, -O3, checked bit for bit against oracle/_ref): the F16C path
 * (kernels.cpp:389-411, built under target("avx2,fma,f16c")) fuses; the target_clones paths for F32, BF16 and
 * dequantized Q8 (kernels.cpp:332, :413-415) multiply and add separately. */
static float tile_dot(const float *w, const float *x, int64_t cols, int fused) {
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 8 <= cols; k += 8)
        for (int l = 0; l < 8; ++l) {
            if (fused) v[l] = fmaf(w[k + l], x[k + l], v[l]);
            else { const float pr = w[k + l] * x[k + l]; v[l] = v[l] + pr; }
        }
    float s = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
    for (; k < cols; ++k) {
        if (fused) s = fmaf(w[k], x[k], s);
        else { const float pr = w[k] * x[k]; s = s + pr; }
    }
    return s;
}

typedef struct { const vo_mat *W; const float *x; int64_t m; float *y; } vo_f32_ctx;

static void f32_rows(void *p, int64_t r0, int64_t r1) {
    const vo_f32_ctx *c = (const vo_f32_ctx *)p;
    const int64_t rows = c->W->rows, cols = c->W->cols;
    float *wr = (float *)malloc(sizeof(float) * (size_t)cols);
    for (int64_t r = r0; r < r1; ++r) {
        vo_mat_row(c->W, r, wr); /* q8 m>8: float(q) * scale, as the dequant pass of kernels.cpp:665-674 */
        const float bz = c->W->bias ? c->W->bias[r] : 0.0f;
        for (int64_t i = 0; i < c->m; ++i) c->y[i * rows + r] = tile_dot(wr, c->x + i * cols, cols, c->W->type == VO_F16) + bz;
    }
    free(wr);
}

void vo_matmul_f32_tiles(const vo_mat *W, const float *x, int64_t m, float *y) {
    vo_f32_ctx c = {W, x, m, y};
    vo_parallel_rows(W->rows, f32_rows, &c);
}

/* matmul dispatcher (kernels.cpp:653-705) */
void vo_matmul(const vo_mat *W, const float *x, int64_t m, float *y, int avx2) {
    if (W->type == VO_Q8 && m <= 8) { vo_matmul_q8_int(W, x, m, y, avx2); return; }
    if (W->type == VO_Q4) { vo_matmul_q4_int(W, x, m, y, avx2); return; }
    vo_matmul_f32_tiles(W, x, m, y);
}

/* dot (kernels.cpp:268-274): 8 lanes, multiply then add (no FMA in the base x86-64 build) */
float vo_dot(const float *a, const float *b, int64_t n) {
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 8 <= n; k += 8)
        for (int l = 0; l < 8; ++l) { const float pr = a[k + l] * b[k + l]; v[l] = v[l] + pr; }
    float s = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
    for (; k < n; ++k) { const float pr = a[k] * b[k]; s = s + pr; }
    return s;
}

/* ------------------------------------------------------------------ elementwise (kernels.cpp:707-757) */
void vo_rmsnorm(const float *x, const float *w, int64_t n, float eps, float *out) {
    float ss = 0;
    for (int64_t i = 0; i < n; ++i) { const float sq = x[i] * x[i]; ss = ss + sq; }
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = w[i] * (x[i] * inv);
}

void vo_layernorm(const float *x, const float *w, const float *b, int64_t n, float eps, float *out) {
    double mean = 0;
    for (int64_t i = 0; i < n; ++i) mean += x[i];
    mean /= (double)n;
    double var = 0;
    for (int64_t i = 0; i < n; ++i) { const double d = x[i] - mean; var += d * d; }
    var /= (double)n;
    const float inv = (float)(1.0 / sqrt(var + (double)eps));
    const float fm = (float)mean;
    for (int64_t i = 0; i < n; ++i) out[i] = (x[i] - fm) * inv * w[i] + (b ? b[i] : 0.0f);
}

void vo_softmax(float *x, int64_t n) {
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) mx = mx < x[i] ? x[i] : mx;
    float sum = 0;
    for (int64_t i = 0; i < n; ++i) { x[i] = expf(x[i] - mx); sum += x[i]; }
    const float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; ++i) x[i] *= inv;
}

float vo_silu(float x) { return x / (1.0f + expf(-x)); }

void vo_rope_inv_freq(int64_t hd, double theta, float *out) {
    for (int64_t i = 0; i < hd / 2; ++i) out[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)hd));
}

void vo_rope_apply(float *x, int64_t heads, int64_t hd, const float *inv_freq, int64_t pos) {
    const int64_t half = hd / 2;
    float *cs = (float *)malloc(sizeof(float) * (size_t)half), *sn = (float *)malloc(sizeof(float) * (size_t)half);
    for (int64_t i = 0; i < half; ++i) {
        const float f = inv_freq[i] * (float)pos;
        cs[i] = cosf(f);
        sn[i] = sinf(f);
    }
    for (int64_t h = 0; h < heads; ++h) {
        float *p = x + h * hd;
        for (int64_t i = 0; i < half; ++i) {
            const float a = p[i], b = p[i + half];
            const float ac = a * cs[i], bs = b * sn[i], bc = b * cs[i], as = a * sn[i];
            p[i] = ac - bs;
            p[i + half] = bc + as;
        }
    }
    free(cs);
    free(sn);
}

/* ------------------------------------------------------------------ transformer (kernels.cpp:760-906) */
static float kv_round(float v, int f16) { return f16 ? vo_f16_to_f32(vo_f32_to_f16(v)) : v; }

/* One query row against keys [0, n) of a layer cache; writes oh[hd]. (kernels.cpp:809-828) */
static void attend(const float *qh, const float *K, const float *V, int64_t n, int64_t kd, int64_t off, int64_t hd, float scale,
                   float *sc, float *oh) {
    for (int64_t j = 0; j < n; ++j) sc[j] = scale * vo_dot(qh, K + j * kd + off, hd);
    vo_softmax(sc, n);
    for (int64_t e = 0; e < hd; ++e) oh[e] = 0;
    for (int64_t j = 0; j < n; ++j) {
        const float p = sc[j];
        const float *vj = V + j * kd + off;
        for (int64_t e = 0; e < hd; ++e) { const float pv = p * vj[e]; oh[e] = oh[e] + pv; }
    }
}

/* Layers [l0, l1) of transformer_forward (kernels.cpp:791-840) on the residual stream h [m][hidden], rows at
 * positions pos0.. (= kv->len); appends their keys/values but does not advance kv->len. */
static void run_layers(const vo_xfmr *w, vo_kv *kv, float *h, int64_t m, int32_t l0, int32_t l1) {
    const int64_t H = w->hidden, nh = w->heads, nkv = w->kv_heads, hd = w->head_dim, I = w->inter;
    const int64_t qd = nh * hd, kd = nkv * hd, group = nh / nkv;
    const int64_t pos0 = kv->len;
    const float scale = 1.0f / sqrtf((float)hd);
    float *xn = (float *)malloc(sizeof(float) * (size_t)(m * H));
    float *q = (float *)malloc(sizeof(float) * (size_t)(m * qd));
    float *k = (float *)malloc(sizeof(float) * (size_t)(m * kd));
    float *v = (float *)malloc(sizeof(float) * (size_t)(m * kd));
    float *ao = (float *)malloc(sizeof(float) * (size_t)(m * qd));
    float *o = (float *)malloc(sizeof(float) * (size_t)(m * H));
    float *g = (float *)malloc(sizeof(float) * (size_t)(m * I));
    float *u = (float *)malloc(sizeof(float) * (size_t)(m * I));
    float *d = (float *)malloc(sizeof(float) * (size_t)(m * H));
    float *sc = (float *)malloc(sizeof(float) * (size_t)(pos0 + m));
    for (int32_t li = l0; li < l1; ++li) {
        const vo_layer *L = &w->layers[li];
        float *K = kv->k + (int64_t)li * kv->cap * kd, *V = kv->v + (int64_t)li * kv->cap * kd;
        for (int64_t i = 0; i < m; ++i) vo_rmsnorm(h + i * H, L->ln1, H, w->eps, xn + i * H);
        vo_matmul(&L->q, xn, m, q, kv->avx2);
        vo_matmul(&L->k, xn, m, k, kv->avx2);
        vo_matmul(&L->v, xn, m, v, kv->avx2);
        for (int64_t i = 0; i < m; ++i) {
            float *qi = q + i * qd, *ki = k + i * kd;
            if (L->qn) for (int64_t hh = 0; hh < nh; ++hh) vo_rmsnorm(qi + hh * hd, L->qn, hd, w->eps, qi + hh * hd);
            if (L->kn) for (int64_t hh = 0; hh < nkv; ++hh) vo_rmsnorm(ki + hh * hd, L->kn, hd, w->eps, ki + hh * hd);
            vo_rope_apply(qi, nh, hd, w->inv_freq, pos0 + i);
            vo_rope_apply(ki, nkv, hd, w->inv_freq, pos0 + i);
        }
        for (int64_t i = 0; i < m; ++i)
            for (int64_t e = 0; e < kd; ++e) {
                K[(pos0 + i) * kd + e] = kv_round(k[i * kd + e], kv->kv_f16);
                V[(pos0 + i) * kd + e] = kv_round(v[i * kd + e], kv->kv_f16);
            }
        for (int64_t t = 0; t < m * nh; ++t) {
            const int64_t i = t / nh, hh = t % nh, gk = hh / group, last = pos0 + i;
            const int64_t first = w->window > 0 && last - w->window + 1 > 0 ? last - w->window + 1 : 0;
            attend(q + i * qd + hh * hd, K + first * kd, V + first * kd, last - first + 1, kd, gk * hd, hd, scale, sc,
                   ao + i * qd + hh * hd);
        }
        vo_matmul(&L->o, ao, m, o, kv->avx2);
        if (L->attn_scale)
            for (int64_t i = 0; i < m; ++i)
                for (int64_t e = 0; e < H; ++e) o[i * H + e] *= L->attn_scale[e];
        for (int64_t i = 0; i < m * H; ++i) h[i] += o[i];
        for (int64_t i = 0; i < m; ++i) vo_rmsnorm(h + i * H, L->ln2, H, w->eps, xn + i * H);
        vo_matmul(&L->gate, xn, m, g, kv->avx2);
        vo_matmul(&L->up, xn, m, u, kv->avx2);
        for (int64_t i = 0; i < m * I; ++i) g[i] = vo_silu(g[i]) * u[i];
        vo_matmul(&L->down, g, m, d, kv->avx2);
        if (L->mlp_scale)
            for (int64_t i = 0; i < m; ++i)
                for (int64_t e = 0; e < H; ++e) d[i * H + e] *= L->mlp_scale[e];
        for (int64_t i = 0; i < m * H; ++i) h[i] += d[i];
    }
    free(xn); free(q); free(k); free(v); free(ao); free(o); free(g); free(u); free(d); free(sc);
}

int vo_transformer_forward(const vo_xfmr *w, vo_kv *kv, const float *x_in, int64_t m, float *out_last, float *out_all) {
    const int64_t H = w->hidden;
    if (kv->len + m > kv->cap) return -1;
    float *h = (float *)malloc(sizeof(float) * (size_t)(m * H));
    memcpy(h, x_in, sizeof(float) * (size_t)(m * H));
    run_layers(w, kv, h, m, 0, w->n_layers);
    kv->len += m;
    if (out_last) vo_rmsnorm(h + (m - 1) * H, w->final_norm, H, w->eps, out_last);
    if (out_all) for (int64_t i = 0; i < m; ++i) vo_rmsnorm(h + i * H, w->final_norm, H, w->eps, out_all + i * H);
    free(h);
    return 0;
}

int vo_transformer_layers(const vo_xfmr *w, vo_kv *kv, const float *x_in, int64_t m, int32_t first, int32_t count, float *h_out) {
    if (kv->len + m > kv->cap || first < 0 || count < 0 || first + count > w->n_layers) return -1;
    memcpy(h_out, x_in, sizeof(float) * (size_t)(m * w->hidden));
    run_layers(w, kv, h_out, m, first, first + count);
    return 0;
}

int vo_transformer_forward_steps(const vo_xfmr *w, vo_kv *const *kvs, int64_t B, const float *x_in, float *out) {
    const int64_t H = w->hidden, nh = w->heads, nkv = w->kv_heads, hd = w->head_dim, I = w->inter;
    const int64_t qd = nh * hd, kd = nkv * hd, group = nh / nkv;
    int64_t maxn = 0;
    for (int64_t b = 0; b < B; ++b) {
        if (kvs[b]->len + 1 > kvs[b]->cap) return -1;
        if (kvs[b]->len + 1 > maxn) maxn = kvs[b]->len + 1;
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const int avx2 = kvs[0]->avx2;
    float *h = (float *)malloc(sizeof(float) * (size_t)(B * H));
    float *xn = (float *)malloc(sizeof(float) * (size_t)(B * H));
    float *q = (float *)malloc(sizeof(float) * (size_t)(B * qd));
    float *k = (float *)malloc(sizeof(float) * (size_t)(B * kd));
    float *v = (float *)malloc(sizeof(float) * (size_t)(B * kd));
    float *ao = (float *)malloc(sizeof(float) * (size_t)(B * qd));
    float *o = (float *)malloc(sizeof(float) * (size_t)(B * H));
    float *g = (float *)malloc(sizeof(float) * (size_t)(B * I));
    float *u = (float *)malloc(sizeof(float) * (size_t)(B * I));
    float *d = (float *)malloc(sizeof(float) * (size_t)(B * H));
    float *sc = (float *)malloc(sizeof(float) * (size_t)maxn);
    memcpy(h, x_in, sizeof(float) * (size_t)(B * H));
    for (int32_t li = 0; li < w->n_layers; ++li) {
        const vo_layer *L = &w->layers[li];
        for (int64_t i = 0; i < B; ++i) vo_rmsnorm(h + i * H, L->ln1, H, w->eps, xn + i * H);
        vo_matmul(&L->q, xn, B, q, avx2);
        vo_matmul(&L->k, xn, B, k, avx2);
        vo_matmul(&L->v, xn, B, v, avx2);
        for (int64_t i = 0; i < B; ++i) {
            float *qi = q + i * qd, *ki = k + i * kd;
            if (L->qn) for (int64_t hh = 0; hh < nh; ++hh) vo_rmsnorm(qi + hh * hd, L->qn, hd, w->eps, qi + hh * hd);
            if (L->kn) for (int64_t hh = 0; hh < nkv; ++hh) vo_rmsnorm(ki + hh * hd, L->kn, hd, w->eps, ki + hh * hd);
            vo_rope_apply(qi, nh, hd, w->inv_freq, kvs[i]->len);
            vo_rope_apply(ki, nkv, hd, w->inv_freq, kvs[i]->len);
            float *K = kvs[i]->k + (int64_t)li * kvs[i]->cap * kd, *V = kvs[i]->v + (int64_t)li * kvs[i]->cap * kd;
            for (int64_t e = 0; e < kd; ++e) {
                K[kvs[i]->len * kd + e] = kv_round(ki[e], kvs[i]->kv_f16);
                V[kvs[i]->len * kd + e] = kv_round(v[i * kd + e], kvs[i]->kv_f16);
            }
        }
        for (int64_t t = 0; t < B * nh; ++t) {
            const int64_t i = t / nh, hh = t % nh, gk = hh / group;
            const float *K = kvs[i]->k + (int64_t)li * kvs[i]->cap * kd, *V = kvs[i]->v + (int64_t)li * kvs[i]->cap * kd;
            attend(q + i * qd + hh * hd, K, V, kvs[i]->len + 1, kd, gk * hd, hd, scale, sc, ao + i * qd + hh * hd);
        }
        vo_matmul(&L->o, ao, B, o, avx2);
        for (int64_t i = 0; i < B * H; ++i) h[i] += o[i];
        for (int64_t i = 0; i < B; ++i) vo_rmsnorm(h + i * H, L->ln2, H, w->eps, xn + i * H);
        vo_matmul(&L->gate, xn, B, g, avx2);
        vo_matmul(&L->up, xn, B, u, avx2);
        for (int64_t i = 0; i < B * I; ++i) g[i] = vo_silu(g[i]) * u[i];
        vo_matmul(&L->down, g, B, d, avx2);
        for (int64_t i = 0; i < B * H; ++i) h[i] += d[i];
    }
    for (int64_t i = 0; i < B; ++i) {
        kvs[i]->len += 1;
        vo_rmsnorm(h + i * H, w->final_norm, H, w->eps, out + i * H);
    }
    free(h); free(xn); free(q); free(k); free(v); free(ao); free(o); free(g); free(u); free(d); free(sc);
    return 0;
}

/* ------------------------------------------------------------------ F5-TTS DiT (f5.cpp, f5_ops.cpp) */
float vo_gelu_tanh(float x) { /* f5.cpp:93-96 */
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}
float vo_mish(float x) { /* f5.cpp:97-100 */
    const float sp = x > 20.f ? x : log1pf(expf(x));
    return x * tanhf(sp);
}

/* Conv1d::forward (f5_ops.cpp:106-147): depthwise directly, else per group im2col [T][K * cig] and the F32 matmul */
void vo_conv1d(const vo_conv *c, const float *x, int32_t T, float *y) {
    const int pad = c->K / 2;
    if (c->groups == c->cin && c->cin == c->cout) { /* depthwise: w [C][K] */
        for (int64_t t = 0; t < T; ++t)
            for (int ch = 0; ch < c->cin; ++ch) {
                float acc = c->b ? c->b[ch] : 0.f;
                const float *wc = c->w + (int64_t)ch * c->K;
                for (int k = 0; k < c->K; ++k) {
                    const int64_t tt = t + k - pad;
                    if (tt >= 0 && tt < T) acc += wc[k] * x[tt * c->cin + ch];
                }
                y[t * c->cout + ch] = acc;
            }
        return;
    }
    const int cig = c->cin / c->groups, cog = c->cout / c->groups;
    const int64_t kc = (int64_t)c->K * cig;
    float *col = (float *)malloc(sizeof(float) * (size_t)(T * kc));
    float *yg = (float *)malloc(sizeof(float) * (size_t)T * (size_t)cog);
    for (int g = 0; g < c->groups; ++g) {
        for (int64_t t = 0; t < T; ++t)
            for (int k = 0; k < c->K; ++k) {
                const int64_t tt = t + k - pad;
                float *dst = col + t * kc + (int64_t)k * cig;
                if (tt >= 0 && tt < T) memcpy(dst, x + tt * c->cin + (int64_t)g * cig, sizeof(float) * (size_t)cig);
                else memset(dst, 0, sizeof(float) * (size_t)cig);
            }
        vo_mat W = {VO_F32, c->w + (int64_t)g * cog * kc, NULL, cog, kc, NULL};
        vo_matmul(&W, col, T, yg, 1);
        for (int64_t t = 0; t < T; ++t)
            for (int o = 0; o < cog; ++o)
                y[t * c->cout + (int64_t)g * cog + o] = yg[t * cog + o] + (c->b ? c->b[g * cog + o] : 0.f);
    }
    free(col);
    free(yg);
}

void vo_f5_modulate(const float *x, int64_t R, int32_t D, const float *sc, const float *sh, float *y) {
    for (int64_t r = 0; r < R; ++r) {
        const float *xr = x + r * D;
        double mean = 0;
        for (int i = 0; i < D; ++i) mean += xr[i];
        mean /= D;
        double var = 0;
        for (int i = 0; i < D; ++i) { const double dd = xr[i] - mean; var += dd * dd; }
        var /= D;
        const float inv = (float)(1.0 / sqrt(var + 1e-6));
        float *yr = y + r * D;
        for (int i = 0; i < D; ++i) yr[i] = (xr[i] - (float)mean) * inv * (1.0f + sc[i]) + sh[i];
    }
}

float vo_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); } /* kernels.hpp:106 */

/* F5Model::vocode (f5.cpp:779-806) up to the head: embed conv, LayerNorm, the ConvNeXt blocks (depthwise conv,
 * LayerNorm, pw1 + GELU-erf, pw2, x += gamma * z), final LayerNorm, head. */
int vo_vocos_head(const vo_vocos *v, const float *mel, int32_t T, float *head) {
    const int D = v->dim, I = v->inter;
    float *x = (float *)malloc(sizeof(float) * (size_t)T * D), *y = (float *)malloc(sizeof(float) * (size_t)T * D);
    float *h = (float *)malloc(sizeof(float) * (size_t)T * I), *z = (float *)malloc(sizeof(float) * (size_t)T * D);
    if (!x || !y || !h || !z) { free(x); free(y); free(h); free(z); return -1; }
    vo_conv1d(&v->embed, mel, T, x);
    for (int64_t t = 0; t < T; ++t) vo_layernorm(x + t * D, v->ln_w, v->ln_b, D, 1e-6f, x + t * D);
    for (int i = 0; i < v->layers; ++i) {
        const vo_vocos_block *b = &v->blocks[i];
        vo_conv1d(&b->dw, x, T, y);
        for (int64_t t = 0; t < T; ++t) vo_layernorm(y + t * D, b->ln_w, b->ln_b, D, 1e-6f, y + t * D);
        vo_matmul(&b->pw1, y, T, h, 1);
        for (int64_t j = 0; j < (int64_t)T * I; ++j) h[j] = vo_gelu_erf(h[j]);
        vo_matmul(&b->pw2, h, T, z, 1);
        for (int64_t t = 0; t < T; ++t)
            for (int c = 0; c < D; ++c) x[t * D + c] += b->gamma[c] * z[t * D + c];
    }
    for (int64_t t = 0; t < T; ++t) vo_layernorm(x + t * D, v->fln_w, v->fln_b, D, 1e-6f, x + t * D);
    vo_matmul(&v->head, x, T, head, 1);
    free(x); free(y); free(h); free(z);
    return 0;
}

int vo_f5_step(const vo_f5 *m, int32_t B, int32_t N, const float *cat, const float *ts, const float *rope, float *out) {
    const int D = m->dim, H = m->heads, HD = m->dim_head, INNER = H * HD, HH = HD / 2, FF = D * m->ff_mult;
    const int64_t R = (int64_t)B * N;
    float *h = (float *)malloc(sizeof(float) * (size_t)(R * D));
    float *a = (float *)malloc(sizeof(float) * (size_t)N * D), *b2 = (float *)malloc(sizeof(float) * (size_t)N * D);
    float *ada = (float *)malloc(sizeof(float) * 6 * (size_t)D), *nrm = (float *)malloc(sizeof(float) * (size_t)(R * D));
    float *q = (float *)malloc(sizeof(float) * (size_t)(R * INNER)), *k = (float *)malloc(sizeof(float) * (size_t)(R * INNER));
    float *v = (float *)malloc(sizeof(float) * (size_t)(R * INNER)), *at = (float *)malloc(sizeof(float) * (size_t)(R * INNER));
    float *o = (float *)malloc(sizeof(float) * (size_t)(R * D)), *ff = (float *)malloc(sizeof(float) * (size_t)(R * FF));
    float *qh = (float *)malloc(sizeof(float) * (size_t)N * HD), *kh = (float *)malloc(sizeof(float) * (size_t)N * HD);
    float *vt = (float *)malloc(sizeof(float) * (size_t)N * HD), *oh = (float *)malloc(sizeof(float) * (size_t)N * HD);
    float *sc = (float *)malloc(sizeof(float) * (size_t)N * N), *fin = (float *)malloc(sizeof(float) * 2 * (size_t)D);
    vo_matmul(&m->in_proj, cat, R, h, 1);
    for (int s = 0; s < B; ++s) { /* convolutional position embedding (f5.cpp:589-598) */
        float *hs = h + (int64_t)s * N * D;
        vo_conv1d(&m->pos1, hs, N, a);
        for (int64_t i = 0; i < (int64_t)N * D; ++i) a[i] = vo_mish(a[i]);
        vo_conv1d(&m->pos2, a, N, b2);
        for (int64_t i = 0; i < (int64_t)N * D; ++i) hs[i] += vo_mish(b2[i]);
    }
    const float scale = 1.0f / sqrtf((float)HD);
    for (int bi = 0; bi < m->depth; ++bi) {
        const vo_f5_block *L = &m->blocks[bi];
        vo_matmul(&L->ada, ts, 1, ada, 1);
        const float *shift_msa = ada, *scale_msa = ada + D, *gate_msa = ada + 2 * D;
        const float *shift_mlp = ada + 3 * D, *scale_mlp = ada + 4 * D, *gate_mlp = ada + 5 * D;
        vo_f5_modulate(h, R, D, scale_msa, shift_msa, nrm);
        vo_matmul(&L->q, nrm, R, q, 1);
        vo_matmul(&L->k, nrm, R, k, 1);
        vo_matmul(&L->v, nrm, R, v, 1);
        for (int64_t r = 0; r < R; ++r) /* RoPE on pairs (2j, 2j+1) (f5.cpp:653-668) */
            for (int hh = 0; hh < H; ++hh) {
                if (m->pe_attn_head > 0 && hh >= m->pe_attn_head) continue;
                const int pos = (int)(r % N);
                float *bufs[2] = {q + r * INNER + (int64_t)hh * HD, k + r * INNER + (int64_t)hh * HD};
                for (int u = 0; u < 2; ++u)
                    for (int j = 0; j < HH; ++j) {
                        const float c = rope[((int64_t)pos * HH + j) * 2], sn = rope[((int64_t)pos * HH + j) * 2 + 1];
                        const float x0 = bufs[u][2 * j], x1 = bufs[u][2 * j + 1];
                        bufs[u][2 * j] = x0 * c - x1 * sn;
                        bufs[u][2 * j + 1] = x1 * c + x0 * sn;
                    }
            }
        for (int s = 0; s < B; ++s) /* attention per head (f5.cpp:626-650) */
            for (int hh = 0; hh < H; ++hh) {
                const int64_t base = (int64_t)s * N * INNER + (int64_t)hh * HD;
                for (int64_t i = 0; i < N; ++i) {
                    memcpy(qh + i * HD, q + base + i * INNER, sizeof(float) * (size_t)HD);
                    memcpy(kh + i * HD, k + base + i * INNER, sizeof(float) * (size_t)HD);
                    for (int d = 0; d < HD; ++d) vt[(int64_t)d * N + i] = v[base + i * INNER + d];
                }
                vo_mat km = {VO_F32, kh, NULL, N, HD, NULL};
                vo_matmul(&km, qh, N, sc, 1);
                for (int64_t i = 0; i < N; ++i) {
                    float *row = sc + i * N, mx = -INFINITY, sum = 0;
                    for (int j = 0; j < N; ++j) { row[j] *= scale; mx = mx < row[j] ? row[j] : mx; }
                    for (int j = 0; j < N; ++j) { row[j] = expf(row[j] - mx); sum += row[j]; }
                    const float inv = 1.0f / sum;
                    for (int j = 0; j < N; ++j) row[j] *= inv;
                }
                vo_mat vm = {VO_F32, vt, NULL, HD, N, NULL};
                vo_matmul(&vm, sc, N, oh, 1);
                for (int64_t i = 0; i < N; ++i) memcpy(at + base + i * INNER, oh + i * HD, sizeof(float) * (size_t)HD);
            }
        vo_matmul(&L->o, at, R, o, 1);
        for (int64_t r = 0; r < R; ++r)
            for (int i = 0; i < D; ++i) h[r * D + i] += gate_msa[i] * o[r * D + i];
        vo_f5_modulate(h, R, D, scale_mlp, shift_mlp, nrm);
        vo_matmul(&L->ff1, nrm, R, ff, 1);
        for (int64_t i = 0; i < R * FF; ++i) ff[i] = vo_gelu_tanh(ff[i]);
        vo_matmul(&L->ff2, ff, R, o, 1);
        for (int64_t r = 0; r < R; ++r)
            for (int i = 0; i < D; ++i) h[r * D + i] += gate_mlp[i] * o[r * D + i];
    }
    vo_matmul(&m->norm_out, ts, 1, fin, 1); /* final modulation: (scale, shift) */
    vo_f5_modulate(h, R, D, fin, fin + D, nrm);
    vo_matmul(&m->proj_out, nrm, R, out, 1);
    free(h); free(a); free(b2); free(ada); free(nrm); free(q); free(k); free(v); free(at); free(o); free(ff);
    free(qh); free(kh); free(vt); free(oh); free(sc); free(fin);
    return 0;
}

/* ------------------------------------------------------------------ CosyVoice2 flow estimator */
float vo_exp_poly(float x) { /* nn.cpp:16-29: x = n ln2 + r, Cephes' degree-6 polynomial for e^r, 2^n in the exponent */
    x = fminf(fmaxf(x, -87.3f), 88.7f);
    const float fn = floorf(x * 1.44269504088896341f + 0.5f);
    const float r = (x - fn * 0.693359375f) - fn * -2.12194440e-4f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * r * r + r + 1.0f;
    const int32_t e = ((int32_t)fn + 127) << 23;
    float sc;
    memcpy(&sc, &e, 4);
    return p * sc;
}

float vo_gelu_poly(float x) { /* nn.cpp:31-38 */
    const float z = fabsf(x) * 0.70710678118654752f;
    const float t = 1.0f / (1.0f + 0.5f * z);
    const float y = t * vo_exp_poly(-z * z - 1.26551223f + t * (1.00002368f + t * (0.37409196f + t * (0.09678418f + t * (-0.18628806f +
                    t * (0.27886807f + t * (-1.13520398f + t * (1.48851587f + t * (-0.82215223f + t * 0.17087277f)))))))));
    const float erf_abs = 1.0f - y;
    return 0.5f * x * (1.0f + (x < 0.f ? -erf_abs : erf_abs));
}

float vo_mish_nn(float x) { /* nn.hpp:103-107 */
    if (x > 20.f) return x;
    const float e = expf(x), n = e * (e + 2.0f);
    return x * (n / (n + 2.0f));
}

void vo_layer_norm_nn(float *x, int64_t T, int32_t C, const float *w, const float *b, float eps) {
    for (int64_t t = 0; t < T; ++t) {
        float *r = x + t * C;
        double mean = 0;
        for (int c = 0; c < C; ++c) mean += r[c];
        mean /= C;
        double var = 0;
        for (int c = 0; c < C; ++c) { const double d = r[c] - mean; var += d * d; }
        var /= C;
        const float inv = (float)(1.0 / sqrt(var + eps));
        for (int c = 0; c < C; ++c) {
            const float n = (r[c] - (float)mean) * inv;
            r[c] = n * w[c] + (b ? b[c] : 0.f);
        }
    }
}

void vo_softmax_fast(float *x, int64_t n) {
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) mx = mx < x[i] ? x[i] : mx;
    for (int64_t i = 0; i < n; ++i) x[i] -= mx;
    for (int64_t i = 0; i < n; ++i) x[i] = vo_exp_poly(x[i]);
    float sum = 0.f;
    for (int64_t i = 0; i < n; ++i) sum += x[i];
    const float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; ++i) x[i] *= inv;
}

void vo_attention_nn(const float *q, const float *k, const float *v, int32_t Tq, int32_t Tk, int32_t H, int32_t dh,
                     float scale, float *out) {
    const int64_t st = (int64_t)H * dh;
    float *Q = (float *)malloc(sizeof(float) * (size_t)Tq * dh), *K = (float *)malloc(sizeof(float) * (size_t)Tk * dh);
    float *Vt = (float *)malloc(sizeof(float) * (size_t)dh * Tk), *S = (float *)malloc(sizeof(float) * (size_t)Tq * Tk);
    float *O = (float *)malloc(sizeof(float) * (size_t)Tq * dh);
    for (int h = 0; h < H; ++h) {
        for (int64_t t = 0; t < Tq; ++t)
            for (int d = 0; d < dh; ++d) Q[t * dh + d] = q[t * st + (int64_t)h * dh + d] * scale;
        for (int64_t t = 0; t < Tk; ++t)
            for (int d = 0; d < dh; ++d) {
                K[t * dh + d] = k[t * st + (int64_t)h * dh + d];
                Vt[(int64_t)d * Tk + t] = v[t * st + (int64_t)h * dh + d];
            }
        const vo_mat km = {VO_F32, K, NULL, Tk, dh, NULL};
        vo_matmul(&km, Q, Tq, S, 1);
        for (int64_t i = 0; i < Tq; ++i) vo_softmax_fast(S + i * Tk, Tk);
        const vo_mat vm = {VO_F32, Vt, NULL, dh, Tk, NULL};
        vo_matmul(&vm, S, Tq, O, 1);
        for (int64_t t = 0; t < Tq; ++t) memcpy(out + t * st + (int64_t)h * dh, O + t * dh, sizeof(float) * (size_t)dh);
    }
    free(Q); free(K); free(Vt); free(S); free(O);
}

void vo_causal_conv(const vo_conv *c, const float *x, int32_t T, float *y) {
    const int64_t kc = (int64_t)c->K * c->cin;
    float *col = (float *)calloc((size_t)(T * kc) + 1, sizeof(float));
    if (!col) return;
    for (int64_t t = 0; t < T; ++t)
        for (int k = 0; k < c->K; ++k) {
            const int64_t s = t + k - (c->K - 1);
            float *dst = col + t * kc + (int64_t)k * c->cin;
            if (s >= 0) memcpy(dst, x + s * c->cin, sizeof(float) * (size_t)c->cin);
            else memset(dst, 0, sizeof(float) * (size_t)c->cin);
        }
    const vo_mat W = {VO_F32, c->w, NULL, c->cout, kc, NULL};
    vo_matmul(&W, col, T, y, 1);
    if (c->b)
        for (int64_t t = 0; t < T; ++t)
            for (int o = 0; o < c->cout; ++o) y[t * c->cout + o] += c->b[o];
    free(col);
}

int32_t vo_convt(const float *w_pt, int32_t cin, int32_t cout, int32_t K, int32_t stride, int32_t pad, int32_t out_pad,
                 const float *bias, const float *x, int32_t T, float *y) {
    if (cin < 1 || cout < 1 || K < 1 || stride < 1 || pad < 0 || out_pad < 0 || T < 1) return -1;
    const int64_t To = (int64_t)(T - 1) * stride - 2 * (int64_t)pad + K + out_pad;
    if (To < 1) return -1;
    const int64_t KO = (int64_t)K * cout;
    float *w = (float *)malloc(sizeof(float) * (size_t)(KO * cin));
    if (!w) return -1;
    for (int c = 0; c < cin; ++c) /* ConvT::load (nn.cpp:205-215) */
        for (int o = 0; o < cout; ++o)
            for (int k = 0; k < K; ++k) w[((int64_t)k * cout + o) * cin + c] = w_pt[((int64_t)c * cout + o) * K + k];
    const vo_mat W = {VO_F32, w, NULL, KO, cin, NULL};
    int64_t blk = ((int64_t)4 << 20) / KO; /* ConvT::forward (nn.cpp:217-245) */
    if (blk < 16) blk = 16;
    float *z = (float *)malloc(sizeof(float) * (size_t)((blk < T ? blk : T) * KO));
    if (!z) { free(w); return -1; }
    memset(y, 0, sizeof(float) * (size_t)(To * cout));
    for (int64_t t0 = 0; t0 < T; t0 += blk) {
        const int64_t n = blk < T - t0 ? blk : T - t0;
        vo_matmul(&W, x + t0 * cin, n, z, 1);
        for (int64_t i = 0; i < n; ++i) {
            const int64_t t = t0 + i;
            for (int k = 0; k < K; ++k) {
                const int64_t to = t * stride + k - pad;
                if (to < 0 || to >= To) continue;
                const float *zr = z + i * KO + (int64_t)k * cout;
                float *yr = y + to * cout;
                for (int o = 0; o < cout; ++o) yr[o] += zr[o];
            }
        }
    }
    if (bias)
        for (int64_t t = 0; t < To; ++t)
            for (int o = 0; o < cout; ++o) y[t * cout + o] += bias[o];
    free(z);
    free(w);
    return (int32_t)To;
}

/* causal_conv_b (cosyvoice.cpp:134-144): per sequence of T rows */
static void cosy_conv_b(const vo_conv *c, const float *x, int32_t T, float *y) {
    for (int b = 0; b < 2; ++b) vo_causal_conv(c, x + (int64_t)b * T * c->cin, T, y + (int64_t)b * T * c->cout);
}

/* CausalBlock1D (cosyvoice.cpp:147-157): causal conv -> LayerNorm (1e-5) -> mish */
static void cosy_block(const vo_conv *c, const float *w, const float *b, const float *x, int32_t T, float *y) {
    cosy_conv_b(c, x, T, y);
    vo_layer_norm_nn(y, 2 * (int64_t)T, c->cout, w, b, 1e-5f);
    for (int64_t i = 0; i < 2 * (int64_t)T * c->cout; ++i) y[i] = vo_mish_nn(y[i]);
}

/* CausalResnetBlock1D::forward (cosyvoice.cpp:169-180) */
static void cosy_resnet(const vo_cosy_res *r, const float *x, int32_t T, const float *tb, float *out) {
    const int C = r->c1.cout;
    const int64_t R = 2 * (int64_t)T;
    float *h = (float *)malloc(sizeof(float) * (size_t)(R * C)), *h2 = (float *)malloc(sizeof(float) * (size_t)(R * C));
    float *rr = (float *)malloc(sizeof(float) * (size_t)(R * C));
    cosy_block(&r->c1, r->n1w, r->n1b, x, T, h);
    for (int64_t t = 0; t < R; ++t)
        for (int c = 0; c < C; ++c) h[t * C + c] += tb[c];
    cosy_block(&r->c2, r->n2w, r->n2b, h, T, h2);
    vo_causal_conv(&r->res, x, (int32_t)R, rr); /* K 1: the linear over all rows (res.forward(x, B T)) */
    for (int64_t i = 0; i < R * C; ++i) out[i] = h2[i] + rr[i];
    free(h); free(h2); free(rr);
}

/* XBlock::forward (cosyvoice.cpp:197-220) on x [2 T][C] in place */
static void cosy_xblock(const vo_cosy_x *L, float *x, int32_t T, int32_t H) {
    const int C = (int)L->o.rows, inner = (int)L->q.rows, dh = inner / H, FF = (int)L->ff1.rows;
    const int64_t R = 2 * (int64_t)T;
    float *xn = (float *)malloc(sizeof(float) * (size_t)(R * C)), *y = (float *)malloc(sizeof(float) * (size_t)(R * C));
    float *Q = (float *)malloc(sizeof(float) * (size_t)(R * inner)), *K = (float *)malloc(sizeof(float) * (size_t)(R * inner));
    float *V = (float *)malloc(sizeof(float) * (size_t)(R * inner)), *A = (float *)malloc(sizeof(float) * (size_t)(R * inner));
    float *hd = (float *)malloc(sizeof(float) * (size_t)(R * FF));
    memcpy(xn, x, sizeof(float) * (size_t)(R * C));
    vo_layer_norm_nn(xn, R, C, L->n1w, L->n1b, 1e-5f);
    vo_matmul(&L->q, xn, R, Q, 1);
    vo_matmul(&L->k, xn, R, K, 1);
    vo_matmul(&L->v, xn, R, V, 1);
    for (int b = 0; b < 2; ++b) {
        const int64_t off = (int64_t)b * T * inner;
        vo_attention_nn(Q + off, K + off, V + off, T, T, H, dh, 1.0f / sqrtf((float)dh), A + off);
    }
    vo_matmul(&L->o, A, R, y, 1);
    for (int64_t i = 0; i < R * C; ++i) x[i] += y[i];
    memcpy(xn, x, sizeof(float) * (size_t)(R * C));
    vo_layer_norm_nn(xn, R, C, L->n3w, L->n3b, 1e-5f);
    vo_matmul(&L->ff1, xn, R, hd, 1);
    for (int64_t i = 0; i < R * FF; ++i) hd[i] = vo_gelu_poly(hd[i]);
    vo_matmul(&L->ff2, hd, R, y, 1);
    for (int64_t i = 0; i < R * C; ++i) x[i] += y[i];
    free(xn); free(y); free(Q); free(K); free(V); free(A); free(hd);
}

int vo_cosy_step(const vo_cosy *m, int32_t T, const float *in, const float *tb, float *out) {
    const int C = m->C;
    const int64_t R = 2 * (int64_t)T;
    float *a = (float *)malloc(sizeof(float) * (size_t)(R * C)), *b = (float *)malloc(sizeof(float) * (size_t)(R * C));
    float *skip = (float *)malloc(sizeof(float) * (size_t)(R * C)), *cat = (float *)malloc(sizeof(float) * (size_t)(R * 2 * C));
    if (!a || !b || !skip || !cat) { free(a); free(b); free(skip); free(cat); return -1; }
    cosy_resnet(&m->down_res, in, T, tb, a);
    for (int i = 0; i < m->n_down_x; ++i) cosy_xblock(&m->down_x[i], a, T, m->heads);
    memcpy(skip, a, sizeof(float) * (size_t)(R * C));
    cosy_conv_b(&m->down_conv, a, T, b);
    int64_t off = 0;
    for (int i = 0; i < m->n_mid; ++i) {
        cosy_resnet(&m->mid_res[i], b, T, tb + (int64_t)(1 + i) * C, a);
        for (int j = 0; j < m->mid_x_count[i]; ++j) cosy_xblock(&m->mid_x[off + j], a, T, m->heads);
        off += m->mid_x_count[i];
        float *t = a; a = b; b = t;
    }
    for (int64_t r = 0; r < R; ++r) {
        memcpy(cat + r * 2 * C, b + r * C, sizeof(float) * (size_t)C);
        memcpy(cat + r * 2 * C + C, skip + r * C, sizeof(float) * (size_t)C);
    }
    cosy_resnet(&m->up_res, cat, T, tb + (int64_t)(1 + m->n_mid) * C, a);
    for (int i = 0; i < m->n_up_x; ++i) cosy_xblock(&m->up_x[i], a, T, m->heads);
    cosy_conv_b(&m->up_out, a, T, b);
    cosy_block(&m->final_conv, m->fn_w, m->fn_b, b, T, a);
    vo_causal_conv(&m->final_proj, a, (int32_t)R, out); /* K 1 over all rows */
    free(a); free(b); free(skip); free(cat);
    return 0;
}

/* ------------------------------------------------------------------ Qwen3-TTS codec decoder */
struct vo_codec_state {
    const vo_codec *c;
    float *pre_h, *conv0_h, *final_h; /* conv histories [(K - 1) dil][cin] */
    float **up_dw_h;                  /* [n_up][(dw_K - 1)][latent] */
    float **tail;                     /* [n_blocks][(K - stride)][cout] */
    float **ru_h;                     /* [n_blocks * 3][(K - 1) dil][cout] */
    vo_kv kv;                         /* f32, [layers][cap][kd] */
    int64_t frames;
};

static size_t hist_elems(const vo_cconv *c) { return (size_t)(c->K - 1) * (size_t)c->dil * (size_t)c->cin; }
static float *zalloc(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

vo_codec_state *vo_codec_state_new(const vo_codec *c, int64_t cap) {
    vo_codec_state *s = (vo_codec_state *)calloc(1, sizeof(vo_codec_state));
    s->c = c;
    s->pre_h = zalloc(hist_elems(&c->pre_conv));
    s->conv0_h = zalloc(hist_elems(&c->conv0));
    s->final_h = zalloc(hist_elems(&c->final_conv));
    s->up_dw_h = (float **)calloc((size_t)c->n_up + 1, sizeof(float *));
    for (int i = 0; i < c->n_up; ++i) s->up_dw_h[i] = zalloc((size_t)(c->ups[i].dw_K - 1) * (size_t)c->latent);
    s->tail = (float **)calloc((size_t)c->n_blocks + 1, sizeof(float *));
    s->ru_h = (float **)calloc(3 * (size_t)c->n_blocks + 1, sizeof(float *));
    for (int b = 0; b < c->n_blocks; ++b) {
        const vo_codec_block *d = &c->blocks[b];
        s->tail[b] = zalloc((size_t)(d->K - d->stride) * (size_t)d->cout);
        for (int u = 0; u < 3; ++u) s->ru_h[3 * b + u] = zalloc(hist_elems(&d->c1[u]));
    }
    const int64_t kd = (int64_t)c->pt.kv_heads * c->pt.head_dim;
    s->kv.k = zalloc((size_t)(c->pt.n_layers * cap * kd));
    s->kv.v = zalloc((size_t)(c->pt.n_layers * cap * kd));
    s->kv.cap = cap;
    return s;
}

static float *dup(const float *p, size_t n) {
    float *d = zalloc(n);
    memcpy(d, p, n * sizeof(float));
    return d;
}

vo_codec_state *vo_codec_state_clone(const vo_codec_state *src) {
    const vo_codec *c = src->c;
    vo_codec_state *s = (vo_codec_state *)calloc(1, sizeof(vo_codec_state));
    *s = *src;
    s->pre_h = dup(src->pre_h, hist_elems(&c->pre_conv));
    s->conv0_h = dup(src->conv0_h, hist_elems(&c->conv0));
    s->final_h = dup(src->final_h, hist_elems(&c->final_conv));
    s->up_dw_h = (float **)calloc((size_t)c->n_up + 1, sizeof(float *));
    for (int i = 0; i < c->n_up; ++i) s->up_dw_h[i] = dup(src->up_dw_h[i], (size_t)(c->ups[i].dw_K - 1) * (size_t)c->latent);
    s->tail = (float **)calloc((size_t)c->n_blocks + 1, sizeof(float *));
    s->ru_h = (float **)calloc(3 * (size_t)c->n_blocks + 1, sizeof(float *));
    for (int b = 0; b < c->n_blocks; ++b) {
        const vo_codec_block *d = &c->blocks[b];
        s->tail[b] = dup(src->tail[b], (size_t)(d->K - d->stride) * (size_t)d->cout);
        for (int u = 0; u < 3; ++u) s->ru_h[3 * b + u] = dup(src->ru_h[3 * b + u], hist_elems(&d->c1[u]));
    }
    const int64_t kd = (int64_t)c->pt.kv_heads * c->pt.head_dim;
    s->kv.k = dup(src->kv.k, (size_t)(c->pt.n_layers * src->kv.cap * kd));
    s->kv.v = dup(src->kv.v, (size_t)(c->pt.n_layers * src->kv.cap * kd));
    return s;
}

void vo_codec_state_free(vo_codec_state *s) {
    if (!s) return;
    const vo_codec *c = s->c;
    free(s->pre_h); free(s->conv0_h); free(s->final_h);
    for (int i = 0; i < c->n_up; ++i) free(s->up_dw_h[i]);
    for (int b = 0; b < c->n_blocks; ++b) {
        free(s->tail[b]);
        for (int u = 0; u < 3; ++u) free(s->ru_h[3 * b + u]);
    }
    free(s->up_dw_h); free(s->tail); free(s->ru_h); free(s->kv.k); free(s->kv.v);
    free(s);
}

int64_t vo_codec_spf(const vo_codec *c) {
    int64_t p = 1;
    for (int i = 0; i < c->n_up; ++i) p *= c->ups[i].K;
    for (int b = 0; b < c->n_blocks; ++b) p *= c->blocks[b].stride;
    return p;
}

int vo_codec_quantize(const vo_codec *c, const int16_t *codes, int32_t F, float *z) {
    const int Q = c->quantizers, dim = c->codebook_dim / 2, CD = c->codebook_dim;
    float *s1 = zalloc((size_t)F * dim), *s2 = zalloc((size_t)F * dim), *tmp = zalloc((size_t)dim), *z2 = zalloc((size_t)F * CD);
    int rc = 0;
    for (int t = 0; t < F && !rc; ++t) {
        const int16_t *cd = codes + (size_t)t * Q;
        for (int q = 0; q < Q; ++q)
            if (cd[q] < 0 || cd[q] >= c->codebook_size) rc = -1;
        if (rc) break;
        vo_mat_row(&c->q_first[0], cd[0], s1 + (size_t)t * dim);
        for (int q = 1; q < Q; ++q) {
            vo_mat_row(&c->q_rest[q - 1], cd[q], tmp);
            for (int i = 0; i < dim; ++i) s2[(size_t)t * dim + i] += tmp[i];
        }
    }
    if (!rc) {
        vo_matmul(&c->q_first_out, s1, F, z, 1);
        vo_matmul(&c->q_rest_out, s2, F, z2, 1);
        for (size_t i = 0; i < (size_t)F * CD; ++i) z[i] += z2[i];
    }
    free(s1); free(s2); free(tmp); free(z2);
    return rc;
}

/* conv_stream (qwen3.cpp:102-121): y = conv([hist; x]) (+ bias through the matmul), hist <- the last rows */
static void conv_stream(const vo_cconv *c, float *hist, const float *x, int64_t T, float *y) {
    const int64_t ctx = (int64_t)(c->K - 1) * c->dil, cin = c->cin;
    if (c->K == 1) { vo_matmul(&c->w, x, T, y, 1); return; }
    float *ext = zalloc((size_t)((ctx + T) * cin)), *col = zalloc((size_t)(T * c->K * cin));
    memcpy(ext, hist, sizeof(float) * (size_t)(ctx * cin));
    memcpy(ext + ctx * cin, x, sizeof(float) * (size_t)(T * cin));
    for (int64_t t = 0; t < T; ++t)
        for (int k = 0; k < c->K; ++k)
            memcpy(col + (t * c->K + k) * cin, ext + (t + (int64_t)k * c->dil) * cin, sizeof(float) * (size_t)cin);
    vo_matmul(&c->w, col, T, y, 1);
    memcpy(hist, ext + T * cin, sizeof(float) * (size_t)(ctx * cin));
    free(ext); free(col);
}

/* dwconv_stream (qwen3.cpp:123-137) */
static void dwconv_stream(const vo_codec_up *u, int C, float *hist, const float *x, int64_t T, float *y) {
    const int64_t ctx = u->dw_K - 1;
    float *ext = zalloc((size_t)((ctx + T) * C));
    memcpy(ext, hist, sizeof(float) * (size_t)(ctx * C));
    memcpy(ext + ctx * C, x, sizeof(float) * (size_t)(T * C));
    for (int64_t t = 0; t < T; ++t)
        for (int ch = 0; ch < C; ++ch) {
            float acc = u->dw_b[ch];
            for (int k = 0; k < u->dw_K; ++k) acc += u->dw_w[(size_t)ch * u->dw_K + k] * ext[(t + k) * C + ch];
            y[t * C + ch] = acc;
        }
    memcpy(hist, ext + T * C, sizeof(float) * (size_t)(ctx * C));
    free(ext);
}

/* trans_stream (qwen3.cpp:139-161): K <= 2 stride; output p gathers frames p / s and p / s - 1; the last K - s rows go
 * to the tail */
static void trans_stream(const vo_mat *w, const float *bias, int K, int s, int co, float *tail, const float *x, int64_t T,
                         float *y) {
    const int64_t tr = K - s;
    float *tmp = zalloc((size_t)(T * K * co)), *nt = zalloc((size_t)(tr * co));
    vo_matmul(w, x, T, tmp, 1);
    for (int64_t p = 0; p < T * s + tr; ++p) {
        const int64_t t = p / s, k = p - t * s;
        for (int o = 0; o < co; ++o) {
            float v = p < tr ? tail[p * co + o] : 0.f;
            if (t < T && k < K) v += tmp[(t * K + k) * co + o];
            if (t >= 1 && k + s < K) v += tmp[((t - 1) * K + k + s) * co + o];
            if (p < T * s) y[p * co + o] = v + bias[o];
            else nt[(p - T * s) * co + o] = v;
        }
    }
    memcpy(tail, nt, sizeof(float) * (size_t)(tr * co));
    free(tmp); free(nt);
}

/* snake_apply (qwen3.cpp:80-89): x + inv_b sin(a x)^2 */
static void snake(const vo_snake *s, float *x, int64_t T, int C) {
    for (int64_t t = 0; t < T; ++t)
        for (int c = 0; c < C; ++c) {
            const float v = x[t * C + c], sn = sinf(v * s->a[c]);
            x[t * C + c] = v + s->inv_b[c] * sn * sn;
        }
}

int64_t vo_codec_forward(const vo_codec *c, vo_codec_state *s, const float *z, int32_t F, float *pcm) {
    const int L = c->latent, H = c->pt.hidden;
    const int64_t T = F;
    if (s->kv.len + T > s->kv.cap) return -1;
    float *lat = zalloc((size_t)(T * L)), *hin = zalloc((size_t)(T * H)), *hout = zalloc((size_t)(T * H));
    conv_stream(&c->pre_conv, s->pre_h, z, T, lat);
    vo_matmul(&c->pt_in, lat, T, hin, 1);
    vo_transformer_forward(&c->pt, &s->kv, hin, T, NULL, hout);
    vo_matmul(&c->pt_out, hout, T, lat, 1);
    free(hin); free(hout);
    float *cur = lat;
    int64_t len = T;
    for (int si = 0; si < c->n_up; ++si) { /* qwen3.cpp:416-441 */
        const vo_codec_up *u = &c->ups[si];
        float *y = zalloc((size_t)(len * u->K * L));
        trans_stream(&u->tr, u->tr_b, u->K, u->K, L, NULL, cur, len, y);
        len *= u->K;
        float *dw = zalloc((size_t)(len * L)), *nrm = zalloc((size_t)(len * L)), *h1 = zalloc((size_t)(len * u->pw1.rows));
        float *h2 = zalloc((size_t)(len * L));
        dwconv_stream(u, L, s->up_dw_h[si], y, len, dw);
        for (int64_t t = 0; t < len; ++t) vo_layernorm(dw + t * L, u->ln_w, u->ln_b, L, 1e-6f, nrm + t * L);
        vo_matmul(&u->pw1, nrm, len, h1, 1);
        for (int64_t i = 0; i < len * u->pw1.rows; ++i) h1[i] = vo_gelu_erf(h1[i]);
        vo_matmul(&u->pw2, h1, len, h2, 1);
        for (int64_t t = 0; t < len; ++t)
            for (int i = 0; i < L; ++i) y[t * L + i] += u->gamma[i] * h2[t * L + i];
        free(dw); free(nrm); free(h1); free(h2); free(cur);
        cur = y;
    }
    float *x = zalloc((size_t)(len * c->conv0.cout));
    conv_stream(&c->conv0, s->conv0_h, cur, len, x);
    free(cur);
    int ch = c->conv0.cout;
    for (int b = 0; b < c->n_blocks; ++b) { /* qwen3.cpp:446-472 */
        const vo_codec_block *d = &c->blocks[b];
        const int out = d->cout;
        snake(&d->act, x, len, ch);
        float *y = zalloc((size_t)(len * d->stride * out));
        trans_stream(&d->tr, d->tr_b, d->K, d->stride, out, s->tail[b], x, len, y);
        len *= d->stride;
        ch = out;
        float *t1 = zalloc((size_t)(len * ch)), *t2 = zalloc((size_t)(len * ch));
        for (int u = 0; u < 3; ++u) {
            memcpy(t1, y, sizeof(float) * (size_t)(len * ch));
            snake(&d->a1[u], t1, len, ch);
            conv_stream(&d->c1[u], s->ru_h[3 * b + u], t1, len, t2);
            snake(&d->a2[u], t2, len, ch);
            conv_stream(&d->c2[u], NULL, t2, len, t1);
            for (int64_t i = 0; i < len * ch; ++i) y[i] += t1[i];
        }
        free(t1); free(t2); free(x);
        x = y;
    }
    snake(&c->final_act, x, len, ch);
    conv_stream(&c->final_conv, s->final_h, x, len, pcm);
    for (int64_t i = 0; i < len; ++i) pcm[i] = fminf(1.0f, fmaxf(-1.0f, pcm[i]));
    free(x);
    s->frames += F;
    return len;
}

void vo_snake_params(const float *alpha, const float *beta, int64_t n, float *a, float *inv_b) {
    for (int64_t i = 0; i < n; ++i) {
        a[i] = expf(alpha[i]);
        inv_b[i] = 1.0f / (expf(beta[i]) + 1e-9f);
    }
}
