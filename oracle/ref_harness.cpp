// ref_harness.cpp — extern "C" wrappers around the reference's own CPU functions.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with
// /root/reference/src/kernels.cpp, f5_ops.cpp and gpu_stub.cpp, where
// they lie, into oracle/_ref/libvoxref.so. tests/ use it to pin the C
// restatement (vox_oracle.c) bit for bit and to write the golden fixtures;
// bench.py may time it as the "reference" CPU baseline. Nothing here is part
// of the product, and no reference source is copied into this repository.
#include <cstring>
#include <vector>

#include "f5_ops.hpp"    // /root/reference/src (Conv1d)
#include "kernels.hpp"   // /root/reference/src
#include "sampling.hpp"  // /root/reference/src
#include "vox_oracle.h"  // struct layouts shared with the restatement

using namespace vox;

namespace {
Mat to_mat(const vo_mat &m) {
    Mat M;
    M.type = WType(m.type);
    M.data = static_cast<const uint8_t *>(m.data);
    M.scale = m.scale;
    M.rows = m.rows;
    M.cols = m.cols;
    M.bias = m.bias;
    M.gpu = -1;
    return M;
}

TransformerW to_xfmr(const vo_xfmr &x, double theta) {
    TransformerW w;
    w.hidden = x.hidden; w.heads = x.heads; w.kv_heads = x.kv_heads; w.head_dim = x.head_dim; w.inter = x.inter;
    w.eps = x.eps; w.theta = theta; w.final_norm = x.final_norm;
    w.inv_freq.assign(x.inv_freq, x.inv_freq + x.head_dim / 2);
    for (int i = 0; i < x.n_layers; ++i) {
        const vo_layer &l = x.layers[i];
        LayerW L;
        L.q = to_mat(l.q); L.k = to_mat(l.k); L.v = to_mat(l.v); L.o = to_mat(l.o);
        L.gate = to_mat(l.gate); L.up = to_mat(l.up); L.down = to_mat(l.down);
        L.qn = l.qn; L.kn = l.kn; L.ln1 = l.ln1; L.ln2 = l.ln2;
        w.layers.push_back(L);
    }
    return w;
}

// Fills a KVCache from a flat [layer][cap][kd] array holding `len` positions.
void load_kv(KVCache &kv, const vo_kv &src, int layers, int64_t kd) {
    kv.init(layers);
    for (int li = 0; li < layers; ++li) {
        const float *k = src.k + int64_t(li) * src.cap * kd, *v = src.v + int64_t(li) * src.cap * kd;
        kv.k[size_t(li)].assign(k, k + src.len * kd);
        kv.v[size_t(li)].assign(v, v + src.len * kd);
    }
    kv.len = src.len;
}

void store_kv(const KVCache &kv, vo_kv &dst, int layers, int64_t kd) {
    for (int li = 0; li < layers; ++li) {
        std::memcpy(dst.k + int64_t(li) * dst.cap * kd, kv.k[size_t(li)].data(), kv.k[size_t(li)].size() * 4);
        std::memcpy(dst.v + int64_t(li) * dst.cap * kd, kv.v[size_t(li)].data(), kv.v[size_t(li)].size() * 4);
    }
    dst.len = kv.len;
}
}  // namespace

extern "C" {
// Conv1d::load + forward (f5_ops.cpp:86-147) on PyTorch-layout weights w [cout][cin/groups][K].
void ref_conv1d(const float *w, int cin, int cout, int K, int groups, const float *bias, const float *x, int T, float *y) {
    Conv1d c;
    c.load(w, cin, cout, K, groups, bias);
    c.forward(x, T, y);
}
float ref_gelu_erf(float x) { return gelu_erf(x); }
void ref_set_threads(int n) { set_num_threads(n); }
void ref_philox(const uint32_t c[4], const uint32_t k[2], uint32_t out[4]) {
    auto r = Philox4x32::block({c[0], c[1], c[2], c[3]}, {k[0], k[1]});
    for (int i = 0; i < 4; ++i) out[i] = r[size_t(i)];
}
float ref_uniform(uint64_t seed, uint64_t frame, uint32_t cb, uint32_t draw) { return DetRng(seed).uniform(frame, cb, draw); }
int32_t ref_sample_logits(float *logits, int32_t n, float temperature, float top_p, int32_t top_k, float rep, const int32_t *hist,
                          int32_t nh, float u) {
    std::vector<float> l(logits, logits + n);
    SampleParams p;
    p.temperature = temperature; p.top_p = top_p; p.top_k = top_k; p.repetition_penalty = rep;
    std::vector<int32_t> h(hist, hist + nh);
    const int32_t r = sample_logits(l, p, u, hist ? &h : nullptr);
    std::memcpy(logits, l.data(), size_t(n) * 4);
    return r;
}
void ref_quantize_q8(const float *w, int64_t rows, int64_t cols, int8_t *q, float *s) {
    std::vector<int8_t> qq; std::vector<float> ss;
    quantize_q8(w, rows, cols, qq, ss);
    std::memcpy(q, qq.data(), qq.size()); std::memcpy(s, ss.data(), ss.size() * 4);
}
void ref_quantize_q4(const float *w, int64_t rows, int64_t cols, uint8_t *q, float *s) {
    std::vector<uint8_t> qq; std::vector<float> ss;
    quantize_q4(w, rows, cols, qq, ss);
    std::memcpy(q, qq.data(), qq.size()); std::memcpy(s, ss.data(), ss.size() * 4);
}
void ref_mat_gather(const vo_mat *m, int64_t r, float *out) { mat_gather(to_mat(*m), r, out); }
void ref_matmul(const vo_mat *m, const float *x, int64_t rows_in, float *y) { matmul(to_mat(*m), x, rows_in, y); }
float ref_dot(const float *a, const float *b, int64_t n) { return dot(a, b, n); }
void ref_rmsnorm(const float *x, const float *w, int64_t n, float eps, float *out) { rmsnorm(x, w, n, eps, out); }
void ref_layernorm(const float *x, const float *w, const float *b, int64_t n, float eps, float *out) { layernorm(x, w, b, n, eps, out); }
void ref_softmax(float *x, int64_t n) { softmax_inplace(x, n); }
float ref_silu(float x) { return silu(x); }
void ref_rope_inv_freq(int64_t hd, double theta, float *out) {
    auto f = rope_inv_freq(hd, theta);
    std::memcpy(out, f.data(), f.size() * 4);
}
void ref_rope_apply(float *x, int64_t heads, int64_t hd, const float *inv_freq, int64_t pos) { rope_apply(x, heads, hd, inv_freq, pos); }
// transformer_forward on a cache given as flat arrays (f32 cache, as KVCache keeps it).
int ref_transformer_forward(const vo_xfmr *x, vo_kv *kv, const float *in, int64_t m, float *out_last, float *out_all) {
    try {
        TransformerW w = to_xfmr(*x, 1e6);
        const int64_t kd = int64_t(x->kv_heads) * x->head_dim;
        if (kv->len + m > kv->cap) return -1;
        KVCache c;
        load_kv(c, *kv, x->n_layers, kd);
        transformer_forward(w, c, in, m, out_last, out_all);
        store_kv(c, *kv, x->n_layers, kd);
        return 0;
    } catch (...) {
        return -2;
    }
}
// A persistent decode session for timing the reference CPU step (the cpu_baseline of bench.py): the
// TransformerW and KVCache are built once; every step rewinds the cache to its initial length, then runs
// transformer_forward (m = 1), the head matmul and sample_logits, as the CPU path of a talker step does.
struct RefSession {
    TransformerW w;
    KVCache kv;
    Mat head;
    int64_t base_len = 0, kd = 0;
    std::vector<float> logits;
};
void *ref_session_new(const vo_xfmr *x, const vo_kv *kv, const vo_mat *head) {
    try {
        auto *s = new RefSession();
        s->w = to_xfmr(*x, 1e6);
        s->kd = int64_t(x->kv_heads) * x->head_dim;
        load_kv(s->kv, *kv, x->n_layers, s->kd);
        s->base_len = kv->len;
        s->head = to_mat(*head);
        s->logits.resize(size_t(head->rows));
        return s;
    } catch (...) {
        return nullptr;
    }
}
int ref_session_step(void *p, const float *x, float *out_last, float temperature, int32_t top_k, float u, int32_t *tok) {
    try {
        auto *s = static_cast<RefSession *>(p);
        for (size_t li = 0; li < s->kv.k.size(); ++li) {
            s->kv.k[li].resize(size_t(s->base_len * s->kd));
            s->kv.v[li].resize(size_t(s->base_len * s->kd));
        }
        s->kv.len = s->base_len;
        transformer_forward(s->w, s->kv, x, 1, out_last);
        matmul(s->head, out_last, 1, s->logits.data());
        SampleParams sp;
        sp.temperature = temperature;
        sp.top_k = top_k;
        *tok = sample_logits(s->logits, sp, u);
        return 0;
    } catch (...) {
        return -2;
    }
}
void ref_session_free(void *p) { delete static_cast<RefSession *>(p); }
int ref_transformer_forward_steps(const vo_xfmr *x, vo_kv *const *kvs, int64_t B, const float *in, float *out) {
    try {
        TransformerW w = to_xfmr(*x, 1e6);
        const int64_t kd = int64_t(x->kv_heads) * x->head_dim;
        std::vector<KVCache> cs(static_cast<size_t>(B));
        std::vector<KVCache *> ps(static_cast<size_t>(B));
        for (int64_t b = 0; b < B; ++b) {
            if (kvs[b]->len + 1 > kvs[b]->cap) return -1;
            load_kv(cs[size_t(b)], *kvs[b], x->n_layers, kd);
            ps[size_t(b)] = &cs[size_t(b)];
        }
        transformer_forward_steps(w, ps.data(), B, in, out);
        for (int64_t b = 0; b < B; ++b) store_kv(cs[size_t(b)], *kvs[b], x->n_layers, kd);
        return 0;
    } catch (...) {
        return -2;
    }
}
}
