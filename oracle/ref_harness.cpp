// ref_harness.cpp — extern "C" wrappers around the reference's own CPU functions.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with
// /root/reference/src/kernels.cpp, f5_ops.cpp, gpu_stub.cpp, nn.cpp, formats.cpp,
// resources.cpp and qwen3.cpp, where they lie, into oracle/_ref/libvoxref.so. tests/ use it to pin the C
// restatement (vox_oracle.c) bit for bit and to write the golden fixtures;
// bench.py may time it as the "reference" CPU baseline. Nothing here is part
// of the product, and no reference source is copied into this repository.
#include <cstring>
#include <vector>

#include "f5_ops.hpp"    // /root/reference/src (Conv1d)
#include "kernels.hpp"   // /root/reference/src
#include "nn.hpp"        // /root/reference/src (the vocoder / estimator layers)
#include "qwen3.hpp"     // /root/reference/src (Qwen3Weights::codec_forward)
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
    w.eps = x.eps; w.theta = theta; w.final_norm = x.final_norm; w.window = x.window;
    w.inv_freq.assign(x.inv_freq, x.inv_freq + x.head_dim / 2);
    for (int i = 0; i < x.n_layers; ++i) {
        const vo_layer &l = x.layers[i];
        LayerW L;
        L.q = to_mat(l.q); L.k = to_mat(l.k); L.v = to_mat(l.v); L.o = to_mat(l.o);
        L.gate = to_mat(l.gate); L.up = to_mat(l.up); L.down = to_mat(l.down);
        L.qn = l.qn; L.kn = l.kn; L.ln1 = l.ln1; L.ln2 = l.ln2;
        L.attn_scale = l.attn_scale; L.mlp_scale = l.mlp_scale;
        w.layers.push_back(L);
    }
    return w;
}

// An nn::Conv (groups 1, stride 1, no padding) over a vo_conv's weights in Conv::w layout [cout][K][cin].
nn::Conv to_nn_conv(const vo_conv &c) {
    nn::Conv o;
    o.cin = c.cin; o.cout = c.cout; o.K = c.K; o.stride = 1; o.pad = 0; o.dil = 1;
    o.w.assign(c.w, c.w + size_t(c.cout) * size_t(c.K) * size_t(c.cin));
    if (c.b) o.b.assign(c.b, c.b + c.cout);
    o.m.type = WType::F32; o.m.data = reinterpret_cast<const uint8_t *>(o.w.data()); o.m.rows = c.cout;
    o.m.cols = int64_t(c.K) * c.cin; o.m.gpu = -1;
    return o;
}
nn::Linear to_linear(const vo_mat &m) {
    nn::Linear L;
    L.w = to_mat(m);
    L.w.bias = nullptr;
    if (m.bias) L.b.assign(m.bias, m.bias + m.rows);
    L.in = m.cols; L.out = m.rows;
    return L;
}
// causal_conv_b (cosyvoice.cpp:127-144) through nn::Conv::forward: K - 1 zero rows in front of each sequence
void ref_causal_conv_b(const nn::Conv &c, const float *x, int T, int B, float *y) {
    std::vector<float> xp, yv;
    for (int b = 0; b < B; ++b) {
        xp.assign(size_t(T + c.K - 1) * size_t(c.cin), 0.f);
        std::memcpy(&xp[size_t(c.K - 1) * size_t(c.cin)], x + size_t(b) * T * c.cin, size_t(T) * c.cin * 4);
        c.forward(xp.data(), T + c.K - 1, yv);
        std::memcpy(y + size_t(b) * T * c.cout, yv.data(), yv.size() * 4);
    }
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
// nn::ConvT with its members set as ConvT::load sets them (nn.cpp:205-215) from PyTorch's weight [cin][cout][K],
// then ConvT::forward (nn.cpp:217-245); returns the output length.
int32_t ref_convt(const float *w_pt, int cin, int cout, int K, int stride, int pad, int out_pad, const float *bias,
                  const float *x, int T, float *y) {
    nn::ConvT c;
    c.cin = cin; c.cout = cout; c.K = K; c.stride = stride; c.pad = pad; c.out_pad = out_pad;
    c.w.resize(size_t(cin) * size_t(cout) * size_t(K));
    for (int ci = 0; ci < cin; ++ci)
        for (int o = 0; o < cout; ++o)
            for (int k = 0; k < K; ++k)
                c.w[(size_t(k) * size_t(cout) + size_t(o)) * size_t(cin) + size_t(ci)] =
                    w_pt[(size_t(ci) * size_t(cout) + size_t(o)) * size_t(K) + size_t(k)];
    if (bias) c.b.assign(bias, bias + cout);
    c.m.type = WType::F32; c.m.data = reinterpret_cast<const uint8_t *>(c.w.data()); c.m.rows = int64_t(K) * cout; c.m.cols = cin;
    std::vector<float> out;
    c.forward(x, T, out);
    std::memcpy(y, out.data(), out.size() * 4);
    return int32_t(out.size() / size_t(cout));
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

// ---- nn.cpp layers (the CosyVoice2 / Chatterbox estimator's)
void ref_gelu_inplace(float *x, int64_t n) { nn::gelu_inplace(x, n); }
float ref_mish_nn(float x) { return nn::mish(x); }
void ref_layer_norm_nn(float *x, int T, int C, const float *w, const float *b, float eps) { nn::layer_norm(x, T, C, w, b, eps); }
void ref_attention_nn(const float *q, const float *k, const float *v, int Tq, int Tk, int H, int dh, float scale, float *out) {
    const int64_t st = int64_t(H) * dh;
    nn::attention(q, st, k, st, v, st, Tq, Tk, H, dh, scale, out);
}
void ref_causal_conv(const vo_conv *c, const float *x, int T, float *y) { ref_causal_conv_b(to_nn_conv(*c), x, T, 1, y); }
// The estimator call of cosyvoice.cpp:839-863 (CResnet :169-180, XBlock :197-220, CBlock :147-157) on the reference's
// own layers, two sequences of T rows.
int ref_cosy_step(const vo_cosy *m, int T, const float *in, const float *tb, float *out) {
    try {
        const int B = 2, C = m->C, R = B * T;
        auto block = [&](const vo_conv &cv, const float *w, const float *b, const float *x, std::vector<float> &y) {
            const nn::Conv c = to_nn_conv(cv);
            y.resize(size_t(R) * size_t(c.cout));
            ref_causal_conv_b(c, x, T, B, y.data());
            nn::layer_norm(y.data(), R, c.cout, w, b, 1e-5f);
            for (float &z : y) z = nn::mish(z);
        };
        auto resnet = [&](const vo_cosy_res &r, const float *x, const float *tbj, std::vector<float> &o) {
            std::vector<float> h, h2, rr;
            block(r.c1, r.n1w, r.n1b, x, h);
            for (int t = 0; t < R; ++t)
                for (int c = 0; c < C; ++c) h[size_t(t) * C + c] += tbj[c];
            block(r.c2, r.n2w, r.n2b, h.data(), h2);
            to_nn_conv(r.res).forward(x, R, rr);
            o.resize(h2.size());
            for (size_t i = 0; i < o.size(); ++i) o[i] = h2[i] + rr[i];
        };
        auto xblock = [&](const vo_cosy_x &L, std::vector<float> &x) {
            const nn::Linear q = to_linear(L.q), k = to_linear(L.k), v = to_linear(L.v), o = to_linear(L.o);
            const nn::Linear f1 = to_linear(L.ff1), f2 = to_linear(L.ff2);
            const int inner = int(q.out), H = m->heads, dh = inner / H;
            std::vector<float> xn = x, Q(size_t(R) * inner), K(Q.size()), V(Q.size()), A(Q.size()), y(size_t(R) * C);
            nn::layer_norm(xn.data(), R, C, L.n1w, L.n1b, 1e-5f);
            q.forward(xn.data(), R, Q.data()); k.forward(xn.data(), R, K.data()); v.forward(xn.data(), R, V.data());
            for (int b = 0; b < B; ++b) {
                const size_t off = size_t(b) * T * inner;
                nn::attention(Q.data() + off, inner, K.data() + off, inner, V.data() + off, inner, T, T, H, dh,
                              1.0f / std::sqrt(float(dh)), A.data() + off);
            }
            o.forward(A.data(), R, y.data());
            for (size_t i = 0; i < x.size(); ++i) x[i] += y[i];
            xn = x;
            nn::layer_norm(xn.data(), R, C, L.n3w, L.n3b, 1e-5f);
            std::vector<float> hd(size_t(R) * size_t(f1.out));
            f1.forward(xn.data(), R, hd.data());
            nn::gelu_inplace(hd.data(), int64_t(hd.size()));
            f2.forward(hd.data(), R, y.data());
            for (size_t i = 0; i < x.size(); ++i) x[i] += y[i];
        };
        std::vector<float> a, b;
        resnet(m->down_res, in, tb, a);
        for (int i = 0; i < m->n_down_x; ++i) xblock(m->down_x[i], a);
        const std::vector<float> skip = a;
        b.resize(a.size());
        ref_causal_conv_b(to_nn_conv(m->down_conv), a.data(), T, B, b.data());
        int64_t off = 0;
        for (int i = 0; i < m->n_mid; ++i) {
            resnet(m->mid_res[i], b.data(), tb + size_t(1 + i) * C, a);
            for (int j = 0; j < m->mid_x_count[i]; ++j) xblock(m->mid_x[off + j], a);
            off += m->mid_x_count[i];
            b.swap(a);
        }
        std::vector<float> cat(size_t(R) * 2 * C);
        for (int r = 0; r < R; ++r) {
            std::memcpy(&cat[size_t(r) * 2 * C], &b[size_t(r) * C], size_t(C) * 4);
            std::memcpy(&cat[size_t(r) * 2 * C + C], &skip[size_t(r) * C], size_t(C) * 4);
        }
        resnet(m->up_res, cat.data(), tb + size_t(1 + m->n_mid) * C, a);
        for (int i = 0; i < m->n_up_x; ++i) xblock(m->up_x[i], a);
        b.resize(a.size());
        ref_causal_conv_b(to_nn_conv(m->up_out), a.data(), T, B, b.data());
        block(m->final_conv, m->fn_w, m->fn_b, b.data(), a);
        std::vector<float> o;
        to_nn_conv(m->final_proj).forward(a.data(), R, o);
        std::memcpy(out, o.data(), o.size() * 4);
        return 0;
    } catch (...) {
        return -2;
    }
}

// ---- Qwen3-TTS codec decoder: a .tmod written by the reference's own tmod_write, loaded as Qwen3Weights, decoded by
// Qwen3Weights::codec_forward on the CPU (qwen3.cpp:366-481)
// tensors: n entries of name, DType index, ndim, shape (flat), data pointer and byte count
int ref_tmod_write(const char *path, const char *manifest, int n, const char *const *names, const int32_t *dtypes,
                   const int32_t *ndims, const int64_t *shapes, const void *const *data, const int64_t *nbytes) {
    try {
        std::map<std::string, Tensor> blobs;
        int64_t so = 0;
        for (int i = 0; i < n; ++i) {
            Tensor t;
            t.dtype = DType(dtypes[i]);
            t.shape.assign(shapes + so, shapes + so + ndims[i]);
            so += ndims[i];
            const uint8_t *p = static_cast<const uint8_t *>(data[i]);
            t.bytes.assign(p, p + nbytes[i]);
            blobs[names[i]] = std::move(t);
        }
        tmod_write(path, json::parse(manifest), blobs);
        return 0;
    } catch (...) {
        return -2;
    }
}
struct RefCodec {
    std::unique_ptr<Qwen3Weights> w;
};
void *ref_codec_open(const char *path) {
    try {
        RefCodec *c = new RefCodec();
        c->w.reset(new Qwen3Weights(std::make_shared<TmodFile>(path)));
        return c;
    } catch (...) {
        return nullptr;
    }
}
void ref_codec_close(void *c) { delete static_cast<RefCodec *>(c); }
void *ref_codec_state_new(void *c) { return new CodecState(static_cast<RefCodec *>(c)->w->new_codec_state()); }
void *ref_codec_state_clone(void *c, void *s) {
    return new CodecState(static_cast<RefCodec *>(c)->w->clone_codec_state(*static_cast<CodecState *>(s)));
}
void ref_codec_state_free(void *s) { delete static_cast<CodecState *>(s); }
// codes [F][quantizers] -> pcm (F * samples per frame); returns the sample count, -2 on an error
int64_t ref_codec_forward(void *c, void *s, const int16_t *codes, int F, float *pcm) {
    try {
        std::vector<float> out;
        static_cast<RefCodec *>(c)->w->codec_forward(*static_cast<CodecState *>(s), codes, F, out);
        std::memcpy(pcm, out.data(), out.size() * 4);
        return int64_t(out.size());
    } catch (...) {
        return -2;
    }
}
}
