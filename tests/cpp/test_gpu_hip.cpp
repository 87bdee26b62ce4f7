// test_gpu_hip.cpp — drives the drop-in through Vox's own C++ device interface, the way Vox's callers do
// (qwen3.cpp:302-344 upload_gpu, kernels.cpp:908-916 transformer_step_fused, kernels.cpp:656 matmul, qwen3.cpp:396-400
// the codec decoder's chunks), and checks the results against the C oracle. Run by tests/test_gpu_dropin.py; exit status 0 = all passed.
#include <cmath>
#include <cstdio>
#include <random>
#include <vector>

#include "gpu.hpp"
#include "qwen3.hpp"
#include "vox_oracle.h"

using namespace vox;

static int g_fail = 0, g_pass = 0;
#define CHECK(c)                                                                                  \
    do {                                                                                          \
        if (c) ++g_pass;                                                                          \
        else { ++g_fail; std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); }      \
    } while (0)

static float rel(const float *a, const float *b, size_t n) {
    double mx = 0, mb = 0;
    for (size_t i = 0; i < n; ++i) { mx = std::max(mx, double(std::fabs(a[i] - b[i]))); mb = std::max(mb, double(std::fabs(b[i]))); }
    return float(mx / std::max(1.0, mb));
}

struct Q8 {
    std::vector<int8_t> q;
    std::vector<float> s;
    int64_t rows, cols;
    Q8(std::mt19937 &rng, int64_t r, int64_t c) : rows(r), cols(c) {
        std::normal_distribution<float> nd(0.f, 0.02f);
        std::vector<float> w(static_cast<size_t>(r * c));
        for (auto &v : w) v = nd(rng);
        q.resize(w.size());
        s.resize(size_t(r * (c / 32)));
        vo_quantize_q8(w.data(), r, c, q.data(), s.data());
    }
    Mat mat() const {
        Mat m;
        m.type = WType::Q8; m.data = reinterpret_cast<const uint8_t *>(q.data()); m.scale = s.data(); m.rows = rows; m.cols = cols;
        return m;
    }
    vo_mat omat() const { return vo_mat{VO_Q8, q.data(), s.data(), rows, cols, nullptr}; }
};

int main() {
    std::string err;
    if (!gpu_init("vulkan:0", err)) {  // the spec create_backend passes (family.cpp:94)
        std::fprintf(stderr, "gpu_init failed: %s\n", err.c_str());
        return 2;
    }
    CHECK(gpu_active());
    auto devs = gpu_enumerate();
    CHECK(!devs.empty() && devs[0].type == "discrete" && !devs[0].software && devs[0].vram_total > (uint64_t(100) << 30));
    CHECK(gpu_mem_info().device_index == 0);
    std::printf("%s", gpu_list_devices().c_str());

    std::mt19937 rng(1);
    std::normal_distribution<float> nd(0.f, 1.f);
    const int H = 256, nh = 4, nkv = 2, hd = 128, I = 512, NL = 2, V = 200;
    // ---- matmul through Mat::gpu (kernels.cpp:656)
    Q8 w(rng, 300, H);
    Mat W = w.mat();
    W.gpu = gpu_upload(W);
    CHECK(W.gpu >= 0);
    std::vector<float> x(5 * H), y(5 * 300), yr(5 * 300);
    for (auto &v : x) v = nd(rng);
    CHECK(gpu_matmul(W, x.data(), 5, y.data()));
    vo_mat ow = w.omat();
    vo_matmul(&ow, x.data(), 5, yr.data(), 1);
    CHECK(rel(y.data(), yr.data(), y.size()) < 1e-5f);

    // ---- a transformer on the device (qwen3.cpp:302-344), stepped like transformer_step_fused
    std::vector<Q8> mats;
    std::vector<std::vector<float>> norms;
    TransformerW T;
    T.hidden = H; T.heads = nh; T.kv_heads = nkv; T.head_dim = hd; T.inter = I; T.eps = 1e-6f; T.theta = 1e6;
    T.inv_freq.resize(hd / 2);
    vo_rope_inv_freq(hd, 1e6, T.inv_freq.data());
    auto vec = [&](int n, float mean) {
        std::vector<float> v(static_cast<size_t>(n));
        for (auto &e : v) e = mean + 0.02f * nd(rng);
        norms.push_back(v);
        return norms.size() - 1;
    };
    const int64_t shapes[7][2] = {{nh * hd, H}, {nkv * hd, H}, {nkv * hd, H}, {H, nh * hd}, {I, H}, {I, H}, {H, I}};
    std::vector<size_t> nidx;
    for (int l = 0; l < NL; ++l) {
        for (int j = 0; j < 7; ++j) mats.emplace_back(rng, shapes[j][0], shapes[j][1]);
        for (int j = 0; j < 2; ++j) nidx.push_back(vec(H, 1.f));
        for (int j = 0; j < 2; ++j) nidx.push_back(vec(hd, 1.f));
    }
    const size_t fin = vec(H, 1.f);
    std::vector<vo_layer> OL(NL);
    for (int l = 0; l < NL; ++l) {
        LayerW L;
        Mat *dst[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
        vo_mat *od[7] = {&OL[l].q, &OL[l].k, &OL[l].v, &OL[l].o, &OL[l].gate, &OL[l].up, &OL[l].down};
        for (int j = 0; j < 7; ++j) { *dst[j] = mats[size_t(7 * l + j)].mat(); *od[j] = mats[size_t(7 * l + j)].omat(); }
        L.ln1 = norms[nidx[size_t(4 * l)]].data(); L.ln2 = norms[nidx[size_t(4 * l + 1)]].data();
        L.qn = norms[nidx[size_t(4 * l + 2)]].data(); L.kn = norms[nidx[size_t(4 * l + 3)]].data();
        OL[l].ln1 = L.ln1; OL[l].ln2 = L.ln2; OL[l].qn = L.qn; OL[l].kn = L.kn;
        T.layers.push_back(L);
    }
    T.final_norm = norms[fin].data();
    int released = 0;
    T.gpu_id = gpu_xfmr_create(T, "talker", -1, [&](const Mat &) { ++released; });
    CHECK(T.gpu_id >= 0);
    CHECK(released == 7 * NL);
    Q8 hw(rng, V, H);
    Mat head = hw.mat();
    head.gpu = gpu_upload(head);
    const int seq = gpu_seq_create(T.gpu_id, 64);
    CHECK(seq >= 0);

    vo_xfmr OX{NL, OL.data(), T.final_norm, H, nh, nkv, hd, I, T.eps, T.inv_freq.data()};
    const int64_t kd = nkv * hd;
    std::vector<float> kc(static_cast<size_t>(NL * 64 * kd)), vc(kc.size());
    vo_kv okv{kc.data(), vc.data(), 64, 0, 1, 1};
    vo_mat ohead = hw.omat();
    int64_t pos = 0;
    for (int step = 0; step < 5; ++step) {
        const int64_t m = step == 0 ? 4 : 1;  // a prompt, then decode steps
        std::vector<float> xi(static_cast<size_t>(m * H)), out(H), logits(V), ro(H), rl(V);
        for (auto &v : xi) v = nd(rng);
        CHECK(gpu_xfmr_forward(T, seq, pos, xi.data(), m, out.data(), nullptr, &head, logits.data()));
        CHECK(vo_transformer_forward(&OX, &okv, xi.data(), m, ro.data(), nullptr) == 0);
        vo_matmul(&ohead, ro.data(), 1, rl.data(), 1);
        const float e1 = rel(out.data(), ro.data(), H), e2 = rel(logits.data(), rl.data(), V);
        std::printf("step %d (m=%lld): hidden rel err %.2e, logits rel err %.2e\n", step, (long long)m, e1, e2);
        CHECK(e1 < 1e-3f && e2 < 1e-3f);
        pos += m;
    }
    // capacity is enforced, and the failure is reported as false (the caller falls back or fails loudly)
    std::vector<float> big(static_cast<size_t>(64 * H), 0.f), o2(H);
    CHECK(!gpu_xfmr_forward(T, seq, pos, big.data(), 64, o2.data()));
    CHECK(!gpu_stats().last_error.empty());
    gpu_seq_free(seq);
    CHECK(gpu_seq_create(T.gpu_id, 32) == seq);  // pooled buffers are reused (gpu_vulkan.cpp:834-837)
    // the code predictor's frame (backend_qwen3.cpp:426-445 calls gpu_pred_frame): the same transformer as a 6-codebook
    // predictor without in_proj, f32 code embeddings; the codes must equal the loop run pass by pass through
    // gpu_xfmr_forward with the oracle's sampler (draw (frame, cb)) and the oracle's mat_row
    {
        const int G = 6;
        std::vector<Q8> hq;
        std::vector<Mat> heads, embs;
        for (int i = 0; i < G - 1; ++i) hq.emplace_back(rng, V, H);
        for (auto &h : hq) {
            heads.push_back(h.mat());
            heads.back().gpu = gpu_upload(heads.back());
        }
        std::vector<std::vector<float>> ew(G - 2, std::vector<float>(size_t(V * H)));
        for (auto &e : ew) for (auto &v : e) v = nd(rng);
        for (auto &e : ew) {
            Mat m;
            m.type = WType::F32; m.data = reinterpret_cast<const uint8_t *>(e.data()); m.rows = V; m.cols = H;
            m.gpu = gpu_upload(m);
            embs.push_back(m);
        }
        GpuSampleCfg c;
        c.temperature = 0.9f; c.top_k = 20; c.top_p = 0.95f; c.key0 = 77; c.key1 = 0; c.frame = 3;
        std::vector<float> in2(static_cast<size_t>(2 * H));
        for (auto &v : in2) v = nd(rng);
        const int s1 = gpu_seq_create(T.gpu_id, 16), s2 = gpu_seq_create(T.gpu_id, 16);
        std::vector<int32_t> codes(G, -1);
        codes[0] = 5;
        CHECK(gpu_pred_frame(T, s1, in2.data(), nullptr, heads, embs, c, codes.data()));
        CHECK(codes[0] == 5);  // the talker's code stays the caller's
        std::vector<float> xin = in2, out(H), logits(V);
        int64_t p = 0;
        bool same = true;
        for (int cb = 1; cb < G; ++cb) {
            const int64_t m = cb == 1 ? 2 : 1;
            CHECK(gpu_xfmr_forward(T, s2, p, xin.data(), m, out.data(), nullptr, &heads[size_t(cb - 1)], logits.data()));
            const int32_t want = vo_sample_logits(logits.data(), V, c.temperature, c.top_p, c.top_k, 1.0f, nullptr, 0,
                                                  vo_uniform(77, 3, uint32_t(cb), 0));
            same = same && codes[size_t(cb)] == want;
            p += m;
            if (cb + 1 < G) {
                vo_mat oe{VO_F32, ew[size_t(cb - 1)].data(), nullptr, V, H, nullptr};
                xin.assign(size_t(H), 0.f);
                vo_mat_row(&oe, want, xin.data());
            }
        }
        std::printf("pred frame codes:");
        for (int cb = 1; cb < G; ++cb) std::printf(" %d", codes[size_t(cb)]);
        std::printf("\n");
        CHECK(same);
        gpu_seq_free(s1);
        gpu_seq_free(s2);
    }
    // an empty F5 / estimator descriptor (no blocks, no matrices) is refused with -1, so the caller keeps its CPU path
    CHECK(gpu_f5_create(GpuF5Desc{}) == -1 && gpu_cosy_create(GpuCosyDesc{}) == -1);

    // ---- the codec decoder: a Qwen3Weights as upload_gpu leaves it (matrices on the device), decoded in two chunks
    {
        std::vector<std::vector<float>> keep;  // host arrays of the weights (the "mmap")
        auto arr = [&](size_t n, float sd, float mean = 0.f) {
            std::normal_distribution<float> d(mean, sd);
            keep.emplace_back(n);
            for (auto &v : keep.back()) v = d(rng);
            return keep.back().data();
        };
        auto fmat = [&](int64_t r, int64_t c, float sd, bool bias) {
            Mat m;
            m.type = WType::F32; m.data = reinterpret_cast<const uint8_t *>(arr(size_t(r * c), sd)); m.rows = r; m.cols = c;
            if (bias) m.bias = arr(size_t(r), 0.05f);
            m.gpu = gpu_upload(m);
            return m;
        };
        auto omat = [](const Mat &m) { return vo_mat{VO_F32, m.data, nullptr, m.rows, m.cols, m.bias}; };
        auto cconv = [&](int K, int cin, int cout, int dil, float gain) {
            CConv c;
            c.w = fmat(cout, int64_t(K) * cin, gain / std::sqrt(float(K * cin)), true);
            c.K = K; c.cin = cin; c.cout = cout; c.dil = dil;
            return c;
        };
        auto snake = [&](int C) {
            Snake sn;
            const float *al = arr(size_t(C), 0.3f), *be = arr(size_t(C), 0.3f);
            sn.a.resize(size_t(C)); sn.inv_b.resize(size_t(C));
            vo_snake_params(al, be, C, sn.a.data(), sn.inv_b.data());
            return sn;
        };
        const int CD = 16, L = 16, HH = 32, heads = 2, hdc = 16, IC = 64, W = 5;
        Qwen3Weights qw;
        qw.cc.codebook_dim = CD; qw.cc.latent = L; qw.cc.hidden = HH; qw.cc.heads = heads; qw.cc.kv_heads = heads;
        qw.cc.head_dim = hdc; qw.cc.window = W; qw.cc.inter = IC; qw.cc.layers = 1; qw.cc.decoder_dim = 16;
        qw.cc.up_rates = {2}; qw.cc.up_ratios = {2};
        qw.pre_conv = cconv(3, CD, L, 1, 1.f);
        qw.pt_in = fmat(HH, L, 0.25f, true);
        qw.pt_out = fmat(L, HH, 0.18f, true);
        TransformerW &pt = qw.pt;
        pt.hidden = HH; pt.heads = heads; pt.kv_heads = heads; pt.head_dim = hdc; pt.inter = IC; pt.eps = 1e-5f;
        pt.theta = 10000.0; pt.window = W;
        pt.inv_freq.resize(size_t(hdc / 2));
        vo_rope_inv_freq(hdc, 10000.0, pt.inv_freq.data());
        LayerW Lw;
        Lw.q = fmat(heads * hdc, HH, 0.18f, false); Lw.k = fmat(heads * hdc, HH, 0.18f, false);
        Lw.v = fmat(heads * hdc, HH, 0.18f, false); Lw.o = fmat(HH, heads * hdc, 0.18f, false);
        Lw.gate = fmat(IC, HH, 0.18f, false); Lw.up = fmat(IC, HH, 0.18f, false); Lw.down = fmat(HH, IC, 0.12f, false);
        Lw.ln1 = arr(size_t(HH), 0.1f, 1.f); Lw.ln2 = arr(size_t(HH), 0.1f, 1.f);
        Lw.attn_scale = arr(size_t(HH), 0.1f, 0.5f); Lw.mlp_scale = arr(size_t(HH), 0.1f, 0.5f);
        pt.layers.push_back(Lw);
        pt.final_norm = arr(size_t(HH), 0.1f, 1.f);
        Qwen3Weights::UpStage u;
        u.tr.w = fmat(2 * L, L, 0.25f, false); u.tr.K = 2; u.tr.stride = 2; u.tr.cin = L; u.tr.cout = L;
        u.tr_b = arr(size_t(L), 0.05f);
        u.dw.w = arr(size_t(L) * 7, 0.3f); u.dw.b = arr(size_t(L), 0.05f); u.dw.K = 7; u.dw.C = L;
        u.ln_w = arr(size_t(L), 0.1f, 1.f); u.ln_b = arr(size_t(L), 0.1f); u.gamma = arr(size_t(L), 0.3f);
        u.pw1 = fmat(4 * L, L, 0.25f, true); u.pw2 = fmat(L, 4 * L, 0.12f, true);
        qw.up.push_back(u);
        qw.conv0 = cconv(7, L, 16, 1, 1.f);
        Qwen3Weights::DecBlock db;
        db.act = snake(16);
        db.tr.w = fmat(4 * 8, 16, 0.18f, false); db.tr.K = 4; db.tr.stride = 2; db.tr.cin = 16; db.tr.cout = 8;
        db.tr_b = arr(8, 0.05f);
        for (int k = 0; k < 3; ++k) {
            db.a1[k] = snake(8); db.a2[k] = snake(8);
            db.c1[k] = cconv(7, 8, 8, k == 0 ? 1 : k == 1 ? 3 : 9, 0.3f);
            db.c2[k] = cconv(1, 8, 8, 1, 0.3f);
        }
        qw.blocks.push_back(db);
        qw.final_act = snake(8);
        qw.final_conv = cconv(7, 8, 1, 1, 0.1f);
        const int codec = gpu_codec_create(qw);
        CHECK(codec >= 0);
        // the same decoder for the oracle
        auto ocv = [&](const CConv &c) { return vo_cconv{omat(c.w), c.K, c.cin, c.cout, c.dil}; };
        auto osn = [](const Snake &sn) { return vo_snake{sn.a.data(), sn.inv_b.data()}; };
        vo_layer ol{};
        ol.q = omat(Lw.q); ol.k = omat(Lw.k); ol.v = omat(Lw.v); ol.o = omat(Lw.o);
        ol.gate = omat(Lw.gate); ol.up = omat(Lw.up); ol.down = omat(Lw.down);
        ol.ln1 = Lw.ln1; ol.ln2 = Lw.ln2; ol.attn_scale = Lw.attn_scale; ol.mlp_scale = Lw.mlp_scale;
        vo_codec_up ou{omat(u.tr.w), u.tr_b, 2, u.dw.w, u.dw.b, 7, u.ln_w, u.ln_b, u.gamma, omat(u.pw1), omat(u.pw2)};
        vo_codec_block ob{};
        ob.act = osn(db.act); ob.tr = omat(db.tr.w); ob.tr_b = db.tr_b; ob.K = 4; ob.stride = 2; ob.cin = 16; ob.cout = 8;
        for (int k = 0; k < 3; ++k) { ob.a1[k] = osn(db.a1[k]); ob.a2[k] = osn(db.a2[k]); ob.c1[k] = ocv(db.c1[k]); ob.c2[k] = ocv(db.c2[k]); }
        vo_codec oc{};
        oc.codebook_dim = CD; oc.latent = L; oc.n_up = 1; oc.n_blocks = 1;
        oc.pre_conv = ocv(qw.pre_conv); oc.pt_in = omat(qw.pt_in); oc.pt_out = omat(qw.pt_out);
        oc.pt = vo_xfmr{1, &ol, pt.final_norm, HH, heads, heads, hdc, IC, 1e-5f, pt.inv_freq.data(), W};
        oc.ups = &ou; oc.conv0 = ocv(qw.conv0); oc.blocks = &ob; oc.final_act = osn(qw.final_act); oc.final_conv = ocv(qw.final_conv);
        const int F = 11;
        std::vector<float> z(size_t(F) * CD);
        for (auto &v : z) v = nd(rng);
        vo_codec_state *os = vo_codec_state_new(&oc, 64);
        std::vector<float> want(size_t(F) * size_t(vo_codec_spf(&oc)));
        CHECK(vo_codec_forward(&oc, os, z.data(), F, want.data()) == int64_t(want.size()));
        vo_codec_state_free(os);
        if (codec >= 0) {
            const int st = gpu_codec_state_new(codec);
            CHECK(st >= 0);
            std::vector<float> pcm;
            CHECK(gpu_codec_forward(codec, st, z.data(), 6, pcm) && gpu_codec_forward(codec, st, z.data() + 6 * CD, F - 6, pcm));
            CHECK(pcm.size() == want.size() && rel(pcm.data(), want.data(), want.size()) < 1e-3f);
            CHECK(!gpu_codec_forward(codec, st, z.data(), kGpuCodecMaxFrames + 1, pcm));  // more than a chunk: false
            gpu_codec_state_free(st);
        }
    }
    std::printf("%d passed, %d failed\n", g_pass, g_fail);
    return g_fail ? 1 : 0;
}
