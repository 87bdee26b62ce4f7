// gpu_hip.cpp — Vox's device interface (src/gpu.hpp + the gpu_* hooks of src/kernels.hpp:88-100) on the
// MI355X backend. Plain C++17: every call goes through the C ABI of include/voxhip.h (libvoxhip.so), which owns
// the HIP context, the device memory and the gfx950 kernels. It replaces gpu_vulkan.cpp + gpu_codec.cpp +
// gpu_f5.cpp in the Vox build the way gpu_stub.cpp does (CMakeLists.txt:42-61), so the resource planner
// (make_plan, via gpu_enumerate) and create_backend (gpu_init("vulkan:N"), family.cpp:90-101) select it unchanged.
//
// Error convention of the reference backend (gpu_vulkan.cpp:568-571, :800-803): no exception escapes, false/-1
// means "compute on the CPU", the reason is kept for gpu_stats().last_error, and one warning goes to stderr.
// gpu_gemm_choice / gpu_gemm_preset (the Vulkan backend's F5 GEMM tuning) answer like gpu_stub.cpp.
#include <cstdio>
#include <cstring>
#include <mutex>

#include "gpu.hpp"
#include "qwen3.hpp"
#include "voxhip.h"

namespace vox {
namespace {

std::once_flag g_warn_once;

void warn_once(const char *what) {
    std::call_once(g_warn_once, [&] { std::fprintf(stderr, "vox: GPU %s failed (%s); falling back to CPU\n", what, voxhip_last_error()); });
}

voxhip_mat to_c(const Mat &m) {
    voxhip_mat c;
    c.type = int32_t(m.type);
    c.data = m.data;
    c.scale = m.scale;
    c.rows = m.rows;
    c.cols = m.cols;
    c.bias = m.bias;
    return c;
}

struct UploadCb {
    const TransformerW *w;
    const std::function<void(const Mat &)> *fn;
};

void on_uploaded(void *user, int32_t layer, int32_t which) {
    auto *cb = static_cast<UploadCb *>(user);
    const LayerW &L = cb->w->layers[size_t(layer)];
    const Mat *m[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
    (*cb->fn)(*m[which]);
}

}  // namespace

bool gpu_init(const std::string &device, std::string &err) {
    char buf[512] = {0};
    if (voxhip_init(device.c_str(), buf, sizeof buf)) return true;
    err = buf;
    return false;
}

bool gpu_active() { return voxhip_active() != 0; }

std::string gpu_device_name() { return voxhip_device_name(); }

int gpu_upload(const Mat &W) {
    const voxhip_mat m = to_c(W);
    return voxhip_upload(&m, 1);
}

GpuStats gpu_stats() {
    voxhip_stats s;
    voxhip_stats_get(&s);
    GpuStats r;
    r.mats_ok = s.mats_ok;
    r.mats_failed = s.mats_failed;
    r.bytes = s.bytes;
    r.bytes_failed = s.bytes_failed;
    r.last_error = voxhip_last_error();
    return r;
}

std::vector<GpuDeviceInfo> gpu_enumerate() {
    std::vector<GpuDeviceInfo> out;
    const int n = voxhip_device_count();
    for (int i = 0; i < n; ++i) {
        voxhip_device_info d;
        if (!voxhip_device_info_get(i, &d)) continue;
        GpuDeviceInfo g;
        g.index = d.index;
        g.name = d.name;
        g.type = d.type;  // "discrete": eligible for make_plan (resources.cpp:376-395)
        g.software = d.software != 0;
        g.unified_memory = d.unified_memory != 0;
        g.vram_total = d.vram_total;
        g.vram_free = d.vram_free;
        g.max_storage_range = d.max_storage_range;
        g.subgroup_arith = d.subgroup_arith != 0;
        g.coop_matrix = d.coop_matrix != 0;
        g.memory_budget = d.memory_budget != 0;
        g.api_version = d.api_version;
        g.vendor_id = d.vendor_id;
        g.driver_version = d.driver_version;
        out.push_back(g);
    }
    return out;
}

std::string gpu_list_devices() {
    const auto devs = gpu_enumerate();
    if (devs.empty()) return "no HIP devices\n";
    std::string out;
    for (const auto &d : devs) {
        char buf[640];
        std::snprintf(buf, sizeof buf, "hip:%d  %s  [%s]  VRAM %.1f GiB, free %.1f GiB\n", d.index, d.name.c_str(), d.type.c_str(),
                      double(d.vram_total) / (1024.0 * 1024 * 1024), double(d.vram_free) / (1024.0 * 1024 * 1024));
        out += buf;
    }
    return out;
}

void gpu_set_vram_limit(uint64_t bytes) { voxhip_set_vram_limit(bytes); }

GpuMemInfo gpu_mem_info() {
    voxhip_mem_info m;
    voxhip_mem_info_get(&m);
    GpuMemInfo r;
    r.used = m.used;
    r.limit = m.limit;
    r.device_free = m.device_free;
    r.device_total = m.device_total;
    r.device_index = m.device_index;
    return r;
}

int gpu_xfmr_create(const TransformerW &w, const char *name, int n_layers, const std::function<void(const Mat &)> &uploaded) {
    if (w.layers.empty()) return -1;
    std::vector<voxhip_layer> L(w.layers.size());
    for (size_t i = 0; i < w.layers.size(); ++i) {
        const LayerW &s = w.layers[i];
        voxhip_layer &d = L[i];
        d.q = to_c(s.q); d.k = to_c(s.k); d.v = to_c(s.v); d.o = to_c(s.o);
        d.gate = to_c(s.gate); d.up = to_c(s.up); d.down = to_c(s.down);
        d.qn = s.qn; d.kn = s.kn; d.ln1 = s.ln1; d.ln2 = s.ln2;
        d.attn_scale = s.attn_scale; d.mlp_scale = s.mlp_scale;
    }
    voxhip_xfmr_desc desc;
    desc.n_layers = int32_t(L.size());
    desc.layers = L.data();
    desc.final_norm = w.final_norm;
    desc.hidden = w.hidden; desc.heads = w.heads; desc.kv_heads = w.kv_heads; desc.head_dim = w.head_dim; desc.inter = w.inter;
    desc.eps = w.eps;
    desc.theta = w.theta;
    desc.window = w.window;
    desc.inv_freq = w.inv_freq.data();
    UploadCb cb{&w, &uploaded};
    const int id = voxhip_xfmr_create(&desc, name, n_layers, uploaded ? on_uploaded : nullptr, &cb);
    if (id < 0) warn_once("transformer setup");
    return id;
}

int gpu_seq_create(int xfmr, int64_t capacity) { return voxhip_seq_create(xfmr, capacity); }

void gpu_seq_free(int seq) { voxhip_seq_free(seq); }

bool gpu_matmul(const Mat &W, const float *x, int64_t m, float *y) {
    if (W.gpu < 0) return false;
    if (voxhip_matmul(W.gpu, x, m, y)) return true;
    warn_once("matmul");
    return false;
}

bool gpu_xfmr_forward(const TransformerW &w, int seq, int64_t pos0, const float *x, int64_t m, float *out_last, const Mat *in_proj,
                      const Mat *head, float *head_out) {
    if (w.gpu_id < 0) return false;
    if (voxhip_xfmr_forward(w.gpu_id, seq, pos0, x, m, out_last, in_proj ? in_proj->gpu : -1, head ? head->gpu : -1, head_out))
        return true;
    std::fprintf(stderr, "vox: GPU transformer failed: %s\n", voxhip_last_error());
    return false;
}

bool gpu_xfmr_forward_hidden(const TransformerW &w, int seq, int64_t pos0, const float *x, int64_t m, float *hidden_out) {
    if (w.gpu_id < 0) return false;
    if (voxhip_xfmr_forward_hidden(w.gpu_id, seq, pos0, x, m, hidden_out)) return true;
    std::fprintf(stderr, "vox: GPU transformer failed: %s\n", voxhip_last_error());
    return false;
}

bool gpu_xfmr_forward_pair(const TransformerW &w, int seq0, int seq1, int64_t pos, const float *x2, const Mat *head, float *out2,
                           float *head_out2) {
    if (w.gpu_id < 0 || (head && head->gpu < 0)) return false;
    if (voxhip_xfmr_forward_pair(w.gpu_id, seq0, seq1, pos, x2, head ? head->gpu : -1, out2, head_out2)) return true;
    std::fprintf(stderr, "vox: GPU transformer (pair) failed: %s\n", voxhip_last_error());
    return false;
}

// ---- F5-TTS DiT step (gpu.hpp:62-91): the description maps field by field; the vocoder fields are ignored
int gpu_f5_create(const GpuF5Desc &d) {
    std::vector<voxhip_f5_block> blocks;
    for (const GpuF5Desc::Block &b : d.blocks) blocks.push_back({b.ada, b.q, b.k, b.v, b.o, b.ff1, b.ff2});
    auto conv = [](const GpuF5Conv &c) { return voxhip_f5_conv{c.w, c.b, c.cin, c.cout, c.K, c.groups}; };
    voxhip_f5_desc c{};
    c.dim = d.dim; c.depth = d.depth; c.heads = d.heads; c.dim_head = d.dim_head; c.ff_mult = d.ff_mult;
    c.mel_dim = d.mel_dim; c.text_dim = d.text_dim; c.pe_attn_head = d.pe_attn_head;
    c.in_proj = d.in_proj; c.norm_out = d.norm_out; c.proj_out = d.proj_out;
    c.blocks = blocks.data(); c.pos1 = conv(d.pos1); c.pos2 = conv(d.pos2);
    if (int(blocks.size()) != d.depth) return -1;
    // Vocos (vocos_dim 0: the vocoder stays on the CPU, f5.cpp:381-385)
    std::vector<voxhip_f5_vblock> vb;
    for (const GpuF5Desc::VBlock &b : d.v_blocks) vb.push_back({conv(b.dw), b.ln_w, b.ln_b, b.gamma, b.pw1, b.pw2});
    c.vocos_dim = d.vocos_dim; c.vocos_inter = d.vocos_inter; c.vocos_out = d.vocos_out;
    c.v_embed = conv(d.v_embed);
    c.v_ln_w = d.v_ln_w; c.v_ln_b = d.v_ln_b; c.v_fln_w = d.v_fln_w; c.v_fln_b = d.v_fln_b;
    c.v_blocks = vb.data(); c.n_vblocks = int32_t(vb.size()); c.v_head = d.v_head;
    const int id = voxhip_f5_create(&c);
    if (id < 0) warn_once("F5 graph");
    return id;
}
bool gpu_f5_begin(int id, int B, int N, const float *cat0, const float *rope) { return voxhip_f5_begin(id, B, N, cat0, rope) != 0; }
bool gpu_f5_step(int id, const float *x, const float *ts, float *out) {
    if (voxhip_f5_step(id, x, ts, out)) return true;
    std::fprintf(stderr, "vox: GPU F5 step failed: %s\n", voxhip_last_error());
    return false;
}
void gpu_f5_end(int id) { (void)voxhip_f5_end(id); }
// Vocos up to the head on the device (gpu_f5.cpp:334-373); false keeps it on the CPU (f5.cpp:787-791)
bool gpu_f5_vocos(int id, const float *mel, int T, std::vector<float> &head) {
    if (id < 0 || T <= 0) return false;
    int vout = 0;
    if (!voxhip_f5_vocos_out(id, &vout) || vout <= 0) return false;  // created without Vocos: the CPU runs it
    head.resize(size_t(T) * size_t(vout));
    if (voxhip_f5_vocos(id, mel, T, head.data())) return true;
    std::fprintf(stderr, "vox: Vocos on the GPU failed: %s\n", voxhip_last_error());
    return false;
}

// The Qwen3-TTS codec decoder (gpu_codec.cpp:205-556): the layers of Qwen3Weights (their matrices already uploaded by
// Qwen3Weights::upload_gpu, qwen3.cpp:326-331) flattened for the C ABI; -1 / false keeps the decoder on the CPU
// (qwen3.cpp:332-338, :396-400).
int gpu_codec_create(const Qwen3Weights &w) {
    auto conv = [](const CConv &c) { return voxhip_codec_conv{c.w.gpu, c.K, c.cin, c.cout, c.dil}; };
    auto snake = [](const Snake &s) { return voxhip_codec_snake{s.a.data(), s.inv_b.data()}; };
    const TransformerW &pt = w.pt;
    std::vector<voxhip_layer> L(pt.layers.size());
    std::vector<int32_t> ids;
    for (size_t i = 0; i < pt.layers.size(); ++i) {
        const LayerW &s = pt.layers[i];
        for (const Mat *m : {&s.q, &s.k, &s.v, &s.o, &s.gate, &s.up, &s.down}) ids.push_back(m->gpu);
        L[i].qn = s.qn; L[i].kn = s.kn; L[i].ln1 = s.ln1; L[i].ln2 = s.ln2;
        L[i].attn_scale = s.attn_scale; L[i].mlp_scale = s.mlp_scale;
    }
    std::vector<voxhip_codec_up> ups;
    for (const Qwen3Weights::UpStage &u : w.up) {
        if (u.tr.K != u.tr.stride) return -1;  // as gpu_codec.cpp:246
        ups.push_back({u.tr.w.gpu, u.tr.K, u.tr_b, u.dw.w, u.dw.b, u.dw.K, u.ln_w, u.ln_b, u.gamma, u.pw1.gpu, u.pw2.gpu});
    }
    std::vector<voxhip_codec_block> blocks;
    for (const Qwen3Weights::DecBlock &d : w.blocks) {
        voxhip_codec_block b{};
        b.act = snake(d.act);
        b.tr = d.tr.w.gpu; b.K = d.tr.K; b.stride = d.tr.stride; b.cin = d.tr.cin; b.cout = d.tr.cout; b.tr_b = d.tr_b;
        for (int u = 0; u < 3; ++u) {
            b.a1[u] = snake(d.a1[u]); b.a2[u] = snake(d.a2[u]);
            b.c1[u] = conv(d.c1[u]); b.c2[u] = conv(d.c2[u]);
        }
        blocks.push_back(b);
    }
    voxhip_codec_desc c{};
    c.codebook_dim = w.cc.codebook_dim; c.latent = w.cc.latent;
    c.pre_conv = conv(w.pre_conv); c.pt_in = w.pt_in.gpu; c.pt_out = w.pt_out.gpu;
    c.pt.n_layers = int32_t(L.size()); c.pt.layers = L.data(); c.pt.final_norm = pt.final_norm;
    c.pt.hidden = pt.hidden; c.pt.heads = pt.heads; c.pt.kv_heads = pt.kv_heads; c.pt.head_dim = pt.head_dim; c.pt.inter = pt.inter;
    c.pt.eps = pt.eps; c.pt.theta = pt.theta; c.pt.window = pt.window; c.pt.inv_freq = pt.inv_freq.data();
    c.pt_mats = ids.data();
    c.ups = ups.data(); c.n_ups = int32_t(ups.size());
    c.conv0 = conv(w.conv0);
    c.blocks = blocks.data(); c.n_blocks = int32_t(blocks.size());
    c.final_act = snake(w.final_act); c.final_conv = conv(w.final_conv);
    const int id = voxhip_codec_create(&c);
    if (id < 0) warn_once("codec decoder");
    return id;
}
int gpu_codec_state_new(int codec) { return voxhip_codec_state_new(codec); }
int gpu_codec_state_clone(int state) { return voxhip_codec_state_clone(state); }
void gpu_codec_state_free(int state) { (void)voxhip_codec_state_free(state); }
// Appends F frames of PCM (F <= kGpuCodecMaxFrames; codec_forward, qwen3.cpp:396-400, calls in such chunks).
bool gpu_codec_forward(int codec, int state, const float *z, int F, std::vector<float> &pcm) {
    if (F <= 0) return true;
    int32_t spf = 0;
    if (!voxhip_codec_spf(codec, &spf)) return false;
    const size_t off = pcm.size();
    pcm.resize(off + size_t(F) * size_t(spf));
    int64_t n = 0;
    if (!voxhip_codec_forward(codec, state, z, F, pcm.data() + off, &n)) {
        pcm.resize(off);
        std::fprintf(stderr, "vox: GPU codec decoder failed: %s\n", voxhip_last_error());
        return false;
    }
    pcm.resize(off + size_t(n));
    return true;
}

// The CosyVoice2 / Chatterbox flow estimator (gpu_f5.cpp:382-556): the description flattened for the C ABI (mid
// block i's transformer list as mid_x_count[i] consecutive entries); -1 / false keeps the flow on the CPU
// (cosyvoice.cpp:557, :828-830).
int gpu_cosy_create(const GpuCosyDesc &d) {
    auto conv = [](const GpuF5Conv &c) { return voxhip_f5_conv{c.w, c.b, c.cin, c.cout, c.K, c.groups}; };
    auto res = [&](const GpuCosyDesc::Res &r) {
        return voxhip_cosy_res{conv(r.c1), conv(r.c2), conv(r.res), r.n1w, r.n1b, r.n2w, r.n2b};
    };
    auto xb = [](const GpuCosyDesc::X &x) {
        return voxhip_cosy_x{x.n1w, x.n1b, x.n3w, x.n3b, x.q, x.k, x.v, x.o, x.ff1, x.ff2, x.ff_dim};
    };
    std::vector<voxhip_cosy_res> mid;
    for (const GpuCosyDesc::Res &r : d.mid_res) mid.push_back(res(r));
    std::vector<voxhip_cosy_x> down, up, midx;
    std::vector<int32_t> counts;
    for (const GpuCosyDesc::X &x : d.down_x) down.push_back(xb(x));
    for (const GpuCosyDesc::X &x : d.up_x) up.push_back(xb(x));
    for (const std::vector<GpuCosyDesc::X> &v : d.mid_x) {
        counts.push_back(int32_t(v.size()));
        for (const GpuCosyDesc::X &x : v) midx.push_back(xb(x));
    }
    if (d.mid_x.size() != d.mid_res.size()) return -1;
    voxhip_cosy_desc c{};
    c.M = d.M; c.C = d.C; c.heads = d.heads; c.head_dim = d.head_dim;
    c.down_res = res(d.down_res); c.up_res = res(d.up_res);
    c.mid_res = mid.data(); c.n_mid = int32_t(mid.size());
    c.down_x = down.data(); c.n_down_x = int32_t(down.size());
    c.up_x = up.data(); c.n_up_x = int32_t(up.size());
    c.mid_x = midx.data(); c.mid_x_count = counts.data();
    c.down_conv = conv(d.down_conv); c.up_out = conv(d.up_out); c.final_conv = conv(d.final_conv);
    c.final_proj = conv(d.final_proj);
    c.fn_w = d.fn_w; c.fn_b = d.fn_b;
    const int id = voxhip_cosy_create(&c);
    if (id < 0) warn_once("flow estimator");
    return id;
}
bool gpu_cosy_begin(int id, int T, const float *in0) { return voxhip_cosy_begin(id, T, in0) != 0; }
bool gpu_cosy_step(int id, const float *x, const float *tb, float *out) {
    if (voxhip_cosy_step(id, x, tb, out)) return true;
    std::fprintf(stderr, "vox: GPU flow estimator step failed: %s\n", voxhip_last_error());
    return false;
}
void gpu_cosy_end(int id) { (void)voxhip_cosy_end(id); }

// The code predictor's frame loop (gpu_vulkan.cpp:968-1045): the same sampler settings for every codebook, the
// draw (frame, cb) of each; matrices the backend does not hold keep the frame on the CPU.
bool gpu_pred_frame(const TransformerW &w, int seq, const float *in2, const Mat *in_proj, const std::vector<Mat> &heads,
                    const std::vector<Mat> &embs, const GpuSampleCfg &c, int32_t *codes) {
    if (w.gpu_id < 0 || heads.empty() || (in_proj && in_proj->gpu < 0)) return false;
    std::vector<int> hid, eid;
    for (const Mat &h : heads) {
        if (h.gpu < 0) return false;
        hid.push_back(h.gpu);
    }
    for (const Mat &e : embs) {
        if (e.gpu < 0) return false;
        eid.push_back(e.gpu);
    }
    voxhip_sample_cfg sc{};
    sc.temperature = c.temperature; sc.top_p = c.top_p; sc.top_k = c.top_k; sc.repetition_penalty = 1.0f;
    sc.key0 = c.key0; sc.key1 = c.key1; sc.frame = c.frame; sc.eos_code = -1;
    if (voxhip_pred_frame(w.gpu_id, seq, in2, in_proj ? in_proj->gpu : -1, hid.data(), int(hid.size()), eid.data(),
                          int(eid.size()), &sc, codes))
        return true;
    std::fprintf(stderr, "vox: GPU predictor loop failed: %s\n", voxhip_last_error());
    return false;
}

// ---- not provided by this backend yet: the callers compute on the CPU (gpu_stub.cpp behaviour)
std::string gpu_gemm_choice() { return ""; }
void gpu_gemm_preset(const std::string &) {}

}  // namespace vox
