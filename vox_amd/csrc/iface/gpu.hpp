// gpu.hpp — Vox's device interface (reference: src/gpu.hpp:10-119), restated with the same declarations so
// that gpu_hip.cpp builds on its own; inside Vox, gpu_hip.cpp includes Vox's own src/gpu.hpp.
#pragma once
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace vox {

bool gpu_init(const std::string &device, std::string &err);
bool gpu_active();
std::string gpu_device_name();
int gpu_upload(const Mat &W);
struct GpuStats {
    int64_t mats_ok = 0, mats_failed = 0;
    uint64_t bytes = 0, bytes_failed = 0;
    std::string last_error;
};
GpuStats gpu_stats();
std::string gpu_list_devices();
struct GpuDeviceInfo {
    int index = 0;
    std::string name, type;
    bool software = false;
    bool unified_memory = false;
    uint64_t vram_total = 0, vram_free = 0, max_storage_range = 0;
    bool subgroup_arith = false, coop_matrix = false, memory_budget = false;
    uint32_t api_version = 0, vendor_id = 0, driver_version = 0;
};
std::vector<GpuDeviceInfo> gpu_enumerate();
void gpu_set_vram_limit(uint64_t bytes);
struct GpuMemInfo {
    uint64_t used = 0, limit = 0, device_free = 0, device_total = 0;
    int device_index = -1;
};
GpuMemInfo gpu_mem_info();
int gpu_xfmr_create(const TransformerW &w, const char *name = "xfmr", int n_layers = -1,
                    const std::function<void(const Mat &)> &uploaded = nullptr);
int gpu_seq_create(int xfmr, int64_t capacity);
void gpu_seq_free(int seq);

struct GpuSampleCfg {
    float temperature = 0.9f, top_p = 1.0f;
    int32_t top_k = 50;
    uint32_t key0 = 0, key1 = 0;
    uint64_t frame = 0;
};
bool gpu_pred_frame(const TransformerW &w, int seq, const float *in2, const Mat *in_proj, const std::vector<Mat> &heads,
                    const std::vector<Mat> &embs, const GpuSampleCfg &cfg, int32_t *codes);

class Qwen3Weights;
int gpu_codec_create(const Qwen3Weights &w);
int gpu_codec_state_new(int codec);
int gpu_codec_state_clone(int state);
void gpu_codec_state_free(int state);
bool gpu_codec_forward(int codec, int state, const float *z, int F, std::vector<float> &pcm);
constexpr int kGpuCodecMaxFrames = 16;

struct GpuF5Conv {
    const float *w = nullptr, *b = nullptr;
    int cin = 0, cout = 0, K = 1, groups = 1;
};
struct GpuF5Desc {
    int dim = 0, depth = 0, heads = 0, dim_head = 0, ff_mult = 2, mel_dim = 100, text_dim = 0, pe_attn_head = 0;
    int in_proj = -1, norm_out = -1, proj_out = -1;
    struct Block {
        int ada = -1, q = -1, k = -1, v = -1, o = -1, ff1 = -1, ff2 = -1;
    };
    std::vector<Block> blocks;
    GpuF5Conv pos1, pos2;
    int vocos_dim = 0, vocos_inter = 0, vocos_out = 0;
    GpuF5Conv v_embed;
    const float *v_ln_w = nullptr, *v_ln_b = nullptr, *v_fln_w = nullptr, *v_fln_b = nullptr;
    struct VBlock {
        GpuF5Conv dw;
        const float *ln_w = nullptr, *ln_b = nullptr, *gamma = nullptr;
        int pw1 = -1, pw2 = -1;
    };
    std::vector<VBlock> v_blocks;
    int v_head = -1;
};
int gpu_f5_create(const GpuF5Desc &d);
bool gpu_f5_begin(int id, int B, int N, const float *cat0, const float *rope);
bool gpu_f5_step(int id, const float *x, const float *ts, float *out);
bool gpu_f5_vocos(int id, const float *mel, int T, std::vector<float> &head);
void gpu_f5_end(int id);
std::string gpu_gemm_choice();
void gpu_gemm_preset(const std::string &choice);

struct GpuCosyDesc {
    int M = 80, C = 256, heads = 8, head_dim = 64;
    struct Res {
        GpuF5Conv c1, c2, res;
        const float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
    };
    struct X {
        const float *n1w = nullptr, *n1b = nullptr, *n3w = nullptr, *n3b = nullptr;
        int q = -1, k = -1, v = -1, o = -1, ff1 = -1, ff2 = -1, ff_dim = 0;
    };
    Res down_res, up_res;
    std::vector<Res> mid_res;
    std::vector<X> down_x, up_x;
    std::vector<std::vector<X>> mid_x;
    GpuF5Conv down_conv, up_out, final_conv, final_proj;
    const float *fn_w = nullptr, *fn_b = nullptr;
};
int gpu_cosy_create(const GpuCosyDesc &d);
bool gpu_cosy_begin(int id, int T, const float *in0);
bool gpu_cosy_step(int id, const float *x, const float *tb, float *out);
void gpu_cosy_end(int id);

}  // namespace vox
