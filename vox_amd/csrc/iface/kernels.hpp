// kernels.hpp — the part of Vox's tensor-op interface that the device backend sees, restated so that
// gpu_hip.cpp builds on its own. In Vox itself gpu_hip.cpp is compiled against Vox's own src/kernels.hpp and
// src/gpu.hpp instead; the declarations here keep the same names, field order and meaning
// (reference: src/kernels.hpp:42-56 Mat/WType, :88-100 gpu hooks, :114-130 LayerW/TransformerW).
#pragma once
#include <cstdint>
#include <vector>

namespace vox {

enum class WType { F32, F16, BF16, Q8, Q4 };

// Weight matrix view [rows][cols] (rows = outputs); data/scale/bias point into host memory (the mmap).
struct Mat {
    WType type = WType::F32;
    const uint8_t *data = nullptr;
    const float *scale = nullptr;  // Q8/Q4: [rows][cols/32]
    int64_t rows = 0, cols = 0;
    const float *bias = nullptr;   // [rows] or null
    int gpu = -1;                  // device handle from gpu_upload, -1 = CPU only
    bool valid() const { return data != nullptr; }
};

// false -> compute on the CPU
bool gpu_matmul(const Mat &W, const float *x, int64_t m, float *y);
struct TransformerW;
bool gpu_xfmr_forward(const TransformerW &w, int seq, int64_t pos0, const float *x, int64_t m, float *out_last,
                      const Mat *in_proj = nullptr, const Mat *head = nullptr, float *head_out = nullptr);
bool gpu_xfmr_forward_hidden(const TransformerW &w, int seq, int64_t pos0, const float *x, int64_t m, float *hidden_out);
bool gpu_xfmr_forward_pair(const TransformerW &w, int seq0, int seq1, int64_t pos, const float *x2, const Mat *head, float *out2,
                           float *head_out2);

struct LayerW {
    Mat q, k, v, o, gate, up, down;
    const float *qn = nullptr, *kn = nullptr;                 // per-head RMSNorm (optional)
    const float *ln1 = nullptr, *ln2 = nullptr;
    const float *attn_scale = nullptr, *mlp_scale = nullptr;  // layer scales (codec decoder only)
};
struct TransformerW {
    std::vector<LayerW> layers;
    const float *final_norm = nullptr;
    int hidden = 0, heads = 0, kv_heads = 0, head_dim = 0, inter = 0;
    float eps = 1e-6f;
    double theta = 10000.0;
    int window = 0;  // 0 = full attention
    std::vector<float> inv_freq;
    int gpu_id = -1;      // gpu_xfmr_create handle
    int gpu_layers = -1;  // first layers on the device, -1 = all
};

}  // namespace vox
