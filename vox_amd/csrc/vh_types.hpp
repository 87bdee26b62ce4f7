// vh_types.hpp — argument blocks shared by the kernels and their host-side launchers.
#pragma once
#include <stdint.h>

namespace vh {

enum { PRO_X = 0, PRO_RMS = 1 };
enum { EPI_STORE = 0, EPI_ACC = 1, EPI_SWIGLU = 2 };
enum { WT_F32 = 0, WT_F16 = 1, WT_BF16 = 2, WT_Q8 = 3, WT_Q4 = 4 };

struct GemvArgs {
    const uint8_t *w;     // weights, reference row layout
    const float *scale;   // [rows][K/32] for Q8/Q4
    const float *bias;    // [rows] or null
    const float *x;       // [m][ldx]
    const float *gamma;   // [K] (PRO_RMS)
    float *y;             // [m][ldy]
    float *xnorm;         // PRO_RMS: normed rows [m][K] written by block 0 (may be null)
    int64_t ldx, ldy;
    int32_t rows, K, m;
    float eps;
};

constexpr int kGemvThreads = 256;

// Cache view of one activation row: the sequence's cache bases (layer 0) and the row's absolute position.
struct RowRef {
    _Float16 *k;
    _Float16 *v;
    int64_t cap;
    int64_t pos;
};

struct QkArgs {
    const float *qkv;   // [m][qd + 2 kd] stacked q|k|v GEMV output
    int64_t ldqkv;
    float *q;           // [m][qd] normed + rotated queries
    const RowRef *rows; // [m]
    const float *qn, *kn;
    const float *rope;  // [positions][hd/2][2] = (cos, sin)
    int32_t heads, kv_heads, hd, layer;
    float eps;
};

constexpr int kAttnSplits = 64;  // grid.x of k_attn_partial; splits beyond the key count exit at once

struct AttnArgs {
    const float *q;      // [m][qd]
    const RowRef *rows;  // [m]
    float *pm, *pl;      // [m][heads][kAttnSplits]
    float *po;           // [m][heads][kAttnSplits][hd]
    float *out;          // [m][qd]
    int32_t heads, kv_heads, layer;
    float scale;
};

struct SampleCfgDev {
    float temperature, top_p, rep;
    int32_t top_k;
    uint32_t key0, key1;
    uint64_t frame;
    uint32_t cb, draw;
    int32_t sup_from, sup_to, eos, block_eos;
    int32_t n_history;
    const int32_t *history;  // device
};

constexpr int kSampleThreads = 1024;
constexpr int kSampleMaxN = 16384;  // 16 values per thread
constexpr int kSampleMaxK = 4096;   // LDS sort capacity

}  // namespace vh
