// voxhip_runtime.hip — host runtime of the gfx950 backend; implements the C ABI of include/voxhip.h.
//
// One context per process (one device, one stream, one lock), as the reference backend
// (gpu_vulkan.cpp:361-374, one mutex taken by every entry point). Weights are copied to HBM once and stay for
// the process lifetime; transformers keep their q|k|v and gate|up matrices stacked (gpu_vulkan.cpp:784-788),
// gate|up interleaved by row pairs so the SwiGLU epilogue sees a (gate, up) pair in one wave. KV caches are f16
// in HBM, [layer][kv_head][capacity][head_dim]. A decode step is a fixed launch sequence that is captured once
// into a HIP graph and replayed; positions and sampler parameters live in small device blocks that are
// refreshed before each replay.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "vh_launch.hpp"
#include "vh_devinfo.hpp"
#include "voxhip.h"

using namespace vh;

// Scratch of voxhip_matmul_dev_noalloc, the entry point that allocates nothing: split-K partial sums and the int
// path's once-quantized input rows of one matrix pass. A fixed array in the code object, so each device the library
// runs on holds its own copy (6.3 MiB) until the process ends. Host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (Ctx::noalloc), never through the array's name.
constexpr int64_t kNoAllocWsFloats = int64_t(3) << 19;               // 1.5 Mi floats of split-K partials (6 MiB)
constexpr int64_t kNoAllocQElems = int64_t(8) * 32768;               // 8 quantized rows of up to 32768 elements
constexpr size_t kNoAllocBytes = size_t(kNoAllocWsFloats) * 4 + size_t(kNoAllocQElems) + size_t(kNoAllocQElems / 32) * 8;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

namespace {

struct Fail : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define HIPCHECK(expr)                                                                                   \
    do {                                                                                                 \
        hipError_t e_ = (expr);                                                                          \
        if (e_ != hipSuccess) throw Fail(std::string(#expr) + " failed: " + hipGetErrorString(e_));      \
    } while (0)

constexpr int kMaxM = 8;          // rows per pass on the int8-activation path; sequences per decode step
constexpr int kMaxPass = 512;     // rows per pass on the f32-activation path (MFMA GEMM above 4 rows)
constexpr int64_t kGemmWsFloats = int64_t(8) << 20;  // split-K workspace: 32 MB
// Passes of at least kQuantRowsMin rows on the int path quantize their input rows once (k_quant_rows) instead of in
// every GEMV block; the buffer holds 8 rows of up to 32768 elements.
constexpr int kQuantRowsMin = 5;
constexpr int64_t kQuantRowsElems = int64_t(8) * 32768;
constexpr int64_t kMaxCap = 65536;

struct GpuMat {
    int32_t type = 0;
    int64_t rows = 0, cols = 0;
    uint8_t *w = nullptr;
    float *s = nullptr;  // [rows][cols/32] block scales (f16 values when s16)
    bool s16 = false;
    float *b = nullptr;
    uint64_t bytes = 0;  // weights + scales + bias bytes (the GEMV's algorithmic stream)
    _Float16 *w16 = nullptr;  // Q8: the int8 values widened to f16 for the split-f16 GEMM, made on first use
    float wmax = 0.f;  // F32: max |w| (NaN when a weight is NaN), which picks the GEMM kernel (f32_wide)
};

struct LayerDev {
    int qkv = -1, o = -1, gu = -1, down = -1;
    size_t ln1 = 0, ln2 = 0, qn = 0, kn = 0;
    bool qk = false;
    // the down weights as 32-column panels for the fused one-row FFN (k_ffn_int), when the transformer has it
    uint8_t *pan = nullptr;
    void *pan_s = nullptr;
};

// A captured decode step: m rows of one sequence (steps = 0), or one row for each of m sequences (steps = 1).
// lng: one row at a position past kAttnSpecKeys (the attention's long first batch).
struct GraphKey {
    std::array<int, 8> seqs;
    int m, head, sample, steps, lng;
    const void *x, *out, *logits, *token;
    bool operator<(const GraphKey &o) const {
        return std::tie(seqs, m, head, sample, steps, lng, x, out, logits, token) <
               std::tie(o.seqs, o.m, o.head, o.sample, o.steps, o.lng, o.x, o.out, o.logits, o.token);
    }
};

// A captured layer pass of forward_rows: the launch sequence of enqueue_layers depends on the pass's row count,
// the caller's row count class (<= 8 rows: int8 path), the layer range, the attention form and row 0's cache view.
struct LayersKey {
    int mc, mt, first, count, fused, pass_attn, lng;
    const void *k, *v;
    int64_t cap;
    bool operator<(const LayersKey &o) const {
        return std::tie(mc, mt, first, count, fused, pass_attn, lng, k, v, cap) <
               std::tie(o.mc, o.mt, o.first, o.count, o.fused, o.pass_attn, o.lng, o.k, o.v, o.cap);
    }
};
constexpr int kMaxLayerGraphs = 64;  // captured layer passes kept per transformer

struct Xfmr {
    std::string name;
    int layers = 0, H = 0, heads = 0, kvh = 0, hd = 0, I = 0;
    float eps = 1e-6f;
    double theta = 1e4;
    std::vector<float> inv_freq;
    std::vector<LayerDev> L;
    float *norms = nullptr;
    size_t final_off = 0;
    float *rope = nullptr;
    int64_t rope_rows = 0;
    // scratch for cap_rows rows (grown by ensure_rows); pre: the GEMM path's prologue output (normed or merged rows)
    int cap_rows = 0;
    float *h = nullptr, *xin = nullptr, *qkv = nullptr, *q = nullptr, *g = nullptr, *xnorm = nullptr, *pre = nullptr;
    // f16 halves (hi plane, then lo plane) of the GEMM inputs of a planes pass: pa16 the normed rows and the attention
    // output (planes of cap_rows x max(H, qd)), pb16 the SwiGLU output (planes of cap_rows x I)
    _Float16 *pa16 = nullptr, *pb16 = nullptr;
    float *pm = nullptr, *pl = nullptr, *po = nullptr, *logits = nullptr;
    int64_t xin_elems = 0, logits_elems = 0;
    // fused one-row FFN: every layer's FFN is one k_ffn_int launch whose down product reaches h through acc
    // ([kAccCopies][H] fixed-point sums, zero between passes)
    bool ffn_fuse = false;
    int64_t *acc = nullptr;
    // per-row cache views of the next pass, followed by each row's RoPE row ([cap_rows][hd] (cos, sin) pairs)
    RowRef *rows_dev = nullptr, *rows_host = nullptr;
    float *rope_rows_dev = nullptr;
    SampleCfgDev *scfg_dev = nullptr, *scfg_host = nullptr;
    int32_t *token_dev = nullptr;
    std::map<GraphKey, hipGraphExec_t> graphs;
    // forward_rows' layer passes: captured on the second use of a key, replayed after
    std::map<LayersKey, hipGraphExec_t> layer_graphs;
    std::map<LayersKey, int> layer_uses;
    std::vector<RowRef> rows_last;
    bool rows_valid = false;
    // CosyVoice2 LM generation: config, state and decoded tokens on the device, pinned copies for the host,
    // optional per-step log-probabilities; graphs of kLmGraphSteps steps keyed by (seq, head, embedding, logp)
    LmCfgDev *lm_cfg = nullptr;
    LmState *lm_state = nullptr;
    int32_t *lm_dec = nullptr;
    float *lm_logp = nullptr;
    int64_t lm_dec_cap = 0, lm_logp_cap = 0;
    std::map<std::array<int64_t, 4>, hipGraphExec_t> lm_graphs;
    // code-predictor frame loop: sampled codes, per-codebook sampler configurations and the code-range flag on the
    // device ([kPredMaxGroups] each; pinned copies for the host); one graph per (seq, in_proj, heads, embeddings)
    int32_t *pred_codes = nullptr, *pred_err = nullptr, *pred_host = nullptr;
    SampleCfgDev *pred_cfg = nullptr, *pred_cfg_host = nullptr;
    std::map<std::vector<int>, hipGraphExec_t> pred_graphs;
};

struct Seq {
    int xfmr = -1;
    int64_t cap = 0;
    _Float16 *k = nullptr, *v = nullptr;
    bool used = false;
    int layers = 0, kvh = 0, hd = 0;
};

struct Ctx {
    std::mutex mu;
    bool ok = false;
    std::string init_error;
    int dev = -1;
    std::string name;
    hipStream_t stream = nullptr;
    std::vector<GpuMat> mats;
    std::vector<Xfmr *> xf;
    std::vector<Seq> seqs;
    std::unordered_map<void *, uint64_t> allocs;
    uint64_t vram_used = 0, vram_limit = 0;
    voxhip_stats stats{};
    std::string last_error;
    bool warned = false;
    // staging for host-pointer entry points
    float *pin = nullptr;
    size_t pin_bytes = 0;
    float *dbuf_x = nullptr, *dbuf_y = nullptr, *dbuf_z = nullptr;
    size_t dbuf_x_bytes = 0, dbuf_y_bytes = 0, dbuf_z_bytes = 0;
    // sampler staging for voxhip_sample_logits
    SampleCfgDev *scfg_dev = nullptr, *scfg_host = nullptr;
    int32_t *hist_dev = nullptr, *tok_dev = nullptr;
    size_t hist_cap = 0;
    std::vector<struct F5 *> f5;
    std::vector<struct Cosy *> cosy;
    std::vector<struct Codec *> codecs;
    std::vector<struct CodecSt *> cstates;
    // split-K partial sums of the MFMA GEMM (allocated at init, so captured graphs can use it)
    float *gemm_ws = nullptr;
    // int-path input rows quantized once per pass (k_quant_rows), kQuantRowsElems elements (allocated at init)
    int8_t *qrows = nullptr;
    float *qrows_s = nullptr;
    int32_t *qrows_sum = nullptr;
    // per device index: the device address of `scratch` (hipGetSymbolAddress at init, with that device current)
    std::array<uint8_t *, 64> noalloc{};
    // LM sampler staging: device config + state, and their pinned host copies (config, state, two state slots)
    LmCfgDev *lm_cfg_dev = nullptr;
    LmState *lm_state_dev = nullptr;
    uint8_t *lm_host = nullptr;
    // the range-status word (allocated and zeroed at init) and its pinned host copy; word 1 of the device block is
    // the scratch of the weight max |w| reduction
    int32_t *status_dev = nullptr, *status_pin = nullptr;
    // VOXHIP_CHECK_HOST=1 at a voxhip_init call: copy_h2d / copy_d2h check each side's memory type (check_copy_side)
    bool check_copies = false;
};

Ctx g;

void set_error(const std::string &e) {
    g.last_error = e;
}
}  // namespace

namespace vh {
int32_t *status_word() { return g.status_dev; }
}  // namespace vh

namespace {

// ------------------------------------------------------------------ device memory with accounting
void *dalloc(size_t bytes) {
    if (bytes == 0) bytes = 16;
    if (g.vram_limit && g.vram_used + bytes > g.vram_limit)
        throw Fail("VRAM limit reached: " + std::to_string(g.vram_limit >> 20) + " MiB allowed, " +
                   std::to_string(g.vram_used >> 20) + " MiB in use, " + std::to_string((bytes + (1u << 20) - 1) >> 20) +
                   " MiB requested");
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) throw Fail(std::string("hipMalloc of ") + std::to_string(bytes >> 20) + " MiB failed: " + hipGetErrorString(e));
    g.allocs[p] = bytes;
    g.vram_used += bytes;
    return p;
}
void dfree(void *p) {
    if (!p) return;
    auto it = g.allocs.find(p);
    if (it != g.allocs.end()) { g.vram_used -= std::min(g.vram_used, it->second); g.allocs.erase(it); }
    (void)hipFree(p);
}
template <class T>
T *dalloc_t(size_t n) { return static_cast<T *>(dalloc(n * sizeof(T))); }

float *pinned(size_t bytes) {
    if (g.pin_bytes < bytes) {
        // an asynchronous copy queued by an earlier call may still read the old block
        if (g.pin) HIPCHECK(hipStreamSynchronize(g.stream));
        if (g.pin) (void)hipHostFree(g.pin);
        g.pin = nullptr;
        g.pin_bytes = 0;
        HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&g.pin), bytes, hipHostMallocDefault));
        g.pin_bytes = bytes;
    }
    return g.pin;
}
float *dev_scratch(float *&p, size_t &cap, size_t bytes) {
    if (cap < bytes) {
        dfree(p);
        p = nullptr;
        cap = 0;
        p = static_cast<float *>(dalloc(bytes));
        cap = bytes;
    }
    return p;
}

// Every copy between host and device memory goes through copy_h2d / copy_d2h. With VOXHIP_CHECK_HOST=1 (read by
// each voxhip_init call) each checks, by hipPointerGetAttributes, that its device side is device memory and its host side is not
// (pinned or unregistered host memory), and fails the call naming the copy otherwise: a device address handed to
// the runtime as host memory would be read or written by the host. s == nullptr: a synchronous copy.
void check_copy_side(const void *p, bool want_device, const char *copy, const char *side) {
    hipPointerAttribute_t a{};
    const hipError_t e = hipPointerGetAttributes(&a, p);
    const bool dev = e == hipSuccess && a.type == hipMemoryTypeDevice;
    if (e != hipSuccess) (void)hipGetLastError();  // unregistered host memory reports an error; clear it
    if (dev != want_device)
        throw Fail(std::string(copy) + ": the " + side + " is " + (dev ? "device" : "host") + " memory, " +
                   (want_device ? "device" : "host") + " memory expected");
}
hipError_t copy_h2d(void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (!bytes) return hipSuccess;
    if (g.check_copies) {
        check_copy_side(dst, true, "host-to-device copy", "destination");
        check_copy_side(src, false, "host-to-device copy", "source");
    }
    return s ? hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s) : hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}
hipError_t copy_d2h(void *dst, const void *src, size_t bytes, hipStream_t s) {
    if (!bytes) return hipSuccess;
    if (g.check_copies) {
        check_copy_side(src, true, "device-to-host copy", "source");
        check_copy_side(dst, false, "device-to-host copy", "destination");
    }
    return s ? hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s) : hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}

// The end of a synchronous call: waits for the stream, then fails the call when one of its kernels set the
// range-status word (an activation beyond the f16 range of a split-f16 product, or a fused-FFN term outside the
// fixed-point range), clearing the word for the next call. The engine then computes the call on the CPU, as for any
// failed device call. Device-resident calls (decode_dev, the no-alloc matmul) are reported by voxhip_sync.
void sync_status() {
    HIPCHECK(copy_d2h(g.status_pin, g.status_dev, sizeof(int32_t), g.stream));
    HIPCHECK(hipStreamSynchronize(g.stream));
    vh::prof_collect();  // VOX_PROFILE=gpu: the call's stamped launches have finished
    const int32_t v = g.status_pin[0];
    if (!v) return;
    g.status_pin[0] = 0;
    HIPCHECK(hipMemsetAsync(g.status_dev, 0, sizeof(int32_t), g.stream));
    HIPCHECK(hipStreamSynchronize(g.stream));
    std::string what;
    if (v & vh::kStatusF16Range) what = "an activation beyond the f16 range of the split-f16 matrix products";
    if (v & vh::kStatusFixRange)
        what += std::string(what.empty() ? "" : "; ") + "a fused-FFN term that is not finite or beyond +-2^18 (fixed-point range)";
    throw Fail("value outside the device arithmetic's range: " + what);
}

void h2d(void *dst, const void *src, size_t bytes) {
    if (!bytes) return;
    HIPCHECK(copy_h2d(dst, src, bytes, nullptr));
}

void require_ok() {
    if (!g.ok) throw Fail(g.init_error.empty() ? "HIP backend is not initialised (voxhip_init)" : g.init_error);
}
GpuMat &mat_at(int id) {
    if (id < 0 || size_t(id) >= g.mats.size() || !g.mats[size_t(id)].w) throw Fail("bad matrix handle " + std::to_string(id));
    return g.mats[size_t(id)];
}
Xfmr &xf_at(int id) {
    if (id < 0 || size_t(id) >= g.xf.size() || !g.xf[size_t(id)]) throw Fail("bad transformer handle " + std::to_string(id));
    return *g.xf[size_t(id)];
}
Seq &seq_at(int id) {
    if (id < 0 || size_t(id) >= g.seqs.size() || !g.seqs[size_t(id)].k) throw Fail("bad sequence handle " + std::to_string(id));
    return g.seqs[size_t(id)];
}

size_t row_bytes(int32_t type, int64_t cols) {
    return type == VOXHIP_F32 ? size_t(cols) * 4 : type == VOXHIP_Q8 ? size_t(cols) : type == VOXHIP_Q4 ? size_t(cols) / 2
                                                                                                         : size_t(cols) * 2;
}
bool quantized(int32_t t) { return t == VOXHIP_Q8 || t == VOXHIP_Q4; }

// Checks the shape rules of the GEMV kernels: Q8/Q4 need cols % 32 (as kernels.cpp:655); the activation
// prologue stages inputs in 8-element slots, so F32/F16/BF16 need cols % 8.
void check_shape(int32_t type, int64_t rows, int64_t cols) {
    if (type < VOXHIP_F32 || type > VOXHIP_Q4) throw Fail("unknown weight type " + std::to_string(type));
    if (rows <= 0 || cols <= 0 || rows > (int64_t(1) << 30)) throw Fail("bad matrix shape");
    if (quantized(type) && cols % 32) throw Fail("Q8/Q4 matrix needs cols % 32 == 0");
    if (!quantized(type) && cols % 8) throw Fail("F32/F16/BF16 matrix needs cols % 8 == 0 on this backend");
}

size_t scale_row_bytes(const GpuMat &m) { return quantized(m.type) ? size_t(m.cols / 32) * (m.s16 ? 2 : 4) : 0; }
int gemv_type(const GpuMat &m) { return m.type == VOXHIP_Q4 && m.s16 ? WT_Q4H : m.type; }
// F32 weights the split-f16 kernel cannot hold (its f16 halves of 2^10 w overflow from |w| >= 64; NaN counts): they
// take the f32 matrix cores (GemmArgs::f32_wide).
constexpr float kF32SplitMaxW = 63.0f;
bool f32_wide(float wmax) { return !(wmax < kF32SplitMaxW); }
bool f32_wide(const GpuMat &m) { return m.type == VOXHIP_F32 && f32_wide(m.wmax); }
// max |w| of n host floats (NaN when one is NaN)
float host_absmax(const float *w, size_t n) {
    float mx = 0.f;
    for (size_t i = 0; i < n; ++i) {
        const float a = std::fabs(w[i]);
        if (!(a <= mx)) mx = a;  // a NaN replaces the max and is never replaced (nothing compares above it)
        if (std::isnan(mx)) break;
    }
    return mx;
}

// f32 -> f16 bits when the value is exactly representable as a normal or zero f16 (the scales a device Q4 matrix
// may store in 2 bytes without changing its arithmetic).
bool f16_exact(float f, uint16_t *out) {
    if (f == 0.f) { *out = std::signbit(f) ? 0x8000 : 0; return true; }
    if (!std::isfinite(f)) return false;
    int e = 0;
    const float mant = std::frexp(std::fabs(f), &e);  // |f| = mant * 2^e, mant in [0.5, 1)
    if (e - 1 < -14 || e - 1 > 15) return false;       // normal f16 range
    const float scaled = std::ldexp(mant, 11);         // 11 significant bits
    if (scaled != std::floor(scaled)) return false;
    const uint32_t m10 = uint32_t(scaled) & 0x3FFu;
    *out = uint16_t((f < 0 ? 0x8000u : 0u) | (uint32_t(e - 1 + 15) << 10) | m10);
    return true;
}

int new_mat(int32_t type, int64_t rows, int64_t cols, bool bias, bool s16 = false) {
    GpuMat m;
    m.type = type; m.rows = rows; m.cols = cols; m.s16 = s16 && type == VOXHIP_Q4;
    const size_t wb = size_t(rows) * row_bytes(type, cols);
    m.w = static_cast<uint8_t *>(dalloc(wb));
    m.bytes = wb;
    if (quantized(type)) {
        const size_t sbytes = size_t(rows) * scale_row_bytes(m);
        m.s = static_cast<float *>(dalloc(sbytes));
        m.bytes += sbytes;
    }
    if (bias) { m.b = dalloc_t<float>(size_t(rows)); m.bytes += size_t(rows) * 4; }
    g.mats.push_back(m);
    return int(g.mats.size()) - 1;
}
void free_mat(int id) {
    if (id < 0 || size_t(id) >= g.mats.size()) return;
    GpuMat &m = g.mats[size_t(id)];
    dfree(m.w); dfree(m.s); dfree(m.b); dfree(m.w16);
    m = GpuMat();
}

// Stacks the parts' rows into one device matrix. interleave2: two parts of equal rows stored as row pairs
// (part0 row r, part1 row r) — the gate|up layout of the SwiGLU epilogue.
int upload_parts(const voxhip_mat *parts, int n, bool interleave2) {
    if (n <= 0) throw Fail("no matrix parts");
    const voxhip_mat &P0 = parts[0];
    int64_t rows = 0;
    bool any_bias = false, all_bias = true;
    for (int i = 0; i < n; ++i) {
        const voxhip_mat &p = parts[i];
        if (p.type != P0.type || p.cols != P0.cols || !p.data) throw Fail("matrix parts differ in type/width or lack data");
        if (quantized(p.type) && !p.scale) throw Fail("quantized matrix without scales");
        rows += p.rows;
        any_bias = any_bias || p.bias;
        all_bias = all_bias && p.bias;
    }
    if (any_bias && !all_bias) throw Fail("bias on some stacked parts only");
    if (interleave2 && (n != 2 || parts[0].rows != parts[1].rows)) throw Fail("interleave needs two equal parts");
    check_shape(P0.type, rows, P0.cols);
    // Q4 scales that are all exact in f16 are stored in 2 bytes (WT_Q4H): same products, less to stream
    const int64_t nbr = P0.cols / 32;
    std::vector<std::vector<uint16_t>> s16(static_cast<size_t>(n));
    bool use16 = P0.type == VOXHIP_Q4;
    for (int i = 0; i < n && use16; ++i) {
        s16[size_t(i)].resize(size_t(parts[i].rows * nbr));
        for (size_t j = 0; j < s16[size_t(i)].size() && use16; ++j) use16 = f16_exact(parts[i].scale[j], &s16[size_t(i)][j]);
    }
    const int id = new_mat(P0.type, rows, P0.cols, all_bias, use16);
    GpuMat &m = g.mats[size_t(id)];
    if (P0.type == VOXHIP_F32)
        for (int i = 0; i < n; ++i)
            m.wmax = std::max(m.wmax, host_absmax(static_cast<const float *>(parts[i].data), size_t(parts[i].rows * P0.cols)),
                              [](float a, float b) { return a < b || std::isnan(b); });
    const size_t rb = row_bytes(P0.type, P0.cols), sb = scale_row_bytes(m);
    auto scale_src = [&](int i) -> const uint8_t * {
        return use16 ? reinterpret_cast<const uint8_t *>(s16[size_t(i)].data()) : reinterpret_cast<const uint8_t *>(parts[i].scale);
    };
    if (!interleave2) {
        int64_t r0 = 0;
        for (int i = 0; i < n; ++i) {
            const voxhip_mat &p = parts[i];
            h2d(m.w + size_t(r0) * rb, p.data, size_t(p.rows) * rb);
            if (sb) h2d(reinterpret_cast<uint8_t *>(m.s) + size_t(r0) * sb, scale_src(i), size_t(p.rows) * sb);
            if (all_bias) h2d(m.b + r0, p.bias, size_t(p.rows) * 4);
            r0 += p.rows;
        }
    } else {
        const int64_t R = parts[0].rows;
        std::vector<uint8_t> tw(size_t(rows) * rb), ts(size_t(rows) * sb);
        std::vector<float> tb(all_bias ? size_t(rows) : 0);
        for (int64_t r = 0; r < R; ++r)
            for (int i = 0; i < 2; ++i) {
                const voxhip_mat &p = parts[i];
                std::memcpy(&tw[size_t(2 * r + i) * rb], static_cast<const uint8_t *>(p.data) + size_t(r) * rb, rb);
                if (sb) std::memcpy(&ts[size_t(2 * r + i) * sb], scale_src(i) + size_t(r) * sb, sb);
                if (all_bias) tb[size_t(2 * r + i)] = p.bias[r];
            }
        h2d(m.w, tw.data(), tw.size());
        if (sb) h2d(m.s, ts.data(), ts.size());
        if (all_bias) h2d(m.b, tb.data(), tb.size() * 4);
    }
    g.stats.mats_ok += n;
    g.stats.bytes += m.bytes;
    return id;
}

// ------------------------------------------------------------------ GEMV launch helpers
// int8 activations for Q8 when the call's row count is <= 8 (kernels.cpp:647, :660) and always for Q4.
bool int_path(const GpuMat &m, int64_t m_total) {
    return m.type == VOXHIP_Q4 || (m.type == VOXHIP_Q8 && m_total <= kMaxM);
}
int rows_per_pass(const GpuMat &m, int64_t m_total) { return int_path(m, m_total) ? kMaxM : kMaxPass; }
// f32-activation passes of more than 4 rows run on the MFMA GEMM (the GEMV holds at most 4 f32 rows in LDS).
bool gemm_path(const GpuMat &m, int64_t m_total, int mc) { return !int_path(m, m_total) && mc > 4; }

// Device scratch of one matrix pass beyond its inputs and outputs: the split-K partial sums of the GEMM (ws_cap
// floats at ws; the launcher splits K only as far as they fit) and the int path's once-quantized input rows
// (q_elems int8 at q, q_elems / 32 scales and block sums; used only when the pass's rows fit).
struct PassScratch {
    float *ws;
    int64_t ws_cap;
    int8_t *q;
    float *qs;
    int32_t *qsum;
    int64_t q_elems;
};
// The library's own scratch, allocated at init.
PassScratch lib_scratch() { return {g.gemm_ws, kGemmWsFloats, g.qrows, g.qrows_s, g.qrows_sum, kQuantRowsElems}; }

// Observer of the launches of one pass (the benchmark's per-kernel timing): before(class) and after() bracket
// every kernel launch enqueue_layers / enqueue_final / the sampler make.
struct Probe {
    virtual void before(int cls) = 0;
    virtual void after() = 0;
    // the launch just made in the current bracket was of class `done`: book it so, and open a new bracket of the
    // bracket's class for the launches that follow (a GEMV pass that quantizes its rows first)
    virtual void split(int done) = 0;
    virtual ~Probe() = default;
};
thread_local Probe *t_probe = nullptr;  // the probe of the bracket being enqueued (gemv() splits it)
template <class F>
void probed(Probe *pr, int cls, F &&f) {
    if (pr) pr->before(cls);
    Probe *prev = t_probe;
    t_probe = pr;
    try {
        f();
    } catch (...) {
        t_probe = prev;
        throw;
    }
    t_probe = prev;
    if (pr) pr->after();
}

// Rows quantized per 32-block as a PRO_Q pass takes them: q [m][K] int8, qs and qsum [m][K/32].
struct QRows {
    int8_t *q;
    float *qs;
    int32_t *qsum;
};

// Whether a pass of mc rows on the int path quantizes its input rows once (k_quant_rows, then PRO_Q).
bool quant_rows_pass(const GpuMat &m, int64_t m_total, int mc, const PassScratch &sc) {
    return int_path(m, m_total) && mc >= kQuantRowsMin && mc <= 8 && int64_t(mc) * m.cols <= sc.q_elems;
}

// The FFN of mc rows on the int path with the SwiGLU output quantized in gate|up's epilogue (EPI_SWIGLU_Q): when
// both passes take pre-quantized rows and the scratch holds gate|up's input rows and the down pass's side by side,
// the down pass's rows (returned in *out, after gate|up's) need no k_quant_rows launch of their own.
// VOXHIP_FFN_QEPI=0 keeps the two quantizations apart (k_quant_rows before the down pass); the rows are the same.
bool ffn_quant_epilogue(const GpuMat &gu, const GpuMat &dn, int64_t m_total, int mc, const PassScratch &sc, QRows *out) {
    const char *e = std::getenv("VOXHIP_FFN_QEPI");
    if (e && e[0] == '0') return false;
    if (!quant_rows_pass(gu, m_total, mc, sc) || !quant_rows_pass(dn, m_total, mc, sc) || gemm_path(gu, m_total, mc) ||
        gemm_path(dn, m_total, mc))
        return false;
    if (gu.rows % 64 || gu.rows / 2 != dn.cols || dn.cols % 32) return false;
    const int64_t oq = (int64_t(mc) * gu.cols + 255) / 256 * 256, os = (int64_t(mc) * (gu.cols / 32) + 63) / 64 * 64;
    if (oq + int64_t(mc) * dn.cols > sc.q_elems || os + int64_t(mc) * (dn.cols / 32) > sc.q_elems / 32) return false;
    *out = {sc.q + oq, sc.qs + os, sc.qsum + os};
    return true;
}

// One matrix pass: y (=, +=, swiglu) W * prologue(x) for mc rows. On the GEMM path the prologue runs as its own
// kernel into pre ([mc][cols]; xnorm instead when the normed rows are wanted). sc: the pass's scratch (null: the
// library's).
// acc (one row on the int path): the fused FFN's pending sums, added to x (PRO_RMS) or to y before the product
// (EPI_ACC, which also clears the rows it consumed).
// qout (EPI_SWIGLU on pre-quantized rows): the SwiGLU output goes to these quantized rows instead of y; qin (PRO_X):
// the input rows arrive quantized there (ffn_quant_epilogue's pair of passes).
void gemv(const GpuMat &m, int64_t m_total, int pro, int epi, const float *x, int64_t ldx, int mc, float *y, int64_t ldy,
          const float *gamma, float eps, float *xnorm, hipStream_t s, const AttnPartials *attn = nullptr,
          float *pre = nullptr, const PassScratch *scp = nullptr, int64_t *acc = nullptr, const float *res = nullptr,
          const float *yscale = nullptr, const QRows *qout = nullptr, const QRows *qin = nullptr) {
    const PassScratch sc = scp ? *scp : lib_scratch();
    if ((qout || qin) && (!quant_rows_pass(m, m_total, mc, sc) || gemm_path(m, m_total, mc) || acc || res || yscale || xnorm ||
                          (qout && (pro != PRO_RMS && pro != PRO_X)) || (qout && epi != EPI_SWIGLU) || (qin && pro != PRO_X)))
        throw Fail("quantized rows on a pass that cannot take them");
    if (acc && (mc != 1 || !int_path(m, m_total) || !(pro == PRO_RMS || epi == EPI_ACC)))
        throw Fail("pending FFN sums on a pass that cannot take them");
    if (res && (epi != EPI_ACC || gemm_path(m, m_total, mc))) throw Fail("separate residual on a pass that cannot take it");
    if (yscale && epi != EPI_ACC) throw Fail("a row scale needs the residual epilogue");
    if (pro == PRO_ATTN && (!attn || int64_t(attn->heads) * attn->hd != m.cols))
        throw Fail("attention partials do not match the o projection");
    if (gemm_path(m, m_total, mc)) {
        const float *A = x;
        int64_t lda = ldx;
        if (pro == PRO_RMS) {
            float *dst = xnorm ? xnorm : pre;
            if (!dst) throw Fail("GEMM pass without prologue scratch");
            HIPCHECK(launch_rmsnorm_rows(x, ldx, gamma, int(m.cols), eps, dst, m.cols, mc, s));
            A = dst; lda = m.cols;
        } else if (pro == PRO_ATTN) {
            if (!pre) throw Fail("GEMM pass without prologue scratch");
            HIPCHECK(launch_attn_merge(*attn, pre, mc, s));
            A = pre; lda = m.cols;
        }
        GemmArgs ga{};
        ga.bias = m.b; ga.y = y; ga.lda = lda; ga.ldy = ldy; ga.m = mc; ga.n = int32_t(m.rows); ga.K = int32_t(m.cols);
        ga.ws = sc.ws; ga.ws_cap = sc.ws_cap;
        ga.gate = yscale;  // a row scale of the GEMV is the GEMM's gated residual (y += gate[col] (c + bias))
        ga.f32_wide = f32_wide(m);
        HIPCHECK(launch_gemm(gemv_type(m), yscale ? EPI_GATED_ACC : epi, m.w, m.s, A, ga, s));
        return;
    }
    GemvArgs a{};
    a.w = m.w; a.scale = m.s; a.bias = m.b; a.x = x; a.gamma = gamma; a.y = y; a.xnorm = xnorm;
    a.ldx = ldx; a.ldy = ldy; a.rows = int32_t(m.rows); a.K = int32_t(m.cols); a.m = mc; a.eps = eps;
    if (pro == PRO_ATTN) a.attn = *attn;
    a.acc = acc;
    a.acc_ld = pro == PRO_RMS ? m.cols : m.rows;
    a.res = res;
    a.yscale = yscale;
    const bool ip = int_path(m, m_total);
    if (qin) {  // the rows were quantized by the previous pass's epilogue
        a.q = qin->q; a.qs = qin->qs; a.qsum = qin->qsum;
        HIPCHECK(launch_gemv(gemv_type(m), true, PRO_Q, epi, a, s));
        return;
    }
    if (quant_rows_pass(m, m_total, mc, sc) && (epi == EPI_STORE || epi == EPI_ACC || epi == EPI_SWIGLU)) {
        // several rows: quantize them once, then every GEMV block copies them instead of recomputing them
        HIPCHECK(launch_quant_rows(pro, a, sc.q, sc.qs, sc.qsum, s));
        if (t_probe) t_probe->split(VOXHIP_K_QUANT);
        a.q = sc.q; a.qs = sc.qs; a.qsum = sc.qsum;
        if (qout) {
            a.yq = qout->q; a.yqs = qout->qs; a.yqsum = qout->qsum;
            HIPCHECK(launch_gemv(gemv_type(m), true, PRO_Q, EPI_SWIGLU_Q, a, s));
            return;
        }
        HIPCHECK(launch_gemv(gemv_type(m), true, PRO_Q, epi, a, s));
        return;
    }
    HIPCHECK(launch_gemv(gemv_type(m), ip, pro, epi, a, s));
}

// ------------------------------------------------------------------ transformer
void drop_graphs(Xfmr &X) {
    for (auto &kv : X.graphs) (void)hipGraphExecDestroy(kv.second);  // graphs captured the old buffer addresses
    X.graphs.clear();
    for (auto &kv : X.layer_graphs) (void)hipGraphExecDestroy(kv.second);
    X.layer_graphs.clear();
    X.layer_uses.clear();
    for (auto &kv : X.lm_graphs) (void)hipGraphExecDestroy(kv.second);
    X.lm_graphs.clear();
    for (auto &kv : X.pred_graphs) (void)hipGraphExecDestroy(kv.second);
    X.pred_graphs.clear();
}

void ensure_rope(Xfmr &X, int64_t rows) {
    if (X.rope_rows >= rows) return;
    const int64_t half = X.hd / 2;
    std::vector<float> t(size_t(rows) * size_t(half) * 2);
    for (int64_t pos = 0; pos < rows; ++pos)
        for (int64_t p = 0; p < half; ++p) {
            const float f = X.inv_freq[size_t(p)] * float(pos);  // as rope_apply (kernels.cpp:744-747)
            t[size_t((pos * half + p) * 2)] = std::cos(f);
            t[size_t((pos * half + p) * 2 + 1)] = std::sin(f);
        }
    float *nr = dalloc_t<float>(t.size());
    h2d(nr, t.data(), t.size() * 4);
    HIPCHECK(hipStreamSynchronize(g.stream));
    dfree(X.rope);
    X.rope = nr;
    X.rope_rows = rows;
    drop_graphs(X);
}

// Row scratch for passes of up to rows rows (at least kMaxM). Growing it frees the old buffers, so the captured
// graphs go and the row table is uploaded again.
void ensure_rows(Xfmr &X, int rows) {
    rows = std::max(rows, kMaxM);
    if (X.cap_rows >= rows) return;
    if (X.cap_rows) HIPCHECK(hipStreamSynchronize(g.stream));
    drop_graphs(X);
    for (float *p : {X.h, X.qkv, X.q, X.g, X.xnorm, X.pre, X.pm, X.pl, X.po}) dfree(p);
    dfree(X.pa16); dfree(X.pb16);
    dfree(X.rows_dev); dfree(X.scfg_dev); dfree(X.token_dev);
    if (X.rows_host) (void)hipHostFree(X.rows_host);
    if (X.scfg_host) (void)hipHostFree(X.scfg_host);
    const size_t M = size_t(rows), qd = size_t(X.heads) * X.hd, kd = size_t(X.kvh) * X.hd;
    X.h = dalloc_t<float>(M * X.H);
    X.qkv = dalloc_t<float>(M * (qd + 2 * kd));
    X.q = dalloc_t<float>(M * qd);
    X.g = dalloc_t<float>(M * X.I);
    X.xnorm = dalloc_t<float>(M * X.H);
    X.pre = dalloc_t<float>(M * std::max<size_t>(size_t(X.H), qd));
    X.pa16 = dalloc_t<_Float16>(2 * M * std::max<size_t>(size_t(X.H), qd));
    X.pb16 = dalloc_t<_Float16>(2 * M * size_t(X.I));
    X.pm = dalloc_t<float>(M * X.heads * kAttnMaxSplits);
    X.pl = dalloc_t<float>(M * X.heads * kAttnMaxSplits);
    X.po = dalloc_t<float>(M * X.heads * kAttnMaxSplits * X.hd);
    const size_t rows_bytes = M * sizeof(RowRef) + M * size_t(X.hd) * 4;
    X.rows_dev = static_cast<RowRef *>(dalloc(rows_bytes));
    X.rope_rows_dev = reinterpret_cast<float *>(X.rows_dev + M);
    HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&X.rows_host), rows_bytes, hipHostMallocDefault));
    X.scfg_dev = dalloc_t<SampleCfgDev>(M);
    HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&X.scfg_host), M * sizeof(SampleCfgDev), hipHostMallocDefault));
    std::memset(X.scfg_host, 0, M * sizeof(SampleCfgDev));
    X.token_dev = dalloc_t<int32_t>(M);
    X.cap_rows = rows;
    X.rows_valid = false;
}

float *ensure_logits(Xfmr &X, int64_t elems) {
    if (X.logits_elems < elems) {
        HIPCHECK(hipStreamSynchronize(g.stream));
        dfree(X.logits);
        X.logits = dalloc_t<float>(size_t(elems));
        X.logits_elems = elems;
        drop_graphs(X);
    }
    return X.logits;
}
float *ensure_xin(Xfmr &X, int64_t elems) {
    if (X.xin_elems < elems) {
        HIPCHECK(hipStreamSynchronize(g.stream));
        dfree(X.xin);
        X.xin = dalloc_t<float>(size_t(elems));
        X.xin_elems = elems;
        drop_graphs(X);  // a captured frame loop reads the old input buffer
    }
    return X.xin;
}

// Uploads the per-row cache views (positions) of the next pass and the RoPE rows at those positions (computed as
// the table rows of ensure_rope); skips the copy when unchanged.
void set_rows(Xfmr &X, const std::vector<RowRef> &rows) {
    if (X.rows_valid && rows.size() == X.rows_last.size() &&
        std::memcmp(rows.data(), X.rows_last.data(), rows.size() * sizeof(RowRef)) == 0)
        return;
    HIPCHECK(hipStreamSynchronize(g.stream));  // the pinned block may still feed an earlier copy
    if (rows.size() > size_t(X.cap_rows)) throw Fail("pass rows exceed the row scratch");
    std::memcpy(X.rows_host, rows.data(), rows.size() * sizeof(RowRef));
    float *rope = reinterpret_cast<float *>(X.rows_host + X.cap_rows);
    const int half = X.hd / 2;
    for (size_t i = 0; i < rows.size(); ++i)
        for (int p = 0; p < half; ++p) {
            const float f = X.inv_freq[size_t(p)] * float(rows[i].pos);
            rope[i * size_t(X.hd) + 2 * size_t(p)] = std::cos(f);
            rope[i * size_t(X.hd) + 2 * size_t(p) + 1] = std::sin(f);
        }
    // the row table and the RoPE rows follow each other only up to the pass rows; copy the two spans
    HIPCHECK(copy_h2d(X.rows_dev, X.rows_host, rows.size() * sizeof(RowRef), g.stream));
    HIPCHECK(copy_h2d(X.rope_rows_dev, rope, rows.size() * size_t(X.hd) * 4, g.stream));
    X.rows_last = rows;
    X.rows_valid = true;
}


AttnPartials partials_of(const Xfmr &X) {
    AttnPartials p;
    p.pm = X.pm; p.pl = X.pl; p.po = X.po; p.rows = X.rows_dev; p.heads = X.heads; p.hd = X.hd;
    return p;
}

// Whether a pass takes the fused one-row FFN: one row, the fused attention, a transformer that has the panels.
bool ffn_pass(const Xfmr &X, int mc, int64_t m_total, bool fused) { return X.ffn_fuse && fused && mc == 1 && m_total == 1; }
// Kernels per layer: fused (rows of distinct sequences: decode, pairs, B sessions) 5, else 6 (+ k_qk_post); the
// fused FFN makes it 4 (and adds one accumulator fold per pass).
int kernels_per_layer(const Xfmr &X, int mc, bool fused) { return ffn_pass(X, mc, mc, fused) ? 4 : fused ? 5 : 6; }

// All layers for mc rows whose input is in X.h (row i at the position in rows_dev[i]).
// m_total: the caller's total row count, which picks the q8 arithmetic (int8 for <= 8, f32 above).
// fused: every row belongs to a different sequence, so the attention kernel can append K/V itself.
// A prefill pass of consecutive rows of one sequence takes attention on the matrix cores straight into the o input.
// A pass of one row whose position (row 0 of the current row table) is past kAttnSpecKeys, so that its cache keys
// 0 .. pos - 1 do not all fit the short first batch: its attention loads a full one (launch_attention's long_ctx).
// Graphs are keyed by it, so a step captured before the position passed kAttnSpecKeys is not the one replayed after.
bool long_row(const Xfmr &X, int mc) {
    return mc == 1 && !X.rows_last.empty() && X.rows_last[0].pos > kAttnSpecKeys;
}

bool pass_attn_of(const Xfmr &X, int mc, bool fused) {
    bool pass_attn = !fused && mc > 4 && (X.hd == 64 || X.hd == 128) && int(X.rows_last.size()) == mc;
    for (int i = 1; i < mc && pass_attn; ++i)
        pass_attn = X.rows_last[size_t(i)].k == X.rows_last[0].k && X.rows_last[size_t(i)].pos == X.rows_last[0].pos + i;
    return pass_attn;
}

// Head sizes other than 64 and 128 take k_qk_post, then k_attn_rows into X.pre, then the o GEMV on those rows.
bool any_hd(const Xfmr &X) { return X.hd != 64 && X.hd != 128; }

// Planes passes: a prefill pass of one sequence on the f32-activation GEMM whose four matrices are F16 or Q8 with K a
// multiple of 64 runs its GEMMs on f16 halves of their inputs that the producers write (the RMSNorms, the attention,
// the SwiGLU epilogue), so no GEMM block splits its A tile again, and Q8 weights as their int8 values widened to f16
// once (planes_weights). The products and their order are those of the f32-activation GEMM.
bool planes_mat(const GpuMat &m, int64_t m_total, int mc) {
    return (m.type == VOXHIP_F16 || m.type == VOXHIP_Q8) && m.cols % 64 == 0 && gemm_path(m, m_total, mc);
}
bool planes_layer(const Xfmr &X, int li, int64_t m_total, int mc, bool need_ready) {
    const LayerDev &L = X.L[size_t(li)];
    for (int id : {L.qkv, L.o, L.gu, L.down}) {
        const GpuMat &m = g.mats[size_t(id)];
        if (!planes_mat(m, m_total, mc) || (need_ready && m.type == VOXHIP_Q8 && !m.w16)) return false;
    }
    return true;
}
// The f16 weights of a planes GEMM: F16 as stored; Q8's int8 values widened into m.w16 on first use (outside any
// graph capture: forward_rows prepares them before its passes).
const _Float16 *planes_weights(GpuMat &m, hipStream_t s) {
    if (m.type == VOXHIP_F16) return reinterpret_cast<const _Float16 *>(m.w);
    if (!m.w16) {
        _Float16 *w16 = dalloc_t<_Float16>(size_t(m.rows) * size_t(m.cols));
        HIPCHECK(launch_q8_to_f16(reinterpret_cast<const int8_t *>(m.w), w16, m.rows * m.cols, s));
        m.w16 = w16;
    }
    return m.w16;
}
// The widened copies are an optimisation: when one cannot be allocated (VRAM limit or device memory), its matrix keeps
// m.w16 null, planes_layer(need_ready) then sends that layer to the f32-activation GEMM, and the pass still runs.
void prepare_planes(Xfmr &X, int first, int count, int64_t m_total, int mc, hipStream_t s) {
    for (int li = first; li < first + count; ++li)
        if (planes_layer(X, li, m_total, mc, false)) {
            const LayerDev &L = X.L[size_t(li)];
            for (int id : {L.qkv, L.o, L.gu, L.down}) {
                try {
                    (void)planes_weights(g.mats[size_t(id)], s);
                } catch (const Fail &) {
                    (void)hipGetLastError();  // a failed hipMalloc leaves its error for the next query
                }
            }
        }
}

// x0 (optional): the input rows ([mc][H]) when they are not in X.h yet. The first layer's q|k|v GEMV then reads them
// and its o GEMV adds its product to them into X.h, where the fused attention path allows; otherwise they are copied.
void enqueue_layers(Xfmr &X, int mc, int64_t m_total, int first, int count, hipStream_t s, bool fused, Probe *pr = nullptr,
                    const float *x0 = nullptr) {
    const int qd = X.heads * X.hd, kd = X.kvh * X.hd, ldqkv = qd + 2 * kd;
    const AttnPartials part = partials_of(X);
    const bool rows_attn = any_hd(X);
    if (rows_attn) fused = false;
    const bool pass_attn = pass_attn_of(X, mc, fused);
    const bool direct = x0 && count > 0 && !rows_attn && !pass_attn && !gemm_path(g.mats[size_t(X.L[size_t(first)].o)], m_total, mc);
    if (x0 && !direct) HIPCHECK(hipMemcpyAsync(X.h, x0, size_t(mc) * X.H * 4, hipMemcpyDeviceToDevice, s));
    const bool ffn = !rows_attn && !pass_attn && ffn_pass(X, mc, m_total, fused);
    bool pa_normed = false;  // planes: the previous layer's down reduce already wrote this layer's first RMSNorm
    bool acc_live = false;   // the previous layer's fused FFN left its down product in X.acc (added by q|k|v and o)
    for (int li = first; li < first + count; ++li) {
        const LayerDev &L = X.L[size_t(li)];
        const GpuMat &Mqkv = g.mats[size_t(L.qkv)], &Mo = g.mats[size_t(L.o)], &Mgu = g.mats[size_t(L.gu)],
                     &Md = g.mats[size_t(L.down)];
        const float *qn = L.qk ? X.norms + L.qn : nullptr, *kn = L.qk ? X.norms + L.kn : nullptr;
        // planes pass: GEMM inputs as f16 halves, hi plane then lo plane PA (PB) halves on
        const bool planes = pass_attn && !rows_attn && planes_layer(X, li, m_total, mc, true);
        const int64_t PA = int64_t(X.cap_rows) * std::max<int64_t>(X.H, qd), PB = int64_t(X.cap_rows) * X.I;
        auto hh_args = [&](const GpuMat &M, const _Float16 *a16, int64_t a_lo, float *y, int64_t ldy) {
            const PassScratch sc = lib_scratch();
            GemmArgs ga{};
            ga.bias = M.b; ga.y = y; ga.ldy = ldy; ga.m = mc; ga.n = int32_t(M.rows); ga.K = int32_t(M.cols);
            ga.a16 = a16; ga.a_lo = a_lo; ga.lda = M.cols; ga.ws = sc.ws; ga.ws_cap = sc.ws_cap;
            return ga;
        };
        auto w16_of = [](const GpuMat &M) {
            return M.type == VOXHIP_F16 ? reinterpret_cast<const _Float16 *>(M.w) : static_cast<const _Float16 *>(M.w16);
        };
        auto hh = [&](const GpuMat &M, int epi, const _Float16 *a16, int64_t a_lo, float *y, int64_t ldy) {
            GemmArgs ga = hh_args(M, a16, a_lo, y, ldy);
            if (epi == EPI_SWIGLU_H16) { ga.y = nullptr; ga.h16 = X.pb16; ga.lo_off = PB; }
            HIPCHECK(launch_gemm_hh(epi, w16_of(M), M.type == VOXHIP_Q8 ? M.s : nullptr, ga, s));
        };
        probed(pr, VOXHIP_K_QKV, [&] {
            if (planes) {
                if (!pa_normed) HIPCHECK(launch_rmsnorm_rows_h16(X.h, X.H, X.norms + L.ln1, int(X.H), X.eps, X.pa16, X.H, PA, mc, s));
                hh(Mqkv, EPI_STORE, X.pa16, PA, X.qkv, ldqkv);
            } else {
                gemv(Mqkv, m_total, PRO_RMS, EPI_STORE, direct && li == first ? x0 : X.h, X.H, mc, X.qkv, ldqkv, X.norms + L.ln1, X.eps,
                     nullptr, s, nullptr, X.pre, nullptr, acc_live ? X.acc : nullptr);
            }
        });
        if (!fused) {
            QkArgs qa;
            qa.qkv = X.qkv; qa.ldqkv = ldqkv; qa.q = X.q; qa.rows = X.rows_dev; qa.qn = qn; qa.kn = kn;
            qa.rope = X.rope; qa.heads = X.heads; qa.kv_heads = X.kvh; qa.hd = X.hd; qa.layer = li; qa.eps = X.eps;
            probed(pr, VOXHIP_K_QKPOST, [&] { HIPCHECK(launch_qk_post(qa, mc, s)); });
        }
        const RowRef &r0 = X.rows_last.at(0);
        if (rows_attn) {
            AttnRowsArgs ra{};
            ra.q = X.q; ra.out = X.pre; ra.rows = X.rows_dev; ra.heads = X.heads; ra.kv_heads = X.kvh; ra.hd = X.hd;
            ra.layer = li; ra.scale = 1.0f / std::sqrt(float(X.hd));
            probed(pr, VOXHIP_K_ATTN, [&] { HIPCHECK(launch_attn_rows(ra, mc, s)); });
            probed(pr, VOXHIP_K_O, [&] { gemv(Mo, m_total, PRO_X, EPI_ACC, X.pre, qd, mc, X.h, X.H, nullptr, 0.f, nullptr, s); });
        } else if (pass_attn && gemm_path(Mo, m_total, mc)) {
            PrefillAttnArgs pa{};
            pa.q = X.q; pa.k = r0.k; pa.v = r0.v; pa.out = X.pre; pa.rows = X.rows_dev; pa.cap = r0.cap; pa.pos0 = r0.pos;
            pa.m = mc;
            pa.heads = X.heads; pa.kv_heads = X.kvh; pa.layer = li; pa.scale = 1.0f / std::sqrt(float(X.hd));
            if (planes) { pa.out16 = X.pa16; pa.lo_off = PA; }
            pa.part = part;  // key-split runs (the partial buffers hold cap_rows rows)
            probed(pr, VOXHIP_K_ATTN, [&] { HIPCHECK(launch_prefill_attn(pa, X.hd, s)); });
            probed(pr, VOXHIP_K_O, [&] {
                if (planes) hh(Mo, EPI_ACC, X.pa16, PA, X.h, X.H);
                else gemv(Mo, m_total, PRO_X, EPI_ACC, X.pre, qd, mc, X.h, X.H, nullptr, 0.f, nullptr, s);
            });
        } else {
            AttnArgs aa;
            aa.ldqkv = ldqkv; aa.q = X.q; aa.qn = qn; aa.kn = kn; aa.part = part;
            aa.kv_heads = X.kvh; aa.scale = 1.0f / std::sqrt(float(X.hd)); aa.eps = X.eps;
            probed(pr, VOXHIP_K_ATTN, [&] {
                HIPCHECK(launch_attention(aa, r0.k, r0.v, r0.cap, X.qkv, X.rope_rows_dev, li, X.hd, X.heads / X.kvh, mc, fused, s,
                                          long_row(X, mc)));
            });
            probed(pr, VOXHIP_K_O, [&] {
                gemv(Mo, m_total, PRO_ATTN, EPI_ACC, nullptr, 0, mc, X.h, X.H, nullptr, 0.f, nullptr, s, &part, X.pre, nullptr,
                     acc_live ? X.acc : nullptr, direct && li == first ? x0 : nullptr);
            });
            acc_live = false;
        }
        if (ffn) {  // RMSNorm, gate|up, SwiGLU and the down product in one launch; h gets the product via X.acc
            FfnArgs fa{};
            fa.gu = Mgu.w; fa.gu_s = Mgu.s; fa.gu_b = Mgu.b;
            fa.dp = L.pan; fa.dp_s = static_cast<const float *>(L.pan_s); fa.d_b = Md.b;
            fa.x = X.h; fa.gamma = X.norms + L.ln2; fa.acc = X.acc;
            fa.H = X.H; fa.I = X.I; fa.parts = ffn_parts(); fa.eps = X.eps;
            probed(pr, VOXHIP_K_FFN, [&] { HIPCHECK(launch_ffn(gemv_type(Mgu), fa, s)); });
            acc_live = true;
            continue;
        }
        QRows gq{};
        const bool gq_on = !planes && ffn_quant_epilogue(Mgu, Md, m_total, mc, lib_scratch(), &gq);
        probed(pr, VOXHIP_K_GATEUP, [&] {
            if (planes) {
                HIPCHECK(launch_rmsnorm_rows_h16(X.h, X.H, X.norms + L.ln2, int(X.H), X.eps, X.pa16, X.H, PA, mc, s));
                hh(Mgu, EPI_SWIGLU_H16, X.pa16, PA, nullptr, X.I);
            } else {
                gemv(Mgu, m_total, PRO_RMS, EPI_SWIGLU, X.h, X.H, mc, X.g, X.I, X.norms + L.ln2, X.eps, nullptr, s, nullptr, X.pre,
                     nullptr, nullptr, nullptr, nullptr, gq_on ? &gq : nullptr);
            }
        });
        pa_normed = false;
        probed(pr, VOXHIP_K_DOWN, [&] {
            // the next layer's first RMSNorm rides on this split-K reduce when that layer is a planes pass too
            if (planes && li + 1 < first + count && planes_layer(X, li + 1, m_total, mc, true)) {
                const GemmArgs ga = hh_args(Md, X.pb16, PB, X.h, X.H);
                HIPCHECK(launch_gemm_hh_acc_rms(w16_of(Md), Md.type == VOXHIP_Q8 ? Md.s : nullptr, ga,
                                                X.norms + X.L[size_t(li + 1)].ln1, X.eps, X.pa16, X.H, PA, s, &pa_normed));
            } else if (planes) {
                hh(Md, EPI_ACC, X.pb16, PB, X.h, X.H);
            } else {
                gemv(Md, m_total, PRO_X, EPI_ACC, X.g, X.I, mc, X.h, X.H, nullptr, 0.f, nullptr, s, nullptr, nullptr, nullptr,
                     nullptr, nullptr, nullptr, nullptr, gq_on ? &gq : nullptr);
            }
        });
    }
    // the last fused FFN's product into h, so every pass leaves h whole and the accumulators at zero
    if (acc_live) probed(pr, VOXHIP_K_FOLD, [&] { HIPCHECK(launch_acc_fold(X.h, X.acc, X.H, s)); });
}

// Final RMSNorm of rows [r0, r0 + mr) of X.h into X.xnorm, and the head on them when head >= 0.
void enqueue_final(Xfmr &X, int r0, int mr, int head, hipStream_t s) {
    if (head >= 0) {
        const GpuMat &Hm = mat_at(head);
        if (Hm.cols != X.H) throw Fail("head width differs from the hidden size");
        float *lg = ensure_logits(X, int64_t(mr) * Hm.rows);
        gemv(Hm, mr, PRO_RMS, EPI_STORE, X.h + size_t(r0) * X.H, X.H, mr, lg, Hm.rows, X.norms + X.final_off, X.eps,
             X.xnorm, s);
    } else {
        HIPCHECK(launch_rmsnorm_rows(X.h + size_t(r0) * X.H, X.H, X.norms + X.final_off, X.H, X.eps, X.xnorm, X.H, mr, s));
    }
}

// enqueue_layers on the library stream for forward_rows, through a captured graph once the same pass shape has been
// seen before. Every launch reads positions, RoPE rows and cache views from the device row table, so a graph replays
// at any position of the same sequence; its buffers are the transformer's row scratch, whose growth drops the graphs.
void run_layers(Xfmr &X, int mc, int64_t m_total, int first, int count, bool fused) {
    if (vh::prof_on()) return enqueue_layers(X, mc, m_total, first, count, g.stream, fused);  // stamped launches
    const RowRef &r0 = X.rows_last.at(0);
    const LayersKey key{mc, int(std::min<int64_t>(m_total, kMaxM + 1)), first, count, fused ? 1 : 0,
                        pass_attn_of(X, mc, fused) ? 1 : 0, long_row(X, mc) ? 1 : 0, r0.k, r0.v, r0.cap};
    auto it = X.layer_graphs.find(key);
    if (it != X.layer_graphs.end()) {
        HIPCHECK(hipGraphLaunch(it->second, g.stream));
        return;
    }
    if (++X.layer_uses[key] < 2 || int(X.layer_graphs.size()) >= kMaxLayerGraphs) {  // one-off shapes run eagerly
        enqueue_layers(X, mc, m_total, first, count, g.stream, fused);
        return;
    }
    hipGraph_t graph = nullptr;
    HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
    try {
        enqueue_layers(X, mc, m_total, first, count, g.stream, fused);
    } catch (...) {
        (void)hipStreamEndCapture(g.stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    HIPCHECK(hipStreamEndCapture(g.stream, &graph));
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HIPCHECK(e);
    X.layer_graphs[key] = exec;
    HIPCHECK(hipGraphLaunch(exec, g.stream));
}

RowRef row_of(const Seq &S, int64_t pos) {
    RowRef r;
    r.k = S.k; r.v = S.v; r.cap = S.cap; r.pos = pos;
    return r;
}

void check_seq_for(Xfmr &X, int xid, const Seq &S) {
    if (S.xfmr != xid && (S.layers < X.layers || S.kvh != X.kvh || S.hd != X.hd)) throw Fail("sequence belongs to another transformer shape");
    ensure_rope(X, S.cap);  // the RoPE table must cover every position the sequence can hold
}

// Generic host-pointer forward for up to any m rows of one sequence (or B rows of B sequences).
// rows_of(i) gives the cache view of row i. x rows are xc wide (in_proj cols or hidden). Returns the row of X.h
// that holds the last input row's hidden state.
template <class RowsOf>
int forward_rows(Xfmr &X, int64_t m, RowsOf rows_of, const float *x, int in_proj, int first_layer, int n_layers, int64_t m_total,
                  float *hidden_out, float *out_last, int head, float *head_out, bool final_all) {
    vh::prof_stage(X.name.c_str());
    const int64_t H = X.H;
    const GpuMat *Pm = in_proj >= 0 ? &mat_at(in_proj) : nullptr;
    if (Pm && Pm->rows != H) throw Fail("in_proj rows differ from the hidden size");
    const int64_t xc = Pm ? Pm->cols : H;
    // rows per pass: the smallest of the passes the used matrices allow (8 on the int8 path, 512 on the f32 path)
    int chunk = kMaxPass, last_row = 0;
    for (int li = first_layer; li < first_layer + n_layers; ++li)
        for (int id : {X.L[size_t(li)].qkv, X.L[size_t(li)].o, X.L[size_t(li)].gu, X.L[size_t(li)].down})
            chunk = std::min(chunk, rows_per_pass(g.mats[size_t(id)], m_total));
    if (Pm) chunk = std::min(chunk, rows_per_pass(*Pm, m_total));
    if (head >= 0 && final_all) chunk = std::min(chunk, rows_per_pass(mat_at(head), m_total));
    const int64_t V = head >= 0 ? mat_at(head).rows : 0;
    chunk = int(std::min<int64_t>(chunk, m));
    ensure_rows(X, chunk);
    float *pin = pinned(size_t(chunk) * size_t(std::max<int64_t>(std::max(xc, H), V)) * 4 + 64);
    for (int64_t c0 = 0; c0 < m; c0 += chunk) {
        const int mc = int(std::min<int64_t>(chunk, m - c0));
        const bool last = c0 + mc == m;
        last_row = mc - 1;
        std::vector<RowRef> rr(static_cast<size_t>(mc));
        for (int i = 0; i < mc; ++i) rr[size_t(i)] = rows_of(c0 + i);
        set_rows(X, rr);
        HIPCHECK(hipStreamSynchronize(g.stream));
        std::memcpy(pin, x + c0 * xc, size_t(mc * xc) * 4);
        if (Pm) {
            float *xin = ensure_xin(X, int64_t(chunk) * xc);
            HIPCHECK(copy_h2d(xin, pin, size_t(mc * xc) * 4, g.stream));
            gemv(*Pm, m_total, PRO_X, EPI_STORE, xin, xc, mc, X.h, H, nullptr, 0.f, nullptr, g.stream);
        } else {
            HIPCHECK(copy_h2d(X.h, pin, size_t(mc * H) * 4, g.stream));
        }
        bool fused = true;
        for (int i = 0; i < mc && fused; ++i)
            for (int j = 0; j < i; ++j)
                if (rr[size_t(i)].k == rr[size_t(j)].k) { fused = false; break; }
        if (pass_attn_of(X, mc, fused)) prepare_planes(X, first_layer, n_layers, m_total, mc, g.stream);
        run_layers(X, mc, m_total, first_layer, n_layers, fused);
        if (hidden_out) {
            HIPCHECK(copy_d2h(pin, X.h, size_t(mc * H) * 4, g.stream));
            HIPCHECK(hipStreamSynchronize(g.stream));
            std::memcpy(hidden_out + c0 * H, pin, size_t(mc * H) * 4);
        }
        if (final_all || last) {
            const int r0 = final_all ? 0 : mc - 1, mr = final_all ? mc : 1;
            if (out_last || head >= 0) {
                enqueue_final(X, r0, mr, head, g.stream);
                if (out_last) {
                    HIPCHECK(copy_d2h(pin, X.xnorm, size_t(mr * H) * 4, g.stream));
                    HIPCHECK(hipStreamSynchronize(g.stream));
                    std::memcpy(out_last + (final_all ? c0 * H : 0), pin, size_t(mr * H) * 4);
                }
                if (head >= 0 && head_out) {
                    HIPCHECK(copy_d2h(pin, X.logits, size_t(mr * V) * 4, g.stream));
                    HIPCHECK(hipStreamSynchronize(g.stream));
                    std::memcpy(head_out + (final_all ? c0 * V : 0), pin, size_t(mr * V) * 4);
                }
            }
        }
    }
    sync_status();
    return last_row;
}

void fill_sample_cfg(SampleCfgDev &d, const voxhip_sample_cfg &c, const int32_t *hist_dev, int32_t n_hist) {
    d.temperature = c.temperature; d.top_p = c.top_p; d.rep = c.repetition_penalty; d.top_k = c.top_k;
    d.key0 = c.key0; d.key1 = c.key1; d.frame = c.frame; d.cb = c.codebook; d.draw = c.draw;
    d.sup_from = c.suppress_from; d.sup_to = c.suppress_to; d.eos = c.eos_code; d.block_eos = c.block_eos;
    d.n_history = n_hist; d.history = hist_dev;
}

template <class F>
int guard_int(F &&f, int fail) {
    std::lock_guard<std::mutex> lk(g.mu);
    try {
        return f();
    } catch (const std::exception &e) {
        set_error(e.what());
        return fail;
    }
}

const char *kWhich[7] = {"q", "k", "v", "o", "gate", "up", "down"};

// codec: the codec's pre-transformer, whose forward (sliding window, layer scales, f32 ring) is the codec's own; only
// its matrices, norms and scratch come from here.
// The fused one-row FFN applies when every layer's four matrices take the int path at one row (Q8 / Q4), gate|up
// and down share a format and the shapes fit k_ffn_int and the staged q|k|v prologue that adds the pending sums
// (H <= 8 * 256); the attention is the fused kernel (head_dim 64 or 128). The down weights are then also kept as
// panels (one more copy of them).
void make_ffn_panels(Xfmr &X) {
    const char *env = std::getenv("VOXHIP_FFN_FUSED");
    // Where it pays: the next layer's q|k|v GEMV must then read the pending sums, which costs about what the second
    // launch saved at FFN width 3 H (the Qwen3-TTS talker and code predictor), while FFNs of 4 H and wider (the
    // CosyVoice2 LM's 896 -> 4864) gain. VOXHIP_FFN_FUSED=1 forces it on, =0 off.
    const bool force = env && env[0] == '1';
    // The q|k|v and o GEMVs that add the pending sums stage their input rows (K = H and K = heads x hd) with one
    // 8-value slot per thread, so both widths must fit 8 x kGemvThreads.
    bool ok = !(env && env[0] == '0') && (force || int64_t(X.I) >= 4 * int64_t(X.H)) && (X.hd == 64 || X.hd == 128) &&
              X.H <= 8 * kGemvThreads && int64_t(X.heads) * X.hd <= 8 * kGemvThreads && !X.L.empty();
    for (const LayerDev &L : X.L) {
        if (!ok) break;
        for (int id : {L.qkv, L.o, L.gu, L.down}) ok = ok && quantized(g.mats[size_t(id)].type);
        const GpuMat &GU = g.mats[size_t(L.gu)], &D = g.mats[size_t(L.down)];
        ok = ok && gemv_type(GU) == gemv_type(D) && ffn_shape_ok(gemv_type(D), X.H, X.I);
    }
    if (!ok) return;
    try {
        for (LayerDev &L : X.L) {
            const GpuMat &D = g.mats[size_t(L.down)];
            const size_t nbytes = size_t(D.rows) * row_bytes(D.type, D.cols), sbytes = size_t(D.rows) * scale_row_bytes(D);
            L.pan = static_cast<uint8_t *>(dalloc(nbytes));
            L.pan_s = dalloc(sbytes);
            HIPCHECK(launch_panel_pack(gemv_type(D), D.w, D.s, X.H, X.I, L.pan, L.pan_s, g.stream));
        }
        X.acc = static_cast<int64_t *>(dalloc(size_t(kAccCopies) * size_t(X.H) * sizeof(int64_t)));
        HIPCHECK(hipMemsetAsync(X.acc, 0, size_t(kAccCopies) * size_t(X.H) * sizeof(int64_t), g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
    } catch (const Fail &) {  // no room for the panels under the VRAM limit: the two-GEMV FFN needs none
        (void)hipStreamSynchronize(g.stream);
        for (LayerDev &L : X.L) {
            dfree(L.pan); dfree(L.pan_s);
            L.pan = nullptr; L.pan_s = nullptr;
        }
        dfree(X.acc);
        X.acc = nullptr;
        return;
    }
    X.ffn_fuse = true;
}

int make_xfmr(const voxhip_xfmr_desc *w, const char *name, int use_layers, const int32_t *mats, voxhip_uploaded_fn uploaded,
              void *user, bool codec = false) {
    require_ok();
    if (!w || w->n_layers <= 0 || !w->layers || !w->final_norm || !w->inv_freq) throw Fail("incomplete transformer description");
    if (w->window != 0 && !codec) throw Fail("sliding-window attention is not supported on the device");
    if (w->head_dim <= 0 || w->head_dim > 128 || w->head_dim % 2) throw Fail("head_dim must be even and at most 128");
    if (w->heads <= 0 || w->kv_heads <= 0 || w->heads % w->kv_heads || w->heads / w->kv_heads > 8)
        throw Fail("heads / kv_heads must be an integer group of at most 8");
    if (w->hidden % 32 || w->inter % 32) throw Fail("hidden and inter must be multiples of 32");
    const int nl = use_layers < 0 || use_layers > w->n_layers ? w->n_layers : use_layers;
    auto X = new Xfmr();
    try {
        X->name = name ? name : "xfmr";
        X->layers = nl; X->H = w->hidden; X->heads = w->heads; X->kvh = w->kv_heads; X->hd = w->head_dim; X->I = w->inter;
        X->eps = w->eps; X->theta = w->theta;
        X->inv_freq.assign(w->inv_freq, w->inv_freq + w->head_dim / 2);
        std::vector<float> nv;
        auto push = [&](const float *p, int n) {
            const size_t off = nv.size();
            nv.insert(nv.end(), p, p + n);
            return off;
        };
        for (int li = 0; li < nl; ++li) {
            const voxhip_layer &L = w->layers[li];
            if ((L.attn_scale || L.mlp_scale) && !codec) throw Fail("layer scales are not supported on the device");
            if (!L.ln1 || !L.ln2) throw Fail("layer without norms");
            if ((L.qn == nullptr) != (L.kn == nullptr)) throw Fail("q_norm and k_norm must both be present or absent");
            LayerDev d;
            if (mats) {
                const int32_t *h = mats + 7 * li;
                for (int j = 0; j < 7; ++j) mat_at(h[j]);
                auto desc_of = [&](int id) {
                    const GpuMat &m = g.mats[size_t(id)];
                    return std::make_tuple(m.type, m.cols);
                };
                if (desc_of(h[0]) != desc_of(h[1]) || desc_of(h[0]) != desc_of(h[2]) || desc_of(h[4]) != desc_of(h[5]))
                    throw Fail("stacked matrices differ in type or width");
                // stack / interleave on the device
                auto stack = [&](std::initializer_list<int> ids, bool inter) {
                    const GpuMat &m0 = g.mats[size_t(*ids.begin())];
                    int64_t rows = 0;
                    bool bias = true;
                    for (int id : ids) { rows += g.mats[size_t(id)].rows; bias = bias && g.mats[size_t(id)].b; }
                    for (int id : ids)
                        if (g.mats[size_t(id)].s16 != m0.s16) throw Fail("stacked matrices differ in scale storage");
                    const int nid = new_mat(m0.type, rows, m0.cols, bias, m0.s16);
                    for (int id : ids) g.mats[size_t(nid)].wmax = std::max(g.mats[size_t(nid)].wmax, g.mats[size_t(id)].wmax,
                                                                          [](float a, float b) { return a < b || std::isnan(b); });
                    const size_t rb = row_bytes(m0.type, m0.cols), sb = scale_row_bytes(m0);
                    int64_t r0 = 0;
                    int part = 0;
                    for (int id : ids) {
                        const GpuMat src = g.mats[size_t(id)];
                        GpuMat &dst = g.mats[size_t(nid)];
                        if (!inter) {
                            HIPCHECK(hipMemcpy(dst.w + size_t(r0) * rb, src.w, size_t(src.rows) * rb, hipMemcpyDeviceToDevice));
                            if (sb) HIPCHECK(hipMemcpy(reinterpret_cast<uint8_t *>(dst.s) + size_t(r0) * sb, src.s, size_t(src.rows) * sb, hipMemcpyDeviceToDevice));
                            if (bias) HIPCHECK(hipMemcpy(dst.b + r0, src.b, size_t(src.rows) * 4, hipMemcpyDeviceToDevice));
                        } else {
                            HIPCHECK(hipMemcpy2D(dst.w + size_t(part) * rb, 2 * rb, src.w, rb, rb, size_t(src.rows), hipMemcpyDeviceToDevice));
                            if (sb) HIPCHECK(hipMemcpy2D(reinterpret_cast<uint8_t *>(dst.s) + size_t(part) * sb, 2 * sb, src.s, sb, sb, size_t(src.rows), hipMemcpyDeviceToDevice));
                            if (bias) HIPCHECK(hipMemcpy2D(dst.b + part, 8, src.b, 4, 4, size_t(src.rows), hipMemcpyDeviceToDevice));
                        }
                        r0 += src.rows;
                        ++part;
                    }
                    return nid;
                };
                d.qkv = stack({h[0], h[1], h[2]}, false);
                d.o = stack({h[3]}, false);
                d.gu = stack({h[4], h[5]}, true);
                d.down = stack({h[6]}, false);
            } else {
                const voxhip_mat qkv[3] = {L.q, L.k, L.v}, gu[2] = {L.gate, L.up};
                d.qkv = upload_parts(qkv, 3, false);
                d.o = upload_parts(&L.o, 1, false);
                d.gu = upload_parts(gu, 2, true);
                d.down = upload_parts(&L.down, 1, false);
                if (uploaded)
                    for (int j = 0; j < 7; ++j) uploaded(user, li, j);
            }
            const GpuMat &Q = g.mats[size_t(d.qkv)], &O = g.mats[size_t(d.o)], &GU = g.mats[size_t(d.gu)], &D = g.mats[size_t(d.down)];
            const int64_t qd = int64_t(w->heads) * w->head_dim, kd = int64_t(w->kv_heads) * w->head_dim;
            if (Q.rows != qd + 2 * kd || Q.cols != w->hidden || O.rows != w->hidden || O.cols != qd || GU.rows != 2 * int64_t(w->inter) ||
                GU.cols != w->hidden || D.rows != w->hidden || D.cols != w->inter)
                throw Fail("layer matrix shapes do not match the transformer description");
            d.ln1 = push(L.ln1, w->hidden);
            d.ln2 = push(L.ln2, w->hidden);
            d.qk = L.qn && L.kn;
            if (d.qk) { d.qn = push(L.qn, w->head_dim); d.kn = push(L.kn, w->head_dim); }
            X->L.push_back(d);
        }
        X->final_off = push(w->final_norm, w->hidden);
        X->norms = dalloc_t<float>(nv.size());
        h2d(X->norms, nv.data(), nv.size() * 4);
        make_ffn_panels(*X);
        ensure_rows(*X, kMaxM);
        ensure_rope(*X, 4096);
    } catch (...) {
        delete X;
        throw;
    }
    g.xf.push_back(X);
    return int(g.xf.size()) - 1;
}

// "<marketing name> (<arch>)". Some driver stacks report an empty marketing name; the label then names the
// product family of the architecture, so device lists and GpuDeviceInfo::name still say what the card is.
std::string device_label(const hipDeviceProp_t &p) {
    return vh::device_label(std::string(p.name, strnlen(p.name, sizeof p.name)), p.gcnArchName);
}

int parse_index(const char *spec) {
    int idx = 0;
    if (spec) {
        const char *c = std::strchr(spec, ':');
        if (c) idx = std::atoi(c + 1);
    }
    if (const char *e = std::getenv("VOX_VK_DEVICE")) idx = std::atoi(e);
    if (const char *e = std::getenv("VOX_HIP_DEVICE")) idx = std::atoi(e);
    return idx;
}

}  // namespace

// ====================================================================== C ABI
extern "C" {

int voxhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int voxhip_device_info_get(int index, voxhip_device_info *out) {
    if (!out) return 0;
    std::memset(out, 0, sizeof *out);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, index) != hipSuccess) return 0;
    DevProps d;
    d.name.assign(p.name, strnlen(p.name, sizeof p.name));
    d.arch = p.gcnArchName;
    d.total = d.free = p.totalGlobalMem;
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur == index) {
        size_t f = 0, t = 0;
        if (hipMemGetInfo(&f, &t) == hipSuccess) d.free = f;
    }
    d.integrated = p.integrated;
    d.major = p.major;
    d.minor = p.minor;
    (void)hipRuntimeGetVersion(&d.runtime);
    device_info_of(index, d, out);
    return 1;
}

int voxhip_init(const char *device, char *err, size_t err_len) {
    std::lock_guard<std::mutex> lk(g.mu);
    auto put_err = [&](const std::string &m) {
        if (err && err_len) { std::snprintf(err, err_len, "%s", m.c_str()); }
    };
    const char *ch = std::getenv("VOXHIP_CHECK_HOST");  // re-read by every call, also after a successful init
    g.check_copies = ch && ch[0] == '1';
    if (g.ok) return 1;
    if (!g.init_error.empty()) { put_err(g.init_error); return 0; }
    try {
        const int idx = parse_index(device);
        int n = 0;
        HIPCHECK(hipGetDeviceCount(&n));
        if (idx < 0 || idx >= n) throw Fail("HIP device " + std::to_string(idx) + " not found (" + std::to_string(n) + " present)");
        HIPCHECK(hipSetDevice(idx));
        hipDeviceProp_t p;
        HIPCHECK(hipGetDeviceProperties(&p, idx));
        if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
            throw Fail(std::string("device is ") + p.gcnArchName + "; this backend is built for gfx950 (MI355X)");
        HIPCHECK(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
        g.dev = idx;
        g.gemm_ws = dalloc_t<float>(size_t(kGemmWsFloats));
        g.qrows = dalloc_t<int8_t>(size_t(kQuantRowsElems));
        g.qrows_s = dalloc_t<float>(size_t(kQuantRowsElems / 32));
        g.qrows_sum = dalloc_t<int32_t>(size_t(kQuantRowsElems / 32));
        g.status_dev = dalloc_t<int32_t>(2);
        HIPCHECK(hipMemset(g.status_dev, 0, 2 * sizeof(int32_t)));
        HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&g.status_pin), 2 * sizeof(int32_t), hipHostMallocDefault));
        g.status_pin[0] = g.status_pin[1] = 0;
        if (idx >= int(g.noalloc.size())) throw Fail("device index above the scratch table");
        void *sp = nullptr;
        HIPCHECK(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
        if (!sp || reinterpret_cast<uintptr_t>(sp) % 256) throw Fail("no device address for the no-alloc scratch");
        g.noalloc[size_t(idx)] = static_cast<uint8_t *>(sp);
        g.name = device_label(p);
        // VOX_PROFILE=gpu (gpu_vulkan.cpp:312-326): per-launch GPU timestamps, the table on stderr at exit
        const char *pe = std::getenv("VOX_PROFILE");
        if (pe && std::strstr(pe, "gpu")) {
            vh::prof_enable();
            std::atexit([] {
                const char *t = vh::prof_report(g.name.c_str());
                if (t && *t) std::fputs(t, stderr);
            });
        }
        g.ok = true;
        return 1;
    } catch (const std::exception &e) {
        g.init_error = std::string("HIP init failed: ") + e.what();
        put_err(g.init_error);
        return 0;
    }
}

int voxhip_active(void) { return g.ok ? 1 : 0; }
const char *voxhip_profile_report(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    return vh::prof_report(g.name.c_str());
}
const char *voxhip_device_name(void) { return g.name.c_str(); }
void voxhip_stats_get(voxhip_stats *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (out) *out = g.stats;
}
const char *voxhip_last_error(void) {
    // a copy taken under the lock: another thread's failure may replace g.last_error meanwhile
    thread_local std::string copy;
    std::lock_guard<std::mutex> lk(g.mu);
    copy = g.last_error;
    return copy.c_str();
}
void voxhip_set_vram_limit(uint64_t bytes) {
    std::lock_guard<std::mutex> lk(g.mu);
    g.vram_limit = bytes;
}
void voxhip_mem_info_get(voxhip_mem_info *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!out) return;
    std::memset(out, 0, sizeof *out);
    out->device_index = -1;
    if (!g.ok) return;
    out->used = g.vram_used;
    out->limit = g.vram_limit;
    out->device_index = g.dev;
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) == hipSuccess) { out->device_free = f; out->device_total = t; }
}

int voxhip_upload(const voxhip_mat *parts, int n_parts) {
    std::lock_guard<std::mutex> lk(g.mu);
    uint64_t bytes = 0;
    try {
        require_ok();
        if (!parts || n_parts <= 0) throw Fail("no matrix");
        for (int i = 0; i < n_parts; ++i) bytes += uint64_t(parts[i].rows) * row_bytes(parts[i].type, parts[i].cols);
        return upload_parts(parts, n_parts, false);
    } catch (const std::exception &e) {
        g.stats.mats_failed += n_parts > 0 ? n_parts : 0;
        g.stats.bytes_failed += bytes;
        set_error(e.what());
        if (!g.warned) { std::fprintf(stderr, "vox: GPU upload failed (%s); some weights will stay on CPU\n", e.what()); g.warned = true; }
        return -1;
    }
}

int voxhip_mat_shape(int mat, int64_t *rows, int64_t *cols) {
    return guard_int([&] {
        const GpuMat &m = mat_at(mat);
        if (rows) *rows = m.rows;
        if (cols) *cols = m.cols;
        return 1;
    }, 0);
}

int voxhip_matmul(int mat, const float *x, int64_t m, float *y) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("matmul");
        const GpuMat &M = mat_at(mat);
        if (m <= 0) return 1;
        const int chunk = rows_per_pass(M, m);
        const size_t xb = size_t(chunk) * size_t(M.cols) * 4, yb = size_t(chunk) * size_t(M.rows) * 4;
        float *pin = pinned(std::max(xb, yb) + 64);
        float *dx = dev_scratch(g.dbuf_x, g.dbuf_x_bytes, xb), *dy = dev_scratch(g.dbuf_y, g.dbuf_y_bytes, yb);
        for (int64_t c0 = 0; c0 < m; c0 += chunk) {
            const int mc = int(std::min<int64_t>(chunk, m - c0));
            std::memcpy(pin, x + c0 * M.cols, size_t(mc) * size_t(M.cols) * 4);
            HIPCHECK(copy_h2d(dx, pin, size_t(mc) * size_t(M.cols) * 4, g.stream));
            gemv(M, m, PRO_X, EPI_STORE, dx, M.cols, mc, dy, M.rows, nullptr, 0.f, nullptr, g.stream);
            HIPCHECK(copy_d2h(pin, dy, size_t(mc) * size_t(M.rows) * 4, g.stream));
            HIPCHECK(hipStreamSynchronize(g.stream));
            std::memcpy(y + c0 * M.rows, pin, size_t(mc) * size_t(M.rows) * 4);
        }
        sync_status();
        return 1;
    }, 0);
}

int voxhip_matmul_dev_noalloc(int mat, const float *d_x, int64_t m, float *d_y) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("matmul");
        const GpuMat &M = mat_at(mat);
        if (m < 0 || (m > 0 && (!d_x || !d_y))) throw Fail("matmul_dev_noalloc: missing argument");
        if (m == 0) return 1;
        uint8_t *base = g.noalloc[size_t(g.dev)];
        if (!base) throw Fail("matmul_dev_noalloc: no scratch address for this device");
        // the fixed scratch: split-K partials, then the quantized rows, their scales and block sums
        PassScratch sc;
        sc.ws = reinterpret_cast<float *>(base);
        sc.ws_cap = kNoAllocWsFloats;
        sc.q = reinterpret_cast<int8_t *>(base + kNoAllocWsFloats * 4);
        sc.qs = reinterpret_cast<float *>(base + kNoAllocWsFloats * 4 + kNoAllocQElems);
        sc.qsum = reinterpret_cast<int32_t *>(base + kNoAllocWsFloats * 4 + kNoAllocQElems + (kNoAllocQElems / 32) * 4);
        sc.q_elems = kNoAllocQElems;
        const int chunk = rows_per_pass(M, m);
        for (int64_t c0 = 0; c0 < m; c0 += chunk) {
            const int mc = int(std::min<int64_t>(chunk, m - c0));
            gemv(M, m, PRO_X, EPI_STORE, d_x + c0 * M.cols, M.cols, mc, d_y + c0 * M.rows, M.rows, nullptr, 0.f, nullptr,
                 g.stream, nullptr, nullptr, &sc);
        }
        return 1;
    }, 0);
}

int voxhip_mat_gather(int mat, const int32_t *ids, int64_t n, float *out) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("gather");
        const GpuMat &M = mat_at(mat);
        if (n < 0 || (n > 0 && (!ids || !out))) throw Fail("mat_gather: missing argument");
        for (int64_t i = 0; i < n; ++i)  // check_id before any gather (backend_qwen3.cpp:305-306)
            if (ids[i] < 0 || ids[i] >= M.rows) throw Fail("mat_gather: row " + std::to_string(ids[i]) + " outside the matrix");
        const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(n, (int64_t(64) << 20) / (M.cols * 4)));
        const size_t ob = size_t(chunk) * size_t(M.cols) * 4, ib = size_t(chunk) * 4;
        float *pin = pinned(std::max(ob, ib) + 64);
        int32_t *dids = reinterpret_cast<int32_t *>(dev_scratch(g.dbuf_x, g.dbuf_x_bytes, ib));
        float *dout = dev_scratch(g.dbuf_y, g.dbuf_y_bytes, ob);
        for (int64_t c0 = 0; c0 < n; c0 += chunk) {
            const int64_t nc = std::min(chunk, n - c0);
            std::memcpy(pin, ids + c0, size_t(nc) * 4);
            HIPCHECK(copy_h2d(dids, pin, size_t(nc) * 4, g.stream));
            HIPCHECK(launch_mat_gather(M.w, M.s, gemv_type(M), M.s16 ? 1 : 0, M.cols, dids, nc, dout, g.stream));
            HIPCHECK(copy_d2h(pin, dout, size_t(nc) * size_t(M.cols) * 4, g.stream));
            HIPCHECK(hipStreamSynchronize(g.stream));
            std::memcpy(out + c0 * M.cols, pin, size_t(nc) * size_t(M.cols) * 4);
        }
        return 1;
    }, 0);
}

int voxhip_convt(int mat, int32_t K, int32_t stride, int32_t pad, int32_t out_pad, const float *bias, const float *x, int32_t T,
                 float *y) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("convt");
        const GpuMat &M = mat_at(mat);
        if (K < 1 || stride < 1 || pad < 0 || out_pad < 0 || T < 1 || !x || !y)
            throw Fail("convt: K, stride and T must be positive, pad and out_pad not negative, x and y given");
        if (M.rows % K) throw Fail("convt: the matrix rows are not K cout");
        if (M.b) throw Fail("convt: the matrix carries a bias; the transposed conv's bias is added after the overlap-add");
        const int64_t cout = M.rows / K, cin = M.cols, KO = M.rows;
        const int64_t To = int64_t(T - 1) * stride - 2 * int64_t(pad) + K + out_pad;
        if (To < 1) throw Fail("convt: no output frames");
        if (To * cout > (int64_t(1) << 31) || int64_t(T) * KO > (int64_t(1) << 31))
            throw Fail("convt: more than 2^31 output or product elements in one call");
        const size_t xb = size_t(T) * size_t(cin) * 4, bb = bias ? size_t(cout) * 4 : 0, zb = size_t(T) * size_t(KO) * 4;
        const size_t yb = size_t(To) * size_t(cout) * 4;
        float *pin = pinned(std::max(xb + bb, yb) + 64);
        float *dx = dev_scratch(g.dbuf_x, g.dbuf_x_bytes, xb + bb), *dz = dev_scratch(g.dbuf_z, g.dbuf_z_bytes, zb);
        float *dy = dev_scratch(g.dbuf_y, g.dbuf_y_bytes, yb);
        float *dbias = bias ? dx + size_t(T) * size_t(cin) : nullptr;
        std::memcpy(pin, x, xb);
        if (bias) std::memcpy(pin + size_t(T) * size_t(cin), bias, bb);
        HIPCHECK(copy_h2d(dx, pin, xb + bb, g.stream));
        // z = x W^T, frames in passes of the matrix's pass height, then the padded overlap-add + bias
        const int chunk = rows_per_pass(M, T);
        for (int64_t c0 = 0; c0 < T; c0 += chunk) {
            const int mc = int(std::min<int64_t>(chunk, T - c0));
            gemv(M, T, PRO_X, EPI_STORE, dx + c0 * cin, cin, mc, dz + c0 * KO, KO, nullptr, 0.f, nullptr, g.stream);
        }
        HIPCHECK(launch_convt_gather(dz, dbias, dy, T, int(To), stride, K, pad, int(cout), g.stream));
        HIPCHECK(copy_d2h(pin, dy, yb, g.stream));
        sync_status();
        std::memcpy(y, pin, yb);
        return 1;
    }, 0);
}

int voxhip_xfmr_create(const voxhip_xfmr_desc *w, const char *name, int n_layers, voxhip_uploaded_fn uploaded, void *user) {
    return guard_int([&] { return make_xfmr(w, name, n_layers, nullptr, uploaded, user); }, -1);
}

int voxhip_xfmr_create_from_mats(const voxhip_xfmr_desc *w, const int32_t *mats, const char *name) {
    return guard_int([&] {
        if (!mats) throw Fail("no matrix handles");
        return make_xfmr(w, name, -1, mats, nullptr, nullptr);
    }, -1);
}

int voxhip_seq_create(int xfmr, int64_t capacity) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        if (capacity <= 0 || capacity > kMaxCap) throw Fail("sequence capacity out of range");
        for (size_t i = 0; i < g.seqs.size(); ++i) {
            Seq &S = g.seqs[i];
            if (S.k && !S.used && S.layers == X.layers && S.kvh == X.kvh && S.hd == X.hd && S.cap >= capacity) {
                S.used = true;
                S.xfmr = xfmr;
                ensure_rope(X, S.cap);
                return int(i);
            }
        }
        Seq S;
        S.xfmr = xfmr; S.cap = capacity; S.layers = X.layers; S.kvh = X.kvh; S.hd = X.hd;
        const size_t n = size_t(X.layers) * size_t(X.kvh) * size_t(capacity) * size_t(X.hd);
        S.k = dalloc_t<_Float16>(n);
        try {
            S.v = dalloc_t<_Float16>(n);
        } catch (...) {
            dfree(S.k);
            throw;
        }
        HIPCHECK(hipMemset(S.k, 0, n * 2));
        HIPCHECK(hipMemset(S.v, 0, n * 2));
        S.used = true;
        ensure_rope(X, capacity);
        g.seqs.push_back(S);
        return int(g.seqs.size()) - 1;
    }, -1);
}

void voxhip_seq_free(int seq) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (seq >= 0 && size_t(seq) < g.seqs.size()) g.seqs[size_t(seq)].used = false;  // buffers stay pooled
}

int voxhip_xfmr_forward(int xfmr, int seq, int64_t pos0, const float *x, int64_t m, float *out_last, int in_proj, int head,
                        float *head_out) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        if (m <= 0) return 1;
        if (pos0 < 0 || pos0 + m > S.cap) throw Fail("context exceeds GPU KV capacity");
        forward_rows(X, m, [&](int64_t i) { return row_of(S, pos0 + i); }, x, in_proj, 0, X.layers, m, nullptr, out_last, head,
                     head_out, false);
        return 1;
    }, 0);
}

int voxhip_xfmr_forward_hidden(int xfmr, int seq, int64_t pos0, const float *x, int64_t m, float *hidden_out) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        if (m <= 0) return 1;
        if (pos0 < 0 || pos0 + m > S.cap) throw Fail("context exceeds GPU KV capacity");
        forward_rows(X, m, [&](int64_t i) { return row_of(S, pos0 + i); }, x, -1, 0, X.layers, m, hidden_out, nullptr, -1,
                     nullptr, false);
        return 1;
    }, 0);
}

int voxhip_xfmr_forward_layers(int xfmr, int seq, int64_t pos0, const float *x, int64_t m, int32_t first, int32_t count,
                               float *hidden_out) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        if (m <= 0 || count == 0) return 1;
        if (first < 0 || count < 0 || first + count > X.layers) throw Fail("layer range outside the transformer");
        if (pos0 < 0 || pos0 + m > S.cap) throw Fail("context exceeds GPU KV capacity");
        forward_rows(X, m, [&](int64_t i) { return row_of(S, pos0 + i); }, x, -1, first, count, m, hidden_out, nullptr, -1,
                     nullptr, false);
        return 1;
    }, 0);
}

int voxhip_xfmr_forward_pair(int xfmr, int seq0, int seq1, int64_t pos, const float *x2, int head, float *out2,
                             float *head_out2) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        if (seq0 == seq1) throw Fail("pair needs two sequences");
        Seq &S0 = seq_at(seq0), &S1 = seq_at(seq1);
        check_seq_for(X, xfmr, S0);
        check_seq_for(X, xfmr, S1);
        if (pos < 0 || pos + 1 > S0.cap || pos + 1 > S1.cap) throw Fail("context exceeds GPU KV capacity");
        forward_rows(X, 2, [&](int64_t i) { return row_of(i == 0 ? S0 : S1, pos); }, x2, -1, 0, X.layers, 2, nullptr, out2, head,
                     head_out2, true);
        return 1;
    }, 0);
}

int voxhip_xfmr_forward_steps(int xfmr, const int32_t *seqs, const int64_t *pos, int64_t B, const float *x, float *out, int head,
                              float *head_out) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        if (B <= 0) return 1;
        if (B > kMaxM) throw Fail("at most 8 sequences per step");
        for (int64_t b = 0; b < B; ++b) {
            Seq &S = seq_at(seqs[b]);
            check_seq_for(X, xfmr, S);
            if (pos[b] < 0 || pos[b] + 1 > S.cap) throw Fail("context exceeds GPU KV capacity");
            for (int64_t c = 0; c < b; ++c)
                if (seqs[c] == seqs[b]) throw Fail("a sequence appears twice in one step");
        }
        forward_rows(X, B, [&](int64_t i) { return row_of(g.seqs[size_t(seqs[i])], pos[i]); }, x, -1, 0, X.layers, B, nullptr, out,
                     head, head_out, true);
        return 1;
    }, 0);
}

int voxhip_sample_logits(const float *logits, int32_t n, const voxhip_sample_cfg *cfg, const int32_t *history, int32_t n_history,
                         int32_t *out_id) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("sample");
        if (!cfg || !out_id || !logits) throw Fail("missing argument");
        if (n <= 0 || n > kSampleMaxN) throw Fail("sampler supports 1..16384 logits");
        if (!g.scfg_dev) {
            g.scfg_dev = dalloc_t<SampleCfgDev>(1);
            HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&g.scfg_host), sizeof(SampleCfgDev), hipHostMallocDefault));
            g.tok_dev = dalloc_t<int32_t>(1);
        }
        if (n_history > 0 && size_t(n_history) > g.hist_cap) {
            dfree(g.hist_dev);
            g.hist_dev = dalloc_t<int32_t>(size_t(n_history));
            g.hist_cap = size_t(n_history);
        }
        HIPCHECK(hipStreamSynchronize(g.stream));
        if (n_history > 0 && history) h2d(g.hist_dev, history, size_t(n_history) * 4);
        fill_sample_cfg(*g.scfg_host, *cfg, n_history > 0 && history ? g.hist_dev : nullptr, history ? n_history : 0);
        HIPCHECK(copy_h2d(g.scfg_dev, g.scfg_host, sizeof(SampleCfgDev), g.stream));
        float *dl = dev_scratch(g.dbuf_x, g.dbuf_x_bytes, size_t(n) * 4);
        float *pin = pinned(size_t(n) * 4 + 64);
        std::memcpy(pin, logits, size_t(n) * 4);
        HIPCHECK(copy_h2d(dl, pin, size_t(n) * 4, g.stream));
        HIPCHECK(launch_sample(g.scfg_dev, dl, n, g.tok_dev, g.stream));
        int32_t tok = -1;
        HIPCHECK(copy_d2h(pin, g.tok_dev, 4, g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
        std::memcpy(&tok, pin, 4);
        if (tok < 0) throw Fail("device sampler rejected the request");
        *out_id = tok;
        return 1;
    }, 0);
}

// ---------------------------------------------------------------- device-resident path
void *voxhip_dev_alloc(size_t bytes) {
    std::lock_guard<std::mutex> lk(g.mu);
    try {
        require_ok();
        return dalloc(bytes);
    } catch (const std::exception &e) {
        set_error(e.what());
        return nullptr;
    }
}
void voxhip_dev_free(void *p) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.ok) { (void)hipStreamSynchronize(g.stream); dfree(p); }
}
int voxhip_memcpy_h2d(void *d_dst, const void *src, size_t bytes) {
    return guard_int([&] {
        require_ok();
        HIPCHECK(hipStreamSynchronize(g.stream));
        HIPCHECK(copy_h2d(d_dst, src, bytes, nullptr));
        return 1;
    }, 0);
}
int voxhip_memcpy_d2h(void *dst, const void *d_src, size_t bytes) {
    return guard_int([&] {
        require_ok();
        HIPCHECK(hipStreamSynchronize(g.stream));
        HIPCHECK(copy_d2h(dst, d_src, bytes, nullptr));
        return 1;
    }, 0);
}
int voxhip_sync(void) {
    return guard_int([&] {
        require_ok();
        sync_status();
        return 1;
    }, 0);
}

}  // extern "C"

namespace {
// Enqueues one device-resident decode step on stream s (no host copies). steps = false: m rows of one sequence at
// pos0 + i; one row takes the fused attention, several rows of the same sequence append their keys first
// (k_qk_post), and the head and sampler run on the last row. steps = true: one row for each of m sequences (fused
// attention), head and sampler on every row.
int enqueue_decode(Xfmr &X, int m, int head, const float *d_x, float *d_out_last, float *d_logits, bool sample, int32_t *d_token,
                   hipStream_t s, Probe *pr = nullptr, bool steps = false) {
    const bool fused = steps || m == 1;
    const int r0 = steps ? 0 : m - 1, mr = steps ? m : 1;
    int kernels = 0;
    enqueue_layers(X, m, m, 0, X.layers, s, fused, pr, d_x);
    kernels += kernels_per_layer(X, m, fused) * X.layers + (ffn_pass(X, m, m, fused) ? 1 : 0);
    probed(head >= 0 ? pr : nullptr, VOXHIP_K_HEAD, [&] { enqueue_final(X, r0, mr, head, s); });
    kernels += 1;
    if (d_out_last) HIPCHECK(hipMemcpyAsync(d_out_last, X.xnorm, size_t(mr) * X.H * 4, hipMemcpyDeviceToDevice, s));
    if (head >= 0) {
        const GpuMat &Hm = g.mats[size_t(head)];
        if (d_logits) HIPCHECK(hipMemcpyAsync(d_logits, X.logits, size_t(mr) * size_t(Hm.rows) * 4, hipMemcpyDeviceToDevice, s));
        if (sample) {
            probed(pr, VOXHIP_K_SAMPLE, [&] {
                HIPCHECK(launch_sample(X.scfg_dev, X.logits, int(Hm.rows), d_token ? d_token : X.token_dev, s, mr));
            });
            kernels += 1;
        }
    }
    return kernels;
}

hipGraphExec_t decode_graph(Xfmr &X, const std::array<int, 8> &seqs, int m, bool steps, int head, const float *d_x,
                            float *d_out_last, float *d_logits, bool sample, int32_t *d_token) {
    GraphKey key{seqs, m, head, sample ? 1 : 0, steps ? 1 : 0, long_row(X, m) ? 1 : 0, d_x, d_out_last, d_logits, d_token};
    auto it = X.graphs.find(key);
    if (it != X.graphs.end()) return it->second;
    hipGraph_t graph = nullptr;
    HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
    try {
        enqueue_decode(X, m, head, d_x, d_out_last, d_logits, sample, d_token, g.stream, nullptr, steps);
    } catch (...) {
        (void)hipStreamEndCapture(g.stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    HIPCHECK(hipStreamEndCapture(g.stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HIPCHECK(e);
    X.graphs[key] = exec;
    return exec;
}
std::array<int, 8> one_seq(int seq) {
    std::array<int, 8> a;
    a.fill(-1);
    a[0] = seq;
    return a;
}

void prepare_head(Xfmr &X, int head, bool sample) {
    if (sample && head < 0) throw Fail("sampling needs a head");
    if (head >= 0) {
        const GpuMat &Hm = mat_at(head);
        if (Hm.cols != X.H) throw Fail("head width differs from the hidden size");
        if (sample && Hm.rows > kSampleMaxN) throw Fail("sampler supports up to 16384 logits");
        ensure_logits(X, int64_t(kMaxM) * Hm.rows);  // no reallocation inside a captured step
    }
}
// Uploads the sampler configurations of rows 0..n-1 when they changed.
void set_sample_cfgs(Xfmr &X, const voxhip_sample_cfg *cfgs, int n) {
    std::vector<SampleCfgDev> d(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) {
        std::memset(&d[size_t(i)], 0, sizeof(SampleCfgDev));
        fill_sample_cfg(d[size_t(i)], cfgs[i], nullptr, 0);
    }
    if (std::memcmp(d.data(), X.scfg_host, size_t(n) * sizeof(SampleCfgDev)) != 0) {
        HIPCHECK(hipStreamSynchronize(g.stream));
        std::memcpy(X.scfg_host, d.data(), size_t(n) * sizeof(SampleCfgDev));
        HIPCHECK(copy_h2d(X.scfg_dev, X.scfg_host, size_t(n) * sizeof(SampleCfgDev), g.stream));
    }
}

void prepare_decode(Xfmr &X, Seq &S, int64_t pos0, int64_t m, int head, const voxhip_sample_cfg *cfg) {
    if (m <= 0 || m > kMaxM) throw Fail("decode_dev takes 1..8 rows");
    if (pos0 < 0 || pos0 + m > S.cap) throw Fail("context exceeds GPU KV capacity");
    prepare_head(X, head, cfg != nullptr);
    std::vector<RowRef> rr(static_cast<size_t>(m));
    for (int64_t i = 0; i < m; ++i) rr[size_t(i)] = row_of(S, pos0 + i);
    set_rows(X, rr);
    if (cfg) set_sample_cfgs(X, cfg, 1);
}

uint64_t gemv_stream_bytes(const Xfmr &X) {
    uint64_t b = 0;
    for (const LayerDev &L : X.L)
        for (int id : {L.qkv, L.o, L.gu, L.down}) b += g.mats[size_t(id)].bytes;
    return b;
}
}  // namespace

extern "C" {

int voxhip_decode_dev(int xfmr, int seq, int64_t pos0, const float *d_x, int64_t m, float *d_out_last, int head, float *d_logits,
                      const voxhip_sample_cfg *cfg, int32_t *d_token) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        prepare_decode(X, S, pos0, m, head, cfg);
        vh::prof_stage(X.name.c_str());
        if (vh::prof_on()) {  // stamped launches are not captured
            enqueue_decode(X, int(m), head, d_x, d_out_last, d_logits, cfg != nullptr, d_token, g.stream);
            return 1;
        }
        hipGraphExec_t exec = decode_graph(X, one_seq(seq), int(m), false, head, d_x, d_out_last, d_logits, cfg != nullptr, d_token);
        HIPCHECK(hipGraphLaunch(exec, g.stream));
        return 1;
    }, 0);
}

int voxhip_decode_steps_dev(int xfmr, const int32_t *seqs, const int64_t *pos, int64_t B, const float *d_x, float *d_out,
                            int head, float *d_logits, const voxhip_sample_cfg *cfgs, int32_t *d_tokens) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        if (!seqs || !pos || !d_x) throw Fail("missing argument");
        if (B <= 0 || B > kMaxM) throw Fail("decode_steps_dev takes 1..8 sequences");
        std::array<int, 8> key;
        key.fill(-1);
        std::vector<RowRef> rr(static_cast<size_t>(B));
        for (int64_t b = 0; b < B; ++b) {
            Seq &S = seq_at(seqs[b]);
            check_seq_for(X, xfmr, S);
            if (pos[b] < 0 || pos[b] + 1 > S.cap) throw Fail("context exceeds GPU KV capacity");
            for (int64_t c = 0; c < b; ++c)
                if (seqs[c] == seqs[b]) throw Fail("a sequence appears twice in one step");
            rr[size_t(b)] = row_of(S, pos[b]);
            key[size_t(b)] = seqs[b];
        }
        prepare_head(X, head, cfgs != nullptr);
        set_rows(X, rr);
        if (cfgs) set_sample_cfgs(X, cfgs, int(B));
        vh::prof_stage(X.name.c_str());
        if (vh::prof_on()) {  // stamped launches are not captured
            enqueue_decode(X, int(B), head, d_x, d_out, d_logits, cfgs != nullptr, d_tokens, g.stream, nullptr, true);
            return 1;
        }
        hipGraphExec_t exec = decode_graph(X, key, int(B), true, head, d_x, d_out, d_logits, cfgs != nullptr, d_tokens);
        HIPCHECK(hipGraphLaunch(exec, g.stream));
        return 1;
    }, 0);
}

}  // extern "C"

namespace {
constexpr int kLmGraphSteps = 8;  // generation steps per captured graph (the host checks for the end between graphs)

LmCfgDev lm_cfg_dev(const voxhip_lm_cfg &c, int32_t max_len) {
    LmCfgDev d{};
    d.top_p = c.top_p; d.tau_r = c.tau_r; d.top_k = c.top_k; d.win_size = c.win_size;
    d.speech_tokens = c.speech_tokens; d.min_len = c.min_len; d.max_len = max_len;
    d.key0 = uint32_t(c.seed); d.key1 = uint32_t(c.seed >> 32);  // DetRng(seed) (sampling.hpp:37)
    d.stream = 0x43560000u + c.piece;                             // "CV" + piece (cosyvoice.cpp:672)
    d.max_trials = 101;                                            // fail after trial 101 (cosyvoice.cpp:681)
    return d;
}
void check_lm_cfg(const voxhip_lm_cfg &c, int64_t n) {
    if (n < 2 || n > kLmMaxN) throw Fail("LM sampler supports 2..8192 logits");
    if (c.top_k < 1 || c.top_k > kLmMaxK) throw Fail("LM top_k must be 1..1024");
    if (!(c.top_p > 0.f)) throw Fail("LM top_p must be positive");
    if (c.win_size < 0 || c.win_size > kLmMaxK) throw Fail("LM win_size must be 0..1024");
    if (c.speech_tokens < 1 || c.speech_tokens > n) throw Fail("LM speech_tokens out of range");
    if (c.min_len < 0 || c.max_len < 0) throw Fail("LM min_len / max_len must not be negative");
}
// Pinned host block of the LM staging: [LmCfgDev][LmState x 3]
LmCfgDev *lm_host_cfg() { return reinterpret_cast<LmCfgDev *>(g.lm_host); }
LmState *lm_host_state(int i) { return reinterpret_cast<LmState *>(g.lm_host + 256) + i; }
void ensure_lm_staging() {
    if (g.lm_host) return;
    g.lm_cfg_dev = dalloc_t<LmCfgDev>(1);
    g.lm_state_dev = dalloc_t<LmState>(1);
    HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&g.lm_host), 256 + 3 * sizeof(LmState), hipHostMallocDefault));
}

void lm_buffers(Xfmr &X, int64_t max_len, int64_t V, bool want_logp) {
    bool changed = false;
    if (!X.lm_cfg) {
        X.lm_cfg = dalloc_t<LmCfgDev>(1);
        X.lm_state = dalloc_t<LmState>(1);
        changed = true;
    }
    if (X.lm_dec_cap < max_len) {
        HIPCHECK(hipStreamSynchronize(g.stream));
        dfree(X.lm_dec);
        X.lm_dec = dalloc_t<int32_t>(size_t(max_len));
        X.lm_dec_cap = max_len;
        changed = true;
    }
    if (want_logp && X.lm_logp_cap < max_len * V) {
        HIPCHECK(hipStreamSynchronize(g.stream));
        dfree(X.lm_logp);
        X.lm_logp = dalloc_t<float>(size_t(max_len * V));
        X.lm_logp_cap = max_len * V;
        changed = true;
    }
    if (changed) drop_graphs(X);
}

// kLmGraphSteps generation steps: final norm + head (+ bias) of row 0 -> sampler -> embedding of the pick and the
// row advanced -> the layers (one fused row). The device state ends the loop; steps after the end write only the
// sequence's spare slot.
void enqueue_lm_steps(Xfmr &X, const Seq &S, int head, int emb, bool want_logp, hipStream_t s) {
    const GpuMat &Hm = mat_at(head), &E = mat_at(emb);
    LmEmbedArgs ea{};
    ea.w = E.w; ea.scale = E.s; ea.type = E.type; ea.s16 = E.s16 ? 1 : 0; ea.rows = E.rows; ea.cols = E.cols;
    ea.st = X.lm_state; ea.decoded = X.lm_dec; ea.x = X.h; ea.row = X.rows_dev; ea.rope_row = X.rope_rows_dev;
    ea.rope = X.rope; ea.hd = X.hd; ea.spare_pos = S.cap - 1;
    for (int i = 0; i < kLmGraphSteps; ++i) {
        enqueue_final(X, 0, 1, head, s);
        HIPCHECK(launch_lm_sample(X.logits, int(Hm.rows), X.lm_cfg, X.lm_state, X.lm_dec, want_logp ? X.lm_logp : nullptr,
                                  Hm.rows, true, s));
        HIPCHECK(launch_lm_embed(ea, s));
        enqueue_layers(X, 1, 1, 0, X.layers, s, true);
    }
}
hipGraphExec_t lm_graph(Xfmr &X, const Seq &S, int seq, int head, int emb, bool want_logp) {
    const std::array<int64_t, 4> key{seq, head, emb, want_logp ? 1 : 0};
    auto it = X.lm_graphs.find(key);
    if (it != X.lm_graphs.end()) return it->second;
    hipGraph_t graph = nullptr;
    HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
    try {
        enqueue_lm_steps(X, S, head, emb, want_logp, g.stream);
    } catch (...) {
        (void)hipStreamEndCapture(g.stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    HIPCHECK(hipStreamEndCapture(g.stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HIPCHECK(e);
    X.lm_graphs[key] = exec;
    return exec;
}

// ------------------------------------------------------------------ code-predictor frame loop (gpu_pred_frame)
constexpr int kPredMaxGroups = 64;  // the reference's bound (gpu_vulkan.cpp:977)

void pred_buffers(Xfmr &X) {
    if (X.pred_codes) return;
    X.pred_codes = dalloc_t<int32_t>(kPredMaxGroups);
    X.pred_err = dalloc_t<int32_t>(1);
    X.pred_cfg = dalloc_t<SampleCfgDev>(kPredMaxGroups);
    HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&X.pred_host), (kPredMaxGroups + 1) * sizeof(int32_t), hipHostMallocDefault));
    HIPCHECK(hipHostMalloc(reinterpret_cast<void **>(&X.pred_cfg_host), kPredMaxGroups * sizeof(SampleCfgDev), hipHostMallocDefault));
}

// The whole frame (gpu_vulkan.cpp:1004-1036) as one graph. Pass cb (1 .. G-1) takes m rows (2 for the first: the
// talker's hidden state and the first code's embedding, staged by the host; 1 after: the embedding of the code the
// previous pass sampled, gathered on the device) at positions pos .. pos + m - 1 of the sequence, then in_proj (or
// the rows as they are), the layers, the final norm and head cb - 1 on the last row, and the sampler with draw
// (frame, cb) into codes[cb]. The first pass's two rows run the unfused layer path (q/k post-processing and the
// K/V append before attention), so row 1 sees row 0.
void enqueue_pred(Xfmr &X, const Seq &S, int in_proj, const int *heads, const int *embs, int G, hipStream_t s) {
    const int64_t din = in_proj >= 0 ? mat_at(in_proj).cols : X.H;
    int64_t pos = 0;
    for (int cb = 1; cb < G; ++cb) {
        const int m = cb == 1 ? 2 : 1;
        PredEmbedArgs pa{};
        pa.codes = X.pred_codes; pa.code_idx = cb - 1; pa.err = X.pred_err;
        pa.x = in_proj >= 0 ? X.xin : X.h;
        pa.row = X.rows_dev; pa.rope_row = X.rope_rows_dev; pa.rope = X.rope; pa.hd = X.hd; pa.m = m;
        pa.base = row_of(S, pos);
        if (cb >= 2) {
            const GpuMat &E = mat_at(embs[cb - 2]);
            pa.w = E.w; pa.scale = E.s; pa.type = E.type; pa.s16 = E.s16 ? 1 : 0; pa.rows = E.rows; pa.cols = E.cols;
        }
        HIPCHECK(launch_pred_embed(pa, s));
        if (in_proj >= 0) gemv(mat_at(in_proj), m, PRO_X, EPI_STORE, X.xin, din, m, X.h, X.H, nullptr, 0.f, nullptr, s);
        enqueue_layers(X, m, m, 0, X.layers, s, m == 1);
        const GpuMat &Hm = mat_at(heads[cb - 1]);
        enqueue_final(X, m - 1, 1, heads[cb - 1], s);
        HIPCHECK(launch_sample(X.pred_cfg + cb, X.logits, int(Hm.rows), X.pred_codes + cb, s));
        pos += m;
    }
}
hipGraphExec_t pred_graph(Xfmr &X, const Seq &S, int seq, int in_proj, const int *heads, const int *embs, int G) {
    std::vector<int> key{seq, in_proj, G};
    key.insert(key.end(), heads, heads + (G - 1));
    key.insert(key.end(), embs, embs + (G - 2));
    auto it = X.pred_graphs.find(key);
    if (it != X.pred_graphs.end()) return it->second;
    hipGraph_t graph = nullptr;
    HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
    try {
        enqueue_pred(X, S, in_proj, heads, embs, G, g.stream);
    } catch (...) {
        (void)hipStreamEndCapture(g.stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    HIPCHECK(hipStreamEndCapture(g.stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HIPCHECK(e);
    X.pred_graphs[key] = exec;
    return exec;
}
}  // namespace

extern "C" {

int voxhip_lm_sample_dev(const float *d_logits, int32_t n, const voxhip_lm_cfg *cfg, int64_t step, const int32_t *d_decoded,
                         int32_t n_decoded, float *d_logp, int32_t *token) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("lm.sample");
        if (!d_logits || !cfg || !token || step < 0 || n_decoded < 0 || (n_decoded > 0 && !d_decoded)) throw Fail("missing argument");
        check_lm_cfg(*cfg, n);
        ensure_lm_staging();
        HIPCHECK(hipStreamSynchronize(g.stream));  // the pinned block may feed an earlier copy
        *lm_host_cfg() = lm_cfg_dev(*cfg, INT32_MAX);
        LmState st{};
        st.step = int32_t(step); st.n_dec = n_decoded; st.last = -1;
        *lm_host_state(0) = st;
        HIPCHECK(copy_h2d(g.lm_cfg_dev, lm_host_cfg(), sizeof(LmCfgDev), g.stream));
        HIPCHECK(copy_h2d(g.lm_state_dev, lm_host_state(0), sizeof(LmState), g.stream));
        HIPCHECK(launch_lm_sample(d_logits, n, g.lm_cfg_dev, g.lm_state_dev, const_cast<int32_t *>(d_decoded), d_logp, 0, false,
                                  g.stream));
        HIPCHECK(copy_d2h(lm_host_state(1), g.lm_state_dev, sizeof(LmState), g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
        const LmState r = *lm_host_state(1);
        if (r.status) throw Fail("CosyVoice: sampling reaches max_trials and still gets eos when ignore_eos is True");
        *token = r.last;
        return 1;
    }, 0);
}

int voxhip_lm_generate(int xfmr, int seq, const float *x, int64_t n, int head, int speech_emb, const voxhip_lm_cfg *cfg,
                       int32_t *tokens, float *logp, int32_t *n_tokens) {
    return guard_int([&] {
        require_ok();
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        if (!x || !cfg || !n_tokens || n <= 0 || (cfg->max_len > 0 && !tokens)) throw Fail("missing argument");
        const GpuMat &Hm = mat_at(head), &E = mat_at(speech_emb);
        if (Hm.cols != X.H || E.cols != X.H) throw Fail("head / embedding width differs from the hidden size");
        const int64_t V = Hm.rows;
        check_lm_cfg(*cfg, V);
        if (cfg->speech_tokens > E.rows) throw Fail("speech embedding has fewer rows than speech tokens");
        if (n + int64_t(cfg->max_len) + 1 > S.cap) throw Fail("context exceeds GPU KV capacity (prompt + max_len + 1 positions)");
        *n_tokens = 0;
        // lm_begin: the prompt rows at positions 0..n-1
        const int last = forward_rows(X, n, [&](int64_t i) { return row_of(S, i); }, x, -1, 0, X.layers, n, nullptr, nullptr,
                                      -1, nullptr, false);
        if (cfg->max_len == 0) return 1;
        if (last) HIPCHECK(hipMemcpyAsync(X.h, X.h + size_t(last) * X.H, size_t(X.H) * 4, hipMemcpyDeviceToDevice, g.stream));
        prepare_head(X, head, false);
        lm_buffers(X, cfg->max_len, V, logp != nullptr);
        ensure_lm_staging();
        HIPCHECK(hipStreamSynchronize(g.stream));
        *lm_host_cfg() = lm_cfg_dev(*cfg, cfg->max_len);
        LmState st{};
        st.last = -1;
        *lm_host_state(0) = st;
        HIPCHECK(copy_h2d(X.lm_cfg, lm_host_cfg(), sizeof(LmCfgDev), g.stream));
        HIPCHECK(copy_h2d(X.lm_state, lm_host_state(0), sizeof(LmState), g.stream));
        set_rows(X, {row_of(S, n - 1)});  // the first step's embedding kernel advances it to position n
        // VOX_PROFILE=gpu: the same steps launched one by one (stamped launches are not captured)
        hipGraphExec_t exec = vh::prof_on() ? nullptr : lm_graph(X, S, seq, head, speech_emb, logp != nullptr);
        auto cleanup = [&] { X.rows_valid = false; };  // the device advanced the row table
        try {
            // One graph ahead: while graph c runs, the host reads the state copied after graph c - 1. The copy's
            // arrival is seen in the pinned slot itself (pad0: -1 set by the host, 0 in the device state), so no
            // events are recorded between graph launches.
            const int chunks = (cfg->max_len + kLmGraphSteps - 1) / kLmGraphSteps;
            for (int c = 0; c < chunks; ++c) {
                LmState *slot = lm_host_state(1 + (c & 1));
                __atomic_store_n(&slot->pad0, -1, __ATOMIC_RELEASE);
                if (exec) HIPCHECK(hipGraphLaunch(exec, g.stream));
                else enqueue_lm_steps(X, S, head, speech_emb, logp != nullptr, g.stream);
                HIPCHECK(copy_d2h(slot, X.lm_state, sizeof(LmState), g.stream));
                if (c >= 1) {
                    LmState *prev = lm_host_state(1 + ((c - 1) & 1));
                    while (__atomic_load_n(&prev->pad0, __ATOMIC_ACQUIRE) == -1) {
                        const hipError_t q = hipStreamQuery(g.stream);
                        if (q == hipSuccess) break;
                        if (q != hipErrorNotReady) HIPCHECK(q);
                        std::this_thread::yield();
                    }
                    if (__atomic_load_n(&prev->done, __ATOMIC_ACQUIRE)) break;
                }
            }
            HIPCHECK(copy_d2h(lm_host_state(0), X.lm_state, sizeof(LmState), g.stream));
            sync_status();
            const LmState r = *lm_host_state(0);
            if (r.status) throw Fail("CosyVoice: sampling reaches max_trials and still gets eos when ignore_eos is True");
            // the counts come from device memory and size the copies into the caller's buffers (max_len entries,
            // max_len x V log-probs): a count outside them is an error, never a copy
            if (r.n_dec < 0 || r.n_dec > cfg->max_len) throw Fail("LM state reports " + std::to_string(r.n_dec) + " tokens of " +
                                                                  std::to_string(cfg->max_len));
            if (r.n_dec > 0) HIPCHECK(copy_d2h(tokens, X.lm_dec, size_t(r.n_dec) * 4, nullptr));
            const int64_t rows = std::min<int64_t>(r.n_dec + (r.last >= cfg->speech_tokens ? 1 : 0), cfg->max_len);
            if (logp && rows > 0) HIPCHECK(copy_d2h(logp, X.lm_logp, size_t(rows * V) * 4, nullptr));
            *n_tokens = r.n_dec;
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();
        return 1;
    }, 0);
}

}  // extern "C"

extern "C" {

int voxhip_pred_frame(int xfmr, int seq, const float *in2, int in_proj, const int *heads, int n_heads, const int *embs,
                      int n_embs, const voxhip_sample_cfg *cfg, int32_t *codes) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("predictor");
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        const int G = n_heads + 1;
        if (!in2 || !heads || !cfg || !codes || n_heads < 1) throw Fail("missing argument");
        if (G > kPredMaxGroups) throw Fail("code predictor supports up to 64 codebooks");
        if (n_embs < G - 2 || (G > 2 && !embs)) throw Fail("code predictor needs an embedding per codebook after the first");
        if (G + 1 > S.cap) throw Fail("context exceeds GPU KV capacity");
        const int64_t din = in_proj >= 0 ? mat_at(in_proj).cols : X.H;
        if (in_proj >= 0 && mat_at(in_proj).rows != X.H) throw Fail("in_proj output differs from the hidden size");
        for (int i = 0; i < G - 1; ++i) {
            const GpuMat &Hm = mat_at(heads[i]);
            if (Hm.cols != X.H) throw Fail("head width differs from the hidden size");
            if (Hm.rows > kSampleMaxN) throw Fail("sampler supports up to 16384 logits");
        }
        for (int i = 0; i < G - 2; ++i)
            if (mat_at(embs[i]).cols != din) throw Fail("embedding width differs from the predictor input");
        ensure_rows(X, 2);
        for (int i = 0; i < G - 1; ++i) prepare_head(X, heads[i], true);
        if (in_proj >= 0) ensure_xin(X, 2 * din);
        pred_buffers(X);
        HIPCHECK(hipStreamSynchronize(g.stream));  // the pinned blocks may feed an earlier copy
        for (int cb = 0; cb < G; ++cb) {
            voxhip_sample_cfg c = *cfg;
            c.codebook = uint32_t(cb); c.draw = 0;
            std::memset(&X.pred_cfg_host[cb], 0, sizeof(SampleCfgDev));
            fill_sample_cfg(X.pred_cfg_host[cb], c, nullptr, 0);
        }
        HIPCHECK(copy_h2d(X.pred_cfg, X.pred_cfg_host, size_t(G) * sizeof(SampleCfgDev), g.stream));
        HIPCHECK(copy_h2d(in_proj >= 0 ? X.xin : X.h, in2, size_t(2 * din) * 4, g.stream));
        HIPCHECK(hipMemsetAsync(X.pred_err, 0, sizeof(int32_t), g.stream));
        // the layer enqueue takes the first row's cache view from the host row table: this sequence's
        set_rows(X, {row_of(S, 0), row_of(S, 1)});
        X.rows_valid = false;  // the frame rewrites the row table
        if (vh::prof_on()) enqueue_pred(X, S, in_proj, heads, embs, G, g.stream);  // stamped launches, not captured
        else HIPCHECK(hipGraphLaunch(pred_graph(X, S, seq, in_proj, heads, embs, G), g.stream));
        HIPCHECK(copy_d2h(X.pred_host, X.pred_codes, size_t(G) * 4, g.stream));
        HIPCHECK(copy_d2h(X.pred_host + kPredMaxGroups, X.pred_err, 4, g.stream));
        sync_status();
        if (X.pred_host[kPredMaxGroups]) throw Fail("code out of the embedding's range");
        for (int cb = 1; cb < G; ++cb) codes[cb] = X.pred_host[cb];
        return 1;
    }, 0);
}

}  // extern "C"

namespace {
// ------------------------------------------------------------------ F5-TTS DiT step (gpu.hpp:62-91)
struct F5Block {
    int ada = -1, qkv = -1, o = -1, ff1 = -1, ff2 = -1;  // q | k | v stacked at create
};
struct F5Conv {
    float *w = nullptr, *b = nullptr;  // w [groups][cout/groups][kpad] (K * cin/groups, zero-padded to a multiple of 8)
    int cin = 0, cout = 0, K = 0, groups = 0, kpad = 0;
    bool wide = false;  // max |w| >= 63 or NaN: the conv GEMM on f32 matrix cores (GemmArgs::f32_wide)
};
struct F5VBlock {  // a Vocos ConvNeXt block (f5.cpp:235-240)
    F5Conv dw;     // depthwise, w [C][K]
    float *ln_w = nullptr, *ln_b = nullptr, *gamma = nullptr;
    int pw1 = -1, pw2 = -1;
};
struct F5 {
    // hd: the model's head_dim (the RoPE table, the softmax scale); hp: the attention layout's (kF5HeadDim, heads of
    // hd < hp padded with zero dims, stack_rows_heads)
    int dim = 0, depth = 0, heads = 0, hd = 0, hp = 0, ff = 0, mel = 0, text = 0, pe = 0;
    int in_proj = -1, norm_out = -1, proj_out = -1;
    // every block's ada matrix and norm_out stacked at create, when they share a type: one GEMV writes all the
    // step's modulation vectors (they depend only on the time embedding) instead of depth + 1 launches; -1: none
    int ada_all = -1;
    std::vector<F5Block> blocks;
    F5Conv pos1, pos2;
    // every block linear F16 and dim, inner, ff multiples of 64: the block's activations travel between kernels as
    // f16 halves (hi, lo planes) and the linears take k_gemm_hh; otherwise f32 rows and k_gemm_h16 / k_gemm_f32
    bool split = false;
    // Vocos (vdim 0: none): embed conv, norms, blocks, head; buffers of the last vocode length vT
    int vdim = 0, vinter = 0, vout = 0, v_head = -1;
    F5Conv v_embed;
    float *v_ln_w = nullptr, *v_ln_b = nullptr, *v_fln_w = nullptr, *v_fln_b = nullptr;
    std::vector<F5VBlock> vblocks;
    int vT = 0;
    float *vm = nullptr, *vx = nullptr, *vy = nullptr, *vh = nullptr, *vhead = nullptr;
    // step buffers of begin(B, N): rows R = B N
    int B = 0, N = 0;
    float *cat = nullptr, *h = nullptr, *a = nullptr, *nrm = nullptr, *at = nullptr, *ffb = nullptr;
    float *ada = nullptr, *fin = nullptr, *ts = nullptr, *x = nullptr, *out = nullptr, *rope = nullptr;
    // q | k rows and v^T ([B heads hd][ldvt], key columns padded with zeros to ldvt) as f16 hi, then lo, planes
    _Float16 *qkv16 = nullptr;
    int64_t lo_off = 0;
    int ldvt = 0;
    // split: the modulated rows, the attention output and the GELU output as hi / lo planes ([R][width] each)
    _Float16 *nrm16 = nullptr, *at16 = nullptr, *ffb16 = nullptr;
};

F5 &f5_at(int id) {
    if (id < 0 || size_t(id) >= g.f5.size() || !g.f5[size_t(id)]) throw Fail("bad F5 handle " + std::to_string(id));
    return *g.f5[size_t(id)];
}

// Stacks matrices of one type and width by rows into a new device matrix (biases zero where a part has none).
// A matrix made by a helper below, freed again when a later step of the helper throws.
struct NewMatGuard {
    int id;
    ~NewMatGuard() {
        if (id >= 0) free_mat(id);
    }
    int release() {
        const int r = id;
        id = -1;
        return r;
    }
};
int stack_rows(const std::vector<int> &ids) {
    const GpuMat m0 = mat_at(ids[0]);
    int64_t rows = 0;
    bool any_bias = false;
    for (int id : ids) {
        const GpuMat &m = mat_at(id);
        if (m.type != m0.type || m.cols != m0.cols || m.s16 != m0.s16) throw Fail("stacked matrices differ in type or width");
        rows += m.rows;
        any_bias = any_bias || m.b;
    }
    const int nid = new_mat(m0.type, rows, m0.cols, any_bias, m0.s16);
    NewMatGuard keep{nid};
    for (int id : ids) g.mats[size_t(nid)].wmax = std::max(g.mats[size_t(nid)].wmax, mat_at(id).wmax,
                                                          [](float a, float b) { return a < b || std::isnan(b); });
    const GpuMat dst = g.mats[size_t(nid)];
    const size_t rb = row_bytes(m0.type, m0.cols), sb = scale_row_bytes(m0);
    int64_t r0 = 0;
    for (int id : ids) {
        const GpuMat src = g.mats[size_t(id)];
        HIPCHECK(hipMemcpy(dst.w + size_t(r0) * rb, src.w, size_t(src.rows) * rb, hipMemcpyDeviceToDevice));
        if (sb) HIPCHECK(hipMemcpy(reinterpret_cast<uint8_t *>(dst.s) + size_t(r0) * sb, src.s, size_t(src.rows) * sb, hipMemcpyDeviceToDevice));
        if (any_bias) {
            if (src.b) HIPCHECK(hipMemcpy(dst.b + r0, src.b, size_t(src.rows) * 4, hipMemcpyDeviceToDevice));
            else HIPCHECK(hipMemset(dst.b + r0, 0, size_t(src.rows) * 4));
        }
        r0 += src.rows;
    }
    return keep.release();
}

// Heads of hd < kF5HeadDim in the F5 / flow-estimator attention, whose tiles hold kF5HeadDim dims a head (the
// reference's device path takes any even head_dim <= 64, gpu_f5.cpp:211, :425). The q | k | v parts are stacked with
// each head's hd rows followed by hp - hd zero rows (zero scales and biases), and to_out gets hp - hd zero columns
// after each head's hd columns: the padding dims are zero in q, k and v, add nothing to q . k, come out of attention
// as zeros and meet zero weights in to_out, so the products are those of the unpadded model.
int stack_rows_heads(const std::vector<int> &ids, int heads, int hd, int hp) {
    if (hd == hp) return stack_rows(ids);
    const GpuMat m0 = mat_at(ids[0]);
    bool any_bias = false;
    for (int id : ids) {
        const GpuMat &m = mat_at(id);
        if (m.type != m0.type || m.cols != m0.cols || m.s16 != m0.s16 || m.rows != int64_t(heads) * hd)
            throw Fail("stacked attention matrices differ in type, width or head rows");
        any_bias = any_bias || m.b;
    }
    const int64_t rows = int64_t(ids.size()) * heads * hp;
    const int nid = new_mat(m0.type, rows, m0.cols, any_bias, m0.s16);
    NewMatGuard keep{nid};
    const GpuMat dst = g.mats[size_t(nid)];
    const size_t rb = row_bytes(m0.type, m0.cols), sb = scale_row_bytes(m0);
    HIPCHECK(hipMemset(dst.w, 0, size_t(rows) * rb));
    if (sb) HIPCHECK(hipMemset(dst.s, 0, size_t(rows) * sb));
    if (any_bias) HIPCHECK(hipMemset(dst.b, 0, size_t(rows) * 4));
    float wmax = 0.f;
    for (size_t p = 0; p < ids.size(); ++p) {
        const GpuMat src = mat_at(ids[p]);
        const size_t r0 = p * size_t(heads) * size_t(hp);  // head h of part p starts at row r0 + h hp
        HIPCHECK(hipMemcpy2D(dst.w + r0 * rb, size_t(hp) * rb, src.w, size_t(hd) * rb, size_t(hd) * rb, size_t(heads),
                             hipMemcpyDeviceToDevice));
        if (sb)
            HIPCHECK(hipMemcpy2D(reinterpret_cast<uint8_t *>(dst.s) + r0 * sb, size_t(hp) * sb, src.s, size_t(hd) * sb,
                                 size_t(hd) * sb, size_t(heads), hipMemcpyDeviceToDevice));
        if (src.b)
            HIPCHECK(hipMemcpy2D(dst.b + r0, size_t(hp) * 4, src.b, size_t(hd) * 4, size_t(hd) * 4, size_t(heads),
                                 hipMemcpyDeviceToDevice));
        wmax = std::max(wmax, src.wmax, [](float a, float b) { return a < b || std::isnan(b); });
    }
    g.mats[size_t(nid)].wmax = wmax;
    return keep.release();
}
// The to_out side of stack_rows_heads: a copy of m [rows][heads hd] as [rows][heads hp], each head's hd columns
// followed by hp - hd zero columns. Q8 needs hd a multiple of 32 (whole scale blocks); Q4 is not taken.
int pad_head_cols(int id, int heads, int hd, int hp) {
    if (hd == hp) return id;
    const GpuMat src = mat_at(id);
    if (src.cols != int64_t(heads) * hd) throw Fail("attention output matrix width is not heads x head_dim");
    int es = 0;
    switch (src.type) {
        case VOXHIP_F32: es = 4; break;
        case VOXHIP_F16: case VOXHIP_BF16: es = 2; break;
        case VOXHIP_Q8: es = 1; break;
        default: throw Fail("head_dim below 64 needs f32 / f16 / bf16 / q8 attention weights");
    }
    if (src.type == VOXHIP_Q8 && hd % 32) throw Fail("q8 attention weights need head_dim a multiple of 32 below 64");
    const int64_t cols = int64_t(heads) * hp;
    const int nid = new_mat(src.type, src.rows, cols, src.b != nullptr);
    NewMatGuard keep{nid};
    const GpuMat dst = g.mats[size_t(nid)];
    const size_t rows = size_t(src.rows);
    HIPCHECK(hipMemset(dst.w, 0, rows * size_t(cols) * size_t(es)));
    HIPCHECK(hipMemcpy2D(dst.w, size_t(hp) * es, src.w, size_t(hd) * es, size_t(hd) * es, rows * size_t(heads),
                         hipMemcpyDeviceToDevice));
    if (src.type == VOXHIP_Q8) {
        const size_t nb = size_t(hd / 32), nbp = size_t(hp / 32);
        HIPCHECK(hipMemset(dst.s, 0, rows * size_t(cols / 32) * 4));
        HIPCHECK(hipMemcpy2D(dst.s, nbp * 4, src.s, nb * 4, nb * 4, rows * size_t(heads), hipMemcpyDeviceToDevice));
    }
    if (src.b) HIPCHECK(hipMemcpy(dst.b, src.b, rows * 4, hipMemcpyDeviceToDevice));
    g.mats[size_t(nid)].wmax = src.wmax;
    return keep.release();
}

// A "same" Conv1d for the implicit-im2col GEMM: Conv1d::w rows [K][cin/groups] (f5_ops.cpp:86-104) padded with zero
// weights to a multiple of 8 (the GEMM's K step), which the A loader meets with zeros.
F5Conv upload_conv_gemm(const voxhip_f5_conv &c, const char *what) {
    if (!c.w || c.cin <= 0 || c.cout <= 0 || c.K <= 0 || c.K % 2 == 0 || c.groups <= 0 || c.cin % c.groups || c.cout % c.groups)
        throw Fail(std::string(what) + ": odd K, groups dividing the channels");
    const int cig = c.cin / c.groups, cog = c.cout / c.groups;
    if (cig % 4) throw Fail(std::string(what) + ": cin/groups must be a multiple of 4");
    F5Conv d;
    d.cin = c.cin; d.cout = c.cout; d.K = c.K; d.groups = c.groups;
    const int64_t kc = int64_t(c.K) * cig;
    d.kpad = int((kc + 7) / 8 * 8);
    std::vector<float> w(size_t(c.cout) * size_t(d.kpad), 0.f);
    for (int64_t r = 0; r < int64_t(c.groups) * cog; ++r) std::memcpy(&w[size_t(r * d.kpad)], c.w + r * kc, size_t(kc) * 4);
    d.wide = f32_wide(host_absmax(w.data(), w.size()));
    d.w = dalloc_t<float>(w.size());
    h2d(d.w, w.data(), w.size() * 4);
    if (c.b) {
        d.b = dalloc_t<float>(size_t(c.cout));
        h2d(d.b, c.b, size_t(c.cout) * 4);
    }
    return d;
}
F5Conv upload_conv(const voxhip_f5_conv &c, int dim) {
    if (c.cin != dim || c.cout != dim) throw Fail("F5 position convolution: cin = cout = dim");
    return upload_conv_gemm(c, "F5 position convolution");
}
// A depthwise "same" Conv1d (groups = cin = cout = dim): w [C][K].
F5Conv upload_dwconv(const voxhip_f5_conv &c, int dim) {
    if (!c.w || c.cin != dim || c.cout != dim || c.groups != dim || c.K <= 0 || c.K % 2 == 0)
        throw Fail("Vocos depthwise convolution: cin = cout = groups = vocos_dim, odd K");
    F5Conv d;
    d.cin = c.cin; d.cout = c.cout; d.K = c.K; d.groups = c.groups; d.kpad = c.K;
    d.w = dalloc_t<float>(size_t(dim) * size_t(c.K));
    h2d(d.w, c.w, size_t(dim) * size_t(c.K) * 4);
    if (c.b) {
        d.b = dalloc_t<float>(size_t(dim));
        h2d(d.b, c.b, size_t(dim) * 4);
    }
    return d;
}
float *upload_vec(const float *v, int n, const char *what) {
    if (!v) throw Fail(std::string("missing ") + what);
    float *d = dalloc_t<float>(size_t(n));
    h2d(d, v, size_t(n) * 4);
    return d;
}

void f5_free_step(F5 &F) {
    for (float *p : {F.cat, F.h, F.a, F.nrm, F.at, F.ffb, F.ada, F.ts, F.x, F.out, F.rope}) dfree(p);  // fin is in ada
    F.cat = F.h = F.a = F.nrm = F.at = F.ffb = F.ada = F.fin = F.ts = F.x = F.out = F.rope = nullptr;
    for (_Float16 *p : {F.qkv16, F.nrm16, F.at16, F.ffb16}) dfree(p);
    F.qkv16 = F.nrm16 = F.at16 = F.ffb16 = nullptr;
    F.B = F.N = F.ldvt = 0;
    F.lo_off = 0;
}

GemmArgs gemm_args(const GpuMat &m, const float *bias, float *y, int64_t lda, int64_t ldy, int64_t rows) {
    GemmArgs ga{};
    ga.bias = bias; ga.y = y; ga.lda = lda; ga.ldy = ldy; ga.m = int32_t(rows); ga.n = int32_t(m.rows); ga.K = int32_t(m.cols);
    ga.ws = g.gemm_ws; ga.ws_cap = kGemmWsFloats;
    ga.f32_wide = f32_wide(m);
    return ga;
}
void f5_gemm(const GpuMat &m, int epi, const float *A, GemmArgs ga, hipStream_t s) {
    // matmul's f32-activation path for these rows (q8 above 8 rows; q4 never)
    if (int_path(m, ga.m)) throw Fail("DiT / flow estimator linears need f32 / f16 / bf16 weights, or q8 with more than 8 rows");
    HIPCHECK(launch_gemm(gemv_type(m), epi, m.w, m.s, A, ga, s));
}
// A block linear: from the f16 planes of A (width ga.K, lo plane R ga.K halves on) when the model is split,
// else from the f32 rows A.
void split_lin(bool split, const GpuMat &m, int epi, const float *A, const _Float16 *A16, GemmArgs ga, hipStream_t s) {
    if (!split) return f5_gemm(m, epi, A, ga, s);
    ga.a16 = A16;
    ga.a_lo = int64_t(ga.m) * ga.K;
    ga.lda = ga.K;
    HIPCHECK(launch_gemm_hh(epi, reinterpret_cast<const _Float16 *>(m.w), nullptr, ga, s));
}
void f5_lin(const F5 &F, const GpuMat &m, int epi, const float *A, const _Float16 *A16, GemmArgs ga, hipStream_t s) {
    split_lin(F.split, m, epi, A, A16, ga, s);
}

// dit_forward on the device (f5.cpp:586-725) for the batches of begin; x [N][mel] and ts [dim] already on the device.
void f5_enqueue(F5 &F, hipStream_t s) {
    const int D = F.dim, INNER = F.heads * F.hp, W = 2 * F.mel + F.text;
    const int64_t R = int64_t(F.B) * F.N;
    HIPCHECK(launch_f5_fill_x(F.x, F.N, F.mel, F.cat, W, F.B, s));
    if (F.ada_all >= 0) {  // the six modulation vectors of every block (f5.cpp:673) and the final (scale, shift)
        const GpuMat &Ma = mat_at(F.ada_all);
        gemv(Ma, 1, PRO_X, EPI_STORE, F.ts, D, 1, F.ada, Ma.rows, nullptr, 0.f, nullptr, s);
    } else {
        for (int i = 0; i < F.depth; ++i) {
            const GpuMat &Ma = mat_at(F.blocks[size_t(i)].ada);
            gemv(Ma, 1, PRO_X, EPI_STORE, F.ts, D, 1, F.ada + size_t(i) * 6 * D, 6 * D, nullptr, 0.f, nullptr, s);
        }
        gemv(mat_at(F.norm_out), 1, PRO_X, EPI_STORE, F.ts, D, 1, F.fin, 2 * D, nullptr, 0.f, nullptr, s);
    }
    const GpuMat &Mi = mat_at(F.in_proj);
    f5_gemm(Mi, EPI_STORE, F.cat, gemm_args(Mi, Mi.b, F.h, W, D, R), s);
    // convolutional position embedding: h += mish(conv2(mish(conv1(h)))) per batch (f5.cpp:589-598)
    for (int c = 0; c < 2; ++c) {
        const F5Conv &cv = c == 0 ? F.pos1 : F.pos2;
        GemmArgs ga{};
        ga.bias = cv.b; ga.y = c == 0 ? F.a : F.h; ga.lda = D; ga.ldy = D; ga.m = int32_t(R);
        ga.n = cv.cout / cv.groups; ga.cig = cv.cin / cv.groups; ga.ksize = cv.K; ga.K = cv.kpad; ga.seq = F.N;
        ga.f32_wide = cv.wide;
        HIPCHECK(launch_conv_gemm(c == 0 ? EPI_MISH : EPI_MISH_ACC, cv.w, c == 0 ? F.h : F.a, ga, cv.groups, s));
    }
    const float scale = 1.0f / std::sqrt(float(F.hd));
    for (int i = 0; i < F.depth; ++i) {
        const F5Block &L = F.blocks[size_t(i)];
        const float *ada = F.ada + size_t(i) * 6 * D;  // shift, scale, gate (msa), shift, scale, gate (mlp)
        float *nrm = F.split ? nullptr : F.nrm;
        HIPCHECK(launch_f5_modulate(F.h, R, D, ada + D, ada, nrm, F.nrm16, R * D, s));
        const GpuMat &Mq = mat_at(L.qkv);
        GemmArgs gq = gemm_args(Mq, Mq.b, nullptr, D, 3 * INNER, R);
        gq.rope = F.rope; gq.seq = F.N; gq.hd = F.hp; gq.rope_hd = F.hd; gq.rope_cols = 2 * INNER; gq.rope_heads = F.pe;
        gq.h16 = F.qkv16; gq.lo_off = F.lo_off; gq.ldvt = F.ldvt;
        f5_lin(F, Mq, EPI_ROPE_H16, F.nrm, F.nrm16, gq, s);
        HIPCHECK(launch_f5_attn(F.qkv16, F.lo_off, F.split ? nullptr : F.at, F.at16, R * INNER, F.B, F.N, F.heads, F.hp,
                                F.ldvt, INNER, scale, s));
        const GpuMat &Mo = mat_at(L.o);
        GemmArgs go = gemm_args(Mo, Mo.b, F.h, INNER, D, R);
        go.gate = ada + 2 * D;
        f5_lin(F, Mo, EPI_GATED_ACC, F.at, F.at16, go, s);
        HIPCHECK(launch_f5_modulate(F.h, R, D, ada + 4 * D, ada + 3 * D, nrm, F.nrm16, R * D, s));
        const GpuMat &M1 = mat_at(L.ff1), &M2 = mat_at(L.ff2);
        GemmArgs g1 = gemm_args(M1, M1.b, F.split ? nullptr : F.ffb, D, F.ff, R);
        g1.h16 = F.ffb16; g1.lo_off = R * F.ff;
        f5_lin(F, M1, F.split ? EPI_GELU_H16 : EPI_GELU, F.nrm, F.nrm16, g1, s);
        GemmArgs g2 = gemm_args(M2, M2.b, F.h, F.ff, D, R);
        g2.gate = ada + 5 * D;
        f5_lin(F, M2, EPI_GATED_ACC, F.ffb, F.ffb16, g2, s);
    }
    HIPCHECK(launch_f5_modulate(F.h, R, D, F.fin, F.fin + D, F.nrm, nullptr, 0, s));  // final modulation: (scale, shift)
    const GpuMat &Mp = mat_at(F.proj_out);
    f5_gemm(Mp, EPI_STORE, F.nrm, gemm_args(Mp, Mp.b, F.out, D, F.mel, R), s);
}
}  // namespace

extern "C" {

int voxhip_f5_create(const voxhip_f5_desc *d) {
    return guard_int([&] {
        require_ok();
        if (!d || d->depth <= 0 || !d->blocks) throw Fail("missing F5 description");
        if (d->dim_head <= 0 || d->dim_head > kF5HeadDim || d->dim_head % 2)
            throw Fail("F5 attention supports even head_dim up to 64");
        const int D = d->dim, INNER = d->heads * d->dim_head, FF = d->dim * d->ff_mult, W = 2 * d->mel_dim + d->text_dim;
        if (D <= 0 || D % 8 || d->heads <= 0 || FF <= 0 || d->mel_dim <= 0 || d->text_dim < 0) throw Fail("bad F5 dimensions");
        auto check = [&](int id, int64_t rows, int64_t cols, const char *what) {
            const GpuMat &m = mat_at(id);
            if (m.rows != rows || m.cols != cols) throw Fail(std::string("F5 ") + what + " has the wrong shape");
        };
        check(d->in_proj, D, W, "in_proj");
        check(d->norm_out, 2 * D, D, "norm_out");
        check(d->proj_out, d->mel_dim, D, "proj_out");
        std::unique_ptr<F5> F(new F5());
        F->dim = D; F->depth = d->depth; F->heads = d->heads; F->hd = d->dim_head; F->hp = kF5HeadDim; F->ff = FF;
        F->mel = d->mel_dim;
        F->text = d->text_dim; F->pe = d->pe_attn_head;
        F->in_proj = d->in_proj; F->norm_out = d->norm_out; F->proj_out = d->proj_out;
        for (int i = 0; i < d->depth; ++i) {
            const voxhip_f5_block &b = d->blocks[i];
            check(b.ada, 6 * D, D, "ada");
            check(b.q, INNER, D, "q"); check(b.k, INNER, D, "k"); check(b.v, INNER, D, "v");
            check(b.o, D, INNER, "o"); check(b.ff1, FF, D, "ff1"); check(b.ff2, D, FF, "ff2");
            F5Block fb;
            fb.ada = b.ada; fb.ff1 = b.ff1; fb.ff2 = b.ff2;
            fb.qkv = stack_rows_heads({b.q, b.k, b.v}, d->heads, d->dim_head, kF5HeadDim);
            fb.o = pad_head_cols(b.o, d->heads, d->dim_head, kF5HeadDim);
            F->blocks.push_back(fb);
        }
        try {  // one modulation GEMV per step; when the matrices differ in type (or VRAM is short) one per block
            std::vector<int> ids;
            for (int i = 0; i < d->depth; ++i) ids.push_back(d->blocks[i].ada);
            ids.push_back(d->norm_out);
            F->ada_all = stack_rows(ids);
        } catch (const Fail &) {
            F->ada_all = -1;
        }
        F->split = D % 64 == 0 && FF % 64 == 0;  // the attention width (heads x 64) always is
        for (const F5Block &fb : F->blocks)
            for (int id : {fb.qkv, fb.o, fb.ff1, fb.ff2}) F->split = F->split && mat_at(id).type == VOXHIP_F16;
        F->pos1 = upload_conv(d->pos1, D);
        F->pos2 = upload_conv(d->pos2, D);
        if (d->vocos_dim > 0) {  // Vocos (f5.cpp:333-346): the linears are matrix handles, the rest host arrays
            const int VD = d->vocos_dim, VI = d->vocos_inter, VO = d->vocos_out;
            if (VD % 4 || VI <= 0 || VO <= 0 || d->n_vblocks < 0 || (d->n_vblocks > 0 && !d->v_blocks))
                throw Fail("bad Vocos dimensions (vocos_dim a multiple of 4)");
            check(d->v_head, VO, VD, "Vocos head");
            if (d->v_embed.cin != d->mel_dim || d->v_embed.cout != VD) throw Fail("Vocos embed: mel_dim -> vocos_dim");
            F->v_embed = upload_conv_gemm(d->v_embed, "Vocos embed");
            F->v_ln_w = upload_vec(d->v_ln_w, VD, "Vocos norm weight");
            F->v_ln_b = d->v_ln_b ? upload_vec(d->v_ln_b, VD, "Vocos norm bias") : nullptr;
            F->v_fln_w = upload_vec(d->v_fln_w, VD, "Vocos final norm weight");
            F->v_fln_b = d->v_fln_b ? upload_vec(d->v_fln_b, VD, "Vocos final norm bias") : nullptr;
            for (int i = 0; i < d->n_vblocks; ++i) {
                const voxhip_f5_vblock &b = d->v_blocks[i];
                check(b.pw1, VI, VD, "Vocos pwconv1");
                check(b.pw2, VD, VI, "Vocos pwconv2");
                F5VBlock vb;
                vb.dw = upload_dwconv(b.dw, VD);
                vb.ln_w = upload_vec(b.ln_w, VD, "Vocos block norm weight");
                vb.ln_b = b.ln_b ? upload_vec(b.ln_b, VD, "Vocos block norm bias") : nullptr;
                vb.gamma = upload_vec(b.gamma, VD, "Vocos gamma");
                vb.pw1 = b.pw1; vb.pw2 = b.pw2;
                F->vblocks.push_back(vb);
            }
            F->vdim = VD; F->vinter = VI; F->vout = VO; F->v_head = d->v_head;
        }
        g.f5.push_back(F.release());
        return int(g.f5.size()) - 1;
    }, -1);
}

int voxhip_f5_begin(int id, int B, int N, const float *cat0, const float *rope) {
    return guard_int([&] {
        require_ok();
        F5 &F = f5_at(id);
        if (B <= 0 || N <= 0 || !cat0 || !rope || int64_t(B) * N > INT32_MAX / 8) throw Fail("bad F5 step shape");
        f5_free_step(F);
        const size_t R = size_t(B) * size_t(N), D = size_t(F.dim), INNER = size_t(F.heads) * F.hp;
        const size_t W = 2 * size_t(F.mel) + F.text;
        F.cat = dalloc_t<float>(R * W); F.h = dalloc_t<float>(R * D); F.a = dalloc_t<float>(R * D);
        F.nrm = dalloc_t<float>(R * D);
        if (F.split) {
            F.nrm16 = dalloc_t<_Float16>(2 * R * D);
            F.at16 = dalloc_t<_Float16>(2 * R * INNER);
            F.ffb16 = dalloc_t<_Float16>(2 * R * size_t(F.ff));
        } else {
            F.at = dalloc_t<float>(R * INNER);
            F.ffb = dalloc_t<float>(R * size_t(F.ff));
        }
        F.ldvt = (N + 63) / 64 * 64;  // whole key tiles, the padding zero
        F.lo_off = int64_t(R * 2 * INNER) + int64_t(B) * int64_t(INNER) * F.ldvt;
        F.qkv16 = dalloc_t<_Float16>(size_t(2 * F.lo_off));
        HIPCHECK(hipMemset(F.qkv16, 0, size_t(2 * F.lo_off) * sizeof(_Float16)));  // the v^T padding stays zero
        F.ada = dalloc_t<float>((size_t(F.depth) * 6 + 2) * D);  // the blocks' vectors, then fin: one GEMV's rows
        F.fin = F.ada + size_t(F.depth) * 6 * D;
        F.ts = dalloc_t<float>(D); F.x = dalloc_t<float>(size_t(N) * F.mel);
        F.out = dalloc_t<float>(R * size_t(F.mel)); F.rope = dalloc_t<float>(size_t(N) * size_t(F.hd));
        h2d(F.cat, cat0, R * W * 4);
        h2d(F.rope, rope, size_t(N) * size_t(F.hd) * 4);
        F.B = B; F.N = N;
        return 1;
    }, 0);
}

int voxhip_f5_step(int id, const float *x, const float *ts, float *out) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("f5.step");
        F5 &F = f5_at(id);
        if (!F.B) throw Fail("F5 step before begin");
        if (!x || !ts || !out) throw Fail("missing argument");
        h2d(F.x, x, size_t(F.N) * F.mel * 4);
        h2d(F.ts, ts, size_t(F.dim) * 4);
        f5_enqueue(F, g.stream);
        sync_status();
        HIPCHECK(copy_d2h(out, F.out, size_t(F.B) * F.N * F.mel * 4, nullptr));
        return 1;
    }, 0);
}

// F5Model::vocode up to the head (f5.cpp:792-806; gpu_f5.cpp:334-373): embed conv, LayerNorm, the ConvNeXt blocks
// (depthwise conv, LayerNorm, pwconv1 + GELU-erf, pwconv2 with x += gamma * (.)), final LayerNorm, head.
int voxhip_f5_vocos(int id, const float *mel, int T, float *head) {
    return guard_int([&] {
        require_ok();
        vh::prof_stage("f5.vocos");
        F5 &F = f5_at(id);
        if (!F.vdim) throw Fail("this F5 model has no Vocos on the device");
        if (!mel || !head || T <= 0 || int64_t(T) * std::max(F.vinter, F.vout) > INT32_MAX / 2) throw Fail("bad Vocos input");
        const int VD = F.vdim;
        if (F.vT < T) {
            HIPCHECK(hipStreamSynchronize(g.stream));
            for (float *p : {F.vm, F.vx, F.vy, F.vh, F.vhead}) dfree(p);
            F.vm = dalloc_t<float>(size_t(T) * F.mel); F.vx = dalloc_t<float>(size_t(T) * VD); F.vy = dalloc_t<float>(size_t(T) * VD);
            F.vh = dalloc_t<float>(size_t(T) * F.vinter); F.vhead = dalloc_t<float>(size_t(T) * F.vout);
            F.vT = T;
        }
        hipStream_t s = g.stream;
        h2d(F.vm, mel, size_t(T) * F.mel * 4);
        const F5Conv &ce = F.v_embed;
        GemmArgs ge{};
        ge.bias = ce.b; ge.y = F.vx; ge.lda = ce.cin; ge.ldy = VD; ge.m = T; ge.n = ce.cout / ce.groups;
        ge.cig = ce.cin / ce.groups; ge.ksize = ce.K; ge.K = ce.kpad; ge.seq = T;
        ge.f32_wide = ce.wide;
        HIPCHECK(launch_conv_gemm(EPI_STORE, ce.w, F.vm, ge, ce.groups, s));
        HIPCHECK(launch_layernorm_rows(F.vx, T, VD, F.v_ln_w, F.v_ln_b, F.vx, s));
        for (const F5VBlock &b : F.vblocks) {
            HIPCHECK(launch_dwconv(F.vx, b.dw.w, b.dw.b, F.vy, T, VD, b.dw.K, T, s));
            HIPCHECK(launch_layernorm_rows(F.vy, T, VD, b.ln_w, b.ln_b, F.vy, s));
            const GpuMat &M1 = mat_at(b.pw1), &M2 = mat_at(b.pw2);
            f5_gemm(M1, EPI_GELU_ERF, F.vy, gemm_args(M1, M1.b, F.vh, VD, F.vinter, T), s);
            GemmArgs g2 = gemm_args(M2, M2.b, F.vx, F.vinter, VD, T);
            g2.gate = b.gamma;
            f5_gemm(M2, EPI_GATED_ACC, F.vh, g2, s);
        }
        HIPCHECK(launch_layernorm_rows(F.vx, T, VD, F.v_fln_w, F.v_fln_b, F.vx, s));
        const GpuMat &Mh = mat_at(F.v_head);
        f5_gemm(Mh, EPI_STORE, F.vx, gemm_args(Mh, Mh.b, F.vhead, VD, F.vout, T), s);
        sync_status();
        HIPCHECK(copy_d2h(head, F.vhead, size_t(T) * F.vout * 4, nullptr));
        return 1;
    }, 0);
}

int voxhip_f5_vocos_out(int id, int32_t *vout) {
    return guard_int([&] {
        require_ok();
        if (!vout) throw Fail("missing argument");
        *vout = f5_at(id).vout;
        return 1;
    }, 0);
}

int voxhip_f5_end(int id) {
    return guard_int([&] {
        require_ok();
        F5 &F = f5_at(id);
        HIPCHECK(hipStreamSynchronize(g.stream));
        f5_free_step(F);
        return 1;
    }, 0);
}

}  // extern "C"

namespace {
// ------------------------------------------------------------------ CosyVoice2 / Chatterbox flow estimator
// (gpu.hpp:100-119; cosyvoice.cpp:126-221 the CPU blocks, :822-863 the step)
struct CosyRes {  // CausalResnetBlock1D
    F5Conv c1, c2, res;
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
};
struct CosyX {  // BasicTransformerBlock; q | k | v stacked at create
    float *n1w = nullptr, *n1b = nullptr, *n3w = nullptr, *n3b = nullptr;
    int qkv = -1, o = -1, ff1 = -1, ff2 = -1, ff = 0;
};
struct Cosy {
    // hd: the model's head_dim; inner: the attention layout's width, heads x kF5HeadDim (heads of hd < 64 padded with
    // zero dims, stack_rows_heads)
    int M = 0, C = 0, heads = 0, hd = 0, inner = 0, ffmax = 0;
    CosyRes down_res, up_res;
    std::vector<CosyRes> mid_res;
    std::vector<CosyX> down_x, up_x;
    std::vector<std::vector<CosyX>> mid_x;
    F5Conv down_conv, up_out, final_conv, final_proj;
    float *fn_w = nullptr, *fn_b = nullptr;
    // every transformer linear F16 and C, inner, ff multiples of 64: the block activations travel as f16 halves
    // and the linears take k_gemm_hh; otherwise f32 rows
    bool split = false;
    // step buffers of begin(T): rows R = 2 T
    int T = 0;
    float *in = nullptr, *a = nullptr, *b = nullptr, *h = nullptr, *cat = nullptr, *xn = nullptr, *at = nullptr,
          *ff = nullptr, *tb = nullptr, *x = nullptr, *out = nullptr;
    _Float16 *qkv16 = nullptr, *xn16 = nullptr, *at16 = nullptr, *ff16 = nullptr;
    int64_t lo_off = 0;
    int ldvt = 0;
    // the step's launches as one graph over the buffers of this begin (captured by the first step after it)
    hipGraphExec_t step_graph = nullptr;
};

Cosy &cosy_at(int id) {
    if (id < 0 || size_t(id) >= g.cosy.size() || !g.cosy[size_t(id)]) throw Fail("bad flow estimator handle " + std::to_string(id));
    return *g.cosy[size_t(id)];
}

void cosy_free_step(Cosy &E) {
    if (E.step_graph) (void)hipGraphExecDestroy(E.step_graph);
    E.step_graph = nullptr;
    for (float *p : {E.in, E.a, E.b, E.h, E.cat, E.xn, E.at, E.ff, E.tb, E.x, E.out}) dfree(p);
    E.in = E.a = E.b = E.h = E.cat = E.xn = E.at = E.ff = E.tb = E.x = E.out = nullptr;
    for (_Float16 *p : {E.qkv16, E.xn16, E.at16, E.ff16}) dfree(p);
    E.qkv16 = E.xn16 = E.at16 = E.ff16 = nullptr;
    E.T = E.ldvt = 0;
    E.lo_off = 0;
}

F5Conv cosy_conv_up(const voxhip_f5_conv &c, int cin, int cout, bool k1, const char *what) {
    if (c.groups != 1 || c.cin != cin || c.cout != cout || (k1 && c.K != 1))
        throw Fail(std::string("flow estimator ") + what + ": wrong shape (groups 1" + (k1 ? ", K 1)" : ")"));
    return upload_conv_gemm(c, what);
}

CosyRes cosy_res_up(const voxhip_cosy_res &r, int cin, int C) {
    CosyRes o;
    o.c1 = cosy_conv_up(r.c1, cin, C, false, "resnet conv 1");
    o.c2 = cosy_conv_up(r.c2, C, C, false, "resnet conv 2");
    o.res = cosy_conv_up(r.res, cin, C, true, "resnet res conv");
    o.n1w = upload_vec(r.n1w, C, "resnet norm 1 weight");
    o.n1b = upload_vec(r.n1b, C, "resnet norm 1 bias");
    o.n2w = upload_vec(r.n2w, C, "resnet norm 2 weight");
    o.n2b = upload_vec(r.n2b, C, "resnet norm 2 bias");
    return o;
}

CosyX cosy_x_up(const voxhip_cosy_x &x, int C, int heads, int hd) {
    const int inner = heads * hd;
    auto check = [&](int id, int64_t rows, int64_t cols, const char *what) {
        const GpuMat &m = mat_at(id);
        if (m.rows != rows || m.cols != cols) throw Fail(std::string("flow estimator ") + what + " has the wrong shape");
    };
    if (x.ff_dim <= 0 || x.ff_dim % 4) throw Fail("flow estimator: ff_dim must be a positive multiple of 4");
    check(x.q, inner, C, "to_q"); check(x.k, inner, C, "to_k"); check(x.v, inner, C, "to_v");
    check(x.o, C, inner, "to_out"); check(x.ff1, x.ff_dim, C, "ff.0"); check(x.ff2, C, x.ff_dim, "ff.2");
    CosyX o;
    o.n1w = upload_vec(x.n1w, C, "norm1 weight"); o.n1b = upload_vec(x.n1b, C, "norm1 bias");
    o.n3w = upload_vec(x.n3w, C, "norm3 weight"); o.n3b = upload_vec(x.n3b, C, "norm3 bias");
    o.qkv = stack_rows_heads({x.q, x.k, x.v}, heads, hd, kF5HeadDim);
    o.o = pad_head_cols(x.o, heads, hd, kF5HeadDim);
    o.ff1 = x.ff1; o.ff2 = x.ff2; o.ff = x.ff_dim;
    return o;
}

// A causal (or K-1) convolution of the R = 2 T rows X (row stride ldx) into Y (row stride ldy) on the conv GEMM.
void cosy_conv(const Cosy &E, const F5Conv &cv, int epi, const float *X, int64_t ldx, float *Y, int64_t ldy, hipStream_t s) {
    GemmArgs ga{};
    ga.bias = cv.b; ga.y = Y; ga.lda = ldx; ga.ldy = ldy; ga.m = int32_t(2 * E.T); ga.n = cv.cout;
    ga.cig = cv.cin; ga.ksize = cv.K; ga.K = cv.kpad; ga.seq = E.T; ga.causal = 1;
    ga.ws = g.gemm_ws; ga.ws_cap = kGemmWsFloats;  // split K when the 64 x 64 tiles leave the CUs idle
    ga.f32_wide = cv.wide;
    HIPCHECK(launch_conv_gemm(epi, cv.w, X, ga, 1, s));
}

// LayerNorm (eps 1e-5f, cosyvoice.cpp:156, :205, :213) of the R rows of C at x into y (or y16 planes), then mish and
// the channel bias tb when given.
void cosy_norm(const Cosy &E, const float *x, const float *w, const float *b, bool mish, const float *tb, float *y,
               _Float16 *y16, hipStream_t s) {
    NormArgs a{};
    a.x = x; a.y = y; a.y16 = y16; a.lo_off = int64_t(2) * E.T * E.C; a.sc = w; a.sh = b; a.tb = tb;
    a.eps = double(1e-5f); a.R = 2 * E.T; a.D = E.C; a.affine = 1; a.mish = mish;
    HIPCHECK(launch_norm_rows(a, s));
}

// CausalResnetBlock1D (cosyvoice.cpp:158-180): O = block2(block1(X) + tb) + res(X), block = causal conv -> LayerNorm
// -> mish; tb the time bias of resnet j.
void cosy_resnet(const Cosy &E, const CosyRes &r, int j, const float *X, int64_t ldx, float *O, hipStream_t s) {
    const int C = E.C;
    cosy_conv(E, r.c1, EPI_STORE, X, ldx, E.h, C, s);
    cosy_norm(E, E.h, r.n1w, r.n1b, true, E.tb + size_t(j) * C, E.h, nullptr, s);
    cosy_conv(E, r.c2, EPI_STORE, E.h, C, O, C, s);
    cosy_norm(E, O, r.n2w, r.n2b, true, nullptr, O, nullptr, s);
    cosy_conv(E, r.res, EPI_ACC, X, ldx, O, C, s);
}

// BasicTransformerBlock (cosyvoice.cpp:182-221) on the rows A in place: LayerNorm -> q | k | v (no bias) -> full
// attention per sequence -> to_out + residual -> LayerNorm -> ff.0 + GELU (erf) -> ff.2 + residual.
void cosy_xblock(const Cosy &E, const CosyX &L, float *A, hipStream_t s) {
    const int C = E.C, INNER = E.inner;
    const int64_t R = int64_t(2) * E.T;
    float *xn = E.split ? nullptr : E.xn;
    cosy_norm(E, A, L.n1w, L.n1b, false, nullptr, xn, E.xn16, s);
    const GpuMat &Mq = mat_at(L.qkv);
    GemmArgs gq = gemm_args(Mq, Mq.b, nullptr, C, 3 * INNER, R);
    gq.rope = nullptr; gq.seq = E.T; gq.hd = kF5HeadDim; gq.rope_cols = 2 * INNER;
    gq.h16 = E.qkv16; gq.lo_off = E.lo_off; gq.ldvt = E.ldvt;
    split_lin(E.split, Mq, EPI_ROPE_H16, E.xn, E.xn16, gq, s);
    HIPCHECK(launch_f5_attn(E.qkv16, E.lo_off, E.split ? nullptr : E.at, E.at16, R * INNER, 2, E.T, E.heads, kF5HeadDim,
                            E.ldvt, INNER, 1.0f / std::sqrt(float(E.hd)), s));
    const GpuMat &Mo = mat_at(L.o);
    split_lin(E.split, Mo, EPI_ACC, E.at, E.at16, gemm_args(Mo, Mo.b, A, INNER, C, R), s);
    cosy_norm(E, A, L.n3w, L.n3b, false, nullptr, xn, E.xn16, s);
    const GpuMat &M1 = mat_at(L.ff1), &M2 = mat_at(L.ff2);
    GemmArgs g1 = gemm_args(M1, M1.b, E.split ? nullptr : E.ff, C, L.ff, R);
    g1.h16 = E.ff16; g1.lo_off = R * L.ff; g1.gelu_erf = 1;
    split_lin(E.split, M1, E.split ? EPI_GELU_H16 : EPI_GELU_ERF, E.xn, E.xn16, g1, s);
    split_lin(E.split, M2, EPI_ACC, E.ff, E.ff16, gemm_args(M2, M2.b, A, L.ff, C, R), s);
}

// The estimator of one Euler step (cosyvoice.cpp:839-863; gpu_f5.cpp:490-547): x and the time biases already on
// the device.
void cosy_enqueue(Cosy &E, hipStream_t s) {
    const int C = E.C, M = E.M;
    const int64_t R = int64_t(2) * E.T;
    HIPCHECK(launch_f5_fill_x(E.x, E.T, M, E.in, 4 * M, 2, s));
    cosy_resnet(E, E.down_res, 0, E.in, 4 * M, E.a, s);
    for (const CosyX &L : E.down_x) cosy_xblock(E, L, E.a, s);
    // the skip half of the up block's input [x | skip]
    HIPCHECK(hipMemcpy2DAsync(E.cat + C, size_t(2 * C) * 4, E.a, size_t(C) * 4, size_t(C) * 4, size_t(R), hipMemcpyDeviceToDevice, s));
    cosy_conv(E, E.down_conv, EPI_STORE, E.a, C, E.b, C, s);
    float *cur = E.b, *oth = E.a;
    for (size_t i = 0; i < E.mid_res.size(); ++i) {
        cosy_resnet(E, E.mid_res[i], int(1 + i), cur, C, oth, s);
        for (const CosyX &L : E.mid_x[i]) cosy_xblock(E, L, oth, s);
        std::swap(cur, oth);
    }
    HIPCHECK(hipMemcpy2DAsync(E.cat, size_t(2 * C) * 4, cur, size_t(C) * 4, size_t(C) * 4, size_t(R), hipMemcpyDeviceToDevice, s));
    cosy_resnet(E, E.up_res, int(1 + E.mid_res.size()), E.cat, 2 * C, oth, s);
    for (const CosyX &L : E.up_x) cosy_xblock(E, L, oth, s);
    cosy_conv(E, E.up_out, EPI_STORE, oth, C, cur, C, s);
    cosy_conv(E, E.final_conv, EPI_STORE, cur, C, oth, C, s);
    cosy_norm(E, oth, E.fn_w, E.fn_b, true, nullptr, oth, nullptr, s);
    cosy_conv(E, E.final_proj, EPI_STORE, oth, C, E.out, M, s);
}
}  // namespace

extern "C" {

int voxhip_cosy_create(const voxhip_cosy_desc *d) {
    return guard_int([&] {
        require_ok();
        if (!d) throw Fail("missing flow estimator description");
        if (d->head_dim <= 0 || d->head_dim > kF5HeadDim || d->head_dim % 2)
            throw Fail("the flow estimator's attention supports even head_dim up to 64");
        const int C = d->C, M = d->M;
        if (C <= 0 || C % 4 || M <= 0 || M % 4 || d->heads <= 0 || d->n_mid < 0 || d->n_down_x < 0 || d->n_up_x < 0)
            throw Fail("bad flow estimator dimensions (C and M multiples of 4)");
        if ((d->n_mid && (!d->mid_res || !d->mid_x_count)) || (d->n_down_x && !d->down_x) || (d->n_up_x && !d->up_x))
            throw Fail("missing flow estimator blocks");
        std::unique_ptr<Cosy> E(new Cosy());
        E->M = M; E->C = C; E->heads = d->heads; E->hd = d->head_dim; E->inner = d->heads * kF5HeadDim;
        E->down_res = cosy_res_up(d->down_res, 4 * M, C);
        E->up_res = cosy_res_up(d->up_res, 2 * C, C);
        for (int i = 0; i < d->n_mid; ++i) E->mid_res.push_back(cosy_res_up(d->mid_res[i], C, C));
        auto xs = [&](const voxhip_cosy_x *v, int n) {
            std::vector<CosyX> o;
            for (int i = 0; i < n; ++i) {
                o.push_back(cosy_x_up(v[i], C, d->heads, d->head_dim));
                E->ffmax = std::max(E->ffmax, v[i].ff_dim);
            }
            return o;
        };
        E->down_x = xs(d->down_x, d->n_down_x);
        E->up_x = xs(d->up_x, d->n_up_x);
        int64_t off = 0;
        for (int i = 0; i < d->n_mid; ++i) {
            if (d->mid_x_count[i] < 0 || (d->mid_x_count[i] && !d->mid_x)) throw Fail("bad mid_x_count");
            E->mid_x.push_back(xs(d->mid_x + off, d->mid_x_count[i]));
            off += d->mid_x_count[i];
        }
        E->down_conv = cosy_conv_up(d->down_conv, C, C, false, "down conv");
        E->up_out = cosy_conv_up(d->up_out, C, C, false, "up conv");
        E->final_conv = cosy_conv_up(d->final_conv, C, C, false, "final block conv");
        E->final_proj = cosy_conv_up(d->final_proj, C, M, true, "final_proj");
        E->fn_w = upload_vec(d->fn_w, C, "final block norm weight");
        E->fn_b = upload_vec(d->fn_b, C, "final block norm bias");
        bool split = C % 64 == 0 && E->inner % 64 == 0;
        for (const auto *v : {&E->down_x, &E->up_x})
            for (const CosyX &x : *v) split = split && x.ff % 64 == 0;
        for (const auto &v : E->mid_x)
            for (const CosyX &x : v) split = split && x.ff % 64 == 0;
        auto all_f16 = [&](const std::vector<CosyX> &v) {
            for (const CosyX &x : v)
                for (int id : {x.qkv, x.o, x.ff1, x.ff2})
                    if (mat_at(id).type != VOXHIP_F16) return false;
            return true;
        };
        split = split && all_f16(E->down_x) && all_f16(E->up_x);
        for (const auto &v : E->mid_x) split = split && all_f16(v);
        E->split = split;
        g.cosy.push_back(E.release());
        return int(g.cosy.size()) - 1;
    }, -1);
}

int voxhip_cosy_begin(int id, int T, const float *in0) {
    return guard_int([&] {
        require_ok();
        Cosy &E = cosy_at(id);
        if (T <= 0 || !in0 || int64_t(T) * 2 * std::max({E.C * 2, E.inner * 3, E.ffmax, 4 * E.M}) > INT32_MAX / 2)
            throw Fail("bad flow estimator length");
        HIPCHECK(hipStreamSynchronize(g.stream));
        cosy_free_step(E);
        const size_t R = size_t(2) * size_t(T), C = size_t(E.C), INNER = size_t(E.inner), FF = size_t(std::max(E.ffmax, 1));
        E.in = dalloc_t<float>(R * 4 * E.M);
        E.a = dalloc_t<float>(R * C); E.b = dalloc_t<float>(R * C); E.h = dalloc_t<float>(R * C);
        E.cat = dalloc_t<float>(R * 2 * C);
        if (E.split) {
            E.xn16 = dalloc_t<_Float16>(2 * R * C);
            E.at16 = dalloc_t<_Float16>(2 * R * INNER);
            E.ff16 = dalloc_t<_Float16>(2 * R * FF);
        } else {
            E.xn = dalloc_t<float>(R * C);
            E.at = dalloc_t<float>(R * INNER);
            E.ff = dalloc_t<float>(R * FF);
        }
        E.ldvt = (T + 63) / 64 * 64;  // whole key tiles, the padding zero
        E.lo_off = int64_t(R * 2 * INNER) + int64_t(2) * int64_t(INNER) * E.ldvt;
        E.qkv16 = dalloc_t<_Float16>(size_t(2 * E.lo_off));
        HIPCHECK(hipMemset(E.qkv16, 0, size_t(2 * E.lo_off) * sizeof(_Float16)));  // the v^T padding stays zero
        E.tb = dalloc_t<float>((2 + E.mid_res.size()) * C);
        E.x = dalloc_t<float>(size_t(T) * E.M);
        E.out = dalloc_t<float>(R * E.M);
        h2d(E.in, in0, R * 4 * E.M * 4);
        E.T = T;
        return 1;
    }, 0);
}

int voxhip_cosy_step(int id, const float *x, const float *tb, float *out) {
    return guard_int([&] {
        require_ok();
        Cosy &E = cosy_at(id);
        if (!E.T) throw Fail("flow estimator step before begin");
        if (!x || !tb || !out) throw Fail("missing argument");
        h2d(E.x, x, size_t(E.T) * E.M * 4);
        h2d(E.tb, tb, (2 + E.mid_res.size()) * size_t(E.C) * 4);
        // the step's ~560 launches as one graph: the buffers of this begin, the weights and the scratch are fixed
        vh::prof_stage("flow.est");
        if (vh::prof_on()) cosy_enqueue(E, g.stream);  // stamped launches are not captured
        else if (!E.step_graph) {
            hipGraph_t graph = nullptr;
            HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
            try {
                cosy_enqueue(E, g.stream);
            } catch (...) {
                (void)hipStreamEndCapture(g.stream, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                throw;
            }
            HIPCHECK(hipStreamEndCapture(g.stream, &graph));
            hipGraphExec_t exec = nullptr;
            const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            HIPCHECK(e);
            E.step_graph = exec;
        }
        if (!vh::prof_on()) HIPCHECK(hipGraphLaunch(E.step_graph, g.stream));
        sync_status();
        HIPCHECK(copy_d2h(out, E.out, size_t(2) * E.T * E.M * 4, nullptr));
        return 1;
    }, 0);
}

int voxhip_cosy_end(int id) {
    return guard_int([&] {
        require_ok();
        Cosy &E = cosy_at(id);
        HIPCHECK(hipStreamSynchronize(g.stream));
        cosy_free_step(E);
        return 1;
    }, 0);
}

}  // extern "C"

namespace {
// ------------------------------------------------------------------ Qwen3-TTS codec decoder (gpu.hpp:53-60)
constexpr int kCodecMaxFrames = 16;  // kGpuCodecMaxFrames (gpu.hpp:61)
struct CodecConv {
    int mat = -1, K = 1, cin = 0, cout = 0, dil = 1;
};
struct CodecSnake {
    float *a = nullptr, *inv_b = nullptr;
};
struct CodecUp {
    int tr = -1, K = 0, pw1 = -1, pw2 = -1, dwK = 0;
    float *tr_b = nullptr, *dw_w = nullptr, *dw_b = nullptr, *ln_w = nullptr, *ln_b = nullptr, *gamma = nullptr;
};
struct CodecBlk {
    CodecSnake act, a1[3], a2[3];
    int tr = -1, K = 0, s = 0, cin = 0, cout = 0;
    float *tr_b = nullptr;
    CodecConv c1[3], c2[3];
};
struct Codec {
    int cdim = 0, latent = 0, H = 0, heads = 0, kvh = 0, hd = 0, I = 0, W = 0, R = 0, layers = 0, spf = 0, dec = 0;
    float eps = 1e-5f;
    std::vector<float> inv_freq;
    int xf = -1;  // the pre-transformer's stacked matrices and norms
    std::vector<float *> sa, sm;  // layer scales [H] or null
    CodecConv pre_conv, conv0, fin;
    int pt_in = -1, pt_out = -1;
    std::vector<CodecUp> ups;
    std::vector<CodecBlk> blocks;
    CodecSnake fin_act;
    // scratch for kCodecMaxFrames frames: S activations (each smax floats), the transformer rows, z, the RoPE rows
    float *S[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
    int64_t smax = 0;
    float *qkv = nullptr, *ao = nullptr, *act = nullptr, *tmp = nullptr, *h = nullptr, *pre = nullptr, *rope = nullptr, *z = nullptr;
};
// A streaming history (or transposed-conv tail) as two buffers: a call reads b[parity] and writes the next call's into
// b[1 - parity]; the state's parity flips after every call, so a call's buffers depend only on (T, parity) and a
// captured call replays.
struct Hist2 {
    float *b[2] = {nullptr, nullptr};
    int rows = 0, C = 0;
};
struct CodecSt {
    int codec = -1;
    int64_t len = 0;   // positions already in the transformer
    int parity = 0;
    int64_t *pos_dev = nullptr;  // len on the device, for the captured kernels
    Hist2 pre, c0, fin;
    std::vector<Hist2> dw, tail, ru;
    std::vector<float *> kr, vr;  // ring caches [R][kv_heads hd] per layer
    std::map<int, hipGraphExec_t> graphs;  // by 2 T + parity
};

Codec &codec_at(int id) {
    if (id < 0 || size_t(id) >= g.codecs.size() || !g.codecs[size_t(id)]) throw Fail("bad codec handle " + std::to_string(id));
    return *g.codecs[size_t(id)];
}
CodecSt &cstate_at(int id) {
    if (id < 0 || size_t(id) >= g.cstates.size() || !g.cstates[size_t(id)]) throw Fail("bad codec state " + std::to_string(id));
    return *g.cstates[size_t(id)];
}

CodecConv codec_conv_up(const voxhip_codec_conv &c, const char *what) {
    const GpuMat &m = mat_at(c.mat);
    if (c.K <= 0 || c.dil <= 0 || c.cin <= 0 || c.cin % 4 || m.rows != c.cout || m.cols != int64_t(c.K) * c.cin)
        throw Fail(std::string("codec ") + what + ": weight must be [cout][K cin], cin a multiple of 4");
    if (m.type != VOXHIP_F32 && m.type != VOXHIP_F16 && m.type != VOXHIP_BF16)
        throw Fail(std::string("codec ") + what + ": f32 / f16 / bf16 weights only");
    CodecConv o;
    o.mat = c.mat; o.K = c.K; o.cin = c.cin; o.cout = c.cout; o.dil = c.dil;
    return o;
}
CodecSnake codec_snake_up(const voxhip_codec_snake &s, int C) {
    CodecSnake o;
    o.a = upload_vec(s.a, C, "Snake a");
    o.inv_b = upload_vec(s.inv_b, C, "Snake inv_b");
    return o;
}
void codec_check_mat(int id, int64_t rows, int64_t cols, const char *what) {
    const GpuMat &m = mat_at(id);
    if (m.rows != rows || m.cols != cols) throw Fail(std::string("codec ") + what + " has the wrong shape");
    if (m.type != VOXHIP_F32 && m.type != VOXHIP_F16 && m.type != VOXHIP_BF16)
        throw Fail(std::string("codec ") + what + ": f32 / f16 / bf16 weights only");
}

Hist2 hist_new(int rows, int C) {
    Hist2 h;
    h.rows = rows; h.C = C;
    for (float *&b : h.b) {
        b = dalloc_t<float>(size_t(std::max(rows, 1)) * size_t(C));
        HIPCHECK(hipMemset(b, 0, size_t(std::max(rows, 1)) * size_t(C) * 4));
    }
    return h;
}
Hist2 hist_clone(const Hist2 &src, int parity) {  // the current buffer into b[0] of a state of parity 0
    Hist2 h = hist_new(src.rows, src.C);
    HIPCHECK(hipMemcpy(h.b[0], src.b[parity], size_t(std::max(src.rows, 1)) * size_t(src.C) * 4, hipMemcpyDeviceToDevice));
    return h;
}
void hist_free(Hist2 &h) {
    for (float *&b : h.b) { dfree(b); b = nullptr; }
}

// A streaming convolution of T rows X (row stride ldx) into Y (row stride ldy): the conv GEMM over [hist; X]; the same
// launch moves the history on (into the other buffer).
// snake: Snake applied in the epilogue (the output then holds Snake(conv(.)), as the residual units consume it).
void codec_conv(const CodecConv &c, Hist2 *h, int par, const float *X, int64_t ldx, int T, float *Y, int64_t ldy, hipStream_t s,
                const CodecSnake *snake = nullptr) {
    const GpuMat &M = mat_at(c.mat);
    GemmArgs ga{};
    if (snake) { ga.snake_a = snake->a; ga.snake_ib = snake->inv_b; }
    ga.bias = M.b; ga.y = Y; ga.lda = ldx; ga.ldy = ldy; ga.m = T; ga.n = c.cout; ga.K = c.K * c.cin;
    ga.cig = c.cin; ga.ksize = c.K; ga.dil = c.dil; ga.ctx = (c.K - 1) * c.dil; ga.hist = h ? h->b[par] : nullptr;
    ga.ws = g.gemm_ws; ga.ws_cap = kGemmWsFloats;
    if (ga.ctx && !h) throw Fail("codec convolution without its history");
    if (ga.ctx) ga.hist_next = h->b[1 - par];
    ga.f32_wide = f32_wide(M);
    HIPCHECK(launch_stream_conv(gemv_type(M), snake ? EPI_SNAKE : EPI_STORE, M.w, M.s, X, ga, s));
}
// y (=, +=, gelu, gamma-gated +=) W x + bias over rows of the f32-activation GEMM (the f32 tile semantics of matmul
// for F32 / F16 / BF16 weights at any row count).
// snake / snake_y (EPI_ACC_SNAKE): Snake of the updated rows into snake_y as well.
void codec_gemm(int mat, int epi, const float *A, int64_t lda, int64_t rows, float *Y, int64_t ldy, const float *gate,
                hipStream_t s, const CodecSnake *snake = nullptr, float *snake_y = nullptr) {
    const GpuMat &M = mat_at(mat);
    GemmArgs ga = gemm_args(M, M.b, Y, lda, ldy, rows);
    ga.gate = gate;
    if (snake) { ga.snake_a = snake->a; ga.snake_ib = snake->inv_b; ga.snake_y = snake_y; }
    HIPCHECK(launch_gemm(gemv_type(M), epi, M.w, M.s, A, ga, s));
}

// gpu_codec_forward's chain for T <= kCodecMaxFrames frames of z already on the device (E.z) and their RoPE rows
// (E.rope); returns the sample count, left in E.S[4].
int64_t codec_enqueue(Codec &E, CodecSt &St, int T, hipStream_t s) {
    Xfmr &X = xf_at(E.xf);
    const int L = E.latent, H = E.H, qd = E.heads * E.hd, QW = (E.heads + 2 * E.kvh) * E.hd, par = St.parity;
    float *A = E.S[0], *B = E.S[1];
    // 1) pre_conv -> A [T][latent]; 2) the pre-transformer (kernels.cpp:760-844 with window and layer scales)
    codec_conv(E.pre_conv, &St.pre, par, E.z, E.cdim, T, A, L, s);
    gemv(mat_at(E.pt_in), T, PRO_X, EPI_STORE, A, L, T, E.h, H, nullptr, 0.f, nullptr, s);
    const float scale = 1.0f / std::sqrt(float(E.hd));
    for (int li = 0; li < E.layers; ++li) {
        const LayerDev &d = X.L[size_t(li)];
        gemv(mat_at(d.qkv), T, PRO_RMS, EPI_STORE, E.h, H, T, E.qkv, QW, X.norms + d.ln1, E.eps, nullptr, s, nullptr, E.pre);
        HIPCHECK(launch_codec_rope_ring(E.qkv, QW, T, E.heads, E.kvh, E.hd, E.rope, St.kr[size_t(li)], St.vr[size_t(li)], E.R,
                                        St.pos_dev, s));
        HIPCHECK(launch_codec_attn(E.qkv, QW, St.kr[size_t(li)], St.vr[size_t(li)], E.R, T, E.heads, E.kvh, E.hd, St.pos_dev, E.W,
                                   scale, E.ao, s));
        // the layer scales (null: none) ride on the residual epilogue: h += scale (W x + b)
        gemv(mat_at(d.o), T, PRO_X, EPI_ACC, E.ao, qd, T, E.h, H, nullptr, 0.f, nullptr, s, nullptr, nullptr, nullptr, nullptr,
             nullptr, E.sa[size_t(li)]);
        gemv(mat_at(d.gu), T, PRO_RMS, EPI_SWIGLU, E.h, H, T, E.act, E.I, X.norms + d.ln2, E.eps, nullptr, s, nullptr, E.pre);
        gemv(mat_at(d.down), T, PRO_X, EPI_ACC, E.act, E.I, T, E.h, H, nullptr, 0.f, nullptr, s, nullptr, nullptr, nullptr, nullptr,
             nullptr, E.sm[size_t(li)]);
    }
    gemv(mat_at(E.pt_out), T, PRO_RMS, EPI_STORE, E.h, H, T, A, L, X.norms + X.final_off, E.eps, nullptr, s, nullptr, E.pre);
    // 3) upsample stages: transposed conv (K = stride: the overlap-add has no tail) + ConvNeXt
    int64_t len = T;
    float *cur = A;
    for (size_t si = 0; si < E.ups.size(); ++si) {
        const CodecUp &U = E.ups[si];
        float *y = cur == A ? B : A;
        codec_gemm(U.tr, EPI_STORE, cur, L, len, E.S[2], int64_t(U.K) * L, nullptr, s);
        HIPCHECK(launch_ola(E.S[2], nullptr, nullptr, U.tr_b, y, int(len), U.K, U.K, L, s));
        len *= U.K;
        Hist2 &hd = St.dw[si];
        HIPCHECK(launch_dwconv_causal(y, hd.b[par], U.dw_w, U.dw_b, E.S[2], int(len), L, U.dwK, s, U.dwK > 1 ? hd.b[1 - par] : nullptr));
        HIPCHECK(launch_layernorm_rows(E.S[2], len, L, U.ln_w, U.ln_b, E.S[3], s));
        codec_gemm(U.pw1, EPI_GELU_ERF, E.S[3], L, len, E.S[4], 4 * int64_t(L), nullptr, s);
        codec_gemm(U.pw2, EPI_GATED_ACC, E.S[4], 4 * int64_t(L), len, y, L, U.gamma, s);
        cur = y;
    }
    // 4) conv0 -> blocks -> Snake -> final conv -> clamp. Every Snake rides on the launch that produces its input
    // (the same float in, the same formula): conv0's epilogue gives the first block's Snake(x) (x itself is not read
    // again), the overlap-add gives each block's first unit its input as well as y, and each unit's residual product
    // (EPI_ACC_SNAKE) the next unit's, the next block's or the final one's.
    float *sa = cur == A ? B : A;  // the Snake of the rows the next product reads
    float *x = cur;                // consumed by conv0: the blocks' rows y go here
    auto next_act = [&](size_t bi) -> const CodecSnake & { return bi < E.blocks.size() ? E.blocks[bi].act : E.fin_act; };
    codec_conv(E.conv0, &St.c0, par, cur, L, int(len), sa, E.dec, s, &next_act(0));
    int ch = E.dec;
    for (size_t bi = 0; bi < E.blocks.size(); ++bi) {
        const CodecBlk &Bk = E.blocks[bi];
        codec_gemm(Bk.tr, EPI_STORE, sa, ch, len, E.S[2], int64_t(Bk.K) * Bk.cout, nullptr, s);
        float *y = x;  // x is consumed
        Hist2 &tl = St.tail[bi];
        HIPCHECK(launch_ola(E.S[2], tl.b[par], tl.b[1 - par], Bk.tr_b, y, int(len), Bk.s, Bk.K, Bk.cout, s, sa, Bk.a1[0].a,
                            Bk.a1[0].inv_b));
        len *= Bk.s;
        ch = Bk.cout;
        for (int u = 0; u < 3; ++u) {
            codec_conv(Bk.c1[u], &St.ru[bi * 3 + size_t(u)], par, sa, ch, int(len), E.S[3], ch, s, &Bk.a2[u]);  // + Snake a2
            const CodecSnake &nx = u < 2 ? Bk.a1[u + 1] : next_act(bi + 1);
            codec_gemm(Bk.c2[u].mat, EPI_ACC_SNAKE, E.S[3], ch, len, y, ch, nullptr, s, &nx, sa);
        }
        x = y;
    }
    codec_conv(E.fin, &St.fin, par, sa, ch, int(len), E.S[4], 1, s);
    HIPCHECK(launch_clamp1(E.S[4], len, s));
    return len;
}
}  // namespace

namespace {
// The object that keeps device pointers into matrix `mat` (a transformer layer, an F5 / estimator / codec instance,
// whose launches or captured graphs read it), or null when none does.
const char *mat_user(int mat) {
    for (const Xfmr *X : g.xf)
        if (X)
            for (const LayerDev &L : X->L)
                if (L.qkv == mat || L.o == mat || L.gu == mat || L.down == mat) return "a transformer";
    for (const F5 *F : g.f5) {
        if (!F) continue;
        if (F->in_proj == mat || F->norm_out == mat || F->proj_out == mat || F->v_head == mat || F->ada_all == mat)
            return "an F5 model";
        for (const F5Block &b : F->blocks)
            if (b.ada == mat || b.qkv == mat || b.o == mat || b.ff1 == mat || b.ff2 == mat) return "an F5 model";
        for (const F5VBlock &b : F->vblocks)
            if (b.pw1 == mat || b.pw2 == mat) return "an F5 model";
    }
    for (const Cosy *E : g.cosy) {
        if (!E) continue;
        for (const auto *xs : {&E->down_x, &E->up_x})
            for (const CosyX &x : *xs)
                if (x.qkv == mat || x.o == mat || x.ff1 == mat || x.ff2 == mat) return "a flow estimator";
        for (const auto &xs : E->mid_x)
            for (const CosyX &x : xs)
                if (x.qkv == mat || x.o == mat || x.ff1 == mat || x.ff2 == mat) return "a flow estimator";
    }
    for (const Codec *C : g.codecs) {
        if (!C) continue;
        if (C->pre_conv.mat == mat || C->conv0.mat == mat || C->fin.mat == mat || C->pt_in == mat || C->pt_out == mat)
            return "a codec decoder";
        for (const CodecUp &u : C->ups)
            if (u.tr == mat || u.pw1 == mat || u.pw2 == mat) return "a codec decoder";
        for (const CodecBlk &b : C->blocks) {
            if (b.tr == mat) return "a codec decoder";
            for (int i = 0; i < 3; ++i)
                if (b.c1[i].mat == mat || b.c2[i].mat == mat) return "a codec decoder";
        }
    }
    return nullptr;
}
}  // namespace

extern "C" {

int voxhip_codec_create(const voxhip_codec_desc *d) {
    return guard_int([&] {
        require_ok();
        if (!d || !d->pt_mats || d->pt.n_layers <= 0 || (d->n_ups && !d->ups) || (d->n_blocks && !d->blocks) || d->n_ups < 0 ||
            d->n_blocks < 0)
            throw Fail("incomplete codec description");
        const voxhip_xfmr_desc &pt = d->pt;
        if (pt.window <= 0 || pt.window > 1024 || pt.head_dim <= 0 || pt.head_dim > 128 || pt.head_dim % 2)
            throw Fail("codec transformer: window 1..1024, even head_dim <= 128");
        for (int li = 0; li < pt.n_layers; ++li) {
            const voxhip_layer &L = pt.layers[li];
            if (L.qn || L.kn) throw Fail("codec transformer with q / k norm is not supported");
            for (int j = 0; j < 7; ++j)
                if (mat_at(d->pt_mats[li * 7 + j]).b) throw Fail("codec transformer with biased projections is not supported");
        }
        std::unique_ptr<Codec> E(new Codec());
        E->cdim = d->codebook_dim; E->latent = d->latent; E->H = pt.hidden; E->heads = pt.heads; E->kvh = pt.kv_heads;
        E->hd = pt.head_dim; E->I = pt.inter; E->W = pt.window; E->R = pt.window + kCodecMaxFrames; E->layers = pt.n_layers;
        E->eps = pt.eps;
        E->inv_freq.assign(pt.inv_freq, pt.inv_freq + pt.head_dim / 2);
        if (E->cdim <= 0 || E->cdim % 4 || E->latent <= 0 || E->latent % 4) throw Fail("codec: codebook_dim and latent multiples of 4");
        E->xf = make_xfmr(&pt, "codec", -1, d->pt_mats, nullptr, nullptr, true);
        for (int li = 0; li < pt.n_layers; ++li) {
            const voxhip_layer &L = pt.layers[li];
            E->sa.push_back(L.attn_scale ? upload_vec(L.attn_scale, pt.hidden, "attn scale") : nullptr);
            E->sm.push_back(L.mlp_scale ? upload_vec(L.mlp_scale, pt.hidden, "mlp scale") : nullptr);
        }
        E->pre_conv = codec_conv_up(d->pre_conv, "pre_conv");
        if (E->pre_conv.cin != E->cdim || E->pre_conv.cout != E->latent) throw Fail("codec pre_conv: codebook_dim -> latent");
        codec_check_mat(d->pt_in, pt.hidden, E->latent, "pre_transformer.input_proj");
        codec_check_mat(d->pt_out, E->latent, pt.hidden, "pre_transformer.output_proj");
        E->pt_in = d->pt_in; E->pt_out = d->pt_out;
        const int L = E->latent;
        int64_t len = kCodecMaxFrames, mx = int64_t(kCodecMaxFrames) * std::max({E->cdim, L, E->H, E->I});
        for (int i = 0; i < d->n_ups; ++i) {
            const voxhip_codec_up &u = d->ups[i];
            if (u.K <= 0 || u.dw_K <= 0) throw Fail("codec upsample stage: K and dw_K positive");
            codec_check_mat(u.tr, int64_t(u.K) * L, L, "upsample transposed conv");
            codec_check_mat(u.pw1, 4 * int64_t(L), L, "upsample pwconv1");
            codec_check_mat(u.pw2, L, 4 * int64_t(L), "upsample pwconv2");
            CodecUp U;
            U.tr = u.tr; U.K = u.K; U.pw1 = u.pw1; U.pw2 = u.pw2; U.dwK = u.dw_K;
            U.tr_b = upload_vec(u.tr_b, L, "upsample bias");
            U.dw_w = upload_vec(u.dw_w, L * u.dw_K, "depthwise weight");
            U.dw_b = upload_vec(u.dw_b, L, "depthwise bias");
            U.ln_w = upload_vec(u.ln_w, L, "norm weight");
            U.ln_b = upload_vec(u.ln_b, L, "norm bias");
            U.gamma = upload_vec(u.gamma, L, "gamma");
            E->ups.push_back(U);
            mx = std::max(mx, len * u.K * L);
            len *= u.K;
            mx = std::max(mx, len * 4 * L);
        }
        E->conv0 = codec_conv_up(d->conv0, "conv0");
        if (E->conv0.cin != L) throw Fail("codec conv0: latent input");
        E->dec = E->conv0.cout;
        mx = std::max(mx, len * E->dec);
        int ch = E->dec;
        for (int b = 0; b < d->n_blocks; ++b) {
            const voxhip_codec_block &k = d->blocks[b];
            if (k.cin != ch || k.stride <= 0 || k.K < k.stride || k.K > 2 * k.stride || k.cout <= 0 || k.cout % 4)
                throw Fail("codec decoder block: cin = the previous width, stride < K <= 2 stride, cout a multiple of 4");
            codec_check_mat(k.tr, int64_t(k.K) * k.cout, k.cin, "decoder transposed conv");
            CodecBlk Bk;
            Bk.act = codec_snake_up(k.act, k.cin);
            Bk.tr = k.tr; Bk.K = k.K; Bk.s = k.stride; Bk.cin = k.cin; Bk.cout = k.cout;
            Bk.tr_b = upload_vec(k.tr_b, k.cout, "decoder transposed conv bias");
            for (int u = 0; u < 3; ++u) {
                Bk.a1[u] = codec_snake_up(k.a1[u], k.cout);
                Bk.a2[u] = codec_snake_up(k.a2[u], k.cout);
                Bk.c1[u] = codec_conv_up(k.c1[u], "residual conv 1");
                Bk.c2[u] = codec_conv_up(k.c2[u], "residual conv 2");
                if (Bk.c1[u].cin != k.cout || Bk.c1[u].cout != k.cout || Bk.c2[u].cin != k.cout || Bk.c2[u].cout != k.cout ||
                    Bk.c2[u].K != 1)
                    throw Fail("codec residual unit: cout -> cout, conv 2 with K 1");
            }
            E->blocks.push_back(Bk);
            mx = std::max(mx, len * k.K * k.cout);
            len *= k.stride;
            mx = std::max(mx, len * k.cout);
            ch = k.cout;
        }
        E->fin_act = codec_snake_up(d->final_act, ch);
        E->fin = codec_conv_up(d->final_conv, "final conv");
        if (E->fin.cin != ch || E->fin.cout != 1) throw Fail("codec final conv: the last width -> 1");
        E->spf = int(len / kCodecMaxFrames);
        E->smax = mx;
        for (float *&p : E->S) p = dalloc_t<float>(size_t(mx));
        const size_t F = kCodecMaxFrames;
        E->qkv = dalloc_t<float>(F * size_t((E->heads + 2 * E->kvh) * E->hd));
        E->ao = dalloc_t<float>(F * size_t(E->heads * E->hd));
        E->act = dalloc_t<float>(F * size_t(E->I));
        E->tmp = dalloc_t<float>(F * size_t(E->H));
        E->h = dalloc_t<float>(F * size_t(E->H));
        E->pre = dalloc_t<float>(F * size_t(std::max(E->H, E->I)));
        E->rope = dalloc_t<float>(F * size_t(E->hd));
        E->z = dalloc_t<float>(F * size_t(E->cdim));
        g.codecs.push_back(E.release());
        return int(g.codecs.size()) - 1;
    }, -1);
}

int voxhip_codec_spf(int codec, int32_t *spf) {
    return guard_int([&] {
        require_ok();
        if (!spf) throw Fail("missing argument");
        *spf = codec_at(codec).spf;
        return 1;
    }, 0);
}

int voxhip_codec_state_new(int codec) {
    return guard_int([&] {
        require_ok();
        const Codec &E = codec_at(codec);
        std::unique_ptr<CodecSt> S(new CodecSt());
        S->codec = codec;
        S->pre = hist_new((E.pre_conv.K - 1) * E.pre_conv.dil, E.pre_conv.cin);
        const size_t kd = size_t(E.kvh) * E.hd;
        for (int l = 0; l < E.layers; ++l) {
            S->kr.push_back(dalloc_t<float>(size_t(E.R) * kd));
            S->vr.push_back(dalloc_t<float>(size_t(E.R) * kd));
            HIPCHECK(hipMemset(S->kr.back(), 0, size_t(E.R) * kd * 4));
            HIPCHECK(hipMemset(S->vr.back(), 0, size_t(E.R) * kd * 4));
        }
        for (const CodecUp &u : E.ups) S->dw.push_back(hist_new(u.dwK - 1, E.latent));
        S->c0 = hist_new((E.conv0.K - 1) * E.conv0.dil, E.conv0.cin);
        for (const CodecBlk &b : E.blocks) {
            S->tail.push_back(hist_new(b.K - b.s, b.cout));
            for (int u = 0; u < 3; ++u) S->ru.push_back(hist_new((b.c1[u].K - 1) * b.c1[u].dil, b.c1[u].cin));
        }
        S->fin = hist_new((E.fin.K - 1) * E.fin.dil, E.fin.cin);
        S->pos_dev = static_cast<int64_t *>(dalloc(sizeof(int64_t)));
        g.cstates.push_back(S.release());
        return int(g.cstates.size()) - 1;
    }, -1);
}

int voxhip_codec_state_clone(int state) {
    return guard_int([&] {
        require_ok();
        HIPCHECK(hipStreamSynchronize(g.stream));
        const CodecSt &src = cstate_at(state);
        const Codec &E = codec_at(src.codec);
        std::unique_ptr<CodecSt> S(new CodecSt());
        S->codec = src.codec;
        S->len = src.len;
        const int par = src.parity;
        S->pre = hist_clone(src.pre, par);
        S->c0 = hist_clone(src.c0, par);
        S->fin = hist_clone(src.fin, par);
        for (const Hist2 &h : src.dw) S->dw.push_back(hist_clone(h, par));
        for (const Hist2 &h : src.tail) S->tail.push_back(hist_clone(h, par));
        for (const Hist2 &h : src.ru) S->ru.push_back(hist_clone(h, par));
        S->pos_dev = static_cast<int64_t *>(dalloc(sizeof(int64_t)));
        const size_t kd = size_t(E.kvh) * E.hd;
        for (size_t l = 0; l < src.kr.size(); ++l) {
            S->kr.push_back(dalloc_t<float>(size_t(E.R) * kd));
            S->vr.push_back(dalloc_t<float>(size_t(E.R) * kd));
            HIPCHECK(hipMemcpy(S->kr.back(), src.kr[l], size_t(E.R) * kd * 4, hipMemcpyDeviceToDevice));
            HIPCHECK(hipMemcpy(S->vr.back(), src.vr[l], size_t(E.R) * kd * 4, hipMemcpyDeviceToDevice));
        }
        g.cstates.push_back(S.release());
        return int(g.cstates.size()) - 1;
    }, -1);
}

int voxhip_codec_state_free(int state) {
    return guard_int([&] {
        require_ok();
        CodecSt &S = cstate_at(state);
        HIPCHECK(hipStreamSynchronize(g.stream));
        for (Hist2 *h : {&S.pre, &S.c0, &S.fin}) hist_free(*h);
        for (auto *v : {&S.dw, &S.tail, &S.ru})
            for (Hist2 &h : *v) hist_free(h);
        for (float *p : S.kr) dfree(p);
        for (float *p : S.vr) dfree(p);
        dfree(S.pos_dev);
        for (auto &kv : S.graphs) (void)hipGraphExecDestroy(kv.second);
        delete g.cstates[size_t(state)];
        g.cstates[size_t(state)] = nullptr;
        return 1;
    }, 0);
}

int voxhip_codec_forward(int codec, int state, const float *z, int F, float *pcm, int64_t *n_out) {
    return guard_int([&] {
        require_ok();
        Codec &E = codec_at(codec);
        CodecSt &St = cstate_at(state);
        if (St.codec != codec) throw Fail("the codec state belongs to another codec");
        if (F <= 0 || F > kCodecMaxFrames) throw Fail("codec forward: 1 to 16 frames per call");
        if (!z || !pcm) throw Fail("missing argument");
        // the RoPE rows of positions len .. len + F - 1 on the host, as rope_apply takes them (kernels.cpp:744-747)
        const int half = E.hd / 2;
        std::vector<float> cs(size_t(F) * size_t(E.hd));
        for (int i = 0; i < F; ++i)
            for (int p = 0; p < half; ++p) {
                const float f = E.inv_freq[size_t(p)] * float(St.len + i);
                cs[size_t(i * E.hd + 2 * p)] = std::cos(f);
                cs[size_t(i * E.hd + 2 * p + 1)] = std::sin(f);
            }
        h2d(E.z, z, size_t(F) * size_t(E.cdim) * 4);
        h2d(E.rope, cs.data(), cs.size() * 4);
        h2d(St.pos_dev, &St.len, sizeof(int64_t));
        // the call's ~150 launches as one graph per (F, parity): the buffers, the weights and the scratch are fixed,
        // the position comes from pos_dev
        const int key = 2 * F + St.parity;
        vh::prof_stage("codec");
        auto it = St.graphs.find(key);
        if (vh::prof_on()) {
            codec_enqueue(E, St, F, g.stream);  // stamped launches are not captured
        } else if (it == St.graphs.end()) {
            hipGraph_t graph = nullptr;
            HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
            try {
                codec_enqueue(E, St, F, g.stream);
            } catch (...) {
                (void)hipStreamEndCapture(g.stream, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                throw;
            }
            HIPCHECK(hipStreamEndCapture(g.stream, &graph));
            hipGraphExec_t exec = nullptr;
            hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            HIPCHECK(e);
            it = St.graphs.emplace(key, exec).first;
        }
        if (!vh::prof_on()) HIPCHECK(hipGraphLaunch(it->second, g.stream));
        sync_status();  // a failure leaves the state as it was (its parity and length unchanged)
        const int64_t n = int64_t(F) * E.spf;
        HIPCHECK(copy_d2h(pcm, E.S[4], size_t(n) * 4, nullptr));
        St.len += F;
        St.parity ^= 1;
        if (n_out) *n_out = n;
        return 1;
    }, 0);
}

int voxhip_mat_synthetic(int32_t type, int64_t rows, int64_t cols, uint64_t seed, uint32_t stream, float mean, float std,
                         int flags) {
    return guard_int([&] {
        require_ok();
        check_shape(type, rows, cols);
        const bool with_bias = (flags & VOXHIP_SYN_BIAS) != 0, s16 = (flags & VOXHIP_SYN_F16_SCALES) && type == VOXHIP_Q4;
        const int id = new_mat(type, rows, cols, with_bias, s16);
        GpuMat &m = g.mats[size_t(id)];
        const size_t n = size_t(rows) * size_t(cols), nsc = quantized(type) ? n / 32 : 0;
        float *tmp = type == VOXHIP_F32 ? reinterpret_cast<float *>(m.w) : dalloc_t<float>(n);
        float *sc32 = nullptr;
        auto release = [&] {
            if (tmp != reinterpret_cast<float *>(m.w)) dfree(tmp);
            dfree(sc32);
        };
        try {
            float *sdst = m.s;
            if (s16) sdst = sc32 = dalloc_t<float>(nsc);  // quantize with f32 scales, then round them to f16
            HIPCHECK(launch_fill_normal(tmp, int64_t(n), seed, stream, mean, std, g.stream));
            switch (type) {
                case VOXHIP_Q8: HIPCHECK(launch_quant_q8(tmp, int64_t(n / 32), reinterpret_cast<int8_t *>(m.w), sdst, g.stream)); break;
                case VOXHIP_Q4: HIPCHECK(launch_quant_q4(tmp, int64_t(n / 32), m.w, sdst, g.stream)); break;
                case VOXHIP_F16: HIPCHECK(launch_to_f16(tmp, int64_t(n), m.w, g.stream)); break;
                case VOXHIP_BF16: HIPCHECK(launch_to_bf16(tmp, int64_t(n), m.w, g.stream)); break;
                default: break;
            }
            if (s16) HIPCHECK(launch_to_f16(sc32, int64_t(nsc), m.s, g.stream));
            if (with_bias) HIPCHECK(launch_fill_normal(m.b, rows, seed, stream + 0x10000u, 0.f, std, g.stream));
            if (type == VOXHIP_F32) {  // max |w|, in word 1 of the status block
                uint32_t *mx = reinterpret_cast<uint32_t *>(g.status_dev + 1);
                HIPCHECK(hipMemsetAsync(mx, 0, 4, g.stream));
                HIPCHECK(launch_absmax(tmp, int64_t(n), mx, g.stream));
                HIPCHECK(copy_d2h(g.status_pin + 1, mx, 4, g.stream));
            }
            HIPCHECK(hipStreamSynchronize(g.stream));
            if (type == VOXHIP_F32) m.wmax = __builtin_bit_cast(float, uint32_t(g.status_pin[1]));
        } catch (...) {
            release();
            throw;
        }
        release();
        g.stats.mats_ok += 1;
        g.stats.bytes += m.bytes;
        return id;
    }, -1);
}

int voxhip_mat_download(int mat, void *data, float *scale, float *bias) {
    return guard_int([&] {
        require_ok();
        const GpuMat &m = mat_at(mat);
        HIPCHECK(hipStreamSynchronize(g.stream));
        if (data) HIPCHECK(copy_d2h(data, m.w, size_t(m.rows) * row_bytes(m.type, m.cols), nullptr));
        if (scale && m.s) {
            const size_t nsc = size_t(m.rows) * size_t(m.cols / 32);
            if (m.s16) {  // widened exactly to the f32 scales the matrix stands for
                std::vector<_Float16> t(nsc);
                HIPCHECK(copy_d2h(t.data(), m.s, nsc * 2, nullptr));
                for (size_t i = 0; i < nsc; ++i) scale[i] = float(t[i]);
            } else {
                HIPCHECK(copy_d2h(scale, m.s, nsc * 4, nullptr));
            }
        }
        if (bias && m.b) HIPCHECK(copy_d2h(bias, m.b, size_t(m.rows) * 4, nullptr));
        return 1;
    }, 0);
}

int voxhip_mat_free(int mat) {
    return guard_int([&] {
        require_ok();
        mat_at(mat);
        HIPCHECK(hipStreamSynchronize(g.stream));
        const char *user = mat_user(mat);
        if (user) throw Fail(std::string("matrix is used by ") + user);
        // decode, generation and frame graphs captured a head, embedding or input projection by address
        for (Xfmr *X : g.xf)
            if (X) drop_graphs(*X);
        free_mat(mat);
        return 1;
    }, 0);
}

int voxhip_seq_fill_synthetic(int seq, int64_t len, uint64_t seed, uint32_t stream, float mean, float std) {
    return guard_int([&] {
        require_ok();
        Seq &S = seq_at(seq);
        if (len < 0 || len > S.cap) throw Fail("fill length exceeds the capacity");
        const int64_t planes = int64_t(S.layers) * S.kvh;
        HIPCHECK(launch_fill_cache(S.k, planes, S.cap, len, S.hd, seed, stream, mean, std, g.stream));
        HIPCHECK(launch_fill_cache(S.v, planes, S.cap, len, S.hd, seed, stream + 1, mean, std, g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
        return 1;
    }, 0);
}

int voxhip_seq_download(int seq, int32_t layer, int64_t len, float *k, float *v) {
    return guard_int([&] {
        require_ok();
        Seq &S = seq_at(seq);
        if (layer < 0 || layer >= S.layers || len < 0 || len > S.cap) throw Fail("bad layer or length");
        HIPCHECK(hipStreamSynchronize(g.stream));
        const size_t plane = size_t(S.cap) * S.hd;
        std::vector<_Float16> tk(static_cast<size_t>(S.kvh) * plane), tv(tk.size());
        HIPCHECK(copy_d2h(tk.data(), S.k + size_t(layer) * S.kvh * plane, tk.size() * 2, nullptr));
        HIPCHECK(copy_d2h(tv.data(), S.v + size_t(layer) * S.kvh * plane, tv.size() * 2, nullptr));
        const size_t kd = size_t(S.kvh) * S.hd;
        for (int64_t p = 0; p < len; ++p)
            for (int h = 0; h < S.kvh; ++h)
                for (int e = 0; e < S.hd; ++e) {
                    const size_t src = size_t(h) * plane + size_t(p) * S.hd + size_t(e), dst = size_t(p) * kd + size_t(h) * S.hd + size_t(e);
                    if (k) k[dst] = float(tk[src]);
                    if (v) v[dst] = float(tv[src]);
                }
        return 1;
    }, 0);
}

int voxhip_quantize_q8_dev(const float *d_w, int64_t rows, int64_t cols, int8_t *d_q, float *d_scale) {
    return guard_int([&] {
        require_ok();
        if (cols % 32) throw Fail("cols % 32 != 0");
        HIPCHECK(launch_quant_q8(d_w, rows * (cols / 32), d_q, d_scale, g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
        return 1;
    }, 0);
}
int voxhip_quantize_q4_dev(const float *d_w, int64_t rows, int64_t cols, uint8_t *d_q, float *d_scale) {
    return guard_int([&] {
        require_ok();
        if (cols % 32) throw Fail("cols % 32 != 0");
        HIPCHECK(launch_quant_q4(d_w, rows * (cols / 32), d_q, d_scale, g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
        return 1;
    }, 0);
}
int voxhip_quantize_act_dev(const float *d_x, int64_t n, int8_t *d_xq, float *d_xs) {
    return guard_int([&] {
        require_ok();
        if (n % 32) throw Fail("n % 32 != 0");
        HIPCHECK(launch_quant_act(d_x, n / 32, d_xq, d_xs, g.stream));
        HIPCHECK(hipStreamSynchronize(g.stream));
        return 1;
    }, 0);
}

}  // extern "C"

namespace {
// rocprofv3 preloads its tool library; kernel-stamped events (hipExtLaunchKernel) are not used under it.
bool profiler_attached() {
    const char *pre = std::getenv("LD_PRELOAD");
    if (pre && std::strstr(pre, "rocprof")) return true;
    return std::getenv("ROCPROF_OUTPUT_PATH") || std::getenv("ROCP_TOOL_LIBRARIES") || std::getenv("ROCPROFILER_LIBRARY_CTOR");
}
}  // namespace

extern "C" {

}  // extern "C"

namespace {
// How long the kernel-by-kernel pass holds the stream before each step's launches: at first kBenchHoldUs, then 1.5x
// the longest host enqueue of a step so far (stamped launches take the host about 10 us each: 1.5 ms for the 142 of
// a 28-layer step), so every step after the first is enqueued whole before its first kernel runs.
constexpr double kBenchHoldUs = 2000.0;

// The decode benchmark for m rows: of one sequence at pos[0] .. (steps_mode false, m = 1 here), or one row of each of
// m sequences at pos[i] (steps_mode true). Region A times the captured graph's replays; region B launches the same
// kernels one by one, each stamped by its own events, for per-class durations and algorithmic bytes.
void bench_decode_impl(Xfmr &X, const std::array<int, 8> &key, int m, bool steps_mode, const std::vector<int64_t> &pos,
                       const float *dx, int head, bool sample, int32_t *d_token, int warmup, int steps, voxhip_bench_result *out) {
    std::memset(out, 0, sizeof *out);
    const bool trace = std::getenv("VOXHIP_TRACE") != nullptr;
    auto mark = [&](const char *what) {
        if (trace) std::fprintf(stderr, "[voxhip bench] %s\n", what);
    };
    std::vector<hipEvent_t> ev;
    auto cleanup = [&] {
        (void)hipStreamSynchronize(g.stream);
        timing_clear();
        for (auto &e : ev) (void)hipEventDestroy(e);
    };
    try {
        // ---- region A: graph replays (the same graph voxhip_decode_dev / _steps_dev replays for these arguments)
        mark("graph");
        hipGraphExec_t exec = decode_graph(X, key, m, steps_mode, head, dx, nullptr, nullptr, sample, d_token);
        for (int i = 0; i < warmup; ++i) HIPCHECK(hipGraphLaunch(exec, g.stream));
        // under a profiler the replays are timed by the host clock around a synchronized stream: the tracer does
        // not survive events recorded around graph launches
        const bool prof = profiler_attached();
        ev.resize(2);
        for (auto &e : ev) HIPCHECK(hipEventCreate(&e));
        HIPCHECK(hipStreamSynchronize(g.stream));
        if (!prof) HIPCHECK(hipEventRecord(ev[0], g.stream));
        const auto h0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; ++i) HIPCHECK(hipGraphLaunch(exec, g.stream));
        const auto h1 = std::chrono::steady_clock::now();
        float ms = 0.f;
        if (!prof) {
            HIPCHECK(hipEventRecord(ev[1], g.stream));
            HIPCHECK(hipEventSynchronize(ev[1]));
            HIPCHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        } else {
            HIPCHECK(hipStreamSynchronize(g.stream));
            ms = float(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - h0).count());
        }
        out->ms_per_step = double(ms) / steps;
        out->launch_ms_per_step = std::chrono::duration<double, std::milli>(h1 - h0).count() / steps;
        mark("kernel by kernel");
        // ---- region B: the same step launched kernel by kernel (same enqueue path as the graph), each launch
        // stamped by its own events: hipExtLaunchKernel start/stop, or plain stream events around the launch
        // when a profiler intercepts launches
        for (auto &e : ev) (void)hipEventDestroy(e);
        ev.clear();
        struct Stamps : Probe {
            std::vector<hipEvent_t> *ev;
            std::vector<int> cls;
            bool stamp;
            hipStream_t s;
            int k = 0, open = -1;
            void before(int c) override {
                while (ev->size() < size_t(2 * k + 2)) {
                    hipEvent_t e = nullptr;
                    HIPCHECK(hipEventCreate(&e));
                    ev->push_back(e);
                }
                if (cls.size() <= size_t(k)) cls.resize(size_t(k) + 1);
                cls[size_t(k)] = c;
                open = c;
                if (stamp) timing_arm((*ev)[size_t(2 * k)], (*ev)[size_t(2 * k + 1)]);
                else HIPCHECK(hipEventRecord((*ev)[size_t(2 * k)], s));
            }
            void after() override {
                if (!stamp) HIPCHECK(hipEventRecord((*ev)[size_t(2 * k + 1)], s));
                ++k;
            }
            void split(int done) override {
                const int c = open;
                cls[size_t(k)] = done;
                after();
                before(c);
            }
        };
        const bool stamp = !profiler_attached();
        Stamps st;
        st.ev = &ev; st.stamp = stamp; st.s = g.stream;
        double sum_ms[VOXHIP_K_CLASSES] = {0};
        int cnt[VOXHIP_K_CLASSES] = {0};
        int per_step = -1;
        double enq_us = 0.0;  // the longest host enqueue of a step so far
        int short_holds = 0;  // timed steps whose enqueue outlasted their hold
        for (int it = 0; it < warmup + steps; ++it) {
            st.k = 0;
            // the stream is held while the host enqueues the step, so its kernels run back to back as in the graph
            // (without the hold each kernel waited for the host's next launch, and the durations moved with the host)
            const double hold = std::min(1e5, std::max(kBenchHoldUs, 1.5 * enq_us));
            HIPCHECK(launch_hold(hold, g.stream));
            const auto e0 = std::chrono::steady_clock::now();
            enqueue_decode(X, m, head, dx, nullptr, nullptr, sample, d_token, g.stream, &st, steps_mode);
            const double enq = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - e0).count();
            if (it >= warmup && enq > hold) ++short_holds;
            enq_us = std::max(enq_us, enq);
            HIPCHECK(hipStreamSynchronize(g.stream));
            if (per_step < 0) per_step = st.k;
            if (st.k != per_step) throw Fail("bench launch count mismatch");
            if (it < warmup) continue;
            for (int i = 0; i < st.k; ++i) {
                float t = 0.f;
                HIPCHECK(hipEventElapsedTime(&t, ev[size_t(2 * i)], ev[size_t(2 * i + 1)]));
                sum_ms[st.cls[size_t(i)]] += t;
                cnt[st.cls[size_t(i)]] += 1;
            }
        }
        if (short_holds)  // the last launches of those steps still waited for the host
            std::fprintf(stderr, "[voxhip bench] %d of %d timed steps took the host longer to enqueue than their hold\n",
                         short_holds, steps);
        if (trace) std::fprintf(stderr, "[voxhip bench] longest host enqueue of a step: %.0f us\n", enq_us);
        const int nl = X.layers;
        // ---- algorithmic bytes per launch of each class: every byte the kernel must move once
        // (weights + scales + bias, every row's activations in and out, cache reads and appends, attention partials)
        const int qd = X.heads * X.hd, kd = X.kvh * X.hd;
        const double partials = double(X.heads) * kAttnMaxSplits * (X.hd + 2) * 4.0;
        double bytes[VOXHIP_K_CLASSES] = {0};
        for (const LayerDev &L : X.L) {
            bytes[VOXHIP_K_QKV] += double(g.mats[size_t(L.qkv)].bytes) + m * (X.H * 4.0 + (qd + 2.0 * kd) * 4.0);
            bytes[VOXHIP_K_O] += double(g.mats[size_t(L.o)].bytes) + m * (partials + 2.0 * X.H * 4.0);
            bytes[VOXHIP_K_GATEUP] += double(g.mats[size_t(L.gu)].bytes) + m * (X.H * 4.0 + X.I * 4.0);
            bytes[VOXHIP_K_DOWN] += double(g.mats[size_t(L.down)].bytes) + m * (X.I * 4.0 + 2.0 * X.H * 4.0);
            // fused FFN: both matrices, the input row in, the down product out
            bytes[VOXHIP_K_FFN] += double(g.mats[size_t(L.gu)].bytes) + double(g.mats[size_t(L.down)].bytes) + 2.0 * X.H * 4.0;
        }
        for (int c = 0; c < 4; ++c) bytes[c] /= nl;
        bytes[VOXHIP_K_FFN] /= nl;
        bytes[VOXHIP_K_FOLD] = X.H * (2.0 * 4.0 + 2.0 * kAccCopies * 8.0);
        // quantized input rows, averaged over a layer's four (K = H, heads x hd, H, I): f32 rows in, int8 rows, block
        // scales and sums out
        bytes[VOXHIP_K_QUANT] = m * (2.0 * X.H + qd + X.I) / 4.0 * (4.0 + 1.0 + 8.0 / 32.0);
        for (int i = 0; i < m; ++i)  // one launch covers every row: each row's cache, q|k|v row, appended K/V, partials
            bytes[VOXHIP_K_ATTN] += 2.0 * double(pos[size_t(i)]) * kd * 2.0 + (qd + 2.0 * kd) * 4.0 + 2.0 * kd * 2.0 + partials;
        const int mr = steps_mode ? m : 1;  // rows through the head and the sampler
        if (head >= 0) {
            const GpuMat &Hm = g.mats[size_t(head)];
            bytes[VOXHIP_K_HEAD] = double(Hm.bytes) + mr * (X.H * 4.0 + double(Hm.rows) * 4.0);
            if (sample) bytes[VOXHIP_K_SAMPLE] = mr * double(Hm.rows) * 4.0;
        }
        double total_ms = 0.0, step_bytes = 0.0;
        for (int c = 0; c < VOXHIP_K_CLASSES; ++c) {
            out->class_launches[c] = steps > 0 ? cnt[c] / steps : 0;
            out->class_ms[c] = cnt[c] ? sum_ms[c] / cnt[c] : 0.0;
            out->class_bytes[c] = bytes[c];
            total_ms += sum_ms[c];
            step_bytes += bytes[c] * out->class_launches[c];
        }
        out->kernel_ms_per_step = total_ms / steps;
        out->step_bytes = step_bytes;
        out->kernels_per_step = per_step;
        out->n_classes = VOXHIP_K_CLASSES;
        out->kernel_stamped = stamp ? 1 : 0;
        mark("done");
    } catch (...) {
        cleanup();
        throw;
    }
    cleanup();
}
}  // namespace

extern "C" {

int voxhip_bench_decode(int xfmr, int seq, int64_t pos0, const float *d_x, int head, const voxhip_sample_cfg *cfg,
                        int32_t *d_token, int warmup, int steps, voxhip_bench_result *out) {
    return guard_int([&] {
        require_ok();
        if (vh::prof_on()) throw Fail("the benchmark entry points capture graphs, which VOX_PROFILE=gpu turns off");
        if (!out || steps <= 0 || !d_x) throw Fail("bad bench arguments");
        Xfmr &X = xf_at(xfmr);
        Seq &S = seq_at(seq);
        check_seq_for(X, xfmr, S);
        prepare_decode(X, S, pos0, 1, head, cfg);
        bench_decode_impl(X, one_seq(seq), 1, false, {pos0}, d_x, head, cfg != nullptr, d_token, warmup, steps, out);
        return 1;
    }, 0);
}

int voxhip_bench_decode_steps(int xfmr, const int32_t *seqs, const int64_t *pos, int64_t B, const float *d_x, int head,
                              const voxhip_sample_cfg *cfgs, int32_t *d_tokens, int warmup, int steps,
                              voxhip_bench_result *out) {
    return guard_int([&] {
        require_ok();
        if (vh::prof_on()) throw Fail("the benchmark entry points capture graphs, which VOX_PROFILE=gpu turns off");
        if (!out || steps <= 0 || !d_x || !seqs || !pos) throw Fail("bad bench arguments");
        Xfmr &X = xf_at(xfmr);
        if (B <= 0 || B > kMaxM) throw Fail("bench_decode_steps takes 1..8 sequences");
        std::array<int, 8> key;
        key.fill(-1);
        std::vector<RowRef> rr(static_cast<size_t>(B));
        std::vector<int64_t> ps(static_cast<size_t>(B));
        for (int64_t b = 0; b < B; ++b) {
            Seq &S = seq_at(seqs[b]);
            check_seq_for(X, xfmr, S);
            if (pos[b] < 0 || pos[b] + 1 > S.cap) throw Fail("context exceeds GPU KV capacity");
            for (int64_t c = 0; c < b; ++c)
                if (seqs[c] == seqs[b]) throw Fail("a sequence appears twice in one step");
            rr[size_t(b)] = row_of(S, pos[b]);
            ps[size_t(b)] = pos[b];
            key[size_t(b)] = seqs[b];
        }
        prepare_head(X, head, cfgs != nullptr);
        set_rows(X, rr);
        if (cfgs) set_sample_cfgs(X, cfgs, int(B));
        bench_decode_impl(X, key, int(B), true, ps, d_x, head, cfgs != nullptr, d_tokens, warmup, steps, out);
        return 1;
    }, 0);
}

int voxhip_bench_gemv_q8(int64_t rows, int64_t cols, int copies, int warmup, int iters, double *ms_per_launch) {
    return guard_int([&] {
        require_ok();
        if (vh::prof_on()) throw Fail("the benchmark entry points capture graphs, which VOX_PROFILE=gpu turns off");
        if (copies <= 0 || iters <= 0 || !ms_per_launch) throw Fail("bad bench arguments");
        check_shape(VOXHIP_Q8, rows, cols);
        std::vector<int> ids;
        float *x = nullptr, *y = nullptr, *gamma = nullptr;
        auto cleanup = [&] {
            (void)hipStreamSynchronize(g.stream);
            for (int id : ids) free_mat(id);
            dfree(x); dfree(y); dfree(gamma);
        };
        try {
            for (int c = 0; c < copies; ++c) {
                const int id = new_mat(VOXHIP_Q8, rows, cols, false);
                ids.push_back(id);
                GpuMat &m = g.mats[size_t(id)];
                float *tmp = dalloc_t<float>(size_t(rows) * size_t(cols));
                HIPCHECK(launch_fill_normal(tmp, rows * cols, 1000 + c, 0x51u, 0.f, 0.02f, g.stream));
                HIPCHECK(launch_quant_q8(tmp, rows * cols / 32, reinterpret_cast<int8_t *>(m.w), m.s, g.stream));
                HIPCHECK(hipStreamSynchronize(g.stream));
                dfree(tmp);
            }
            x = dalloc_t<float>(size_t(cols));
            y = dalloc_t<float>(size_t(rows));
            gamma = dalloc_t<float>(size_t(cols));
            HIPCHECK(launch_fill_normal(x, cols, 3, 0x52u, 0.f, 1.f, g.stream));
            HIPCHECK(launch_fill_normal(gamma, cols, 4, 0x53u, 1.f, 0.02f, g.stream));
            for (int i = 0; i < warmup; ++i)
                gemv(g.mats[size_t(ids[size_t(i % copies)])], 1, PRO_RMS, EPI_STORE, x, cols, 1, y, rows, gamma, 1e-6f, nullptr, g.stream);
            hipEvent_t e0, e1;
            HIPCHECK(hipEventCreate(&e0));
            HIPCHECK(hipEventCreate(&e1));
            HIPCHECK(hipEventRecord(e0, g.stream));
            for (int i = 0; i < iters; ++i)
                gemv(g.mats[size_t(ids[size_t(i % copies)])], 1, PRO_RMS, EPI_STORE, x, cols, 1, y, rows, gamma, 1e-6f, nullptr, g.stream);
            HIPCHECK(hipEventRecord(e1, g.stream));
            HIPCHECK(hipEventSynchronize(e1));
            float ms = 0.f;
            HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
            *ms_per_launch = double(ms) / iters;
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();
        return 1;
    }, 0);
}

int voxhip_bench_ffn_q8(int64_t hidden, int64_t inter, int copies, int warmup, int iters, double *us_per_block, float *check) {
    return guard_int([&] {
        require_ok();
        if (vh::prof_on()) throw Fail("the benchmark entry points capture graphs, which VOX_PROFILE=gpu turns off");
        if (copies <= 0 || iters <= 0 || !us_per_block || hidden % 32 || inter % 32) throw Fail("bad bench arguments");
        std::vector<int> ids;
        float *x = nullptr, *h = nullptr, *gbuf = nullptr, *gamma = nullptr;
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        auto cleanup = [&] {
            (void)hipStreamSynchronize(g.stream);
            if (exec) (void)hipGraphExecDestroy(exec);
            if (graph) (void)hipGraphDestroy(graph);
            if (e0) (void)hipEventDestroy(e0);
            if (e1) (void)hipEventDestroy(e1);
            for (int id : ids) free_mat(id);
            dfree(x); dfree(h); dfree(gbuf); dfree(gamma);
        };
        try {
            // per copy: gate|up interleaved [2 inter][hidden] and down [hidden][inter], q8, ~N(0, 0.02)
            for (int c = 0; c < copies; ++c)
                for (int part = 0; part < 2; ++part) {
                    const int64_t rows = part ? hidden : 2 * inter, cols = part ? inter : hidden;
                    const int id = new_mat(VOXHIP_Q8, rows, cols, false);
                    ids.push_back(id);
                    GpuMat &m = g.mats[size_t(id)];
                    float *tmp = dalloc_t<float>(size_t(rows) * size_t(cols));
                    HIPCHECK(launch_fill_normal(tmp, rows * cols, 2000 + c, 0x60u + part, 0.f, 0.02f, g.stream));
                    HIPCHECK(launch_quant_q8(tmp, rows * cols / 32, reinterpret_cast<int8_t *>(m.w), m.s, g.stream));
                    HIPCHECK(hipStreamSynchronize(g.stream));
                    dfree(tmp);
                }
            x = dalloc_t<float>(size_t(hidden));
            h = dalloc_t<float>(size_t(hidden));
            gbuf = dalloc_t<float>(size_t(inter));
            gamma = dalloc_t<float>(size_t(hidden));
            HIPCHECK(launch_fill_normal(x, hidden, 7, 0x70u, 0.f, 1.f, g.stream));
            HIPCHECK(launch_fill_normal(gamma, hidden, 8, 0x71u, 1.f, 0.02f, g.stream));
            HIPCHECK(hipMemcpyAsync(h, x, size_t(hidden) * 4, hipMemcpyDeviceToDevice, g.stream));
            if (check) {  // copy 0's block once on x, as the graph launches it: x, gamma and the block's output
                gemv(g.mats[size_t(ids[0])], 1, PRO_RMS, EPI_SWIGLU, h, hidden, 1, gbuf, inter, gamma, 1e-6f, nullptr, g.stream);
                gemv(g.mats[size_t(ids[1])], 1, PRO_X, EPI_ACC, gbuf, inter, 1, h, hidden, nullptr, 0.f, nullptr, g.stream);
                HIPCHECK(copy_d2h(check, x, size_t(hidden) * 4, g.stream));
                HIPCHECK(copy_d2h(check + hidden, gamma, size_t(hidden) * 4, g.stream));
                HIPCHECK(copy_d2h(check + 2 * hidden, h, size_t(hidden) * 4, g.stream));
                HIPCHECK(hipMemcpyAsync(h, x, size_t(hidden) * 4, hipMemcpyDeviceToDevice, g.stream));
            }
            HIPCHECK(hipStreamSynchronize(g.stream));
            // one graph over all copies: RMSNorm + gate|up + SwiGLU, then down + residual (two kernels per block)
            HIPCHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal));
            try {
                for (int c = 0; c < copies; ++c) {
                    const GpuMat &gu = g.mats[size_t(ids[size_t(2 * c)])], &dn = g.mats[size_t(ids[size_t(2 * c + 1)])];
                    gemv(gu, 1, PRO_RMS, EPI_SWIGLU, h, hidden, 1, gbuf, inter, gamma, 1e-6f, nullptr, g.stream);
                    gemv(dn, 1, PRO_X, EPI_ACC, gbuf, inter, 1, h, hidden, nullptr, 0.f, nullptr, g.stream);
                }
            } catch (...) {
                (void)hipStreamEndCapture(g.stream, &graph);
                throw;
            }
            HIPCHECK(hipStreamEndCapture(g.stream, &graph));
            HIPCHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
            for (int i = 0; i < warmup; ++i) HIPCHECK(hipGraphLaunch(exec, g.stream));
            HIPCHECK(hipEventCreate(&e0));
            HIPCHECK(hipEventCreate(&e1));
            HIPCHECK(hipEventRecord(e0, g.stream));
            for (int i = 0; i < iters; ++i) HIPCHECK(hipGraphLaunch(exec, g.stream));
            HIPCHECK(hipEventRecord(e1, g.stream));
            HIPCHECK(hipEventSynchronize(e1));
            float ms = 0.f;
            HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
            *us_per_block = double(ms) * 1000.0 / (double(iters) * copies);
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();
        return 1;
    }, 0);
}

int voxhip_bench_gemm_hh(int64_t m, int64_t n, int64_t K, int q8, int tile, int warmup, int iters, double *us_per_launch,
                         float *y_out) {
    return guard_int([&] {
        require_ok();
        if (vh::prof_on()) throw Fail("the benchmark entry points time launches, which VOX_PROFILE=gpu serialises");
        if (m <= 0 || n <= 0 || K <= 0 || K % 64 || tile < 0 || tile > 4 || warmup < 0 || iters <= 0 || !us_per_launch)
            throw Fail("bad bench arguments");
        if (m > (int64_t(1) << 20) || n > (int64_t(1) << 20) || m * K > (int64_t(1) << 28) || n * K > (int64_t(1) << 28))
            throw Fail("bench_gemm_hh: shape too large");
        _Float16 *a16 = nullptr, *w16 = nullptr;
        float *tmp = nullptr, *sc = nullptr, *y = nullptr;
        int8_t *q = nullptr;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        auto cleanup = [&] {
            (void)hipStreamSynchronize(g.stream);
            vh::set_gemm_hh_tile(0);
            dfree(a16); dfree(w16); dfree(tmp); dfree(sc); dfree(y); dfree(q);
            if (e0) (void)hipEventDestroy(e0);
            if (e1) (void)hipEventDestroy(e1);
        };
        try {
            // A: hi plane ~N(0, 1) as f16, lo plane ~N(0, 1e-3) as f16; W: ~N(0, 0.02) as f16, or its q8 form (int8
            // values as f16 and the block scales)
            a16 = dalloc_t<_Float16>(size_t(2 * m * K));
            w16 = dalloc_t<_Float16>(size_t(n * K));
            tmp = dalloc_t<float>(size_t(std::max(m, n) * K));
            y = dalloc_t<float>(size_t(m * n));
            HIPCHECK(launch_fill_normal(tmp, m * K, 11, 0x90u, 0.f, 1.f, g.stream));
            HIPCHECK(launch_to_f16(tmp, m * K, a16, g.stream));
            HIPCHECK(launch_fill_normal(tmp, m * K, 12, 0x91u, 0.f, 1e-3f, g.stream));
            HIPCHECK(launch_to_f16(tmp, m * K, a16 + m * K, g.stream));
            HIPCHECK(launch_fill_normal(tmp, n * K, 13, 0x92u, 0.f, 0.02f, g.stream));
            if (q8) {
                q = dalloc_t<int8_t>(size_t(n * K));
                sc = dalloc_t<float>(size_t(n * K / 32));
                HIPCHECK(launch_quant_q8(tmp, n * K / 32, q, sc, g.stream));
                HIPCHECK(launch_q8_to_f16(q, w16, n * K, g.stream));
            } else {
                HIPCHECK(launch_to_f16(tmp, n * K, w16, g.stream));
            }
            GemmArgs ga{};
            ga.m = int32_t(m);
            ga.n = int32_t(n);
            ga.K = int32_t(K);
            ga.a16 = a16;
            ga.a_lo = m * K;
            ga.lda = int32_t(K);
            ga.y = y;
            ga.ldy = int32_t(n);
            vh::set_gemm_hh_tile(tile);
            for (int i = 0; i < warmup; ++i) HIPCHECK(launch_gemm_hh(EPI_STORE, w16, sc, ga, g.stream));
            HIPCHECK(hipEventCreate(&e0));
            HIPCHECK(hipEventCreate(&e1));
            HIPCHECK(hipEventRecord(e0, g.stream));
            for (int i = 0; i < iters; ++i) HIPCHECK(launch_gemm_hh(EPI_STORE, w16, sc, ga, g.stream));
            HIPCHECK(hipEventRecord(e1, g.stream));
            HIPCHECK(hipEventSynchronize(e1));
            float ms = 0.f;
            HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
            *us_per_launch = double(ms) * 1000.0 / iters;
            if (y_out) HIPCHECK(copy_d2h(y_out, y, size_t(m * n) * 4, nullptr));
            sync_status();
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();
        return 1;
    }, 0);
}

int voxhip_selftest_split_f16(int64_t pairs, int64_t *mismatches) {
    return guard_int([&] {
        require_ok();
        if (pairs <= 0 || !mismatches) throw Fail("bad self-test arguments");
        unsigned long long *bad = nullptr;
        try {
            bad = dalloc_t<unsigned long long>(1);
            HIPCHECK(hipMemsetAsync(bad, 0, sizeof *bad, g.stream));
            const int64_t chunk = int64_t(1) << 26;
            for (int64_t p = 0; p < pairs; p += chunk)
                HIPCHECK(launch_check_split(uint64_t(2 * p), uint64_t(std::min(chunk, pairs - p)), bad, g.stream));
            unsigned long long h = 0;
            HIPCHECK(copy_d2h(&h, bad, sizeof h, g.stream));
            HIPCHECK(hipStreamSynchronize(g.stream));
            *mismatches = int64_t(h);
        } catch (...) {
            (void)hipStreamSynchronize(g.stream);
            dfree(bad);
            throw;
        }
        dfree(bad);
        return 1;
    }, 0);
}

int voxhip_bench_copy(int64_t bytes, int warmup, int iters, double *ms_per_copy) {
    return guard_int([&] {
        require_ok();
        if (vh::prof_on()) throw Fail("the benchmark entry points capture graphs, which VOX_PROFILE=gpu turns off");
        if (bytes < 16 || iters <= 0 || !ms_per_copy) throw Fail("bad bench arguments");
        void *a = nullptr, *b = nullptr;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        auto cleanup = [&] {
            (void)hipStreamSynchronize(g.stream);
            dfree(a); dfree(b);
            if (e0) (void)hipEventDestroy(e0);
            if (e1) (void)hipEventDestroy(e1);
        };
        try {
            a = dalloc(size_t(bytes));
            b = dalloc(size_t(bytes));
            HIPCHECK(launch_fill_normal(static_cast<float *>(a), bytes / 4, 5, 0x55u, 0.f, 1.f, g.stream));
            for (int i = 0; i < warmup; ++i) HIPCHECK(launch_copy16(a, b, bytes, g.stream));
            HIPCHECK(hipEventCreate(&e0));
            HIPCHECK(hipEventCreate(&e1));
            HIPCHECK(hipEventRecord(e0, g.stream));
            for (int i = 0; i < iters; ++i) HIPCHECK(launch_copy16(a, b, bytes, g.stream));
            HIPCHECK(hipEventRecord(e1, g.stream));
            HIPCHECK(hipEventSynchronize(e1));
            float ms = 0.f;
            HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
            *ms_per_copy = double(ms) / iters;
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();
        return 1;
    }, 0);
}

}  // extern "C"
