// vh_launch.hpp — host-side launchers of the gfx950 kernels (one translation unit per kernel family).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <string>

#include "vh_types.hpp"

namespace vh {

// Kernel timing hook: timing_arm() queues (start, stop) event pairs; each kernel launch takes the next pair, if
// any, and is launched with hipExtLaunchKernel so the events are stamped at that kernel's own start and end on
// its stream. The benchmark arms it around single launches; an empty queue costs one branch per launch.
void timing_arm(hipEvent_t start, hipEvent_t stop);
void timing_clear();
bool timing_take(hipEvent_t *start, hipEvent_t *stop);

// VOX_PROFILE=gpu (the reference's GPU profile, gpu_vulkan.cpp:62-87, :312-326): every launch is stamped with HIP
// events at its own start and end and booked under "<stage>/<kernel>", the stage being the entry point's
// (prof_stage); prof_collect() books the launches of a synchronized stream, prof_report() is the table sorted by
// time. The library runs its graphs' launches one by one meanwhile (stamped launches cannot be captured).
bool prof_on();
void prof_enable();
void prof_stage(const char *stage);
void prof_take(const void *kernel, hipStream_t s, hipEvent_t *start, hipEvent_t *stop);
void prof_collect();
// The table (one line per label: calls, total ms, average us, share of the GPU busy time); empty when off.
const char *prof_report(const char *device);

template <typename K, typename... Args>
hipError_t launch(K kernel, dim3 grid, dim3 block, size_t smem, hipStream_t s, Args... args) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (timing_take(&e0, &e1)) {
        hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(smem), s, e0, e1, 0u, args...);
    } else if (prof_on()) {
        prof_take(reinterpret_cast<const void *>(kernel), s, &e0, &e1);
        hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(smem), s, e0, e1, 0u, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, smem, s, args...);
    }
    return hipGetLastError();
}

// The library's range-status word (kStatusF16Range, kStatusFixRange), in device memory; null before init. The
// launchers of kernels that can meet an unrepresentable value hand it to them.
int32_t *status_word();

// GEMV launch: rows/K/m etc. in a; wt = weight type; int_path = int8 activations (Q8 m <= 8, Q4 always).
// Picks the row block M and the tile (R rows per wave, IT 1 KiB chunks in flight per row) from the shape.
// The int path's prologue of a pass of m rows, once per row, into q [m][K] int8, qs / qsum [m][K/32]; the GEMV
// then runs with PRO_Q and a.q / a.qs / a.qsum set.
hipError_t launch_quant_rows(int pro, const GemvArgs &a, int8_t *q, float *qs, int32_t *qsum, hipStream_t s);
hipError_t launch_gemv(int wt, bool int_path, int pro, int epi, const GemvArgs &a, hipStream_t s);
void gemv_tile(int rows, int nchunk, int M, bool swiglu, int *R, int *IT);

hipError_t launch_qk_post(const QkArgs &a, int m, hipStream_t s);

// Multi-row f32 GEMM on the matrix cores (F32 / F16 / BF16 / Q8 weights).
hipError_t launch_gemm(int wt, int epi, const uint8_t *w, const float *scale, const float *A, const GemmArgs &g, hipStream_t s);
// Grouped "same" Conv1d as an implicit-im2col GEMM (f32 weights [groups][cout/groups][K][cin/groups]).
// Split-f16 GEMM with A already split by its producer (g.a16 hi, g.a16 + g.a_lo lo), K % 64 == 0: F16 weights
// (q8_scale null), or Q8 weights as their int8 values widened to f16 with the block scales [n][K / 32] in q8_scale;
// epilogues STORE, ACC, GATED_ACC, GELU, SWIGLU, GELU_H16, SWIGLU_H16, ROPE_H16 (split K uses g.ws).
hipError_t launch_gemm_hh(int epi, const _Float16 *w, const float *q8_scale, const GemmArgs &g, hipStream_t s);
// Forces launch_gemm_hh's block tile (0: its shape policy); voxhip_bench_gemm_hh only.
void set_gemm_hh_tile(int tile);
// The same with EPI_ACC, and when the product splits K, the next RMSNorm (gamma, eps) of the updated rows of y written
// as f16 halves (out16, ldo, lo_off as launch_rmsnorm_rows_h16) by the split-K reduce itself: *normed tells whether
// it did (otherwise the caller runs the norm).
hipError_t launch_gemm_hh_acc_rms(const _Float16 *w, const float *q8_scale, const GemmArgs &g, const float *gamma, float eps,
                                  _Float16 *out16, int64_t ldo, int64_t lo_off, hipStream_t s, bool *normed);
hipError_t launch_conv_gemm(int epi, const float *w, const float *A, const GemmArgs &g, int groups, hipStream_t s);
// Merge of the split attention partials of m rows into ao [m][heads * hd].
hipError_t launch_attn_merge(const AttnPartials &P, float *ao, int m, hipStream_t s);
// Split-K attention partials of m rows (merged by the PRO_ATTN GEMV prologue). fused: rows of distinct sequences,
// q/k post-processing and the K/V append happen inside; otherwise k_qk_post ran first. kc0/vc0/cap0: row 0's cache
// (the same as the first row view); qkv: [m][a.ldqkv]; rope_rows: [m][hd] (fused). long_ctx: a fused row at a position
// past kAttnSpecKeys, whose first batch then holds as many keys as a launch of several rows takes (a graph
// captured with it replays correctly at any position).
hipError_t launch_attention(const AttnArgs &a, const _Float16 *kc0, const _Float16 *vc0, int64_t cap0, const float *qkv,
                            const float *rope_rows, int layer, int hd, int group, int m, bool fused, hipStream_t s,
                            bool long_ctx = false);
// rows samplers at once: cfg[b], logits [b][n], out[b].
hipError_t launch_sample(const SampleCfgDev *cfg, const float *logits, int n, int32_t *out, hipStream_t s, int rows = 1);

hipError_t launch_quant_q8(const float *w, int64_t nblocks, int8_t *q, float *scale, hipStream_t s);
hipError_t launch_quant_q4(const float *w, int64_t nblocks, uint8_t *q, float *scale, hipStream_t s);
hipError_t launch_quant_act(const float *x, int64_t nblocks, int8_t *xq, float *xs, hipStream_t s);
hipError_t launch_to_f16(const float *x, int64_t n, void *y, hipStream_t s);
hipError_t launch_to_bf16(const float *x, int64_t n, void *y, hipStream_t s);
hipError_t launch_rmsnorm_rows(const float *x, int64_t ldx, const float *w, int K, float eps, float *out, int64_t ldo,
                               int m, hipStream_t s);
// The same RMSNorm written as f16 halves (hi rows of ldo halves at out16, lo rows at out16 + lo_off).
hipError_t launch_rmsnorm_rows_h16(const float *x, int64_t ldx, const float *w, int K, float eps, _Float16 *out16,
                                   int64_t ldo, int64_t lo_off, int m, hipStream_t s);
// int8 values widened to f16 (n a multiple of 8).
hipError_t launch_q8_to_f16(const int8_t *q, _Float16 *out, int64_t n, hipStream_t s);
hipError_t launch_fill_normal(float *out, int64_t n, uint64_t seed, uint32_t stream, float mean, float std,
                              hipStream_t s);
hipError_t launch_fill_cache(void *c, int64_t planes, int64_t cap, int64_t len, int hd, uint64_t seed, uint32_t stream,
                             float mean, float std, hipStream_t s);

// max |x| over n floats into *out as float bits (the caller zeroes *out; NaN reads as above every value)
hipError_t launch_absmax(const float *x, int64_t n, uint32_t *out, hipStream_t s);
hipError_t launch_copy16(const void *src, void *dst, int64_t bytes, hipStream_t s);
// A one-wave kernel that holds the stream for about `us` microseconds (0 < us <= 1e5), by the device's real-time clock.
hipError_t launch_hold(double us, hipStream_t s);
// k_check_split over pairs base/2 .. base/2 + pairs - 1; *bad (device) accumulates the pairs that differ.
hipError_t launch_check_split(uint64_t base, uint64_t pairs, unsigned long long *bad, hipStream_t s);
// Attention one block per (head, row) for any even head_dim <= 128 (q from k_qk_post, keys from each row's cache).
hipError_t launch_attn_rows(const AttnRowsArgs &a, int m, hipStream_t s);
// Causal attention of a prefill pass (consecutive rows of one sequence) on the matrix cores, head_dim 64 or 128.
hipError_t launch_prefill_attn(const PrefillAttnArgs &a, int hd, hipStream_t s);
// F5-TTS DiT step: AdaLN modulation of R rows of D, the step input's x columns, attention (head_dim 64).
hipError_t launch_f5_modulate(const float *x, int64_t R, int D, const float *sc, const float *sh, float *y, _Float16 *y16,
                              int64_t lo_off, hipStream_t s);
hipError_t launch_f5_fill_x(const float *x, int N, int mel, float *cat, int W, int B, hipStream_t s);
// Vocos: LayerNorm with weight and bias (double statistics, eps 1e-6) of R rows of D; depthwise "same" conv over
// batches of seq rows (w [C][K], bias or null).
hipError_t launch_layernorm_rows(const float *x, int64_t R, int D, const float *w, const float *b, float *y, hipStream_t s);
// Any row norm of NormArgs (LayerNorm / modulation, optional mish and channel bias; the CosyVoice2 estimator's blocks).
hipError_t launch_norm_rows(const NormArgs &a, hipStream_t s);
hipError_t launch_dwconv(const float *x, const float *w, const float *b, float *y, int64_t R, int C, int K, int seq, hipStream_t s);
hipError_t launch_f5_attn(const _Float16 *qkv16, int64_t lo_off, float *out, _Float16 *out16, int64_t out_lo, int B, int N,
                          int heads, int hd, int ldvt, int ldo, float scale, hipStream_t s);
// Qwen3-TTS codec decoder: streaming histories (dst != old), the causal depthwise conv, the transposed conv's
// overlap-add (tail_old -> tail_new, K <= 2 stride, with an optional Snake output), the pre-transformer's RoPE + ring
// append and windowed attention,
// layer-scaled residual adds, the final clamp; and the streaming conv GEMM (A = im2col of [hist; x]).
hipError_t launch_hist_shift(float *dst, const float *old, const float *x, int64_t ldx, int T, int ctx, int C, hipStream_t s);
hipError_t launch_dwconv_causal(const float *x, const float *hist, const float *w, const float *b, float *y, int T, int C, int K,
                                hipStream_t s, float *hist_next = nullptr);
// snake_y (optional, another buffer than y): Snake (snake_a, snake_ib per channel) of the rows written to y, as well.
hipError_t launch_ola(const float *tmp, const float *tail_old, float *tail_new, const float *bias, float *y, int T, int stride,
                      int K, int co, hipStream_t s, float *snake_y = nullptr, const float *snake_a = nullptr,
                      const float *snake_ib = nullptr);
// nn::ConvT's padded overlap-add (gather form) from the GEMM output z [T][K co] to y [To][co] (+ bias when not null).
hipError_t launch_convt_gather(const float *z, const float *bias, float *y, int T, int To, int stride, int K, int pad, int co,
                               hipStream_t s);
hipError_t launch_codec_rope_ring(float *qkv, int ld, int F, int heads, int kvh, int hd, const float *rope, float *ring_k,
                                  float *ring_v, int R, const int64_t *pos, hipStream_t s);
hipError_t launch_codec_attn(const float *qkv, int ld, const float *ring_k, const float *ring_v, int R, int F, int heads, int kvh,
                             int hd, const int64_t *pos, int W, float scale, float *ao, hipStream_t s);
hipError_t launch_scale_acc(float *h, const float *t, const float *sc, int64_t rows, int H, hipStream_t s);
hipError_t launch_clamp1(float *y, int64_t n, hipStream_t s);
hipError_t launch_stream_conv(int wt, int epi, const uint8_t *w, const float *scale, const float *x, const GemmArgs &g,
                              hipStream_t s);
// CosyVoice2 LM: one sampling step (log-softmax, RAS trial loop) and the next step's embedding + row advance.
hipError_t launch_lm_sample(const float *logits, int n, const LmCfgDev *cfg, LmState *st, int32_t *decoded, float *logp_out,
                            int64_t logp_stride, bool append, hipStream_t s);
hipError_t launch_lm_embed(const LmEmbedArgs &a, hipStream_t s);
// mat_gather of n rows ids[0..n) (device, already range-checked) into out [n][cols]; wt a WT_* weight format.
hipError_t launch_mat_gather(const uint8_t *w, const void *scale, int wt, int s16, int64_t cols, const int32_t *ids,
                             int64_t n, float *out, hipStream_t s);
// A pass of the code-predictor frame loop: row table + RoPE rows of the pass, the sampled code's embedding row.
hipError_t launch_pred_embed(const PredEmbedArgs &a, hipStream_t s);

// The fused one-row FFN (k_ffn_int): Q8 / Q4 / Q4H layers with H % 32 == 0, I % 32 == 0, H <= kFfnMaxH (2048); the down weights
// as panels (launch_panel_pack); adds its down product to a.acc (zero on entry) in fixed point.
bool ffn_shape_ok(int wt, int H, int I);
int ffn_parts();
hipError_t launch_ffn(int wt, const FfnArgs &a, hipStream_t s);
// Down weights [H][I] + scales [H][I/32] into panels [I/32][H][32 columns] + [I/32][H] (pw, ps hold as many bytes).
hipError_t launch_panel_pack(int wt, const uint8_t *w, const void *scale, int H, int I, uint8_t *pw, void *ps, hipStream_t s);
// h += the pending sums of acc [kAccCopies][H]; acc back to zero.
hipError_t launch_acc_fold(float *h, int64_t *acc, int H, hipStream_t s);

// Shared-memory opt-in above 64 KiB, once per kernel.
hipError_t ensure_smem(const void *kernel, size_t bytes);

}  // namespace vh
