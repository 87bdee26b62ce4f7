// vh_types.hpp — argument blocks shared by the kernels and their host-side launchers.
#pragma once
#include <stdint.h>

namespace vh {

// The library's range-status word: a kernel whose arithmetic cannot represent a value it was given sets a bit, and
// the synchronous entry points fail the call when one is set (so the engine computes it on the CPU instead).
enum : int32_t { kStatusF16Range = 1, kStatusFixRange = 2 };

// GEMV input prologues: x as is; RMSNorm(x, gamma); or the merge of split-K attention partials.
// GEMV prologues; PRO_Q (int path only): the input rows arrive already quantized (k_quant_rows)
enum { PRO_X = 0, PRO_RMS = 1, PRO_ATTN = 2, PRO_Q = 3 };
enum { EPI_STORE = 0, EPI_ACC = 1, EPI_SWIGLU = 2 };
// Int-path GEMV on pre-quantized rows (PRO_Q) only: SwiGLU, then the output rows quantized per 32-block into
// GemvArgs::yq / yqs / yqsum for the next pass (which takes them as its PRO_Q rows) instead of stored as floats
enum { EPI_SWIGLU_Q = 13 };
// GEMM-only epilogues (F5 DiT, Vocos, the codec): y += gate * c; y = gelu_tanh(c); y = mish(c); y += mish(c); RoPE on
// q|k columns; y = gelu_erf(c); y = snake(c); y += c, then snake(y) into snake_y as well
enum { EPI_GATED_ACC = 3, EPI_GELU = 4, EPI_MISH = 5, EPI_MISH_ACC = 6, EPI_ROPE = 7, EPI_ROPE_H16 = 8, EPI_GELU_H16 = 9,
       EPI_GELU_ERF = 10, EPI_SNAKE = 11, EPI_SWIGLU_H16 = 12, EPI_ACC_SNAKE = 14 };
// GEMM A operand: rows of a matrix, or the implicit im2col rows of a grouped "same" Conv1d
enum { ASRC_ROWS = 0, ASRC_CONV = 1, ASRC_STREAM = 2 };
// Weight formats of the GEMV kernels: the reference's types, plus Q4 with f16 block scales (WT_Q4H), the
// device storage of a Q4 matrix whose f32 scales are all exact in f16 (same arithmetic, 2 bytes less per block).
enum { WT_F32 = 0, WT_F16 = 1, WT_BF16 = 2, WT_Q8 = 3, WT_Q4 = 4, WT_Q4H = 5 };

// Cache view of one activation row: the sequence's cache bases (layer 0) and the row's absolute position.
struct RowRef {
    _Float16 *k;
    _Float16 *v;
    int64_t cap;
    int64_t pos;
};

constexpr int kAttnMaxSplits = 8;  // split-K blocks per (row, kv head); the merge happens in the o-GEMV prologue
constexpr int kAttnSpecKeys = 512; // cache keys each (row, kv head) loads before its position is known

// Split s of a row holds the keys j with j % kAttnMaxSplits == s (interleaved, so a split's key set does not
// depend on the row's length). Every split writes partials; one with no keys (s >= n) writes an empty one
// (max -inf, denominator 0, output 0), so readers merge a fixed count.

// Split-K attention partials of m rows: running max, denominator and unnormalized output per (row, head, split).
// Every split of every row is written by each attention launch.
struct AttnPartials {
    float *pm, *pl;  // [m][heads][kAttnMaxSplits]
    float *po;       // [m][heads][kAttnMaxSplits][hd]
    const RowRef *rows;
    int32_t heads, hd;
};

struct GemvArgs {
    const uint8_t *w;     // weights, reference row layout
    const float *scale;   // [rows][K/32] for Q8/Q4 (f16 values for WT_Q4H)
    const float *bias;    // [rows] or null
    const float *x;       // [m][ldx] (PRO_X, PRO_RMS)
    const float *gamma;   // [K] (PRO_RMS)
    float *y;             // [m][ldy]
    float *xnorm;         // PRO_RMS / PRO_ATTN: block 0 writes the prologue's f32 rows [m][K] here (may be null)
    AttnPartials attn;    // PRO_ATTN: K = heads * hd
    int64_t ldx, ldy;
    int32_t rows, K, m;
    float eps;
    // PRO_Q: the rows quantized per 32-block, q [m][K] int8, qs [m][K/32] scales, qsum [m][K/32] block sums
    const int8_t *q;
    const float *qs;
    const int32_t *qsum;
    // EPI_SWIGLU_Q: the SwiGLU output rows quantized as PRO_Q takes them, yq [m][rows/2], yqs and yqsum [m][rows/64]
    int8_t *yq;
    float *yqs;
    int32_t *yqsum;
    // One-row passes after a fused FFN (k_ffn_int): the FFN's down product still pending as fixed-point sums
    // [kAccCopies][acc_ld]. PRO_RMS adds them to x before the norm; EPI_ACC adds them to y before its own product
    // (the two residual adds in the reference's order) and sets the rows it consumed to zero.
    int64_t *acc;
    int64_t acc_ld;
    // EPI_ACC: the residual rows to add to ([m][ldy]); null: y itself (y += product)
    const float *res;
    // EPI_ACC: per output row scale of the product, y = residual + yscale[r] (product + bias) (the codec's layer
    // scales); null: 1
    const float *yscale;
};

// Copies of the fixed-point down accumulators: FFN blocks of group g add into copy g % kAccCopies, so fewer
// blocks meet on one cache line; readers sum the copies.
constexpr int kAccCopies = 4;

// The decode FFN of one row as one launch (k_ffn_int): RMSNorm(x, gamma), the gate|up GEMV, SwiGLU, the
// activation quantization of the SwiGLU output per 32-block, and the down product split by its input columns:
// block group g owns SwiGLU outputs 32g .. 32g+31 (one quantization block) and adds its share of every down row
// into acc. The down weights come repacked as panels of 32 columns, so a group's share is contiguous.
struct FfnArgs {
    const uint8_t *gu;    // gate|up rows (2u, 2u + 1) = (gate u, up u), [2I][row bytes of H]
    const float *gu_s;    // [2I][H/32] block scales (f16 values for WT_Q4H)
    const float *gu_b;    // [2I] or null
    const uint8_t *dp;    // down panels [I/32][H][row bytes of 32 columns]
    const float *dp_s;    // panel scales [I/32][H] (f16 values for WT_Q4H)
    const float *d_b;     // down bias [H] or null (added once, by group 0)
    const float *x;       // the input row [H]
    const float *gamma;   // [H]
    int64_t *acc;         // [kAccCopies][H] fixed-point (2^-32) sums of the down product
    int32_t H, I, parts;  // parts: blocks per group, each taking H / parts of the down rows
    float eps;
    int32_t *status;      // the range-status word (a down term outside the fixed-point range); set by the launcher
};

constexpr int kGemvThreads = 256;

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

// Attention over each row's f16 cache. fused: the kernel also does what k_qk_post does (q/k RMSNorm, RoPE, K/V
// append) for rows whose sequences differ (decode, pairs, B sessions); otherwise q comes from `q` and the keys of
// this pass are already in the cache (prefill of one sequence).
struct AttnArgs {
    int64_t ldqkv;           // row stride of the fused q|k|v input (passed to the kernel as its own argument)
    const float *q;          // not fused: [m][qd]
    const float *qn, *kn;
    AttnPartials part;
    int32_t kv_heads;
    int32_t group;           // query heads per kv head (a block takes G of them: group / G blocks per kv head)
    float scale, eps;
};

// Causal attention of m consecutive rows of one sequence (prefill) on the matrix cores: row r sits at position
// pos0 + r and attends keys 0 .. pos0 + r of the f16 cache (the pass's keys already appended by k_qk_post).
struct PrefillAttnArgs {
    const float *q;        // [m][heads hd] normed + rotated queries
    const _Float16 *k, *v; // the sequence's cache bases ([layer][kv_head][cap][hd])
    float *out;            // [m][heads hd]
    _Float16 *out16;       // or, when set, the output as f16 halves: hi [m][heads hd] at out16, lo at out16 + lo_off
    int64_t lo_off;
    const RowRef *rows;    // the pass's row table: the kernel takes pos0 from rows[0].pos, so a captured pass
                           // replays at whatever position the host last wrote there
    int64_t cap, pos0;     // pos0: the host's copy of rows[0].pos at launch, checked against cap
    int32_t m, heads, kv_heads, layer;
    float scale;
    // key splits: with splits > 1 block z of a query tile takes the z-th of `splits` contiguous runs of its key tiles
    // and writes (max, sum, unnormalized output) to part's slot z; k_pattn_merge then writes out / out16
    AttnPartials part;
    int32_t splits;
    int32_t *status;  // the range-status word (queries beyond the f16 range of the split products)
};

// Attention of m rows, one block per (head, row), for any even head_dim <= 128: q [m][heads hd] already normed and
// rotated (k_qk_post), each row over keys 0 .. rows[i].pos of its own cache, output [m][heads hd] normalized.
struct AttnRowsArgs {
    const float *q;
    float *out;
    const RowRef *rows;
    int32_t heads, kv_heads, hd, layer;
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

// The multi-row MFMA GEMM (y[i][r] = sum_k A[i][k] W[r][k] + bias[r], then the epilogue).
struct GemmArgs {
    const float *bias;  // [n] or null
    float *y;           // [m][ldy]
    int64_t lda, ldy;
    int32_t m, n, K;
    const float *gate;  // EPI_GATED_ACC: [n]
    // EPI_ROPE: table [seq][hd/2][2] (cos, sin) at position row % seq; pairs (2j, 2j + 1) of the columns below
    // rope_cols rotate (q | k heads), heads >= rope_heads of each of q and k are left as they are
    const float *rope;
    int32_t seq, hd, rope_cols, rope_heads;
    // heads padded with zero dims to hd (the attention tiles' 64): the table's head dim and the dims that rotate,
    // d < rope_hd (0: hd)
    int32_t rope_hd;
    // EPI_ROPE_H16: the rotated q | k and v as f16 halves (x = hi + lo) for the attention's matrix cores, written to
    // h16 instead of y: plane hi then plane lo (lo_off halves apart), each = q | k rows [m][rope_cols] followed by
    // v transposed per batch and head, [m / seq][heads][hd][ldvt] (ldvt >= seq, a multiple of 8); rope null: the
    // same layout without the rotation
    // EPI_GELU_H16: gelu(c + bias) as f16 halves into h16 (hi) and h16 + lo_off (lo), rows of ldy halves; the tanh
    // form, or the erf form when gelu_erf is set. EPI_SWIGLU_H16: EPI_SWIGLU's silu(gate) up written the same way.
    _Float16 *h16;
    int64_t lo_off;
    int32_t ldvt;
    // k_gemm_hh: A already split into f16 halves, hi plane a16 and lo plane a16 + a_lo, rows of lda halves
    const _Float16 *a16;
    int64_t a_lo;
    // ASRC_CONV: x [m][lda] rows of `seq`-row batches; group g = blockIdx.z reads channels [g cig, (g + 1) cig) at
    // rows t + k - ksize / 2 of the same batch (causal: t + k - (ksize - 1)) (zeros outside) for A column k cig + i;
    // W and y are offset per group
    int32_t ksize, cig, causal;
    int32_t gelu_erf;
    // ASRC_STREAM (the codec's streaming convolutions): A column k cig + i of row t is channel i of row t + k dil of
    // [hist (ctx rows of cig); x (rows of lda)], ctx = (ksize - 1) dil
    const float *hist;
    int32_t ctx, dil;
    // EPI_SNAKE: y = v + snake_ib[col] sin(snake_a[col] v)^2 of v = c + bias (the codec's Snake after a convolution);
    // EPI_ACC_SNAKE: y += c + bias, then the same Snake of the updated y into snake_y ([m][ldy]; the next residual
    // unit's or block's input)
    const float *snake_a, *snake_ib;
    float *snake_y;
    // ASRC_STREAM: when set, the launch also writes the history of the next call, the last ctx rows of [hist; x], to
    // hist_next (another buffer than hist), each block a share
    float *hist_next;
    // split K (k_gemm_h16): block z sums K columns [z kchunk, (z + 1) kchunk) into ws + z m n ([m][n]); a reduce
    // pass adds the slices in order and applies the epilogue. kchunk 0: no split.
    int32_t kchunk;
    float *ws;
    int64_t ws_cap;  // floats available at ws (0: no split)
    // the range-status word (kStatusF16Range when a value split into f16 halves is beyond the f16 range); the public
    // launchers set it
    int32_t *status;
    // F32 weights with max |w| >= 63 (or NaN): the split kernel's 2^10-scaled f16 halves cannot hold them, so they
    // take k_gemm_f32
    int32_t f32_wide;
};

// CosyVoice2 LM sampling (lm_logp + ras_sample + lm_generate's trial loop, cosyvoice.cpp:598-690).
struct LmCfgDev {
    float top_p, tau_r;
    int32_t top_k, win_size;
    int32_t speech_tokens;  // ids >= speech_tokens end the generation
    int32_t min_len, max_len;  // lm_generate's bounds; a step at i >= max_len ends the generation
    uint32_t key0, key1;    // DetRng(seed)
    uint32_t stream;        // 0x43560000 + piece
    int32_t max_trials;     // the reference fails after trial 101
};
// Device state of a generation: step i, decoded count, done flag, status (0 ok, 1 trial limit), last token.
struct LmState {
    int32_t step, n_dec, done, status, last, pad0, pad1, pad2;
};
struct LmEmbedArgs {
    const uint8_t *w;
    const void *scale;     // f32 [rows][cols/32], or f16 bits when s16 (Q4)
    int32_t type, s16;
    int64_t rows, cols;
    const LmState *st;
    const int32_t *decoded;
    float *x;
    RowRef *row;
    float *rope_row;       // [hd] (cos, sin) pairs of the row
    const float *rope;     // table [positions][hd]
    int32_t hd;
    int64_t spare_pos;
};
// Row LayerNorm of R rows of D (k_f5_modulate), one wave per row, double statistics:
// n = (x - float(mean)) * float(1 / sqrt(var + eps)); modulate (affine 0): y = n * (1 + sc) + sh; affine:
// y = n * sc + sh (sh null: 0); then mish (the nn.hpp form) when set, then + tb (null: none). y as f32 rows, or as
// f16 halves (hi at y16, lo at y16 + lo_off) when y16 is set. x and y may be the same rows.
struct NormArgs {
    const float *x;
    float *y;
    _Float16 *y16;
    int64_t lo_off;
    const float *sc, *sh, *tb;
    double eps;
    int32_t R, D, affine, mish;
    int32_t *status;  // the range-status word (y16 values beyond the f16 range); set by the launcher
};

// One pass of the code-predictor frame loop (gpu_pred_frame): the pass's m rows of the sequence at positions
// pos0 .. pos0 + m - 1 (row table + RoPE rows), and for a pass after the first the embedding row of the code the
// previous pass sampled (codes[code_idx]) into x.
struct PredEmbedArgs {
    const uint8_t *w;      // embedding [rows][cols] (null: no gather)
    const void *scale;     // f32 [rows][cols/32], or f16 bits when s16 (Q4)
    int32_t type, s16;
    int64_t rows, cols;
    const int32_t *codes;
    int32_t code_idx;
    float *x;              // [cols]
    RowRef *row;           // [m]
    float *rope_row;       // [m][hd]
    const float *rope;     // table [positions][hd]
    int32_t hd, m;
    RowRef base;           // cache view of the sequence; pos = pos0
    int32_t *err;          // set to 1 when a code falls outside the embedding
};
constexpr int kF5HeadDim = 64;   // head_dim of the F5 attention kernel
constexpr int kLmMaxK = 1024;  // top_k limit of the device RAS sampler (sorted in LDS above 64)
constexpr int kLmMaxN = 8192;  // vocabulary limit of the device RAS sampler (8 entries per thread)

constexpr int kSampleThreads = 1024;
constexpr int kSampleMaxN = 16384;  // logits per call (keys sorted in LDS)

}  // namespace vh
