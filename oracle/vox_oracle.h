/*
 * vox_oracle.h — CPU restatement of the reference's tensor-op hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * backend in vox_amd/. It may be loaded only by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg. The product path never links or calls it.
 *
 * Every function restates one reference function (cited file:line under
 * /root/reference). Floating-point operation order follows the reference
 * where the reference fixes it. The build uses -ffp-contract=off, so the only
 * fused multiply-adds are explicit fmaf() calls, placed where the reference
 * compiles to vfmadd.
 *
 * Parity pins: every function is checked by tests/test_oracle.py against one
 * of these: the Random123 KAT vectors (test_core.cpp:35-43), the sampler rule
 * tests (test_core.cpp:45-79), the Q4 bounds (test_core.cpp:461-521), golden
 * vectors written by the compiled reference (oracle/_ref, fixtures under
 * tests/golden/), or a float64 brute force. No function here is "parity
 * unpinned".
 */
#ifndef VOX_ORACLE_H
#define VOX_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight types, in the order of vox::WType (kernels.hpp:42). */
enum { VO_F32 = 0, VO_F16 = 1, VO_BF16 = 2, VO_Q8 = 3, VO_Q4 = 4 };

/* Non-owning weight view, field meaning as vox::Mat (kernels.hpp:44-56):
 * [rows][cols] row-major, rows = outputs. Q8: int8 data + f32 scale
 * [rows][cols/32]. Q4: 16 bytes per 32-block, byte j = w[j] | w[j+16] << 4,
 * value (u - 8) * scale; f32 scale [rows][cols/32]. bias: [rows] or NULL. */
typedef struct {
    int32_t type;
    const void *data;
    const float *scale;
    int64_t rows, cols;
    const float *bias;
} vo_mat;

/* ---- counter RNG and sampling (sampling.hpp) ---- */
void vo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float vo_uniform(uint64_t seed, uint64_t frame, uint32_t codebook, uint32_t draw);
int32_t vo_sample_logits(float *logits, int32_t n, float temperature, float top_p, int32_t top_k,
                         float repetition_penalty, const int32_t *history, int32_t n_history, float u);
/* CosyVoice2 repetition-aware sampler (cosyvoice.cpp:617-664). logp is modified like the reference
 * (the chosen token is set to -inf when it is resampled). */
int32_t vo_ras_sample(float *logp, int32_t n, const int32_t *decoded, int32_t n_decoded, float top_p, int32_t top_k,
                      int32_t win_size, float tau_r, float u0, float u1);
/* lm_logp's log-softmax (cosyvoice.cpp:602-606) in place on v = head output + bias: mx = max, lse = mx +
 * float(log(sum of exp(double(v - mx)))) summed in index order, v -= lse. */
void vo_lm_logp(float *v, int32_t n);
/* One step of lm_generate's trial loop (cosyvoice.cpp:677-682): u0, u1 = uniform(step, 0x43560000 + piece,
 * 2 trial (+1)) under key seed; ras_sample until step >= min_len or the token is below speech_tokens. Returns the
 * token (>= speech_tokens: the end), or -2 when the reference fails after trial 101. logp is modified as there. */
int32_t vo_lm_step(float *logp, int32_t n, const int32_t *decoded, int32_t n_decoded, int64_t step, int32_t min_len,
                   int32_t speech_tokens, float top_p, int32_t top_k, int32_t win_size, float tau_r, uint64_t seed,
                   uint32_t piece);
/* Philox Box-Muller normal stream (f5.cpp:402-414): out[2p], out[2p+1] from draws (p, stream, 0/1). */
void vo_noise(uint64_t seed, uint32_t stream, size_t n, float *out);

/* ---- formats (kernels.hpp:59-76, kernels.cpp:432-471, :606-645, :918-929) ---- */
float vo_f16_to_f32(uint16_t h);
uint16_t vo_f32_to_f16(float f); /* round to nearest even (used to model an f16 KV cache) */
float vo_bf16_to_f32(uint16_t h);
void vo_mat_row(const vo_mat *W, int64_t r, float *out);
void vo_quantize_q8(const float *w, int64_t rows, int64_t cols, int8_t *q, float *scale);
void vo_quantize_q4(const float *w, int64_t rows, int64_t cols, uint8_t *q, float *scale);
/* Per-32-block int8 activation quantization of the q8/q4 GEMV (kernels.cpp:515-523). */
void vo_quantize_act(const float *x, int64_t n, int8_t *xq, float *xs);

/* ---- matmul (kernels.cpp:475-705) ----
 * avx2 = 1 restates the AVX2/FMA dot (kernels.cpp:485-501, :554-573), 0 the scalar one (:475-483, :541-552).
 * Dispatch as matmul(): Q8 with m <= 8 and Q4 use int8 activations; Q8 with m > 8 and F32/F16/BF16 use the
 * f32 tile path (kernels.cpp:230-251, :661-679); only F16 fuses its lane steps, as the F16C build does. */
void vo_matmul(const vo_mat *W, const float *x, int64_t m, float *y, int avx2);
void vo_matmul_q8_int(const vo_mat *W, const float *x, int64_t m, float *y, int avx2);
void vo_matmul_q4_int(const vo_mat *W, const float *x, int64_t m, float *y, int avx2);
void vo_matmul_f32_tiles(const vo_mat *W, const float *x, int64_t m, float *y);
/* dot() of kernels.cpp:268-274: 8 lanes, separate multiply and add (not multiversioned, no FMA). */
float vo_dot(const float *a, const float *b, int64_t n);

/* ---- elementwise (kernels.cpp:707-757, kernels.hpp:105) ---- */
void vo_rmsnorm(const float *x, const float *w, int64_t n, float eps, float *out);
void vo_layernorm(const float *x, const float *w, const float *b, int64_t n, float eps, float *out);
void vo_softmax(float *x, int64_t n);
float vo_silu(float x);
void vo_rope_inv_freq(int64_t hd, double theta, float *out);
void vo_rope_apply(float *x, int64_t heads, int64_t hd, const float *inv_freq, int64_t pos);

/* ---- transformer (kernels.hpp:114-147, kernels.cpp:760-906) ---- */
typedef struct {
    vo_mat q, k, v, o, gate, up, down;
    const float *qn, *kn; /* per-head RMSNorm weights [head_dim] or NULL */
    const float *ln1, *ln2;
    const float *attn_scale, *mlp_scale; /* layer scales [hidden] or NULL (the codec's pre-transformer) */
} vo_layer;

typedef struct {
    int32_t n_layers;
    const vo_layer *layers;
    const float *final_norm;
    int32_t hidden, heads, kv_heads, head_dim, inter;
    float eps;
    const float *inv_freq; /* [head_dim/2] */
    int32_t window;        /* sliding window (0: full attention): a row at position p sees keys (p - window, p] */
} vo_xfmr;

/* KV cache: k, v are [n_layers][cap][kv_heads*head_dim] floats. kv_f16 = 1 rounds every appended
 * key/value to f16 (a cache stored in f16, read back exactly widened); 0 keeps f32 like KVCache. */
typedef struct {
    float *k, *v;
    int64_t cap;
    int64_t len;
    int32_t kv_f16;
    int32_t avx2;
} vo_kv;

/* transformer_forward (kernels.cpp:760-844), with its sliding window and layer scales.
 * Returns 0, or -1 when the cache is too small. */
int vo_transformer_forward(const vo_xfmr *w, vo_kv *kv, const float *x, int64_t m, float *out_last, float *out_all);
/* Layers [first, first + count) of transformer_forward on the residual stream x [m][hidden] (rows at positions
 * kv->len ..), writing the residual stream after them to h_out (no final norm) and their keys/values to the cache;
 * kv->len is not advanced. The CPU side of the reference's hybrid placement (kernels.cpp:764-791) and the
 * per-layer parity probe of the tests. */
int vo_transformer_layers(const vo_xfmr *w, vo_kv *kv, const float *x, int64_t m, int32_t first, int32_t count, float *h_out);
/* transformer_forward_steps (kernels.cpp:846-906): one token for each of B sequences. */
int vo_transformer_forward_steps(const vo_xfmr *w, vo_kv *const *kvs, int64_t B, const float *x, float *out);

/* ---- F5-TTS DiT step (f5.cpp:86-106, :563-725; f5_ops.cpp:86-147) ---- */
float vo_gelu_tanh(float x); /* f5.cpp:93-96 */
float vo_mish(float x);      /* f5.cpp:97-100 */
/* Conv1d with "same" zero padding (odd K) and groups (f5_ops.cpp:106-147). w in Conv1d::w layout
 * [groups][cout/groups][K][cin/groups] (= GpuF5Conv, gpu.hpp:65), bias [cout] or NULL; x [T][cin] -> y [T][cout]. */
typedef struct {
    const float *w, *b;
    int32_t cin, cout, K, groups;
} vo_conv;
void vo_conv1d(const vo_conv *c, const float *x, int32_t T, float *y);
/* LayerNorm without parameters + modulation (f5.cpp:608-625): double mean / variance, eps 1e-6,
 * y = (x - float(mean)) * float(1 / sqrt(var + eps)) * (1 + scale) + shift, per row of D. */
void vo_f5_modulate(const float *x, int64_t R, int32_t D, const float *scale, const float *shift, float *y);
typedef struct {
    vo_mat ada, q, k, v, o, ff1, ff2;
} vo_f5_block;
typedef struct {
    int32_t dim, depth, heads, dim_head, ff_mult, mel_dim, text_dim, pe_attn_head;
    vo_mat in_proj, norm_out, proj_out;
    const vo_f5_block *blocks;
    vo_conv pos1, pos2;
} vo_f5;
/* dit_forward from the input projection on (f5.cpp:586-725), B batches of N rows: cat [B*N][2 mel + text] (x, cond,
 * text), ts [dim] (SiLU of the time embedding), rope [N][dim_head/2][2] (cos, sin) -> out [B*N][mel]. */
int vo_f5_step(const vo_f5 *m, int32_t B, int32_t N, const float *cat, const float *ts, const float *rope, float *out);

/* ---- F5-TTS Vocos backbone and head (f5.cpp:779-806), the iSTFT left out ---- */
float vo_gelu_erf(float x); /* kernels.hpp:106 */
typedef struct {
    vo_conv dw; /* depthwise, K 7 */
    const float *ln_w, *ln_b, *gamma;
    vo_mat pw1, pw2;
} vo_vocos_block;
typedef struct {
    int32_t dim, inter, mel_dim, layers;
    vo_conv embed;
    const float *ln_w, *ln_b, *fln_w, *fln_b;
    const vo_vocos_block *blocks;
    vo_mat head;
} vo_vocos;
/* F5Model::vocode up to the head output: mel [T][mel_dim] -> head [T][head.rows] (log-magnitude | phase). */
int vo_vocos_head(const vo_vocos *v, const float *mel, int32_t T, float *head);

/* ---- CosyVoice2 / Chatterbox flow estimator (cosyvoice.cpp:126-221, :839-863; nn.cpp, nn.hpp) ---- */
float vo_exp_poly(float x);  /* nn.cpp:16-29 */
float vo_gelu_poly(float x); /* nn.cpp:31-38: erf GELU through Numerical Recipes' erfc fit */
float vo_mish_nn(float x);   /* nn.hpp:103-107 */
/* LayerNorm with weight and bias over channels of [T][C] rows, in place (nn.cpp:248-265, modulate false). */
void vo_layer_norm_nn(float *x, int64_t T, int32_t C, const float *w, const float *b, float eps);
/* softmax_fast (nn.cpp:97-106): max, subtract, exp_poly, sum, * (1 / sum). */
void vo_softmax_fast(float *x, int64_t n);
/* attention without the score term (nn.cpp:448-500 from :473): per head, Q * scale, S = Q K^T through the F32
 * matmul, softmax_fast rows, O = S V; q/k/v/out rows of H dh floats. */
void vo_attention_nn(const float *q, const float *k, const float *v, int32_t Tq, int32_t Tk, int32_t H, int32_t dh,
                     float scale, float *out);
/* causal_conv (cosyvoice.cpp:127-131): Conv::forward (nn.cpp:179-202, groups 1, w [cout][K][cin]) of x [T][cin]
 * with K - 1 zero rows in front, bias added after the product (nn.cpp:146-155). K 1: the plain linear. */
void vo_causal_conv(const vo_conv *c, const float *x, int32_t T, float *y);
/* nn::ConvT, ConvTranspose1d with groups 1 (nn.cpp:205-245): w_pt in PyTorch's layout [cin][cout][K] is laid out as
 * rows k cout + o of cin (ConvT::load), z = x W^T through the F32 matmul in blocks of max(16, 4 Mi / (K cout)) input
 * rows, then y[t s + k - pad] += z[t][k][o] in the order t, k for 0 <= t s + k - pad < To, and the bias last.
 * x [T][cin] -> y [To][cout], To = (T - 1) s - 2 pad + K + out_pad; returns To (or -1 on bad arguments). */
int32_t vo_convt(const float *w_pt, int32_t cin, int32_t cout, int32_t K, int32_t stride, int32_t pad, int32_t out_pad,
                 const float *bias, const float *x, int32_t T, float *y);
typedef struct {
    vo_conv c1, c2, res;
    const float *n1w, *n1b, *n2w, *n2b;
} vo_cosy_res;
typedef struct {
    const float *n1w, *n1b, *n3w, *n3b;
    vo_mat q, k, v, o, ff1, ff2; /* q, k, v without bias */
} vo_cosy_x;
typedef struct {
    int32_t M, C, heads, head_dim;
    vo_cosy_res down_res, up_res;
    const vo_cosy_res *mid_res;
    int32_t n_mid;
    const vo_cosy_x *down_x, *up_x, *mid_x; /* mid block i: mid_x_count[i] consecutive entries of mid_x */
    int32_t n_down_x, n_up_x;
    const int32_t *mid_x_count;
    vo_conv down_conv, up_out, final_conv, final_proj;
    const float *fn_w, *fn_b;
} vo_cosy;
/* One estimator call (cosyvoice.cpp:839-863): in [2][T][4 M] ([x | mu | spks | cond] of both passes), tb
 * [2 + n_mid][C] (the resnets' time biases) -> out [2][T][M]. */
int vo_cosy_step(const vo_cosy *m, int32_t T, const float *in, const float *tb, float *out);

/* ---- Qwen3-TTS codec decoder (qwen3.cpp:102-161, :366-481) ---- */
/* A streaming conv: w [cout][K * cin] (+ bias in w.bias), dilation dil, causal with a history of (K - 1) dil rows. */
typedef struct {
    vo_mat w;
    int32_t K, cin, cout, dil;
} vo_cconv;
/* Snake: a = exp(alpha), inv_b = 1 / (exp(beta) + 1e-9) per channel (qwen3.cpp:80-89). */
typedef struct {
    const float *a, *inv_b;
} vo_snake;
/* An upsample stage (qwen3.cpp:254-267): transposed conv K = stride, w [K latent][latent] + bias tr_b, then a
 * ConvNeXt block: causal depthwise conv (w [C][dw_K], bias), LayerNorm (1e-6), pw1 + GELU-erf, pw2, x += gamma (.). */
typedef struct {
    vo_mat tr;
    const float *tr_b;
    int32_t K;
    const float *dw_w, *dw_b;
    int32_t dw_K;
    const float *ln_w, *ln_b, *gamma;
    vo_mat pw1, pw2;
} vo_codec_up;
/* A decoder block (qwen3.cpp:269-283): Snake, transposed conv (K = 2 stride, w [K cout][cin] + tr_b) with its
 * overlap tail, three residual units (Snake, conv K 7 dilation 1 / 3 / 9, Snake, conv K 1). */
typedef struct {
    vo_snake act;
    vo_mat tr;
    const float *tr_b;
    int32_t K, stride, cin, cout;
    vo_snake a1[3], a2[3];
    vo_cconv c1[3], c2[3];
} vo_codec_block;
typedef struct {
    int32_t codebook_size, codebook_dim, latent, quantizers, n_up, n_blocks;
    const vo_mat *q_first, *q_rest; /* [1], [quantizers - 1]: [codebook_size][codebook_dim / 2] */
    vo_mat q_first_out, q_rest_out; /* [codebook_dim][codebook_dim / 2] */
    vo_cconv pre_conv;
    vo_mat pt_in, pt_out;
    vo_xfmr pt; /* window, layer scales, no q/k norm */
    const vo_codec_up *ups;
    vo_cconv conv0;
    const vo_codec_block *blocks;
    vo_snake final_act;
    vo_cconv final_conv;
} vo_codec;
/* Streaming state (CodecState, qwen3.hpp:58-66): histories, transposed-conv tails, the transformer's f32 cache.
 * Created zeroed for a codec and a cache capacity (positions); vo_codec_state_free releases it. */
typedef struct vo_codec_state vo_codec_state;
vo_codec_state *vo_codec_state_new(const vo_codec *c, int64_t cap);
vo_codec_state *vo_codec_state_clone(const vo_codec_state *s);
void vo_codec_state_free(vo_codec_state *s);
/* The quantizer of codec_forward (qwen3.cpp:371-388): codes [F][quantizers] -> z [F][codebook_dim]. Returns -1 for a
 * code out of range. */
int vo_codec_quantize(const vo_codec *c, const int16_t *codes, int32_t F, float *z);
/* The rest of codec_forward (qwen3.cpp:405-480): z [F][codebook_dim] -> pcm [F * samples per frame], clamped to
 * [-1, 1]; the state advances. Returns the sample count, or -1 when the cache is full. */
int64_t vo_codec_forward(const vo_codec *c, vo_codec_state *s, const float *z, int32_t F, float *pcm);
/* load_snake (qwen3.cpp:80-89): a = exp(alpha), inv_b = 1 / (exp(beta) + 1e-9), in float. */
void vo_snake_params(const float *alpha, const float *beta, int64_t n, float *a, float *inv_b);
/* Samples per codec frame (the product of the upsample strides). */
int64_t vo_codec_spf(const vo_codec *c);

/* Thread count for the row-parallel loops (matmul); 1 = scalar single-thread. Results do not depend on it. */
void vo_set_threads(int n);
int vo_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
