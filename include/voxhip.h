/*
 * voxhip.h — C ABI of the MI355X (gfx950) compute backend for Vox.
 *
 * This is the drop-in boundary. Every entry point flattens one function of the
 * reference's device interface (/root/reference/src/gpu.hpp plus the gpu_* hooks
 * declared in /root/reference/src/kernels.hpp:88-100) into plain pointers and
 * sizes. No C++ or HIP types cross it. vox_amd/csrc/gpu_hip.cpp implements the
 * unchanged vox::gpu_* C++ interface on top of it.
 *
 * Conventions (as the reference backend, gpu_vulkan.cpp:568-571, :800-803):
 *  - no exception crosses the boundary;
 *  - failure returns -1 (handles) or 0 (bool-like int), and the reason is
 *    kept in voxhip_last_error();
 *  - one device per process; every entry point takes one global lock, so the
 *    library is thread-safe, and calls serialise.
 * Handles are small non-negative ints, as in the reference.
 */
#ifndef VOXHIP_H
#define VOXHIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VOXHIP_ABI_VERSION 1

/* Weight element types, numbered as vox::WType (kernels.hpp:42). */
enum voxhip_wtype { VOXHIP_F32 = 0, VOXHIP_F16 = 1, VOXHIP_BF16 = 2, VOXHIP_Q8 = 3, VOXHIP_Q4 = 4 };

/* Host view of a weight matrix; fields as vox::Mat (kernels.hpp:44-56): [rows][cols] row-major,
 * rows = outputs. Q8: int8 data + f32 scale [rows][cols/32]. Q4: 16 bytes per 32-block
 * (byte j = w[j] | w[j+16] << 4, value (u - 8) * scale), f32 scale [rows][cols/32].
 * bias: f32 [rows] or NULL. All pointers are host memory, read during the call only. */
typedef struct voxhip_mat {
    int32_t type;
    const void *data;
    const float *scale;
    int64_t rows, cols;
    const float *bias;
} voxhip_mat;

/* vox::GpuDeviceInfo (gpu.hpp:22-30); strings are fixed-size, NUL-terminated. */
typedef struct voxhip_device_info {
    int32_t index;
    char name[256];
    char type[16];
    int32_t software, unified_memory;
    uint64_t vram_total, vram_free, max_storage_range;
    int32_t subgroup_arith, coop_matrix, memory_budget;
    uint32_t api_version, vendor_id, driver_version;
} voxhip_device_info;

/* vox::GpuStats (gpu.hpp:16) without last_error (see voxhip_last_error). */
typedef struct voxhip_stats {
    int64_t mats_ok, mats_failed;
    uint64_t bytes, bytes_failed;
} voxhip_stats;

/* vox::GpuMemInfo (gpu.hpp:35). */
typedef struct voxhip_mem_info {
    uint64_t used, limit, device_free, device_total;
    int32_t device_index;
} voxhip_mem_info;

/* ---------------------------------------------------------------- device, init, accounting */
/* gpu_enumerate (gpu.hpp:31): number of devices; 0 when the HIP runtime finds none. */
int voxhip_device_count(void);
/* gpu_enumerate entry `index`: 1 on success. */
int voxhip_device_info_get(int index, voxhip_device_info *out);
/* gpu_init (gpu.hpp:10). device: "hip", "hip:N", "gpu:N", or "vulkan:N" as family.cpp:94 passes it
 * (N = device index, also taken from VOX_VK_DEVICE like gpu_vulkan.cpp:160). Failure is sticky,
 * as gpu_vulkan.cpp:364. Returns 1 on success; on failure writes the reason to err. */
int voxhip_init(const char *device, char *err, size_t err_len);
int voxhip_active(void);                                   /* gpu_active (gpu.hpp:11) */
/* The GPU profile of VOX_PROFILE=gpu (gpu_vulkan.cpp:62-87, :312-326): when the variable holds "gpu" at init, every
 * kernel launch is timed on the device and booked under "<stage>/<kernel>" (stage: the transformer's name, "matmul",
 * "predictor", "f5.step", "f5.vocos", "flow.est", "codec", ...); this returns the table of the launches booked so far
 * (calls, total ms, average us, share, sorted by time; launches are booked when a synchronous call or voxhip_sync
 * returns), and the library prints it to stderr at exit. Empty when the profile is off. Graphs are not captured while
 * it is on (stamped launches cannot be), so timings are those of launches issued one by one; the voxhip_bench_*
 * entry points refuse to run. The text stays valid until the next call. */
const char *voxhip_profile_report(void);
const char *voxhip_device_name(void);                      /* gpu_device_name (gpu.hpp:12) */
void voxhip_stats_get(voxhip_stats *out);                  /* gpu_stats (gpu.hpp:17) */
/* GpuStats::last_error (gpu.hpp:16): copied under the library lock into a buffer of the calling thread, valid
 * until that thread's next voxhip_last_error call (a failure on another thread cannot change it). */
const char *voxhip_last_error(void);
void voxhip_set_vram_limit(uint64_t bytes);                /* gpu_set_vram_limit (gpu.hpp:34) */
void voxhip_mem_info_get(voxhip_mem_info *out);            /* gpu_mem_info (gpu.hpp:36) */

/* ---------------------------------------------------------------- matrices */
/* gpu_upload (gpu.hpp:14). n_parts > 1 stacks the parts' rows into one device matrix (same type
 * and cols, all or none with bias), as upload_parts (gpu_vulkan.cpp:476-536). Returns a handle or -1.
 * Q4 matrices whose block scales are all exact in f16 keep them in 2 bytes on the device (identical products,
 * a 10% smaller stream); voxhip_mat_download returns them widened to f32. */
int voxhip_upload(const voxhip_mat *parts, int n_parts);
/* gpu_matmul (kernels.hpp:89): y[m][rows] = x[m][cols] . W^T (+ bias), host x and y.
 * Semantics of matmul (kernels.cpp:653-705): Q8 with m <= 8 and Q4 quantize x per 32-block to int8
 * and use integer dots; Q8 with m > 8 and F32/F16/BF16 use f32 activations. Returns 1 or 0. */
int voxhip_matmul(int mat, const float *x, int64_t m, float *y);
/* voxhip_matmul on device-resident rows, allocating nothing: d_y [m][rows] = d_x [m][cols] . W^T (+ bias), with the
 * arithmetic of voxhip_matmul (the same kernels and m-dependent paths). No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). It calls no hipMalloc / hipFree: the split-K partial sums and the int path's once-quantized
 * input rows live in a fixed 6.3 MiB array in the library's code object (one copy per device, held until the
 * process ends); passes whose scratch would not fit (more than 1.5 Mi floats of partials, or more than 8 x 32768
 * quantized elements) run the same kernels without it, so no size is refused for lack of scratch. Every call on a
 * device shares that array: calls are serialised on the library's stream, and calls that overlap on one GPU (for
 * example the same call captured into graphs replayed on two streams at once) race on it. Asynchronous on the
 * library's stream (voxhip_sync waits). Returns 1 or 0. */
int voxhip_matmul_dev_noalloc(int mat, const float *d_x, int64_t m, float *d_y);
/* mat_gather (kernels.cpp:468-471, through mat_row :432-466) on the device: out [n][cols] = row ids[i] of the
 * matrix widened to f32 (F16 / BF16 exactly, Q8 float(q) * s, Q4 float(u - 8) * s), the unpack the device
 * embedding gathers of the LM and the code predictor use. Host ids and out; an id outside the rows fails (0) before
 * anything is written, as check_id does before the gathers (backend_qwen3.cpp:305-306). No counterpart in gpu.hpp. */
int voxhip_mat_gather(int mat, const int32_t *ids, int64_t n, float *out);
/* Rows and cols of a device matrix (0 on a bad handle). */
int voxhip_mat_shape(int mat, int64_t *rows, int64_t *cols);
/* nn::ConvT::forward (nn.cpp:217-245; ConvTranspose1d, groups 1) on the device: `mat` holds the transposed conv's
 * weights as ConvT::load lays them out (nn.cpp:205-215), K cout rows of cin (row k cout + o; the reference's ConvT
 * matrix is F32, any uploaded type is accepted) and no bias. x [T][cin] (host) -> y [To][cout] (host),
 * To = (T - 1) stride - 2 pad + K + out_pad; bias [cout] or NULL is added after the overlap-add. 1 on success, 0 on
 * error (voxhip_last_error). */
int voxhip_convt(int mat, int32_t K, int32_t stride, int32_t pad, int32_t out_pad, const float *bias, const float *x, int32_t T,
                 float *y);

/* ---------------------------------------------------------------- transformer */
/* vox::LayerW (kernels.hpp:114-119). attn_scale / mlp_scale must be NULL (as gpu_vulkan.cpp:782). */
typedef struct voxhip_layer {
    voxhip_mat q, k, v, o, gate, up, down;
    const float *qn, *kn;  /* per-head RMSNorm [head_dim] or NULL (both or none) */
    const float *ln1, *ln2;
    const float *attn_scale, *mlp_scale;
} voxhip_layer;

/* vox::TransformerW (kernels.hpp:120-130). window must be 0 and head_dim even and <= 128 (as gpu_vulkan.cpp:770;
 * 64 and 128 run the split-K decode and MFMA prefill attention, other sizes a one-block-per-head kernel);
 * heads / kv_heads <= 8. inv_freq: [head_dim/2], as rope_inv_freq (kernels.cpp:734-738). */
typedef struct voxhip_xfmr_desc {
    int32_t n_layers;
    const voxhip_layer *layers;
    const float *final_norm;
    int32_t hidden, heads, kv_heads, head_dim, inter;
    float eps;
    double theta;
    int32_t window;
    const float *inv_freq;
} voxhip_xfmr_desc;

/* Called once per uploaded matrix (layer, which = 0..6 for q,k,v,o,gate,up,down) right after its
 * upload, so the caller may release the host pages (gpu.hpp:37-40, qwen3.cpp:309-316). */
typedef void (*voxhip_uploaded_fn)(void *user, int32_t layer, int32_t which);

/* gpu_xfmr_create (gpu.hpp:40). n_layers < 0 = all layers. Returns a handle or -1. */
int voxhip_xfmr_create(const voxhip_xfmr_desc *w, const char *name, int n_layers, voxhip_uploaded_fn uploaded, void *user);
/* gpu_seq_create (gpu.hpp:42): a KV cache of `capacity` positions (f16, on the device). The reference
 * caps capacity at 3072 (gpu_vk_internal.hpp:34); this backend accepts up to 65536. Returns a handle or -1. */
int voxhip_seq_create(int xfmr, int64_t capacity);
void voxhip_seq_free(int seq);                             /* gpu_seq_free (gpu.hpp:43); buffers stay pooled */
/* gpu_xfmr_forward (kernels.hpp:92-93): x [m][in_proj ? in_proj.cols : hidden] at positions pos0..pos0+m-1;
 * out_last [hidden] = final RMSNorm of the last row (may be NULL); head >= 0: head_out [head.rows] = head
 * applied to out_last. in_proj / head are matrix handles or -1. Returns 1 or 0. */
int voxhip_xfmr_forward(int xfmr, int seq, int64_t pos0, const float *x, int64_t m, float *out_last, int in_proj,
                        int head, float *head_out);
/* gpu_xfmr_forward_hidden (kernels.hpp:96): the device layers only, no final norm: hidden_out [m][hidden]. */
int voxhip_xfmr_forward_hidden(int xfmr, int seq, int64_t pos0, const float *x, int64_t m, float *hidden_out);
/* Layers [first, first + count) only, on the residual stream x [m][hidden] (no input projection, no final norm):
 * hidden_out [m][hidden]. Generalizes the hybrid placement of gpu_xfmr_forward_hidden (the reference runs the first
 * gpu_layers layers on the device and the rest on the CPU, kernels.cpp:764-791) to any contiguous range. */
int voxhip_xfmr_forward_layers(int xfmr, int seq, int64_t pos0, const float *x, int64_t m, int32_t first, int32_t count,
                               float *hidden_out);
/* gpu_xfmr_forward_pair (kernels.hpp:99-100): one token of each of two sequences at the same position. */
int voxhip_xfmr_forward_pair(int xfmr, int seq0, int seq1, int64_t pos, const float *x2, int head, float *out2,
                             float *head_out2);
/* transformer_forward_steps (kernels.hpp:144-147) on the device: one token for each of B sequences
 * (seqs[b] at position pos[b]); weights are read once for all B. out [B][hidden] normed; head >= 0:
 * head_out [B][head.rows]. B <= 8. Returns 1 or 0. */
int voxhip_xfmr_forward_steps(int xfmr, const int32_t *seqs, const int64_t *pos, int64_t B, const float *x,
                              float *out, int head, float *head_out);

/* ---------------------------------------------------------------- sampling */
/* vox::SampleParams (sampling.hpp:52-57) + the Philox counter of DetRng::uniform (sampling.hpp:40-44)
 * + the logit mask the engine applies before sampling code 0 (engine.cpp:664-668):
 * logits[suppress_from .. suppress_to) = -inf except eos_code; eos_code also -inf when block_eos. */
typedef struct voxhip_sample_cfg {
    float temperature, top_p;
    int32_t top_k;
    float repetition_penalty;
    uint32_t key0, key1;       /* DetRng key: seed low / high 32 bits */
    uint64_t frame;
    uint32_t codebook, draw;
    int32_t suppress_from, suppress_to, eos_code, block_eos;
} voxhip_sample_cfg;

/* sample_logits (sampling.hpp:61-119) on the device, from host logits [n] and history [n_history].
 * Writes the sampled index to *out_id. n <= 65536. Returns 1 or 0. */
int voxhip_sample_logits(const float *logits, int32_t n, const voxhip_sample_cfg *cfg, const int32_t *history,
                         int32_t n_history, int32_t *out_id);

/* gpu_pred_frame (gpu.hpp:51-52; gpu_vulkan.cpp:968-1045): the code predictor's whole frame on the device. With
 * G = n_heads + 1 codebooks: pass 1 runs the 2 rows of in2 ([2][din]: the talker's hidden state and the first
 * code's embedding) at positions 0 and 1 of seq, pass cb >= 2 one row at position cb, the embedding row
 * embs[cb - 2][codes[cb - 1]]; each pass goes through in_proj (or none: din = hidden), the layers, the final norm
 * and heads[cb - 1] on its last row, and sample_logits with cfg's temperature / top-k / top-p and the draw
 * (cfg->frame, cb) into codes[cb]. codes[0] is not written. Returns 1, or 0 with the error set. */
int voxhip_pred_frame(int xfmr, int seq, const float *in2, int in_proj, const int *heads, int n_heads, const int *embs,
                      int n_embs, const voxhip_sample_cfg *cfg, int32_t *codes);

/* ---------------------------------------------------------------- device-resident path
 * Entry points for callers that keep activations in device memory (bench, tests, a device-side
 * generate loop). Pointers named d_* are device pointers from voxhip_dev_alloc. */
void *voxhip_dev_alloc(size_t bytes);
void voxhip_dev_free(void *p);
int voxhip_memcpy_h2d(void *d_dst, const void *src, size_t bytes);
int voxhip_memcpy_d2h(void *dst, const void *d_src, size_t bytes);
int voxhip_sync(void);

/* One decode step with everything on the device: d_x [m][hidden] -> layers -> final norm of the last row
 * (d_out_last [hidden], may be NULL) -> head (d_logits [head.rows]) -> sampler (d_token, when cfg != NULL).
 * Launched as one captured HIP graph per (xfmr, seq, m, head, cfg != NULL); asynchronous on the library's
 * stream. Returns 1 or 0. */
int voxhip_decode_dev(int xfmr, int seq, int64_t pos0, const float *d_x, int64_t m, float *d_out_last, int head,
                      float *d_logits, const voxhip_sample_cfg *cfg, int32_t *d_token);

/* transformer_forward_steps (kernels.hpp:144-147) on device-resident inputs: one token for each of B (1..8)
 * distinct sequences at its own position pos[b], in one captured graph per sequence list (weights read once for
 * the B rows). d_x [B][hidden]; d_out (or NULL) [B][hidden] normed states; with head >= 0, d_logits (or NULL)
 * [B][head rows]; with cfgs != NULL, row b is sampled with cfgs[b] into d_tokens[b]. Asynchronous. */
int voxhip_decode_steps_dev(int xfmr, const int32_t *seqs, const int64_t *pos, int64_t B, const float *d_x, float *d_out,
                            int head, float *d_logits, const voxhip_sample_cfg *cfgs, int32_t *d_tokens);

/* ---------------------------------------------------------------- CosyVoice2 LM (cosyvoice.cpp:598-690)
 * The reference runs this loop on the host around gpu_xfmr_forward and gpu_matmul (cosyvoice.cpp:573-575,
 * :598-607); these entry points keep it on the device: head + bias -> lm_logp -> ras_sample with the trial loop
 * of lm_generate -> the speech-token embedding of the pick -> the layers at the next position. */
typedef struct voxhip_lm_cfg {
    float top_p;            /* CosyCfg::top_p: keep while the sorted cumulative probability < top_p (> 0) */
    int32_t top_k;          /* CosyCfg::top_k: at most top_k kept, 1..1024 */
    int32_t win_size;       /* CosyCfg::win_size: repetition window of decoded tokens, 0..1024 */
    float tau_r;            /* CosyCfg::tau_r: resample when the pick occurs >= win_size * tau_r times */
    int32_t speech_tokens;  /* CosyCfg::speech_tokens: ids >= speech_tokens end the generation */
    int32_t min_len;        /* lm_generate's min_len (text length * min_ratio): no end before this step */
    int32_t max_len;        /* lm_generate's max_len (text length * max_ratio): at most max_len steps */
    uint32_t piece;         /* Philox stream 0x43560000 + piece (cosyvoice.cpp:672) */
    uint64_t seed;          /* DetRng(seed) */
} voxhip_lm_cfg;
/* lm_logp + the trial loop of lm_generate for step `step` (cosyvoice.cpp:598-607, :674-683) on device logits
 * [n] (head output + bias, n 2..8192) with the decoded tokens d_decoded [n_decoded] (device). d_logp (optional,
 * device [n]): the log-probabilities before the trials. *token: the pick (>= speech_tokens: the end). Fails
 * (0) where the reference fails: more than 101 trials that end before min_len. */
int voxhip_lm_sample_dev(const float *d_logits, int32_t n, const voxhip_lm_cfg *cfg, int64_t step, const int32_t *d_decoded,
                         int32_t n_decoded, float *d_logp, int32_t *token);
/* lm_begin's prefill + lm_generate's loop (cosyvoice.cpp:564-596, :666-690) on the device: x [n][hidden] (host,
 * the gathered prompt embeddings) at positions 0..n-1 of seq, then up to max_len steps of final norm -> head
 * (with its bias) -> lm_logp -> RAS trial loop -> row `token` of speech_emb -> layers at the next position.
 * tokens [max_len] receives the decoded tokens (the end token excluded), *n_tokens their count; logp (optional,
 * host [max_len][head rows]) the log-probabilities of every step that sampled. The sequence needs
 * n + max_len + 1 positions (its last slot takes the writes of steps launched after the end). */
int voxhip_lm_generate(int xfmr, int seq, const float *x, int64_t n, int head, int speech_emb, const voxhip_lm_cfg *cfg,
                       int32_t *tokens, float *logp, int32_t *n_tokens);

/* ---------------------------------------------------------------- F5-TTS DiT step (gpu.hpp:62-91)
 * The whole dit_forward (f5.cpp:586-725) of a sampling step on the device, and Vocos up to its head. */
/* GpuF5Conv (gpu.hpp:66): f32 weights in Conv1d::w layout [groups][cout/groups][K][cin/groups], bias [cout] or NULL.
 * The position convolutions need cin = cout = dim, odd K and cin/groups a multiple of 4. */
typedef struct voxhip_f5_conv {
    const float *w, *b;
    int32_t cin, cout, K, groups;
} voxhip_f5_conv;
/* GpuF5Desc::Block (gpu.hpp:70): matrix handles of one DiT block. q, k, v are stacked on the device at create. */
typedef struct voxhip_f5_block {
    int32_t ada, q, k, v, o, ff1, ff2;
} voxhip_f5_block;
/* GpuF5Desc::VBlock (gpu.hpp:78): a Vocos ConvNeXt block; dw depthwise (groups = cin = cout, w [C][K]). */
typedef struct voxhip_f5_vblock {
    voxhip_f5_conv dw;
    const float *ln_w, *ln_b, *gamma; /* [vocos_dim] */
    int32_t pw1, pw2;                 /* matrix handles: vocos_inter x vocos_dim, vocos_dim x vocos_inter */
} voxhip_f5_vblock;
/* GpuF5Desc (gpu.hpp:67-81). dim_head even and <= 64 (as gpu_f5.cpp:211; heads below 64 run on zero-padded
 * attention tiles). vocos_dim 0: no Vocos (gpu_f5_vocos then fails and the caller
 * runs the vocoder on the CPU); else v_embed (mel_dim -> vocos_dim), the norms, n_vblocks blocks and v_head
 * (vocos_out x vocos_dim). */
typedef struct voxhip_f5_desc {
    int32_t dim, depth, heads, dim_head, ff_mult, mel_dim, text_dim, pe_attn_head;
    int32_t in_proj, norm_out, proj_out;
    const voxhip_f5_block *blocks; /* [depth] */
    voxhip_f5_conv pos1, pos2;
    int32_t vocos_dim, vocos_inter, vocos_out;
    voxhip_f5_conv v_embed;
    const float *v_ln_w, *v_ln_b, *v_fln_w, *v_fln_b;
    const voxhip_f5_vblock *v_blocks; /* [n_vblocks] */
    int32_t n_vblocks, v_head;
} voxhip_f5_desc;
int voxhip_f5_create(const voxhip_f5_desc *d);  /* gpu_f5_create (gpu.hpp:82): a handle or -1 */
/* gpu_f5_begin (gpu.hpp:85): B sequences of N rows; cat0 [B][N][2 mel + text] (zeros in the x columns),
 * rope [N][dim_head/2][2] (cos, sin). */
int voxhip_f5_begin(int id, int B, int N, const float *cat0, const float *rope);
/* gpu_f5_step (gpu.hpp:87): x [N][mel] (the same for every sequence), ts [dim] = SiLU(time embedding) ->
 * out [B][N][mel]. */
int voxhip_f5_step(int id, const float *x, const float *ts, float *out);
int voxhip_f5_end(int id);  /* gpu_f5_end (gpu.hpp:90): frees the step buffers, keeps the weights */
/* gpu_f5_vocos (gpu.hpp:88-89; gpu_f5.cpp:334-373, the CPU path f5.cpp:792-806): mel [T][mel_dim] -> the Vocos head
 * output head [T][vocos_out] (log-magnitude | phase); the iSTFT stays with the caller. */
int voxhip_f5_vocos(int id, const float *mel, int T, float *head);
/* The Vocos head width of an F5 handle into *vout (0 when created without Vocos). Returns 1, or 0 for a bad handle.
 * No counterpart in gpu.hpp: gpu_hip.cpp sizes gpu_f5_vocos's output with it. */
int voxhip_f5_vocos_out(int id, int32_t *vout);

/* ---------------------------------------------------------------- CosyVoice2 / Chatterbox flow estimator
 * (gpu.hpp:100-119; the CPU estimator cosyvoice.cpp:126-221, :822-863). One Euler step runs the conditional and the
 * unconditional pass together as sequences 0 and 1 of T rows each (rows R = 2 T). Convolutions are f32 in
 * Conv1d::w layout [cout][K][cin] (groups 1), causal (left zero padding K - 1 per sequence) for the K-3 block and
 * level convolutions, K 1 for res and final_proj; linears are matrix handles (q, k, v without bias). */
/* GpuCosyDesc::Res (gpu.hpp:105): CausalResnetBlock1D, c1 (cin -> C), c2 (C -> C), res (cin -> C, K 1), the two
 * LayerNorms (weight, bias [C]). */
typedef struct voxhip_cosy_res {
    voxhip_f5_conv c1, c2, res;
    const float *n1w, *n1b, *n2w, *n2b;
} voxhip_cosy_res;
/* GpuCosyDesc::X (gpu.hpp:106): a BasicTransformerBlock, norms [C] and matrix handles (q, k, v: inner x C; o:
 * C x inner; ff1: ff_dim x C; ff2: C x ff_dim). */
typedef struct voxhip_cosy_x {
    const float *n1w, *n1b, *n3w, *n3b;
    int32_t q, k, v, o, ff1, ff2, ff_dim;
} voxhip_cosy_x;
/* GpuCosyDesc (gpu.hpp:103-113). The reference's vector of mid transformer lists is flattened: mid block i owns
 * mid_x_count[i] consecutive entries of mid_x. head_dim even and <= 64 (as gpu_f5.cpp:425), C a multiple of 4. */
typedef struct voxhip_cosy_desc {
    int32_t M, C, heads, head_dim;
    voxhip_cosy_res down_res, up_res;
    const voxhip_cosy_res *mid_res; /* [n_mid] */
    int32_t n_mid;
    const voxhip_cosy_x *down_x, *up_x, *mid_x;
    int32_t n_down_x, n_up_x;
    const int32_t *mid_x_count; /* [n_mid] */
    voxhip_f5_conv down_conv, up_out, final_conv, final_proj;
    const float *fn_w, *fn_b;
} voxhip_cosy_desc;
int voxhip_cosy_create(const voxhip_cosy_desc *d); /* gpu_cosy_create (gpu.hpp:114): a handle or -1 */
/* gpu_cosy_begin (gpu.hpp:116): in0 [2][T][4 M], the estimator input [x | mu | spks | cond] of both passes with the
 * x columns left zero. */
int voxhip_cosy_begin(int id, int T, const float *in0);
/* gpu_cosy_step (gpu.hpp:118): x [T][M] (the same for both passes), tb [2 + n_mid][C] the time-embedding bias of
 * every resnet (down, mid..., up) -> out [2][T][M]. */
int voxhip_cosy_step(int id, const float *x, const float *tb, float *out);
int voxhip_cosy_end(int id); /* gpu_cosy_end (gpu.hpp:119): frees the step buffers, keeps the weights */

/* ---------------------------------------------------------------- Qwen3-TTS codec decoder (gpu.hpp:53-60)
 * gpu_codec_forward's chain (gpu_codec.cpp:400-556; the CPU path qwen3.cpp:390-480) from the quantizer output z on:
 * pre_conv (causal K 3) -> pre-transformer (sliding window, layer scales, an f32 ring cache) -> upsample stages
 * (transposed conv K = stride + causal ConvNeXt) -> conv0 -> decoder blocks (Snake, transposed conv K = 2 stride
 * with its overlap tail, 3 residual units) -> Snake -> final conv -> clamp. Streaming state (conv histories, tails,
 * ring) lives on the device. Weights are matrix handles of F32 / F16 / BF16 type; the rest host arrays. */
typedef struct voxhip_codec_conv {
    int32_t mat;              /* [cout][K cin] with its bias (CConv::w, qwen3.hpp:45) */
    int32_t K, cin, cout, dil;
} voxhip_codec_conv;
typedef struct voxhip_codec_snake {
    const float *a, *inv_b;   /* exp(alpha), 1 / (exp(beta) + 1e-9) [C] (Snake, qwen3.hpp:48) */
} voxhip_codec_snake;
/* Qwen3Weights::UpStage (qwen3.hpp:96): tr [K latent][latent], K = stride. */
typedef struct voxhip_codec_up {
    int32_t tr, K;
    const float *tr_b;          /* [latent] */
    const float *dw_w, *dw_b;   /* depthwise [latent][dw_K], [latent] */
    int32_t dw_K;
    const float *ln_w, *ln_b, *gamma;
    int32_t pw1, pw2;
} voxhip_codec_up;
/* Qwen3Weights::DecBlock (qwen3.hpp:99): tr [K cout][cin], stride < K <= 2 stride. */
typedef struct voxhip_codec_block {
    voxhip_codec_snake act;
    int32_t tr, K, stride, cin, cout;
    const float *tr_b;          /* [cout] */
    voxhip_codec_snake a1[3], a2[3];
    voxhip_codec_conv c1[3], c2[3];
} voxhip_codec_block;
/* The decoder of Qwen3Weights (qwen3.hpp:90-104, CodecCfg :29-41). pt: the pre-transformer's TransformerW (window,
 * eps, inv_freq, norms and layer scales; its voxhip_mat entries are ignored), pt_mats its matrix handles [layers][7]
 * (q, k, v, o, gate, up, down; no biases, no q / k norm). */
typedef struct voxhip_codec_desc {
    int32_t codebook_dim, latent;
    voxhip_codec_conv pre_conv;
    int32_t pt_in, pt_out;
    voxhip_xfmr_desc pt;
    const int32_t *pt_mats;
    const voxhip_codec_up *ups;
    int32_t n_ups;
    voxhip_codec_conv conv0;
    const voxhip_codec_block *blocks;
    int32_t n_blocks;
    voxhip_codec_snake final_act;
    voxhip_codec_conv final_conv;
} voxhip_codec_desc;
int voxhip_codec_create(const voxhip_codec_desc *d);   /* gpu_codec_create (gpu.hpp:55): a handle or -1 */
int voxhip_codec_state_new(int codec);                 /* gpu_codec_state_new (gpu.hpp:56): zeroed state, or -1 */
int voxhip_codec_state_clone(int state);               /* gpu_codec_state_clone (gpu.hpp:57): a deep copy, or -1 */
int voxhip_codec_state_free(int state);                /* gpu_codec_state_free (gpu.hpp:58) */
/* gpu_codec_forward (gpu.hpp:60): z [F][codebook_dim], 1 <= F <= 16 (kGpuCodecMaxFrames, gpu.hpp:61) -> pcm
 * [F samples_per_frame] (clamped), *n_out the count; the state advances. */
int voxhip_codec_forward(int codec, int state, const float *z, int F, float *pcm, int64_t *n_out);
/* Samples per codec frame into *spf (no counterpart in gpu.hpp: the adapter sizes gpu_codec_forward's output). */
int voxhip_codec_spf(int codec, int32_t *spf);

/* Synthetic weights and caches, generated on the device (Philox4x32-10 Box-Muller, mean + std * z).
 * voxhip_mat_synthetic: f32 values, then quantized on the device to `type` with the reference's
 * quantizer (Q8: kernels.cpp:918-929; Q4: kernels.cpp:606-645; F16/BF16: nearest even). Returns a handle.
 * flags: VOXHIP_SYN_BIAS adds an f32 bias ~N(0, std); VOXHIP_SYN_F16_SCALES rounds Q4 block scales to f16 (the
 * "4-bit + f16 scale" format; the matrix then stores 2-byte scales, see voxhip_upload). */
enum { VOXHIP_SYN_BIAS = 1, VOXHIP_SYN_F16_SCALES = 2 };
int voxhip_mat_synthetic(int32_t type, int64_t rows, int64_t cols, uint64_t seed, uint32_t stream, float mean,
                         float std, int flags);
/* Copies a device matrix back in the reference host layout (data, scale, bias may be NULL). */
int voxhip_mat_download(int mat, void *data, float *scale, float *bias);
/* Releases a device matrix that no transformer uses (the reference keeps uploads for the process lifetime;
 * this is for synthetic setups that restack matrices). Returns 1 or 0. */
int voxhip_mat_free(int mat);
/* Creates a transformer from matrices already on the device: per layer the handles of q,k,v,o,gate,up,down
 * (7 ints per layer, in that order) and host norm vectors from desc (desc->layers[i].ln1 etc; the voxhip_mat
 * fields of desc->layers are ignored). */
int voxhip_xfmr_create_from_mats(const voxhip_xfmr_desc *w, const int32_t *mats, const char *name);
/* Fills positions [0, len) of every layer of a KV cache with N(mean, std) values rounded to f16. */
int voxhip_seq_fill_synthetic(int seq, int64_t len, uint64_t seed, uint32_t stream, float mean, float std);
/* Copies positions [0, len) of layer `layer` of a KV cache to host f32 k, v [len][kv_heads*head_dim]. */
int voxhip_seq_download(int seq, int32_t layer, int64_t len, float *k, float *v);

/* Device quantizers of the reference formats (kernels.cpp:918-929, :606-645, :515-523) on device memory. */
int voxhip_quantize_q8_dev(const float *d_w, int64_t rows, int64_t cols, int8_t *d_q, float *d_scale);
int voxhip_quantize_q4_dev(const float *d_w, int64_t rows, int64_t cols, uint8_t *d_q, float *d_scale);
int voxhip_quantize_act_dev(const float *d_x, int64_t n, int8_t *d_xq, float *d_xs);

/* ---------------------------------------------------------------- measurement */
/* Kernel classes of one decode step, for voxhip_bench_result. */
enum voxhip_kernel_class {
    VOXHIP_K_QKV = 0,      /* RMSNorm + q|k|v GEMV */
    VOXHIP_K_O = 1,        /* o GEMV + residual */
    VOXHIP_K_GATEUP = 2,   /* RMSNorm + gate|up GEMV + SwiGLU */
    VOXHIP_K_DOWN = 3,     /* down GEMV + residual */
    VOXHIP_K_HEAD = 4,     /* final RMSNorm + head GEMV */
    VOXHIP_K_ATTN = 5,     /* split-K attention over the f16 cache */
    VOXHIP_K_COMBINE = 6,  /* merge of the attention splits */
    VOXHIP_K_QKPOST = 7,   /* q/k RMSNorm, RoPE, f16 K/V append */
    VOXHIP_K_SAMPLE = 8,   /* device sampler */
    VOXHIP_K_FFN = 9,      /* one-row FFN in one launch: RMSNorm + gate|up + SwiGLU + down, product into accumulators */
    VOXHIP_K_FOLD = 10,    /* the last layer's accumulated FFN product into h */
    VOXHIP_K_QUANT = 11,   /* the input rows of a several-row int-path GEMV quantized once (k_quant_rows) */
    VOXHIP_K_CLASSES = 12
};

/* Times `steps` replays of the captured decode graph (after `warmup` untimed ones) with HIP events on the
 * library's stream: ms_per_step. Then runs `steps` more steps launching the same kernels one by one, each with
 * start/stop events stamped at that kernel's own start and end (hipExtLaunchKernel): per-class average launch
 * durations and the algorithmic bytes one launch of each class moves. */
typedef struct voxhip_bench_result {
    double ms_per_step;         /* whole decode step (graph replay), average */
    double launch_ms_per_step;  /* host time of one hipGraphLaunch call in the timed loop (a step is host-bound when this
                                   approaches ms_per_step) */
    double kernel_ms_per_step;  /* sum of the kernel durations of one step (event-stamped run) */
    double step_bytes;          /* algorithmic HBM bytes per step (weights + scales, KV read + write, norms) */
    int32_t kernels_per_step;
    int32_t n_classes;
    int32_t kernel_stamped;     /* 1: hipExtLaunchKernel events at kernel start/end; 0: stream events around each launch
                                   (used when a profiler intercepts launches) */
    double class_ms[VOXHIP_K_CLASSES];        /* average duration of one launch of the class */
    double class_bytes[VOXHIP_K_CLASSES];     /* algorithmic bytes of one launch of the class */
    int32_t class_launches[VOXHIP_K_CLASSES]; /* launches per step */
} voxhip_bench_result;
int voxhip_bench_decode(int xfmr, int seq, int64_t pos0, const float *d_x, int head, const voxhip_sample_cfg *cfg,
                        int32_t *d_token, int warmup, int steps, voxhip_bench_result *out);
/* The same for a step of B sessions (voxhip_decode_steps_dev: row b at position pos[b] of sequence seqs[b]); the
 * per-class bytes count every row's activations and cache. */
int voxhip_bench_decode_steps(int xfmr, const int32_t *seqs, const int64_t *pos, int64_t B, const float *d_x, int head,
                              const voxhip_sample_cfg *cfgs, int32_t *d_tokens, int warmup, int steps,
                              voxhip_bench_result *out);

/* Times one GEMV kernel configuration on `copies` distinct device copies of a synthetic q8 matrix
 * (rotating, so the working set exceeds the 256 MB Infinity Cache): average ms per launch. */
int voxhip_bench_gemv_q8(int64_t rows, int64_t cols, int copies, int warmup, int iters, double *ms_per_launch);

/* Times the split-f16 MFMA GEMM of the multi-row passes (prefill, DiT and flow-estimator linears) on one product
 * shape: y [m][n] = (A_hi + A_lo) [m][K] . W [n][K]^T, A_hi ~N(0, 1) and A_lo ~N(0, 1e-3) as f16 planes, W ~N(0,
 * 0.02) as f16 or (q8 != 0) in its q8 form (int8 values widened to f16, per-32 block scales). tile 0 takes the
 * library's shape policy; 1..4 force one of its block tiles (rows of A x rows of W: 32x32, 32x64, 64x64, 64x128 of
 * 8 waves); every tile gives the same bits (the same MFMA sequence per output). The inputs are those of
 * voxhip_mat_synthetic(F16, m, K, 11, 0x90, 0, 1) (A_hi), (F16, m, K, 12, 0x91, 0, 1e-3) (A_lo) and (F16 or Q8, n, K,
 * 13, 0x92, 0, 0.02) (W). Average microseconds per launch; y_out (host, may be NULL) receives y of
 * the last launch. K must be a multiple of 64. No reference counterpart (benchmark helper). */
int voxhip_bench_gemm_hh(int64_t m, int64_t n, int64_t K, int q8, int tile, int warmup, int iters, double *us_per_launch,
                         float *y_out);

/* BASELINE configs[0] on the device: one q8 FFN block (RMSNorm -> gate|up GEMV + SwiGLU -> down GEMV + residual,
 * two kernels) over `copies` distinct weight sets in one graph, so the working set exceeds the 256 MB Infinity
 * Cache: average microseconds per block. Copy c's gate|up matrix [2 inter][hidden] (gate row u at row 2u, up row u
 * at 2u + 1) is voxhip_mat_synthetic(Q8, 2 inter, hidden, 2000 + c, 0x60, 0, 0.02), its down matrix the same with
 * (hidden, inter, stream 0x61); x ~N(0, 1) and gamma ~N(1, 0.02) come from the same generator (seeds 7 / 8, streams
 * 0x70 / 0x71), eps 1e-6. check (host, may be NULL): [3][hidden] = x, gamma and copy 0's block applied once to x,
 * for the parity test. No reference counterpart (benchmark helper). */
int voxhip_bench_ffn_q8(int64_t hidden, int64_t inter, int copies, int warmup, int iters, double *us_per_block, float *check);

/* Times a plain 16-byte device copy of `bytes` (STREAM copy; reads and writes `bytes` each): average ms per copy.
 * The same kernel calibrates the HBM traffic counters. No reference counterpart (benchmark helper). */
int voxhip_bench_copy(int64_t bytes, int warmup, int iters, double *ms_per_copy);

/* Self-test of the packed f16 split the F5 / flow-estimator attention uses for P (v_cvt_pk_f16_f32 and
 * v_fma_mix{lo,hi}_f16): `pairs` pseudo-random f32 pairs (half of them in the f16 subnormal .. overflow range) split
 * both that way and as hi = f16(x), lo = f16(x - hi); *mismatches = the pairs whose bits differ (NaN inputs skipped).
 * No reference counterpart (a check of this build's instruction sequence). */
int voxhip_selftest_split_f16(int64_t pairs, int64_t *mismatches);

#ifdef __cplusplus
}
#endif
#endif
