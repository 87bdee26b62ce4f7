"""Synthetic decoder stacks built directly in HBM (weights generated and quantized on the device).

The workloads of BASELINE.json: random-init weights ~N(0, 0.02) in the reference's storage formats, norm
weights ~N(1, 0.02), a KV cache of prior tokens ~N(0, 1) stored in f16. Nothing here reads a checkpoint.
"""
import math

import numpy as np

from . import voxhip as vh

# Qwen3-TTS-0.6B-shaped talker
TALKER_0_6B = dict(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072, theta=1e6, eps=1e-6,
                   kv_len=512, head_rows=3072, wtype=vh.Q8, head_type=vh.Q8)
# Qwen3-TTS-1.7B-shaped talker with q4 body
TALKER_1_7B_Q4 = dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, theta=1e6, eps=1e-6,
                      kv_len=1024, head_rows=3072, wtype=vh.Q4, head_type=vh.Q8, f16_scales=True)
# CosyVoice2-0.5B-shaped LM: Qwen2 body (q/k/v biases, no q/k norm) in q8, f32 head 6564 x 896 with
# bias (cosyvoice.cpp:405 keeps it out of q8), f32 speech-token embedding; prefill 512, then 256 decode steps
COSY_LM_0_5B = dict(layers=24, hidden=896, heads=14, kv_heads=2, head_dim=64, inter=4864, theta=1e6, eps=1e-6,
                    kv_len=0, head_rows=6564, wtype=vh.Q8, head_type=vh.F32, qkv_bias=True, qk_norm=False,
                    head_bias=True, speech_tokens=6561, prefill=512, decode_steps=256)
# Qwen3-TTS-0.6B-shaped code predictor (the frame loop of gpu_pred_frame): 5 layers of the talker's widths, 16
# codebooks (15 passes), q8 heads of 2048 codes per codebook, bf16 code embeddings; the talker's hidden is the
# predictor's (no in_proj)
PRED_0_6B = dict(layers=5, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072, theta=1e6, eps=1e-6,
                 kv_len=0, head_rows=0, wtype=vh.Q8, head_type=vh.Q8, groups=16, vocab=2048, emb_type=vh.BF16)
NAMES = ("q", "k", "v", "o", "gate", "up", "down")


def rope_inv_freq(head_dim, theta):
    """rope_inv_freq (kernels.cpp:734-738): float(1 / theta^(2i/hd)) with the C library's pow."""
    return np.array([1.0 / math.pow(theta, (2 * i) / head_dim) for i in range(head_dim // 2)], np.float64).astype(np.float32)


class Decoder:
    """A device-resident decoder stack: per-layer matrix handles, the stacked transformer, one KV sequence, a head."""

    def __init__(self, cfg, seed=0, capacity=None, keep_mats=True):
        c = dict(cfg)
        self.cfg = c
        H, nh, nkv, hd, I, L = c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["inter"], c["layers"]
        qd, kd = nh * hd, nkv * hd
        shapes = {"q": (qd, H), "k": (kd, H), "v": (kd, H), "o": (H, qd), "gate": (I, H), "up": (I, H), "down": (H, I)}
        rng = np.random.default_rng(seed)
        self.mats = []
        layers = []
        for li in range(L):
            ids = {}
            for j, n in enumerate(NAMES):
                r, cc = shapes[n]
                ids[n] = vh.mat_synthetic(c["wtype"], r, cc, seed, 0x100 * li + j, 0.0, 0.02,
                                          bias=c.get("qkv_bias", False) and n in ("q", "k", "v"),
                                          f16_scales=c.get("f16_scales", False))
            self.mats.append(ids)
            norms = {n: (1.0 + 0.02 * rng.standard_normal(H)).astype(np.float32) for n in ("ln1", "ln2")}
            if c.get("qk_norm", True):
                norms.update({n: (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32) for n in ("qn", "kn")})
            layers.append(norms)
        self.layers = layers
        self.final_norm = (1.0 + 0.02 * rng.standard_normal(H)).astype(np.float32)
        self.inv_freq = rope_inv_freq(hd, c["theta"])
        self.desc = vh.XfmrHost(layers, self.final_norm, H, nh, nkv, hd, I, c["eps"], c["theta"], self.inv_freq)
        handles = [self.mats[li][n] for li in range(L) for n in NAMES]
        self.xfmr = vh.xfmr_create_from_mats(self.desc, handles, "talker")
        if not keep_mats:
            for ids in self.mats:
                for h in ids.values():
                    vh.mat_free(h)
            self.mats = None
        self.capacity = capacity or max(c["kv_len"] + 64, 1024)
        self.seq = vh.seq_create(self.xfmr, self.capacity)
        if c["kv_len"]:
            vh.seq_fill_synthetic(self.seq, c["kv_len"], seed, 0xC0DE, 0.0, 1.0)
        self.head = vh.mat_synthetic(c["head_type"], c["head_rows"], H, seed, 0xF00D, 0.0, 0.02,
                                     bias=c.get("head_bias", False)) if c.get("head_rows") else -1

    def extra_seq(self, stream):
        """Another sequence of the same capacity whose first kv_len positions are filled from Philox stream `stream`
        (independent sessions for the B-session step)."""
        s = vh.seq_create(self.xfmr, self.capacity)
        vh.seq_fill_synthetic(s, self.cfg["kv_len"], 0, stream, 0.0, 1.0)
        return s

    def linear_flops(self, m):
        """FLOPs of the layer matrices for m rows (2 per multiply-add)."""
        c = self.cfg
        H, qd, kd, I = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]
        return 2 * m * c["layers"] * ((qd + 2 * kd) * H + H * qd + 2 * I * H + H * I)

    def attention_flops(self, m, pos0=0):
        """FLOPs of causal attention for m rows at positions pos0..pos0+m-1 (scores and weighted values)."""
        c = self.cfg
        keys = sum(pos0 + i + 1 for i in range(m))
        return 4 * c["layers"] * c["heads"] * c["head_dim"] * keys

    def weight_bytes(self):
        """Algorithmic bytes of one decode step's weight stream (layers + head), as stored."""
        c = self.cfg
        H, qd, kd, I = c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"], c["inter"]

        def mb(t, rows, cols, bias=False):
            b = rows * 4 if bias else 0
            if t == vh.Q8:
                return rows * cols + rows * (cols // 32) * 4 + b
            if t == vh.Q4:
                return rows * cols // 2 + rows * (cols // 32) * (2 if c.get("f16_scales") else 4) + b
            return rows * cols * (4 if t == vh.F32 else 2) + b
        qb = c.get("qkv_bias", False)
        per_layer = sum(mb(c["wtype"], r, cc, bb) for r, cc, bb in ((qd + 2 * kd, H, qb), (H, qd, False), (2 * I, H, False),
                                                                     (H, I, False)))
        head = mb(c["head_type"], c["head_rows"], H, c.get("head_bias", False)) if c.get("head_rows") else 0
        return per_layer * c["layers"] + head

    def step_bytes(self, pos):
        """Algorithmic HBM bytes of one decode step at position pos: weights, f16 KV read (pos + 1 keys and values
        per layer), norm weights, and the new token's f16 K/V write."""
        c = self.cfg
        kd = c["kv_heads"] * c["head_dim"]
        kv = c["layers"] * 2 * (pos + 1) * kd * 2
        norms = c["layers"] * (2 * c["hidden"] + (2 * c["head_dim"] if c.get("qk_norm", True) else 0)) * 4 + c["hidden"] * 4
        kv_write = c["layers"] * 2 * kd * 2
        return self.weight_bytes() + kv + norms + kv_write


# F5-TTS-shaped DiT: 22 blocks, dim 1024, 16 x 64 heads, FFN 2048 (GELU-tanh), adaLN-zero, mel 100,
# text 512 (in_proj 712 -> 1024), position convolutions K 31 / 16 groups (f32); f16 linear weights ~N(0, 0.02)
F5_DIT = dict(dim=1024, depth=22, heads=16, dim_head=64, ff_mult=2, mel=100, text=512, K=31, groups=16, pe_attn_head=0,
              wtype=vh.F16, frames=1000)
# F5-TTS's Vocos (mel 100, dim 512, intermediate 1536, 8 ConvNeXt blocks, head 2 x (n_fft 1024 / 2 + 1)); 938 frames
# of hop 256 at 24 kHz are 10 s of audio
F5_VOCOS = dict(dim=512, inter=1536, layers=8, out=1026, frames=938)


# CosyVoice2's flow estimator (CosyCfg, cosyvoice.hpp:30-33): mel 80, 256 channels, 8 x 64 heads, FFN 1024 (erf GELU),
# 4 transformer blocks per level, 12 mid resnets; 512 frames = the mel of configs[4]'s 256 speech tokens
# (token_mel_ratio 2); 10 Euler steps per utterance
COSY_FLOW = dict(M=80, C=256, heads=8, head_dim=64, ff=1024, n_x=4, n_mid=12, frames=512, steps=10, wtype=vh.F16)


# Qwen3-TTS's codec decoder (the 12 Hz tokenizer, python/vox/build.py:35-38 CODEC_DEFAULTS, codebook_dim 512): 16
# codebooks of 2048, pre_conv 512 -> 1024, an 8-layer windowed transformer (hidden 1024, 16 x 64 heads, window 72,
# FFN 3072, layer scales), upsampling ratios [2, 2], decoder 1536 channels with rates [8, 5, 4, 3]: 1920 samples of
# 24 kHz per frame (80 ms); f32 weights (the converter's default codec precision)
QWEN3_CODEC = dict(codebook_dim=512, latent=1024, hidden=1024, heads=16, kv_heads=16, head_dim=64, window=72, inter=3072,
                   layers=8, ratios=[2, 2], rates=[8, 5, 4, 3], dec=1536, wtype=vh.F32)


class CodecDec:
    """A device-resident Qwen3-TTS codec decoder with synthetic weights (matrices generated on the device, the norms,
    Snake parameters and depthwise taps on the host)."""

    def __init__(self, cfg, seed=0):
        c = dict(cfg)
        self.cfg = c
        rng = np.random.default_rng(seed)
        stream = [0x9000]
        self.mats = []
        CD, L, H, hd, I, dec = c["codebook_dim"], c["latent"], c["hidden"], c["head_dim"], c["inter"], c["dec"]

        def mat(rows, cols, std, bias):
            stream[0] += 1
            h = vh.mat_synthetic(c["wtype"], rows, cols, seed, stream[0], 0.0, std, bias=bias)
            self.mats.append(h)
            return h

        def conv(K, cin, cout, dil=1, gain=1.0):
            return (mat(cout, K * cin, gain / np.sqrt(K * cin), True), K, cin, cout, dil)

        def vec(n, m, sd):
            return (m + sd * rng.standard_normal(n)).astype(np.float32)

        def snake(C):
            return (np.exp(vec(C, 0, 0.3)).astype(np.float32), (1.0 / (np.exp(vec(C, 0, 0.3)) + 1e-9)).astype(np.float32))
        qd, kd = c["heads"] * hd, c["kv_heads"] * hd
        ids, layers = [], []
        for _ in range(c["layers"]):
            ids.append([mat(qd, H, H ** -0.5, False), mat(kd, H, H ** -0.5, False), mat(kd, H, H ** -0.5, False),
                        mat(H, qd, qd ** -0.5, False), mat(I, H, H ** -0.5, False), mat(I, H, H ** -0.5, False),
                        mat(H, I, I ** -0.5, False)])
            layers.append(dict(ln1=vec(H, 1, 0.1), ln2=vec(H, 1, 0.1), attn_scale=vec(H, 0.01, 0.001),
                               mlp_scale=vec(H, 0.01, 0.001)))
        inv = (1.0 / (10000.0 ** (np.arange(0, hd, 2, dtype=np.float64) / hd))).astype(np.float32)
        pt = dict(hidden=H, heads=c["heads"], kv_heads=c["kv_heads"], head_dim=hd, inter=I, eps=1e-5, theta=10000.0,
                  window=c["window"], inv_freq=inv, final_norm=vec(H, 1, 0.1), layers=layers)
        ups = [dict(tr=mat(r * L, L, L ** -0.5, False), K=r, tr_b=vec(L, 0, 0.02), dw_w=vec(L * 7, 0, 0.3),
                    dw_b=vec(L, 0, 0.02), dw_K=7, ln_w=vec(L, 1, 0.1), ln_b=vec(L, 0, 0.1), gamma=vec(L, 0, 0.1),
                    pw1=mat(4 * L, L, L ** -0.5, True), pw2=mat(L, 4 * L, (4 * L) ** -0.5, True)) for r in c["ratios"]]
        blocks = []
        for b, r in enumerate(c["rates"]):
            ind, outd = dec >> b, dec >> (b + 1)
            blocks.append(dict(act=snake(ind), tr=mat(2 * r * outd, ind, (2 * ind) ** -0.5, False), K=2 * r, stride=r, cin=ind,
                               cout=outd, tr_b=vec(outd, 0, 0.02), a1=[snake(outd) for _ in range(3)],
                               a2=[snake(outd) for _ in range(3)],
                               c1=[conv(7, outd, outd, dil, 0.3) for dil in (1, 3, 9)],
                               c2=[conv(1, outd, outd, 1, 0.3) for _ in range(3)]))
        nb = len(c["rates"])
        self.codec = vh.codec_create(CD, L, conv(3, CD, L), mat(H, L, L ** -0.5, True), mat(L, H, H ** -0.5, True), pt, ids,
                                     ups, conv(7, L, dec), blocks, snake(dec >> nb), conv(7, dec >> nb, 1, 1, 0.1))
        self.spf = vh.codec_spf(self.codec)

    def flops_per_frame(self):
        """FLOPs of one frame (2 per multiply-add), as the layers run: pre_conv, transformer, upsampling, conv0, blocks."""
        c = self.cfg
        CD, L, H, hd, I, dec = c["codebook_dim"], c["latent"], c["hidden"], c["head_dim"], c["inter"], c["dec"]
        qd, kd = c["heads"] * hd, c["kv_heads"] * hd
        fl = 2 * 3 * CD * L + 2 * 2 * L * H
        fl += c["layers"] * (2 * H * (qd + 2 * kd + 2 * I) + 2 * qd * H + 2 * I * H + 4 * c["window"] * qd)
        pos = 1
        for r in c["ratios"]:
            fl += 2 * L * L * r * pos
            pos *= r
            fl += pos * (2 * 7 * L + 2 * 2 * 4 * L * L)
        fl += pos * 2 * 7 * L * dec
        ch = dec
        for r in c["rates"]:
            out = ch // 2
            fl += pos * 2 * ch * out * 2 * r
            pos *= r
            fl += pos * 3 * (2 * 7 * out * out + 2 * out * out)
            ch = out
        return fl + pos * 2 * 7 * ch


class CosyFlow:
    """A device-resident CosyVoice2 flow estimator with synthetic weights (linears generated on the device, the causal
    convolutions and the norms on the host)."""

    def __init__(self, cfg, seed=0):
        c = dict(cfg)
        self.cfg = c
        M, C, inner, FF = c["M"], c["C"], c["heads"] * c["head_dim"], c["ff"]
        rng = np.random.default_rng(seed)
        stream = [0x7000]
        self.mats = []

        def mat(rows, cols, bias):
            stream[0] += 1
            h = vh.mat_synthetic(c["wtype"], rows, cols, seed, stream[0], 0.0, 1.0 / np.sqrt(cols), bias=bias)
            self.mats.append(h)
            return h

        def conv(cin, cout, K):
            return ((rng.standard_normal((cout, K, cin)) / np.sqrt(K * cin)).astype(np.float32),
                    (rng.standard_normal(cout) * 0.02).astype(np.float32), cin, cout, K, 1)

        def vec(n, m, sd):
            return (m + sd * rng.standard_normal(n)).astype(np.float32)

        def res(cin):
            return dict(c1=conv(cin, C, 3), c2=conv(C, C, 3), res=conv(cin, C, 1), n1w=vec(C, 1, 0.02), n1b=vec(C, 0, 0.02),
                        n2w=vec(C, 1, 0.02), n2b=vec(C, 0, 0.02))

        def xb():
            return dict(n1w=vec(C, 1, 0.02), n1b=vec(C, 0, 0.02), n3w=vec(C, 1, 0.02), n3b=vec(C, 0, 0.02),
                        q=mat(inner, C, False), k=mat(inner, C, False), v=mat(inner, C, False), o=mat(C, inner, True),
                        ff1=mat(FF, C, True), ff2=mat(C, FF, True), ff_dim=FF)
        n_x, n_mid = c["n_x"], c["n_mid"]
        self.est = vh.cosy_create(M, C, c["heads"], c["head_dim"], res(4 * M), res(2 * C), [res(C) for _ in range(n_mid)],
                                  [xb() for _ in range(n_x)], [xb() for _ in range(n_x)],
                                  [[xb() for _ in range(n_x)] for _ in range(n_mid)], conv(C, C, 3), conv(C, C, 3),
                                  conv(C, C, 3), conv(C, M, 1), vec(C, 1, 0.02), vec(C, 0, 0.02))

    def flops(self, T):
        """FLOPs of one estimator call (both passes, 2 T rows; 2 per multiply-add)."""
        c = self.cfg
        M, C, inner, FF, R = c["M"], c["C"], c["heads"] * c["head_dim"], c["ff"], 2 * T
        resnet = lambda cin: 2 * R * C * (3 * cin + 3 * C + cin)
        xblock = 2 * R * (3 * inner * C + inner * C + 2 * FF * C) + 2 * 4 * T * T * inner
        n_x = c["n_x"] * (2 + c["n_mid"])
        convs = 3 * 2 * R * C * 3 * C + 2 * R * M * C
        return resnet(4 * M) + resnet(2 * C) + c["n_mid"] * resnet(C) + n_x * xblock + convs


class DiT:
    """A device-resident F5 DiT with synthetic weights (linears generated on the device, convolutions on the host)."""

    def __init__(self, cfg, seed=0, vocos=None):
        c = dict(cfg)
        self.cfg = c
        D, H, HD, FF, mel, text = c["dim"], c["heads"], c["dim_head"], c["dim"] * c["ff_mult"], c["mel"], c["text"]
        inner = H * HD
        stream = [0x5000]

        def mat(rows, cols):
            stream[0] += 1
            return vh.mat_synthetic(c["wtype"], rows, cols, seed, stream[0], 0.0, 0.02, bias=True)
        self.in_proj, self.norm_out, self.proj_out = mat(D, 2 * mel + text), mat(2 * D, D), mat(mel, D)
        self.blocks = [{"ada": mat(6 * D, D), "q": mat(inner, D), "k": mat(inner, D), "v": mat(inner, D), "o": mat(D, inner),
                        "ff1": mat(FF, D), "ff2": mat(D, FF)} for _ in range(c["depth"])]
        rng = np.random.default_rng(seed)
        G, K = c["groups"], c["K"]
        self.pos = [((rng.standard_normal((G, D // G, K, D // G)) * 0.02).astype(np.float32),
                     (rng.standard_normal(D) * 0.02).astype(np.float32), D, D, K, G) for _ in range(2)]
        self.vocos = None
        vk = {}
        if vocos:  # the vocoder's linears on the device, its convolutions and norms from the host
            v = dict(vocos)
            VD, VI = v["dim"], v["inter"]
            vec = lambda n, m, sd: (m + sd * rng.standard_normal(n)).astype(np.float32)
            self.vocos = v
            self.vmats = [mat(VI, VD) if i % 2 == 0 else mat(VD, VI) for i in range(2 * v["layers"])] + [mat(v["out"], VD)]
            vk = dict(vocos=dict(dim=VD, inter=VI, out=v["out"],
                                 embed=((rng.standard_normal((1, VD, 7, mel)) * 0.02).astype(np.float32), vec(VD, 0, 0.02),
                                        mel, VD, 7, 1),
                                 ln_w=vec(VD, 1, 0.02), ln_b=vec(VD, 0, 0.02), fln_w=vec(VD, 1, 0.02), fln_b=vec(VD, 0, 0.02),
                                 head=self.vmats[-1],
                                 blocks=[dict(dw=((rng.standard_normal((VD, 7)) * 0.1).astype(np.float32), vec(VD, 0, 0.02),
                                                  VD, VD, 7, VD),
                                              ln_w=vec(VD, 1, 0.02), ln_b=vec(VD, 0, 0.02), gamma=vec(VD, 0, 0.1),
                                              pw1=self.vmats[2 * i], pw2=self.vmats[2 * i + 1]) for i in range(v["layers"])]))
        self.f5 = vh.f5_create(D, c["depth"], H, HD, c["ff_mult"], mel, text, c["pe_attn_head"], self.in_proj, self.norm_out,
                               self.proj_out, self.blocks, self.pos[0], self.pos[1], **vk)

    def vocos_flops(self, T):
        """FLOPs of the Vocos backbone and head for T frames (2 per multiply-add)."""
        v, mel = self.vocos, self.cfg["mel"]
        VD, VI = v["dim"], v["inter"]
        return 2 * T * (VD * 7 * mel + v["layers"] * (VD * 7 + 2 * VD * VI) + v["out"] * VD)

    def flops(self, B, N):
        """FLOPs of one step (2 per multiply-add): linears, attention, position convolutions, ada / final GEMVs."""
        c = self.cfg
        D, HD, H, FF = c["dim"], c["dim_head"], c["heads"], c["dim"] * c["ff_mult"]
        R, inner = B * N, H * HD
        lin = 2 * R * c["depth"] * (3 * inner * D + inner * D + 2 * FF * D)
        att = 4 * B * N * N * HD * H * c["depth"]
        conv = 2 * 2 * R * D * c["K"] * (D // c["groups"])
        io = 2 * R * (2 * c["mel"] + c["text"]) * D + 2 * R * D * c["mel"]
        ada = 2 * c["depth"] * 6 * D * D + 2 * 2 * D * D
        return {"linears": lin, "attention": att, "pos_conv": conv, "in_out": io, "ada": ada}
