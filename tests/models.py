"""Random Qwen3-shaped transformers and matrices for the parity tests.

Weights are built once on the host in the reference layout (vox::Mat) and handed to both sides: the oracle
(pyoracle) and the HIP backend (vox_amd.voxhip) consume the same stored int8 / u4 / f16 / bf16 / f32 bytes.
"""
import numpy as np

import pyoracle as po

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4


def to_bf16_bits(w):
    u = np.ascontiguousarray(w, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_round(w):
    """w rounded to bfloat16 values (nearest even), as f32."""
    b = to_bf16_bits(np.ascontiguousarray(w, np.float32)).astype(np.uint32) << 16
    return b.view(np.float32).reshape(w.shape)


def make_mat(rng, wtype, rows, cols, std=0.02, bias=False):
    """Returns (data, scale, bias) in the reference layout for wtype."""
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    b = (rng.standard_normal(rows) * std).astype(np.float32) if bias else None
    if wtype == Q8:
        q, s = po.quantize_q8(w)
        return q, s, b
    if wtype == Q4:
        q, s = po.quantize_q4(w)
        return q, s, b
    if wtype == F16:
        return w.astype(np.float16).view(np.uint16), None, b
    if wtype == BF16:
        return to_bf16_bits(w), None, b
    return w, None, b


class Model:
    """A transformer in both host descriptions: `ox` for the oracle, `hx` for the HIP backend."""

    def __init__(self, seed, n_layers, hidden, heads, kv_heads, head_dim, inter, wtype=Q8, qk_norm=True, bias=False, theta=1e6,
                 eps=1e-6, head_rows=0, head_type=None, ffn_bias=False):
        from vox_amd import voxhip
        rng = np.random.default_rng(seed)
        self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter = hidden, heads, kv_heads, head_dim, inter
        self.n_layers, self.eps, self.wtype = n_layers, eps, wtype
        qd, kd = heads * head_dim, kv_heads * head_dim
        self.inv_freq = np.empty(head_dim // 2, np.float32)
        po.lib().vo_rope_inv_freq(head_dim, theta, self.inv_freq.ctypes.data)
        olayers, hlayers = [], []
        self.keep = []
        shapes = {"q": (qd, hidden), "k": (kd, hidden), "v": (kd, hidden), "o": (hidden, qd), "gate": (inter, hidden),
                  "up": (inter, hidden), "down": (hidden, inter)}
        for _ in range(n_layers):
            oL, hL = {}, {}
            for n, (r, c) in shapes.items():
                d, s, b = make_mat(rng, wtype, r, c, bias=(bias and n in ("q", "k", "v")) or (ffn_bias and n in ("gate", "up", "down")))
                oL[n] = po.Mat(wtype, d, r, c, s, b)
                hL[n] = voxhip.HostMat(wtype, d, r, c, s, b)
            for n in ("ln1", "ln2"):
                v = (1.0 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
                oL[n] = hL[n] = v
            if qk_norm:
                for n in ("qn", "kn"):
                    v = (1.0 + 0.02 * rng.standard_normal(head_dim)).astype(np.float32)
                    oL[n] = hL[n] = v
            olayers.append(oL)
            hlayers.append(hL)
        self.final_norm = (1.0 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
        self.ox = po.Xfmr(olayers, self.final_norm, hidden, heads, kv_heads, head_dim, inter, eps, self.inv_freq)
        self.hx = voxhip.XfmrHost(hlayers, self.final_norm, hidden, heads, kv_heads, head_dim, inter, eps, theta, self.inv_freq)
        self.head = None
        if head_rows:
            ht = head_type if head_type is not None else wtype
            d, s, b = make_mat(rng, ht, head_rows, hidden)
            self.head = (po.Mat(ht, d, head_rows, hidden, s, b), voxhip.HostMat(ht, d, head_rows, hidden, s, b))

    def oracle_kv(self, cap, kv_f16=1):
        return po.KV(self.n_layers, cap, self.kv_heads * self.head_dim, kv_f16=kv_f16)


def f5_rope(N, hd):
    """The rope table of gpu_f5_begin: [N][hd/2][2] (cos, sin) at angle i * theta^(-2j/hd), theta 10000 (f5.cpp:528-539)."""
    HH = hd // 2
    inv = np.array([np.float32(1.0 / 10000.0 ** (2 * j / hd)) for j in range(HH)], np.float32)
    a = (np.arange(N, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return np.stack([np.cos(a), np.sin(a)], axis=-1).astype(np.float32)


class F5Model:
    """A random F5-TTS DiT in both descriptions: `ox` for the oracle, `hip` (create kwargs with host matrices) for the
    backend. Linear weights of type wtype (~N(0, std)) with biases; position convolutions f32 in Conv1d::w layout."""

    def __init__(self, seed, dim, depth, heads, dim_head=64, ff_mult=2, mel=20, text=32, K=7, groups=4, pe_attn_head=0,
                 wtype=F16, std=0.05, vocos=None):
        rng = np.random.default_rng(seed)
        self.dim, self.depth, self.heads, self.hd, self.mel, self.text = dim, depth, heads, dim_head, mel, text
        self.ff_mult, self.pe = ff_mult, pe_attn_head
        inner, ff, W = heads * dim_head, dim * ff_mult, 2 * mel + text

        def mat(rows, cols, s=std):
            d, sc, b = make_mat(rng, wtype, rows, cols, std=s, bias=True)
            return (wtype, d, rows, cols, sc, b)
        self.mats = {"in_proj": mat(dim, W), "norm_out": mat(2 * dim, dim), "proj_out": mat(mel, dim)}
        self.blocks = []
        for _ in range(depth):
            self.blocks.append({"ada": mat(6 * dim, dim), "q": mat(inner, dim), "k": mat(inner, dim), "v": mat(inner, dim),
                                "o": mat(dim, inner), "ff1": mat(ff, dim), "ff2": mat(dim, ff)})
        cig = dim // groups

        def conv():
            w = (rng.standard_normal((groups, dim // groups, K, cig)) * 0.05).astype(np.float32)
            b = (rng.standard_normal(dim) * 0.05).astype(np.float32)
            return (w, b, dim, dim, K, groups)
        self.pos = [conv(), conv()]
        om = {k: po.Mat(*v) for k, v in self.mats.items()}
        ob = [{k: po.Mat(*v) for k, v in b.items()} for b in self.blocks]
        oc = [po.Conv(*c) for c in self.pos]
        self.ox = po.F5(dim, depth, heads, dim_head, ff_mult, mel, text, pe_attn_head, om["in_proj"], om["norm_out"],
                        om["proj_out"], ob, oc[0], oc[1])
        self.vocos = None
        if vocos:  # dict(dim, inter, layers, out[, wtype]): Vocos backbone + head (f5.cpp:333-346)
            vd, vi, vt = vocos["dim"], vocos["inter"], vocos.get("wtype", wtype)

            def vmat(rows, cols, s=0.05):
                d, sc, b = make_mat(rng, vt, rows, cols, std=s, bias=True)
                return (vt, d, rows, cols, sc, b)

            def vec(n, mean, sd):
                return (mean + sd * rng.standard_normal(n)).astype(np.float32)
            v = {"dim": vd, "inter": vi, "out": vocos["out"],
                 "embed": ((rng.standard_normal((1, vd, 7, mel)) * 0.1).astype(np.float32), vec(vd, 0, 0.05), mel, vd, 7, 1),
                 "ln_w": vec(vd, 1, 0.1), "ln_b": vec(vd, 0, 0.1), "fln_w": vec(vd, 1, 0.1), "fln_b": vec(vd, 0, 0.1),
                 "head": vmat(vocos["out"], vd), "blocks": []}
            for _ in range(vocos["layers"]):
                v["blocks"].append({"dw": ((rng.standard_normal((vd, 7)) * 0.3).astype(np.float32), vec(vd, 0, 0.05), vd, vd, 7, vd),
                                    "ln_w": vec(vd, 1, 0.1), "ln_b": vec(vd, 0, 0.1), "gamma": vec(vd, 0, 0.1),
                                    "pw1": vmat(vi, vd), "pw2": vmat(vd, vi)})
            self.vocos = v
            self.vox = po.Vocos(vd, vi, mel, po.Conv(*v["embed"]), v["ln_w"], v["ln_b"],
                                [{"dw": po.Conv(*b["dw"]), "ln_w": b["ln_w"], "ln_b": b["ln_b"], "gamma": b["gamma"],
                                  "pw1": po.Mat(*b["pw1"]), "pw2": po.Mat(*b["pw2"])} for b in v["blocks"]],
                                v["fln_w"], v["fln_b"], po.Mat(*v["head"]))

    def create(self, hip):
        h = {k: hip.upload(hip.HostMat(*v)) for k, v in self.mats.items()}
        hb = [{k: hip.upload(hip.HostMat(*v)) for k, v in b.items()} for b in self.blocks]
        vk = {}
        if self.vocos:
            v = self.vocos
            vk = dict(vocos=dict(dim=v["dim"], inter=v["inter"], out=v["out"], embed=v["embed"], ln_w=v["ln_w"],
                                 ln_b=v["ln_b"], fln_w=v["fln_w"], fln_b=v["fln_b"], head=hip.upload(hip.HostMat(*v["head"])),
                                 blocks=[dict(dw=b["dw"], ln_w=b["ln_w"], ln_b=b["ln_b"], gamma=b["gamma"],
                                              pw1=hip.upload(hip.HostMat(*b["pw1"])), pw2=hip.upload(hip.HostMat(*b["pw2"])))
                                         for b in v["blocks"]]))
        return hip.f5_create(self.dim, self.depth, self.heads, self.hd, self.ff_mult, self.mel, self.text, self.pe,
                             h["in_proj"], h["norm_out"], h["proj_out"], hb, self.pos[0], self.pos[1], **vk)

    def inputs(self, rng, B, N):
        """cat0 [B N][2 mel + text] with zeros in the x columns, x [N][mel], ts [dim], rope."""
        cat0 = rng.standard_normal((B * N, 2 * self.mel + self.text)).astype(np.float32)
        cat0[:, :self.mel] = 0.0
        x = rng.standard_normal((N, self.mel)).astype(np.float32)
        ts = rng.standard_normal(self.dim).astype(np.float32)
        return cat0, x, ts, f5_rope(N, self.hd)

    @staticmethod
    def with_x(cat0, x, B):
        cat = cat0.copy()
        N = x.shape[0]
        for b in range(B):
            cat[b * N:(b + 1) * N, :x.shape[1]] = x
        return cat


class CosyModel:
    """A random CosyVoice2 / Chatterbox flow estimator (CausalConditionalDecoder with one channel level) in both
    descriptions: `ox` for the oracle, `create(hip)` for the backend. Convolutions f32 in Conv::w layout
    [cout][K][cin] with std 1 / sqrt(K cin); linears of type wtype, q / k / v without bias."""

    def __init__(self, seed, M=8, C=64, heads=2, head_dim=64, n_mid=1, n_x=1, ff=128, wtype=F32, std=None):
        rng = np.random.default_rng(seed)
        self.M, self.C, self.heads, self.hd, self.ff, self.wtype = M, C, heads, head_dim, ff, wtype
        inner = heads * head_dim

        def conv(cin, cout, K):
            w = (rng.standard_normal((cout, K, cin)) / np.sqrt(K * cin)).astype(np.float32)
            return (w, (rng.standard_normal(cout) * 0.05).astype(np.float32), cin, cout, K, 1)

        def vec(n, mean, sd):
            return (mean + sd * rng.standard_normal(n)).astype(np.float32)

        def mat(rows, cols, bias):
            d, sc, b = make_mat(rng, wtype, rows, cols, std=std or 1.0 / np.sqrt(cols), bias=bias)
            if b is not None:
                b = (b * 0.05 * np.sqrt(cols)).astype(np.float32)
            return (wtype, d, rows, cols, sc, b)

        def res(cin):
            return {"c1": conv(cin, C, 3), "c2": conv(C, C, 3), "res": conv(cin, C, 1), "n1w": vec(C, 1, 0.1),
                    "n1b": vec(C, 0, 0.1), "n2w": vec(C, 1, 0.1), "n2b": vec(C, 0, 0.1)}

        def xb():
            return {"n1w": vec(C, 1, 0.1), "n1b": vec(C, 0, 0.1), "n3w": vec(C, 1, 0.1), "n3b": vec(C, 0, 0.1),
                    "q": mat(inner, C, False), "k": mat(inner, C, False), "v": mat(inner, C, False), "o": mat(C, inner, True),
                    "ff1": mat(ff, C, True), "ff2": mat(C, ff, True)}
        self.down_res, self.up_res = res(4 * M), res(2 * C)
        self.mid_res = [res(C) for _ in range(n_mid)]
        self.down_x, self.up_x = [xb() for _ in range(n_x)], [xb() for _ in range(n_x)]
        self.mid_x = [[xb() for _ in range(n_x)] for _ in range(n_mid)]
        self.convs = {"down_conv": conv(C, C, 3), "up_out": conv(C, C, 3), "final_conv": conv(C, C, 3),
                      "final_proj": conv(C, M, 1)}
        self.fn = (vec(C, 1, 0.1), vec(C, 0, 0.1))
        self.n_res = 2 + n_mid

        def ores(r):
            return {**{k: po.Conv(*r[k]) for k in ("c1", "c2", "res")}, **{k: r[k] for k in ("n1w", "n1b", "n2w", "n2b")}}

        def ox(x):
            return {k: (po.Mat(*v) if isinstance(v, tuple) else v) for k, v in x.items()}
        oc = {k: po.Conv(*v) for k, v in self.convs.items()}
        self.ox = po.Cosy(M, C, heads, head_dim, ores(self.down_res), ores(self.up_res), [ores(r) for r in self.mid_res],
                          [ox(x) for x in self.down_x], [ox(x) for x in self.up_x], [[ox(x) for x in v] for v in self.mid_x],
                          oc["down_conv"], oc["up_out"], oc["final_conv"], oc["final_proj"], *self.fn)

    def create(self, hip):
        def hx(x):
            d = {k: (hip.upload(hip.HostMat(*v)) if isinstance(v, tuple) else v) for k, v in x.items()}
            d["ff_dim"] = self.ff
            return d
        return hip.cosy_create(self.M, self.C, self.heads, self.hd, self.down_res, self.up_res, self.mid_res,
                               [hx(x) for x in self.down_x], [hx(x) for x in self.up_x], [[hx(x) for x in v] for v in self.mid_x],
                               self.convs["down_conv"], self.convs["up_out"], self.convs["final_conv"],
                               self.convs["final_proj"], *self.fn)

    def inputs(self, rng, T):
        """in0 [2 T][4 M] as cosyvoice.cpp:806-815 fills it (pass 0: [0 | mu | spks | cond], pass 1 all zero),
        x [T][M], tb [2 + n_mid][C]."""
        M = self.M
        in0 = np.zeros((2 * T, 4 * M), np.float32)
        in0[:T, M:] = rng.standard_normal((T, 3 * M)).astype(np.float32)
        in0[:T, 2 * M:3 * M] = in0[0, 2 * M:3 * M]  # spks: one vector for every row
        x = rng.standard_normal((T, M)).astype(np.float32)
        tb = (rng.standard_normal((self.n_res, self.C)) * 0.5).astype(np.float32)
        return in0, x, tb

    def with_x(self, in0, x):
        inp = in0.copy()
        T = x.shape[0]
        inp[:T, :self.M] = x
        inp[T:, :self.M] = x
        return inp


CODEC_TINY = dict(codebook_size=16, hidden_size=32, latent_dim=16, num_attention_heads=2, num_key_value_heads=2,
                  head_dim=16, sliding_window=5, intermediate_size=64, layer_scale_initial_scale=0.5, rms_norm_eps=1e-5,
                  num_hidden_layers=2, num_quantizers=4, upsample_rates=[2, 3], upsampling_ratios=[2, 2],
                  decoder_dim=32, codebook_dim=16, rope_theta=10000.0)


class CodecModel:
    """A random Qwen3-TTS codec decoder by .tmod tensor name (f32, the layouts qwen3.cpp:225-283 reads): `t` the
    tensors, `ox` the oracle's Codec, `write_tmod` a whole Qwen3-TTS .tmod for the compiled reference (a minimal
    talker and predictor beside the codec, which Qwen3Weights loads too)."""

    def __init__(self, seed, cc=None, wround=F32):
        cc = dict(CODEC_TINY if cc is None else cc)
        self.cc = cc
        rng = np.random.default_rng(seed)
        t = {}

        def w(name, rows, cols, std=None):
            t[name] = (rng.standard_normal((rows, cols)) * (std or 1.0 / np.sqrt(cols))).astype(np.float32)

        def v(name, n, mean=0.0, sd=0.1):
            t[name] = (mean + sd * rng.standard_normal(n)).astype(np.float32)
        Q, CD, L, H = cc["num_quantizers"], cc["codebook_dim"], cc["latent_dim"], cc["hidden_size"]
        heads, kvh, hd, I = cc["num_attention_heads"], cc["num_key_value_heads"], cc["head_dim"], cc["intermediate_size"]
        dim, cs = CD // 2, cc["codebook_size"]
        w("codec.quantizer.rvq_first.vq.layers.0._codebook.embedding", cs, dim, 1.0)
        for i in range(Q - 1):
            w(f"codec.quantizer.rvq_rest.vq.layers.{i}._codebook.embedding", cs, dim, 0.5)
        w("codec.quantizer.rvq_first.output_proj.weight", CD, dim)
        w("codec.quantizer.rvq_rest.output_proj.weight", CD, dim)

        def conv(p, K, cin, cout, std=None):
            w(p + ".weight", cout, K * cin, std)
            v(p + ".bias", cout, 0.0, 0.05)
        conv("codec.pre_conv.conv", 3, CD, L)
        w("codec.pre_transformer.input_proj.weight", H, L)
        v("codec.pre_transformer.input_proj.bias", H)
        w("codec.pre_transformer.output_proj.weight", L, H)
        v("codec.pre_transformer.output_proj.bias", L)
        for i in range(cc["num_hidden_layers"]):
            p = f"codec.pre_transformer.layers.{i}."
            w(p + "self_attn.q_proj.weight", heads * hd, H)
            w(p + "self_attn.k_proj.weight", kvh * hd, H)
            w(p + "self_attn.v_proj.weight", kvh * hd, H)
            w(p + "self_attn.o_proj.weight", H, heads * hd)
            w(p + "mlp.gate_proj.weight", I, H)
            w(p + "mlp.up_proj.weight", I, H)
            w(p + "mlp.down_proj.weight", H, I)
            v(p + "input_layernorm.weight", H, 1.0)
            v(p + "post_attention_layernorm.weight", H, 1.0)
            v(p + "self_attn_layer_scale.scale", H, cc["layer_scale_initial_scale"], 0.1)
            v(p + "mlp_layer_scale.scale", H, cc["layer_scale_initial_scale"], 0.1)
        v("codec.pre_transformer.norm.weight", H, 1.0)
        for s_, r in enumerate(cc["upsampling_ratios"]):
            p = f"codec.upsample.{s_}."
            w(p + "0.conv.weight", r * L, L)
            v(p + "0.conv.bias", L)
            w(p + "1.dwconv.conv.weight", L, 7, 0.3)
            v(p + "1.dwconv.conv.bias", L)
            v(p + "1.norm.weight", L, 1.0)
            v(p + "1.norm.bias", L)
            v(p + "1.gamma", L, 0.0, 0.3)
            w(p + "1.pwconv1.weight", 4 * L, L)
            v(p + "1.pwconv1.bias", 4 * L)
            w(p + "1.pwconv2.weight", L, 4 * L)
            v(p + "1.pwconv2.bias", L)
        dec = cc["decoder_dim"]
        conv("codec.decoder.0.conv", 7, L, dec)

        def snake(p, C):
            v(p + ".alpha", C, 0.0, 0.3)
            v(p + ".beta", C, 0.0, 0.3)
        for b, r in enumerate(cc["upsample_rates"]):
            ind, outd = dec >> b, dec >> (b + 1)
            p = f"codec.decoder.{b + 1}.block."
            snake(p + "0", ind)
            w(p + "1.conv.weight", 2 * r * outd, ind, 1.0 / np.sqrt(2 * ind))  # two taps overlap per output
            v(p + "1.conv.bias", outd)
            for u in range(3):  # residual units scaled down so the stack keeps unit-size activations
                q = p + f"{u + 2}."
                snake(q + "act1", outd)
                conv(q + "conv1.conv", 7, outd, outd, 0.3 / np.sqrt(7 * outd))
                snake(q + "act2", outd)
                conv(q + "conv2.conv", 1, outd, outd, 0.3 / np.sqrt(outd))
        nb = len(cc["upsample_rates"])
        snake(f"codec.decoder.{nb + 1}", dec >> nb)
        conv(f"codec.decoder.{nb + 2}.conv", 7, dec >> nb, 1, 0.1 / np.sqrt(7 * (dec >> nb)))
        if wround == F16:  # the matrices as the device stores them, so both sides see the same weights
            t = {k: (a.astype(np.float16).astype(np.float32) if a.ndim == 2 else a) for k, a in t.items()}
        elif wround == BF16:
            t = {k: (bf16_round(a) if a.ndim == 2 else a) for k, a in t.items()}
        self.t = t
        self.ox = po.Codec(cc, t)
        self.spf = self.ox.spf

    def create(self, hip, wtype=F32):
        """The device codec (gpu_codec_create) over the same tensors, linears and convs uploaded as wtype."""
        cc, t = self.cc, self.t
        mats = []

        def up(name, bias=None):
            w = t[name]
            d = w.astype(np.float16).view(np.uint16) if wtype == F16 else (to_bf16_bits(w) if wtype == BF16 else w)
            h = hip.upload(hip.HostMat(wtype, d, w.shape[0], w.shape[1], None, None if bias is None else t[bias]))
            mats.append(h)
            return h

        def conv(p, K, cin, cout, dil=1):
            return (up(p + ".weight", p + ".bias"), K, cin, cout, dil)

        def snake(p):
            a = np.empty(t[p + ".alpha"].size, np.float32)
            ib = np.empty_like(a)
            po.lib().vo_snake_params(t[p + ".alpha"].ctypes.data, t[p + ".beta"].ctypes.data, a.size, a.ctypes.data,
                                     ib.ctypes.data)
            return (a, ib)
        CD, L, H = cc["codebook_dim"], cc["latent_dim"], cc["hidden_size"]
        heads, hd = cc["num_attention_heads"], cc["head_dim"]
        layers, ids = [], []
        for i in range(cc["num_hidden_layers"]):
            p = f"codec.pre_transformer.layers.{i}."
            ids.append([up(p + k + ".weight") for k in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                                        "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")])
            layers.append(dict(ln1=t[p + "input_layernorm.weight"], ln2=t[p + "post_attention_layernorm.weight"],
                               attn_scale=t[p + "self_attn_layer_scale.scale"], mlp_scale=t[p + "mlp_layer_scale.scale"]))
        inv = np.empty(hd // 2, np.float32)
        po.lib().vo_rope_inv_freq(hd, cc.get("rope_theta", 10000.0), inv.ctypes.data)
        pt = dict(hidden=H, heads=heads, kv_heads=cc["num_key_value_heads"], head_dim=hd, inter=cc["intermediate_size"],
                  eps=cc.get("rms_norm_eps", 1e-5), theta=cc.get("rope_theta", 10000.0), window=cc["sliding_window"],
                  inv_freq=inv, final_norm=t["codec.pre_transformer.norm.weight"], layers=layers)
        ups = []
        for s_, r in enumerate(cc["upsampling_ratios"]):
            p = f"codec.upsample.{s_}."
            ups.append(dict(tr=up(p + "0.conv.weight"), K=r, tr_b=t[p + "0.conv.bias"], dw_w=t[p + "1.dwconv.conv.weight"],
                            dw_b=t[p + "1.dwconv.conv.bias"], dw_K=7, ln_w=t[p + "1.norm.weight"], ln_b=t[p + "1.norm.bias"],
                            gamma=t[p + "1.gamma"], pw1=up(p + "1.pwconv1.weight", p + "1.pwconv1.bias"),
                            pw2=up(p + "1.pwconv2.weight", p + "1.pwconv2.bias")))
        dec, blocks = cc["decoder_dim"], []
        for b, r in enumerate(cc["upsample_rates"]):
            ind, outd = dec >> b, dec >> (b + 1)
            p = f"codec.decoder.{b + 1}.block."
            blocks.append(dict(act=snake(p + "0"), tr=up(p + "1.conv.weight"), K=2 * r, stride=r, cin=ind, cout=outd,
                               tr_b=t[p + "1.conv.bias"], a1=[snake(p + f"{u + 2}.act1") for u in range(3)],
                               a2=[snake(p + f"{u + 2}.act2") for u in range(3)],
                               c1=[conv(p + f"{u + 2}.conv1.conv", 7, outd, outd, dil) for u, dil in enumerate((1, 3, 9))],
                               c2=[conv(p + f"{u + 2}.conv2.conv", 1, outd, outd) for u in range(3)]))
        nb = len(cc["upsample_rates"])
        self.mats = mats
        return hip.codec_create(CD, L, conv("codec.pre_conv.conv", 3, CD, L), up("codec.pre_transformer.input_proj.weight",
                                "codec.pre_transformer.input_proj.bias"), up("codec.pre_transformer.output_proj.weight",
                                "codec.pre_transformer.output_proj.bias"), pt, ids, ups, conv("codec.decoder.0.conv", 7, L, dec),
                                blocks, snake(f"codec.decoder.{nb + 1}"), conv(f"codec.decoder.{nb + 2}.conv", 7, dec >> nb, 1))

    def codes(self, rng, F):
        return rng.integers(0, self.cc["codebook_size"], (F, self.cc["num_quantizers"])).astype(np.int16)

    def write_tmod(self, path):
        hid = 8
        tc = dict(hidden_size=hid, intermediate_size=hid, num_hidden_layers=1, num_attention_heads=1, num_key_value_heads=1,
                  head_dim=hid, vocab_size=8, text_hidden_size=hid, text_vocab_size=8, num_code_groups=2,
                  codec_eos_token_id=1, codec_think_id=2, codec_nothink_id=3, codec_think_bos_id=4, codec_think_eos_id=5,
                  codec_pad_id=6, codec_bos_id=7)
        pc = dict(hidden_size=hid, intermediate_size=hid, num_hidden_layers=1, num_attention_heads=1, num_key_value_heads=1,
                  head_dim=hid, vocab_size=8)
        ids = dict(im_start=0, im_end=1, tts_pad=2, tts_bos=3, tts_eos=4)
        t = dict(self.t)
        z = lambda *s: np.zeros(s, np.float32)
        for p in ("talker.model.", "talker.code_predictor.model."):
            L = p + "layers.0."
            for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
                      "mlp.up_proj", "mlp.down_proj"):
                t[L + n + ".weight"] = z(hid, hid)
            for n in ("input_layernorm", "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm"):
                t[L + n + ".weight"] = z(hid)
            t[p + "norm.weight"] = z(hid)
        for n in ("talker.model.codec_embedding.weight", "talker.model.text_embedding.weight", "talker.codec_head.weight",
                  "talker.text_projection.linear_fc1.weight", "talker.text_projection.linear_fc2.weight",
                  "talker.code_predictor.model.codec_embedding.0.weight", "talker.code_predictor.lm_head.0.weight"):
            t[n] = z(8, hid)
        t["talker.text_projection.linear_fc1.weight"] = z(hid, hid)
        t["talker.text_projection.linear_fc2.weight"] = z(hid, hid)
        po.tmod_write(path, {"qwen3": {"talker": tc, "predictor": pc, "codec": self.cc, "ids": ids}}, t)
