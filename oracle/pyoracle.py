"""ctypes binding of the CPU parity checker (oracle/liboracle.so) and of the
compiled reference harness (oracle/_ref/libvoxref.so, present only where it
was built from /root/reference).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py. The product (vox_amd/) never imports it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libvoxref.so")

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4


class VoMat(C.Structure):
    _fields_ = [("type", C.c_int32), ("data", C.c_void_p), ("scale", C.c_void_p),
                ("rows", C.c_int64), ("cols", C.c_int64), ("bias", C.c_void_p)]


class VoLayer(C.Structure):
    _fields_ = [(n, VoMat) for n in ("q", "k", "v", "o", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("qn", "kn", "ln1", "ln2", "attn_scale", "mlp_scale")]


class VoXfmr(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("layers", C.POINTER(VoLayer)), ("final_norm", C.c_void_p),
                ("hidden", C.c_int32), ("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("inter", C.c_int32), ("eps", C.c_float), ("inv_freq", C.c_void_p), ("window", C.c_int32)]


class VoCConv(C.Structure):
    _fields_ = [("w", VoMat), ("K", C.c_int32), ("cin", C.c_int32), ("cout", C.c_int32), ("dil", C.c_int32)]


class VoSnake(C.Structure):
    _fields_ = [("a", C.c_void_p), ("inv_b", C.c_void_p)]


class VoCodecUp(C.Structure):
    _fields_ = [("tr", VoMat), ("tr_b", C.c_void_p), ("K", C.c_int32), ("dw_w", C.c_void_p), ("dw_b", C.c_void_p),
                ("dw_K", C.c_int32), ("ln_w", C.c_void_p), ("ln_b", C.c_void_p), ("gamma", C.c_void_p), ("pw1", VoMat),
                ("pw2", VoMat)]


class VoCodecBlock(C.Structure):
    _fields_ = [("act", VoSnake), ("tr", VoMat), ("tr_b", C.c_void_p), ("K", C.c_int32), ("stride", C.c_int32),
                ("cin", C.c_int32), ("cout", C.c_int32), ("a1", VoSnake * 3), ("a2", VoSnake * 3), ("c1", VoCConv * 3),
                ("c2", VoCConv * 3)]


class VoCodec(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("codebook_size", "codebook_dim", "latent", "quantizers", "n_up", "n_blocks")] + \
               [("q_first", C.POINTER(VoMat)), ("q_rest", C.POINTER(VoMat)), ("q_first_out", VoMat), ("q_rest_out", VoMat),
                ("pre_conv", VoCConv), ("pt_in", VoMat), ("pt_out", VoMat), ("pt", VoXfmr),
                ("ups", C.POINTER(VoCodecUp)), ("conv0", VoCConv), ("blocks", C.POINTER(VoCodecBlock)),
                ("final_act", VoSnake), ("final_conv", VoCConv)]


class VoKV(C.Structure):
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("cap", C.c_int64), ("len", C.c_int64),
                ("kv_f16", C.c_int32), ("avx2", C.c_int32)]


class VoConv(C.Structure):
    _fields_ = [("w", C.c_void_p), ("b", C.c_void_p), ("cin", C.c_int32), ("cout", C.c_int32), ("K", C.c_int32),
                ("groups", C.c_int32)]


class VoF5Block(C.Structure):
    _fields_ = [(n, VoMat) for n in ("ada", "q", "k", "v", "o", "ff1", "ff2")]


class VoF5(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "depth", "heads", "dim_head", "ff_mult", "mel_dim", "text_dim",
                                         "pe_attn_head")] + \
               [(n, VoMat) for n in ("in_proj", "norm_out", "proj_out")] + \
               [("blocks", C.POINTER(VoF5Block)), ("pos1", VoConv), ("pos2", VoConv)]


class VoVocosBlock(C.Structure):
    _fields_ = [("dw", VoConv), ("ln_w", C.c_void_p), ("ln_b", C.c_void_p), ("gamma", C.c_void_p), ("pw1", VoMat),
                ("pw2", VoMat)]


class VoVocos(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "inter", "mel_dim", "layers")] + \
               [("embed", VoConv)] + [(n, C.c_void_p) for n in ("ln_w", "ln_b", "fln_w", "fln_b")] + \
               [("blocks", C.POINTER(VoVocosBlock)), ("head", VoMat)]


class VoCosyRes(C.Structure):
    _fields_ = [("c1", VoConv), ("c2", VoConv), ("res", VoConv)] + [(n, C.c_void_p) for n in ("n1w", "n1b", "n2w", "n2b")]


class VoCosyX(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("n1w", "n1b", "n3w", "n3b")] + \
               [(n, VoMat) for n in ("q", "k", "v", "o", "ff1", "ff2")]


class VoCosy(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("M", "C", "heads", "head_dim")] + \
               [("down_res", VoCosyRes), ("up_res", VoCosyRes), ("mid_res", C.POINTER(VoCosyRes)), ("n_mid", C.c_int32),
                ("down_x", C.POINTER(VoCosyX)), ("up_x", C.POINTER(VoCosyX)), ("mid_x", C.POINTER(VoCosyX)),
                ("n_down_x", C.c_int32), ("n_up_x", C.c_int32), ("mid_x_count", C.c_void_p)] + \
               [(n, VoConv) for n in ("down_conv", "up_out", "final_conv", "final_proj")] + \
               [("fn_w", C.c_void_p), ("fn_b", C.c_void_p)]


def _p(a):
    return None if a is None else a.ctypes.data


def _declare(lib, prefix):
    P, I64, I32, F, D, U32, U64 = C.c_void_p, C.c_int64, C.c_int32, C.c_float, C.c_double, C.c_uint32, C.c_uint64
    sig = {
        "philox4x32_10" if prefix == "vo_" else "philox": (None, [P, P, P]),
        "uniform": (F, [U64, U64, U32, U32]),
        "sample_logits": (I32, [P, I32, F, F, I32, F, P, I32, F]),
        "quantize_q8": (None, [P, I64, I64, P, P]),
        "quantize_q4": (None, [P, I64, I64, P, P]),
        "dot": (F, [P, P, I64]),
        "rmsnorm": (None, [P, P, I64, F, P]),
        "layernorm": (None, [P, P, P, I64, F, P]),
        "rope_inv_freq": (None, [I64, D, P]),
        "rope_apply": (None, [P, I64, I64, P, I64]),
        "silu": (F, [F]),
        "gelu_erf": (F, [F]),
        "transformer_forward": (C.c_int, [P, P, P, I64, P, P]),
        "transformer_forward_steps": (C.c_int, [P, P, I64, P, P]),
    }
    if prefix == "vo_":
        sig.update({
            "softmax": (None, [P, I64]),
            "ras_sample": (I32, [P, I32, P, I32, F, I32, I32, F, F, F]),
            "lm_logp": (None, [P, I32]),
            "gelu_tanh": (F, [F]),
            "mish": (F, [F]),
            "conv1d": (None, [P, P, I32, P]),
            "f5_modulate": (None, [P, I64, I32, P, P, P]),
            "f5_step": (C.c_int, [P, I32, I32, P, P, P, P]),
            "vocos_head": (C.c_int, [P, P, I32, P]),
            "exp_poly": (F, [F]),
            "gelu_poly": (F, [F]),
            "mish_nn": (F, [F]),
            "layer_norm_nn": (None, [P, I64, I32, P, P, F]),
            "softmax_fast": (None, [P, I64]),
            "attention_nn": (None, [P, P, P, I32, I32, I32, I32, F, P]),
            "causal_conv": (None, [P, P, I32, P]),
            "convt": (I32, [P, I32, I32, I32, I32, I32, I32, P, P, I32, P]),
            "cosy_step": (C.c_int, [P, I32, P, P, P]),
            "snake_params": (None, [P, P, I64, P, P]),
            "codec_state_new": (P, [P, I64]),
            "codec_state_clone": (P, [P]),
            "codec_state_free": (None, [P]),
            "codec_quantize": (C.c_int, [P, P, I32, P]),
            "codec_forward": (I64, [P, P, P, I32, P]),
            "codec_spf": (I64, [P]),
            "lm_step": (I32, [P, I32, P, I32, I64, I32, I32, F, I32, I32, F, U64, U32]),
            "noise": (None, [U64, U32, C.c_size_t, P]),
            "f16_to_f32": (F, [C.c_uint16]),
            "f32_to_f16": (C.c_uint16, [F]),
            "mat_row": (None, [P, I64, P]),
            "quantize_act": (None, [P, I64, P, P]),
            "matmul": (None, [P, P, I64, P, C.c_int]),
            "matmul_q8_int": (None, [P, P, I64, P, C.c_int]),
            "matmul_q4_int": (None, [P, P, I64, P, C.c_int]),
            "matmul_f32_tiles": (None, [P, P, I64, P]),
            "set_threads": (None, [C.c_int]),
            "get_threads": (C.c_int, []),
            "transformer_layers": (C.c_int, [P, P, P, I64, I32, I32, P]),
        })
    else:
        sig.update({
            "softmax": (None, [P, I64]),
            "mat_gather": (None, [P, I64, P]),
            "conv1d": (None, [P, I32, I32, I32, I32, P, P, I32, P]),
            "matmul": (None, [P, P, I64, P]),
            "set_threads": (None, [C.c_int]),
            "session_new": (P, [P, P, P]),
            "session_step": (C.c_int, [P, P, P, F, I32, F, P]),
            "session_free": (None, [P]),
            "gelu_inplace": (None, [P, I64]),
            "mish_nn": (F, [F]),
            "layer_norm_nn": (None, [P, I32, I32, P, P, F]),
            "attention_nn": (None, [P, P, P, I32, I32, I32, I32, F, P]),
            "causal_conv": (None, [P, P, I32, P]),
            "convt": (I32, [P, I32, I32, I32, I32, I32, I32, P, P, I32, P]),
            "cosy_step": (C.c_int, [P, I32, P, P, P]),
            "tmod_write": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int, P, P, P, P, P, P]),
            "codec_open": (P, [C.c_char_p]),
            "codec_close": (None, [P]),
            "codec_state_new": (P, [P]),
            "codec_state_clone": (P, [P, P]),
            "codec_state_free": (None, [P]),
            "codec_forward": (I64, [P, P, P, C.c_int, P]),
        })
    for name, (res, args) in sig.items():
        fn = getattr(lib, prefix + name)
        fn.restype = res
        fn.argtypes = args
    return lib


_oracle = None
_ref = None


def lib():
    """The C restatement (always built by __graft_entry__.build())."""
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} is not built; run __graft_entry__.build() or make -C oracle")
        _oracle = _declare(C.CDLL(ORACLE_SO), "vo_")
    return _oracle


def ref():
    """The compiled reference harness, or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        _ref = _declare(C.CDLL(REF_SO), "ref_")
    return _ref


# ---------------------------------------------------------------- helpers
class Mat:
    """A weight matrix in the reference layout with its ctypes view."""

    def __init__(self, wtype, data, rows, cols, scale=None, bias=None):
        self.type, self.rows, self.cols = wtype, rows, cols
        self.data = np.ascontiguousarray(data)
        self.scale = None if scale is None else np.ascontiguousarray(scale, dtype=np.float32)
        self.bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self.c = VoMat(wtype, _p(self.data), _p(self.scale), rows, cols, _p(self.bias))


def quantize_q8(w, use_ref=False):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // 32), np.float32)
    getattr(ref() if use_ref else lib(), ("ref_" if use_ref else "vo_") + "quantize_q8")(_p(w), rows, cols, _p(q), _p(s))
    return q, s


def quantize_q4(w, use_ref=False):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols // 2), np.uint8)
    s = np.empty((rows, cols // 32), np.float32)
    getattr(ref() if use_ref else lib(), ("ref_" if use_ref else "vo_") + "quantize_q4")(_p(w), rows, cols, _p(q), _p(s))
    return q, s


def quantize_act(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    xq = np.empty(x.size, np.int8)
    xs = np.empty(x.size // 32, np.float32)
    lib().vo_quantize_act(_p(x), x.size, _p(xq), _p(xs))
    return xq, xs


def matmul(M, x, avx2=1, use_ref=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0] if x.ndim == 2 else 1
    y = np.empty((m, M.rows), np.float32)
    if use_ref:
        ref().ref_matmul(C.byref(M.c), _p(x), m, _p(y))
    else:
        lib().vo_matmul(C.byref(M.c), _p(x), m, _p(y), avx2)
    return y


def mat_row(M, r, use_ref=False):
    out = np.empty(M.cols, np.float32)
    if use_ref:
        ref().ref_mat_gather(C.byref(M.c), r, _p(out))
    else:
        lib().vo_mat_row(C.byref(M.c), r, _p(out))
    return out


def sample_logits(logits, temperature=0.9, top_p=1.0, top_k=50, rep=1.0, history=None, u=0.5, use_ref=False):
    l = np.ascontiguousarray(logits, dtype=np.float32).copy()
    h = None if history is None else np.ascontiguousarray(history, dtype=np.int32)
    fn = ref().ref_sample_logits if use_ref else lib().vo_sample_logits
    return fn(_p(l), l.size, temperature, top_p, top_k, rep, _p(h), 0 if h is None else h.size, u)


def lm_logp(v):
    """lm_logp after the head and bias: a log-softmax copy of v (cosyvoice.cpp:602-606)."""
    l = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().vo_lm_logp(_p(l), l.size)
    return l


def lm_step(logp, decoded, step, min_len, speech_tokens, top_p=0.8, top_k=25, win_size=10, tau_r=0.1, seed=1234, piece=0):
    """One step of lm_generate's trial loop on log-probabilities; returns (token or -2, logp as modified)."""
    l = np.ascontiguousarray(logp, dtype=np.float32).copy()
    d = np.ascontiguousarray(decoded, dtype=np.int32)
    tok = lib().vo_lm_step(_p(l), l.size, _p(d) if d.size else None, d.size, step, min_len, speech_tokens, top_p, top_k,
                           win_size, tau_r, seed, piece)
    return tok, l


class Conv:
    """A Conv1d in Conv1d::w layout [groups][cout/groups][K][cin/groups] (GpuF5Conv), with its ctypes view."""

    def __init__(self, w, b, cin, cout, K, groups):
        self.w = np.ascontiguousarray(w, np.float32)
        self.b = None if b is None else np.ascontiguousarray(b, np.float32)
        self.cin, self.cout, self.K, self.groups = cin, cout, K, groups
        self.c = VoConv(_p(self.w), _p(self.b), cin, cout, K, groups)

    @staticmethod
    def from_torch(w_pt, b, groups):
        """From PyTorch Conv1d.weight [cout][cin/groups][K] (the conversion of Conv1d::load, f5_ops.cpp:86-104)."""
        cout, cig, K = w_pt.shape
        cog = cout // groups
        if groups == cig * groups and cout == groups and cig == 1:  # depthwise: [C][K]
            return Conv(w_pt.reshape(cout, K), b, groups, cout, K, groups)
        w = w_pt.reshape(groups, cog, cig, K).transpose(0, 1, 3, 2)  # [g][o][k][i]
        return Conv(w, b, cig * groups, cout, K, groups)


def conv1d(cv, x, use_ref=False, w_pt=None):
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    y = np.empty((T, cv.cout), np.float32)
    if use_ref:
        ref().ref_conv1d(_p(np.ascontiguousarray(w_pt, np.float32)), cv.cin, cv.cout, cv.K, cv.groups, _p(cv.b), _p(x), T, _p(y))
    else:
        lib().vo_conv1d(C.byref(cv.c), _p(x), T, _p(y))
    return y


def convt(w_pt, bias, x, stride, pad, out_pad=0, use_ref=False):
    """nn::ConvT (nn.cpp:205-245) of x [T][cin] with PyTorch's ConvTranspose1d weight [cin][cout][K] and bias [cout]
    (or None): y [(T - 1) stride - 2 pad + K + out_pad][cout]. use_ref runs the compiled reference instead."""
    w_pt = np.ascontiguousarray(w_pt, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    cin, cout, K = w_pt.shape
    T = x.shape[0]
    To = (T - 1) * stride - 2 * pad + K + out_pad
    y = np.empty((max(To, 1), cout), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    fn = ref().ref_convt if use_ref else lib().vo_convt
    n = fn(_p(w_pt), cin, cout, K, stride, pad, out_pad, _p(b) if b is not None else None, _p(x), T, _p(y))
    if n != To:
        raise ValueError(f"convt: bad arguments (output length {n})")
    return y


def f5_modulate(x, scale, shift):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().vo_f5_modulate(_p(x), x.shape[0], x.shape[1], _p(np.ascontiguousarray(scale, np.float32)),
                         _p(np.ascontiguousarray(shift, np.float32)), _p(y))
    return y


class F5:
    """An F5-TTS DiT in the oracle's struct layout: blocks = list of dicts ada,q,k,v,o,ff1,ff2 -> Mat."""

    def __init__(self, dim, depth, heads, dim_head, ff_mult, mel_dim, text_dim, pe_attn_head, in_proj, norm_out, proj_out,
                 blocks, pos1, pos2):
        self.keep = (in_proj, norm_out, proj_out, blocks, pos1, pos2)
        arr = (VoF5Block * len(blocks))()
        for i, b in enumerate(blocks):
            for n in ("ada", "q", "k", "v", "o", "ff1", "ff2"):
                setattr(arr[i], n, b[n].c)
        self._arr = arr
        self.c = VoF5(dim, depth, heads, dim_head, ff_mult, mel_dim, text_dim, pe_attn_head, in_proj.c, norm_out.c,
                      proj_out.c, arr, pos1.c, pos2.c)
        self.mel_dim = mel_dim


def f5_step(m, B, N, cat, ts, rope):
    cat = np.ascontiguousarray(cat, np.float32)
    out = np.empty((B * N, m.mel_dim), np.float32)
    lib().vo_f5_step(C.byref(m.c), B, N, _p(cat), _p(np.ascontiguousarray(ts, np.float32)),
                     _p(np.ascontiguousarray(rope, np.float32)), _p(out))
    return out


def gelu_erf(x, use_ref=False):
    return (ref().ref_gelu_erf if use_ref else lib().vo_gelu_erf)(x)


class Vocos:
    """F5's Vocos backbone + head in the oracle's struct layout: embed Conv, ln (w, b), blocks = list of dicts
    dw (Conv), ln_w, ln_b, gamma, pw1, pw2 (Mat), fln (w, b), head Mat."""

    def __init__(self, dim, inter, mel_dim, embed, ln_w, ln_b, blocks, fln_w, fln_b, head):
        f = lambda a: np.ascontiguousarray(a, np.float32)
        self.vecs = [f(a) for a in (ln_w, ln_b, fln_w, fln_b)]
        self.bvecs = [[f(b[n]) for n in ("ln_w", "ln_b", "gamma")] for b in blocks]
        self.keep = (embed, blocks, head)
        arr = (VoVocosBlock * max(1, len(blocks)))()
        for i, b in enumerate(blocks):
            arr[i] = VoVocosBlock(b["dw"].c, _p(self.bvecs[i][0]), _p(self.bvecs[i][1]), _p(self.bvecs[i][2]), b["pw1"].c,
                                  b["pw2"].c)
        self._arr = arr
        self.c = VoVocos(dim, inter, mel_dim, len(blocks), embed.c, *[_p(a) for a in self.vecs], arr, head.c)
        self.out = head.rows


def vocos_head(v, mel):
    mel = np.ascontiguousarray(mel, np.float32)
    out = np.empty((mel.shape[0], v.out), np.float32)
    rc = lib().vo_vocos_head(C.byref(v.c), _p(mel), mel.shape[0], _p(out))
    assert rc == 0
    return out


def uniform(seed, frame, cb, draw=0):
    return lib().vo_uniform(seed, frame, cb, draw)


def noise(seed, stream, n):
    out = np.empty(n, np.float32)
    lib().vo_noise(seed, stream, n, _p(out))
    return out


class Xfmr:
    """A Qwen3-shaped transformer in the oracle's struct layout (keeps its arrays alive)."""

    def __init__(self, layers, final_norm, hidden, heads, kv_heads, head_dim, inter, eps, inv_freq):
        self.layers = layers  # list of dicts: q,k,v,o,gate,up,down (Mat), qn,kn,ln1,ln2 (np or None)
        self.final_norm = np.ascontiguousarray(final_norm, np.float32)
        self.inv_freq = np.ascontiguousarray(inv_freq, np.float32)
        self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter, self.eps = hidden, heads, kv_heads, head_dim, inter, eps
        arr = (VoLayer * len(layers))()
        for i, L in enumerate(layers):
            for n in ("q", "k", "v", "o", "gate", "up", "down"):
                setattr(arr[i], n, L[n].c)
            for n in ("qn", "kn", "ln1", "ln2"):
                setattr(arr[i], n, _p(L.get(n)))
        self._arr = arr
        self.c = VoXfmr(len(layers), arr, _p(self.final_norm), hidden, heads, kv_heads, head_dim, inter, eps,
                        _p(self.inv_freq))


class KV:
    """Flat [layer][cap][kv_heads*head_dim] f32 cache."""

    def __init__(self, n_layers, cap, kd, kv_f16=0, avx2=1, k=None, v=None, length=0):
        self.k = np.zeros((n_layers, cap, kd), np.float32) if k is None else np.ascontiguousarray(k, np.float32)
        self.v = np.zeros((n_layers, cap, kd), np.float32) if v is None else np.ascontiguousarray(v, np.float32)
        self.c = VoKV(_p(self.k), _p(self.v), cap, length, kv_f16, avx2)

    @property
    def len(self):
        return self.c.len

    def copy(self):
        n = KV(self.k.shape[0], self.k.shape[1], self.k.shape[2], self.c.kv_f16, self.c.avx2, self.k.copy(), self.v.copy(), self.c.len)
        return n


def transformer_forward(X, kv, x, want_all=False, use_ref=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    out_last = np.empty(X.hidden, np.float32)
    out_all = np.empty((m, X.hidden), np.float32) if want_all else None
    fn = ref().ref_transformer_forward if use_ref else lib().vo_transformer_forward
    rc = fn(C.byref(X.c), C.byref(kv.c), _p(x), m, _p(out_last), _p(out_all))
    if rc != 0:
        raise RuntimeError(f"transformer_forward failed ({rc})")
    return (out_last, out_all) if want_all else out_last


def transformer_layers(X, kv, x, first, count):
    """Residual stream after layers [first, first + count) (no final norm); kv.len is not advanced."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty_like(x)
    if lib().vo_transformer_layers(C.byref(X.c), C.byref(kv.c), _p(x), x.shape[0], first, count, _p(h)) != 0:
        raise RuntimeError("transformer_layers failed")
    return h


def transformer_forward_steps(X, kvs, x, use_ref=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    B = x.shape[0]
    ptrs = (C.POINTER(VoKV) * B)(*[C.pointer(k.c) for k in kvs])
    out = np.empty((B, X.hidden), np.float32)
    fn = ref().ref_transformer_forward_steps if use_ref else lib().vo_transformer_forward_steps
    rc = fn(C.byref(X.c), ptrs, B, _p(x), _p(out))
    if rc != 0:
        raise RuntimeError(f"transformer_forward_steps failed ({rc})")
    return out


# ---- the CosyVoice2 / Chatterbox flow estimator (cosyvoice.cpp:126-221, :839-863)
def gelu_poly(x, use_ref=False):
    """nn.cpp's GELU on an array: the oracle's scalar restatement, or the reference's gelu_inplace."""
    x = np.array(x, np.float32, copy=True).ravel()
    if use_ref:
        ref().ref_gelu_inplace(_p(x), x.size)
        return x
    return np.array([lib().vo_gelu_poly(float(v)) for v in x], np.float32)


def mish_nn(x, use_ref=False):
    return (ref().ref_mish_nn if use_ref else lib().vo_mish_nn)(x)


def layer_norm_nn(x, w, b, eps, use_ref=False):
    y = np.array(x, np.float32, copy=True)
    f = np.ascontiguousarray
    (ref().ref_layer_norm_nn if use_ref else lib().vo_layer_norm_nn)(_p(y), y.shape[0], y.shape[1], _p(f(w, np.float32)),
                                                                     _p(None if b is None else f(b, np.float32)), eps)
    return y


def attention_nn(q, k, v, H, dh, scale, use_ref=False):
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    out = np.empty_like(q)
    (ref().ref_attention_nn if use_ref else lib().vo_attention_nn)(_p(q), _p(k), _p(v), q.shape[0], k.shape[0], H, dh,
                                                                   scale, _p(out))
    return out


def causal_conv(cv, x, use_ref=False):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty((x.shape[0], cv.cout), np.float32)
    (ref().ref_causal_conv if use_ref else lib().vo_causal_conv)(C.byref(cv.c), _p(x), x.shape[0], _p(y))
    return y


class Cosy:
    """The estimator in the oracle's struct layout. res: dict c1, c2, res (Conv), n1w, n1b, n2w, n2b; x: dict n1w,
    n1b, n3w, n3b, q, k, v, o, ff1, ff2 (Mat); mid_x: a list per mid block."""

    def __init__(self, M, C_, heads, head_dim, down_res, up_res, mid_res, down_x, up_x, mid_x, down_conv, up_out,
                 final_conv, final_proj, fn_w, fn_b):
        f = lambda a: np.ascontiguousarray(a, np.float32)
        self.keep = []

        def res(r):
            v = [f(r[n]) for n in ("n1w", "n1b", "n2w", "n2b")]
            self.keep += [r, v]
            return VoCosyRes(r["c1"].c, r["c2"].c, r["res"].c, *[_p(a) for a in v])

        def xs(lst):
            arr = (VoCosyX * max(1, len(lst)))()
            for i, x in enumerate(lst):
                v = [f(x[n]) for n in ("n1w", "n1b", "n3w", "n3b")]
                self.keep += [x, v]
                arr[i] = VoCosyX(*[_p(a) for a in v], *[x[n].c for n in ("q", "k", "v", "o", "ff1", "ff2")])
            self.keep.append(arr)
            return arr

        mids = (VoCosyRes * max(1, len(mid_res)))()
        for i, r in enumerate(mid_res):
            mids[i] = res(r)
        self.counts = np.array([len(v) for v in mid_x] or [0], np.int32)
        flat = [x for v in mid_x for x in v]
        self.fn = [f(fn_w), f(fn_b)]
        self.keep += [mids, down_conv, up_out, final_conv, final_proj]
        self.c = VoCosy(M, C_, heads, head_dim, res(down_res), res(up_res), mids, len(mid_res), xs(down_x), xs(up_x),
                        xs(flat), len(down_x), len(up_x), _p(self.counts), down_conv.c, up_out.c, final_conv.c,
                        final_proj.c, _p(self.fn[0]), _p(self.fn[1]))
        self.M, self.C, self.n_res = M, C_, 2 + len(mid_res)


def cosy_step(m, T, inp, tb, use_ref=False):
    """One estimator call: inp [2 T][4 M], tb [2 + n_mid][C] -> [2 T][M]."""
    inp = np.ascontiguousarray(inp, np.float32)
    tb = np.ascontiguousarray(tb, np.float32)
    assert inp.shape == (2 * T, 4 * m.M) and tb.shape == (m.n_res, m.C)
    out = np.empty((2 * T, m.M), np.float32)
    rc = (ref().ref_cosy_step if use_ref else lib().vo_cosy_step)(C.byref(m.c), T, _p(inp), _p(tb), _p(out))
    assert rc == 0, rc
    return out


# ---- the Qwen3-TTS codec decoder (qwen3.cpp:225-283 load_codec, :366-481 codec_forward)
class Codec:
    """The codec decoder in the oracle's struct layout, from its tensors by .tmod name (t: name -> f32 array, 2-D
    weights as qwen3.cpp reads them) and the codec config cc (the manifest's codec keys)."""

    def __init__(self, cc, t):
        f = lambda a: np.ascontiguousarray(a, np.float32)
        self.keep = []
        self.cc = cc

        def mat(name, bias=None):
            w = f(t[name])
            b = None if bias is None else f(t[bias])
            m = Mat(F32, w, w.shape[0], w.shape[1] if w.ndim > 1 else 1, None, b)
            self.keep.append(m)
            return m.c

        def vec(name):
            a = f(t[name]).ravel()
            self.keep.append(a)
            return _p(a)

        def conv(p, K, cin, cout, dil=1):
            return VoCConv(mat(p + ".weight", p + ".bias"), K, cin, cout, dil)

        def snake(p):
            al, be = f(t[p + ".alpha"]).ravel(), f(t[p + ".beta"]).ravel()
            a, ib = np.empty_like(al), np.empty_like(be)
            lib().vo_snake_params(_p(al), _p(be), al.size, _p(a), _p(ib))
            self.keep += [a, ib]
            return VoSnake(_p(a), _p(ib))
        Q, CD, L = cc["num_quantizers"], cc["codebook_dim"], cc["latent_dim"]
        H, heads, kvh = cc["hidden_size"], cc["num_attention_heads"], cc["num_key_value_heads"]
        hd = cc.get("head_dim", H // heads)
        qf = (VoMat * 1)(mat("codec.quantizer.rvq_first.vq.layers.0._codebook.embedding"))
        qr = (VoMat * max(1, Q - 1))(*[mat(f"codec.quantizer.rvq_rest.vq.layers.{i}._codebook.embedding") for i in range(Q - 1)])
        layers = (VoLayer * cc["num_hidden_layers"])()
        for i in range(cc["num_hidden_layers"]):
            p = f"codec.pre_transformer.layers.{i}."
            lw = layers[i]
            for n, k in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"), ("o", "self_attn.o_proj"),
                         ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"), ("down", "mlp.down_proj")):
                setattr(lw, n, mat(p + k + ".weight"))
            lw.ln1, lw.ln2 = vec(p + "input_layernorm.weight"), vec(p + "post_attention_layernorm.weight")
            lw.attn_scale, lw.mlp_scale = vec(p + "self_attn_layer_scale.scale"), vec(p + "mlp_layer_scale.scale")
        theta = cc.get("rope_theta", 10000.0)
        inv = np.empty(hd // 2, np.float32)
        lib().vo_rope_inv_freq(hd, theta, _p(inv))
        self.keep += [qf, qr, layers, inv]
        pt = VoXfmr(cc["num_hidden_layers"], layers, vec("codec.pre_transformer.norm.weight"), H, heads, kvh, hd,
                    cc["intermediate_size"], cc.get("rms_norm_eps", 1e-5), _p(inv), cc["sliding_window"])
        ratios, rates, dec = cc["upsampling_ratios"], cc["upsample_rates"], cc["decoder_dim"]
        ups = (VoCodecUp * max(1, len(ratios)))()
        for s_, r in enumerate(ratios):
            p = f"codec.upsample.{s_}."
            ups[s_] = VoCodecUp(mat(p + "0.conv.weight"), vec(p + "0.conv.bias"), r, vec(p + "1.dwconv.conv.weight"),
                                vec(p + "1.dwconv.conv.bias"), 7, vec(p + "1.norm.weight"), vec(p + "1.norm.bias"),
                                vec(p + "1.gamma"), mat(p + "1.pwconv1.weight", p + "1.pwconv1.bias"),
                                mat(p + "1.pwconv2.weight", p + "1.pwconv2.bias"))
        blocks = (VoCodecBlock * max(1, len(rates)))()
        for b, r in enumerate(rates):
            ind, outd = dec >> b, dec >> (b + 1)
            p = f"codec.decoder.{b + 1}.block."
            blk = blocks[b]
            blk.act = snake(p + "0")
            blk.tr, blk.tr_b, blk.K, blk.stride, blk.cin, blk.cout = mat(p + "1.conv.weight"), vec(p + "1.conv.bias"), 2 * r, r, ind, outd
            for u, dil in enumerate((1, 3, 9)):
                q = p + f"{u + 2}."
                blk.a1[u], blk.a2[u] = snake(q + "act1"), snake(q + "act2")
                blk.c1[u] = conv(q + "conv1.conv", 7, outd, outd, dil)
                blk.c2[u] = conv(q + "conv2.conv", 1, outd, outd)
        nb = len(rates)
        self.keep += [ups, blocks]
        self.c = VoCodec(cc["codebook_size"], CD, L, Q, len(ratios), nb, qf, qr,
                         mat("codec.quantizer.rvq_first.output_proj.weight"), mat("codec.quantizer.rvq_rest.output_proj.weight"),
                         conv("codec.pre_conv.conv", 3, CD, L), mat("codec.pre_transformer.input_proj.weight",
                                                                    "codec.pre_transformer.input_proj.bias"),
                         mat("codec.pre_transformer.output_proj.weight", "codec.pre_transformer.output_proj.bias"), pt, ups,
                         conv("codec.decoder.0.conv", 7, L, dec), blocks, snake(f"codec.decoder.{nb + 1}"),
                         conv(f"codec.decoder.{nb + 2}.conv", 7, dec >> nb, 1))
        self.spf = lib().vo_codec_spf(C.byref(self.c))


class CodecState:
    """The oracle's streaming state of a Codec (cap: transformer positions it can hold)."""

    def __init__(self, codec, cap=512, _ptr=None):
        self.codec = codec
        self.p = _ptr if _ptr else lib().vo_codec_state_new(C.byref(codec.c), cap)

    def clone(self):
        return CodecState(self.codec, _ptr=lib().vo_codec_state_clone(self.p))

    def __del__(self):
        if getattr(self, "p", None):
            lib().vo_codec_state_free(self.p)
            self.p = None


def codec_quantize(codec, codes):
    codes = np.ascontiguousarray(codes, np.int16)
    z = np.empty((codes.shape[0], codec.cc["codebook_dim"]), np.float32)
    assert lib().vo_codec_quantize(C.byref(codec.c), _p(codes), codes.shape[0], _p(z)) == 0
    return z


def codec_forward(state, z):
    """z [F][codebook_dim] -> pcm [F * spf]; the state advances."""
    z = np.ascontiguousarray(z, np.float32)
    out = np.empty(z.shape[0] * state.codec.spf, np.float32)
    n = lib().vo_codec_forward(C.byref(state.codec.c), state.p, _p(z), z.shape[0], _p(out))
    assert n == out.size, n
    return out


def tmod_write(path, manifest, tensors):
    """Writes a .tmod with the compiled reference's tmod_write (f32 tensors by name)."""
    import json
    names = sorted(tensors)
    arrs = [np.ascontiguousarray(tensors[n], np.float32) for n in names]
    nm = (C.c_char_p * len(names))(*[n.encode() for n in names])
    dt = np.zeros(len(names), np.int32)  # DType::F32
    nd = np.array([a.ndim for a in arrs], np.int32)
    sh = np.array([d for a in arrs for d in a.shape], np.int64)
    ptr = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    nb = np.array([a.nbytes for a in arrs], np.int64)
    rc = ref().ref_tmod_write(path.encode(), json.dumps(manifest).encode(), len(names), nm, _p(dt), _p(nd), _p(sh), ptr, _p(nb))
    assert rc == 0, rc


class RefCodec:
    """The reference's Qwen3Weights (codec_forward on the CPU) loaded from a .tmod written by tmod_write."""

    def __init__(self, path, spf):
        self.h = ref().ref_codec_open(path.encode())
        assert self.h, "the reference could not load " + path
        self.spf = spf

    def state(self):
        return ref().ref_codec_state_new(self.h)

    def clone(self, s):
        return ref().ref_codec_state_clone(self.h, s)

    def free_state(self, s):
        ref().ref_codec_state_free(s)

    def forward(self, s, codes):
        codes = np.ascontiguousarray(codes, np.int16)
        out = np.empty(codes.shape[0] * self.spf, np.float32)
        n = ref().ref_codec_forward(self.h, s, _p(codes), codes.shape[0], _p(out))
        assert n == out.size, n
        return out

    def __del__(self):
        if getattr(self, "h", None):
            ref().ref_codec_close(self.h)
            self.h = None
