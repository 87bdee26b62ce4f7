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
                 eps=1e-6, head_rows=0, head_type=None):
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
                d, s, b = make_mat(rng, wtype, r, c, bias=bias and n in ("q", "k", "v"))
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
