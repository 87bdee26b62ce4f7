"""Writes tests/golden/golden_ref.npz from the compiled reference harness (oracle/_ref/libvoxref.so).

Run here (where /root/reference exists and `make -C oracle ref` has built the harness):
    python tests/golden/make_golden.py          # golden_ref.npz
    python tests/golden/make_golden.py cosy     # golden_cosy.npz (the flow estimator's nn.cpp layers)
    python tests/golden/make_golden.py codec    # golden_codec.npz (the Qwen3-TTS codec decoder)
    python tests/golden/make_golden.py q4       # golden_q4.npz (quantize_q4 blocks on float-rounding ties)
The fixtures hold inputs and the reference's outputs only (data, no reference source; the estimator's weights are
regenerated from a seed by tests/models.py's CosyModel). Tests compare the
C restatement (oracle/liboracle.so) against it on machines without the reference.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import pyoracle as po  # noqa: E402

OUT = os.path.join(HERE, "golden_ref.npz")
OUT_COSY = os.path.join(HERE, "golden_cosy.npz")
COSY_SEED, COSY_T = 77, 13  # CosyModel(COSY_SEED, n_mid=1, n_x=1) at T frames
OUT_CODEC = os.path.join(HERE, "golden_codec.npz")
OUT_Q4 = os.path.join(HERE, "golden_q4.npz")
CODEC_SEED, CODEC_F = 91, 9  # CodecModel(CODEC_SEED) on F frames, decoded as 4 + 5


def main():
    R = po.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libvoxref.so is not built")
    po.ref().ref_set_threads(4)
    rng = np.random.default_rng(20261201)
    g = {}
    # Philox / DetRng
    ctr = rng.integers(0, 2**32, size=(64, 4), dtype=np.uint64).astype(np.uint32)
    key = rng.integers(0, 2**32, size=(64, 2), dtype=np.uint64).astype(np.uint32)
    outs = np.empty((64, 4), np.uint32)
    for i in range(64):
        c, k, o = np.ascontiguousarray(ctr[i]), np.ascontiguousarray(key[i]), np.empty(4, np.uint32)
        R.ref_philox(c.ctypes.data, k.ctypes.data, o.ctypes.data)
        outs[i] = o
    g["philox_ctr"], g["philox_key"], g["philox_out"] = ctr, key, outs
    uargs = rng.integers(0, 2**40, size=(64, 4), dtype=np.uint64)
    g["uniform_args"] = uargs
    g["uniform_out"] = np.array([R.ref_uniform(int(a[0]), int(a[1]), int(a[2]) & 0xFFFFFFFF, int(a[3]) & 0xFFFFFFFF)
                                 for a in uargs], np.float32)
    # sample_logits: random logits, ties, -inf masks, penalties
    cases = []
    for i in range(200):
        n = int(rng.choice([4, 50, 100, 3072]))
        l = (rng.standard_normal(n) * rng.uniform(0.5, 4)).astype(np.float32)
        if i % 7 == 0:
            l = np.round(l).astype(np.float32)  # many ties
        if i % 5 == 0:
            l[rng.integers(0, n, n // 4)] = -np.inf
        T = float(rng.choice([0.0, 0.5, 0.9, 1.0, 1.3]))
        top_k = int(rng.choice([0, 1, 5, 50, n + 3]))
        top_p = float(rng.choice([1.0, 0.8, 0.5, 0.95]))
        rep = float(rng.choice([1.0, 1.1, 2.0]))
        hist = rng.integers(-2, n + 2, int(rng.integers(0, 20))).astype(np.int32)
        u = float(np.float32(rng.uniform()))
        ll = l.copy()
        idx = R.ref_sample_logits(ll.ctypes.data, n, T, top_p, top_k, rep, hist.ctypes.data if hist.size else None, hist.size, u)
        cases.append((l, T, top_p, top_k, rep, hist, u, idx))
    g["sample_n"] = np.array([c[0].size for c in cases], np.int64)
    g["sample_logits"] = np.concatenate([c[0] for c in cases])
    g["sample_params"] = np.array([[c[1], c[2], c[3], c[4], c[6]] for c in cases], np.float64)
    g["sample_hist_n"] = np.array([c[5].size for c in cases], np.int64)
    g["sample_hist"] = np.concatenate([c[5] for c in cases]).astype(np.int32)
    g["sample_idx"] = np.array([c[7] for c in cases], np.int32)
    # quantizers
    w = (rng.standard_normal((37, 160)) * np.linspace(0.01, 2, 160)).astype(np.float32)
    w[3, :32] = 0.0
    w[4, 32:64] = 0.5  # equal magnitudes
    g["quant_w"] = w
    g["q8_q"], g["q8_s"] = po.quantize_q8(w, use_ref=True)
    g["q4_q"], g["q4_s"] = po.quantize_q4(w, use_ref=True)
    # matmul paths
    x = rng.standard_normal((12, 160)).astype(np.float32)
    g["mm_x"] = x
    bias = rng.standard_normal(37).astype(np.float32)
    g["mm_bias"] = bias
    for name, wt, data, scale in (("q8", po.Q8, g["q8_q"], g["q8_s"]), ("q4", po.Q4, g["q4_q"], g["q4_s"]),
                                  ("f32", po.F32, w, None), ("f16", po.F16, w.astype(np.float16).view(np.uint16), None)):
        M = po.Mat(wt, data, 37, 160, scale, bias)
        for m in (1, 3, 8, 12):
            g[f"mm_{name}_m{m}"] = po.matmul(M, x[:m], use_ref=True)
    # norms / rope / softmax
    v = rng.standard_normal(1024).astype(np.float32)
    gam = (1 + 0.02 * rng.standard_normal(1024)).astype(np.float32)
    out = np.empty(1024, np.float32)
    R.ref_rmsnorm(v.ctypes.data, gam.ctypes.data, 1024, np.float32(1e-6), out.ctypes.data)
    g["rms_x"], g["rms_w"], g["rms_out"] = v, gam, out.copy()
    R.ref_layernorm(v.ctypes.data, gam.ctypes.data, None, 1024, np.float32(1e-6), out.ctypes.data)
    g["ln_out"] = out.copy()
    s = v[:513].copy()
    R.ref_softmax(s.ctypes.data, 513)
    g["softmax_out"] = s
    inv = np.empty(64, np.float32)
    R.ref_rope_inv_freq(128, 1e6, inv.ctypes.data)
    g["rope_inv"] = inv
    qh = rng.standard_normal(16 * 128).astype(np.float32)
    g["rope_x"] = qh.copy()
    R.ref_rope_apply(qh.ctypes.data, 16, 128, inv.ctypes.data, 512)
    g["rope_out"] = qh
    # tiny transformer: 2 layers, hidden 64, 4 heads / 2 kv x 32... head_dim 32, inter 96, q8, prompt of 5 then 2 tokens
    from models import Model
    mdl = Model(7, 2, 64, 4, 2, 32, 96, wtype=po.Q8)
    kv = mdl.oracle_kv(16, kv_f16=0)
    xs = rng.standard_normal((7, 64)).astype(np.float32)
    g["xf_x"] = xs
    o1, oa = po.transformer_forward(mdl.ox, kv, xs[:5], want_all=True, use_ref=True)
    o2 = po.transformer_forward(mdl.ox, kv, xs[5:6], use_ref=True)
    o3 = po.transformer_forward(mdl.ox, kv, xs[6:7], use_ref=True)
    g["xf_out_all5"], g["xf_out6"], g["xf_out7"] = oa, o2, o3
    np.savez_compressed(OUT, **g)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


def main_cosy():
    """The nn.cpp layers of the CosyVoice2 / Chatterbox estimator (gelu_inplace, mish, layer_norm, attention,
    Conv::forward on a causally padded input) and one whole estimator call composed from them."""
    R = po.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libvoxref.so is not built")
    R.ref_set_threads(4)
    rng = np.random.default_rng(20261202)
    g = {}
    x = np.concatenate([rng.standard_normal(997) * 3, [0.0, -0.0, 1e-30, -1e-30, 9.0, -9.0, 30.0, -30.0, 87.0, -87.0],
                        np.linspace(-6, 6, 61)]).astype(np.float32)
    g["act_x"] = x
    g["gelu_out"] = po.gelu_poly(x, use_ref=True)
    g["mish_out"] = np.array([po.mish_nn(float(v), use_ref=True) for v in x], np.float32)
    ln_x = (rng.standard_normal((9, 72)) * 2 + 0.5).astype(np.float32)
    ln_w, ln_b = (1 + 0.1 * rng.standard_normal(72)).astype(np.float32), (0.1 * rng.standard_normal(72)).astype(np.float32)
    g["ln_x"], g["ln_w"], g["ln_b"] = ln_x, ln_w, ln_b
    g["ln_out"] = po.layer_norm_nn(ln_x, ln_w, ln_b, 1e-5, use_ref=True)
    q, k, v = (rng.standard_normal((11, 3 * 16)).astype(np.float32) for _ in range(3))
    g["attn_q"], g["attn_k"], g["attn_v"] = q, k, v
    g["attn_out"] = po.attention_nn(q, k, v, 3, 16, 0.25, use_ref=True)
    w = (rng.standard_normal((6, 3, 8)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(6) * 0.1).astype(np.float32)
    cx = rng.standard_normal((10, 8)).astype(np.float32)
    g["conv_w"], g["conv_b"], g["conv_x"] = w, b, cx
    g["conv_out"] = po.causal_conv(po.Conv(w, b, 8, 6, 3, 1), cx, use_ref=True)
    from models import CosyModel
    m = CosyModel(COSY_SEED, n_mid=1, n_x=1)
    in0, xx, tb = m.inputs(np.random.default_rng(COSY_SEED), COSY_T)
    inp = m.with_x(in0, xx)
    g["cosy_in"], g["cosy_tb"] = inp, tb
    g["cosy_out"] = po.cosy_step(m.ox, COSY_T, inp, tb, use_ref=True)
    np.savez_compressed(OUT_COSY, **g)
    print("wrote", OUT_COSY, os.path.getsize(OUT_COSY), "bytes")


def main_codec():
    """Qwen3Weights::codec_forward of the compiled reference on a CodecModel written as a .tmod by its own tmod_write:
    the codes, the quantizer output and the PCM of two streaming calls."""
    import tempfile
    if po.ref() is None:
        raise SystemExit("oracle/_ref/libvoxref.so is not built")
    from models import CodecModel
    m = CodecModel(CODEC_SEED)
    codes = m.codes(np.random.default_rng(CODEC_SEED), CODEC_F)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "codec.tmod")
        m.write_tmod(path)
        R = po.RefCodec(path, m.spf)
        s = R.state()
        pcm = np.concatenate([R.forward(s, codes[:4]), R.forward(s, codes[4:])])
        R.free_state(s)
        del R
    np.savez_compressed(OUT_CODEC, codes=codes, pcm=pcm)
    print("wrote", OUT_CODEC, os.path.getsize(OUT_CODEC), "bytes")


def q4_block_errors(p):
    """Float64 squared errors of quantize_q4's nine candidate scales and of the least-squares refit of the best one
    (kernels.cpp:606-645), for blocks p [n][32] f32. Numpy sums in its own order, so the values are close to the
    reference's, not equal: they only rank blocks by how near a rounding of the stored error they are."""
    a = np.abs(p)
    mx = p[np.arange(p.shape[0]), np.argmax(a, axis=1)]  # first value of largest magnitude
    errs, qs = [], []
    for k in range(9):
        d = (mx / np.float32(-(7.0 + 0.25 * k))).astype(np.float32)
        inv = (np.float32(1) / d).astype(np.float32)
        c = np.clip(np.floor((p * inv[:, None]).astype(np.float32) + np.float32(8.5)), 0, 15)
        q = c.astype(np.int64) - 8
        errs.append(((p.astype(np.float64) - q * d[:, None].astype(np.float64)) ** 2).sum(1))
        qs.append(q)
    errs = np.stack(errs, 1)
    best = np.argmin(errs, 1)
    bq = np.stack(qs, 1)[np.arange(p.shape[0]), best]
    num = (p.astype(np.float64) * bq).sum(1)
    den = (bq * bq).sum(1).astype(np.float64)
    d2 = (num / np.where(den > 0, den, 1)).astype(np.float32)
    ls = ((p.astype(np.float64) - bq * d2[:, None].astype(np.float64)) ** 2).sum(1)
    return errs, ls


def main_q4():
    """quantize_q4 on blocks where the float best_err of kernels.cpp:616 decides: the best candidate's error and a
    rival (another candidate or the least-squares refit) lie within a few float ulps of each other, so storing the
    double error as a float can flip the choice. Drawn from N(0, 0.02), U(-1, 1) and near-grid matrices."""
    if po.ref() is None:
        raise SystemExit("oracle/_ref/libvoxref.so is not built")
    rng = np.random.default_rng(20261203)
    picked = []
    for kind in range(3):
        n = 1 << 20
        if kind == 0:
            p = (rng.standard_normal((n, 32)) * 0.02).astype(np.float32)
        elif kind == 1:
            p = rng.uniform(-1, 1, (n, 32)).astype(np.float32)
        else:
            p = (rng.integers(-8, 8, (n, 32)) * 0.01 + rng.standard_normal((n, 32)) * 1e-6).astype(np.float32)
        errs, ls = q4_block_errors(p)
        srt = np.sort(errs, 1)
        best = srt[:, 0]
        gap = np.minimum(np.abs(srt[:, 1] - best), np.abs(ls - best)) / np.maximum(best, 1e-300)
        sel = np.nonzero(gap < 2.0 ** -22)[0]
        picked.append(p[sel[:700]])
    w = np.ascontiguousarray(np.concatenate(picked), np.float32)
    q, s = po.quantize_q4(w, use_ref=True)
    np.savez_compressed(OUT_Q4, w=w, q=q, s=s)
    print("wrote", OUT_Q4, w.shape[0], "blocks", os.path.getsize(OUT_Q4), "bytes")


if __name__ == "__main__":
    mode = sys.argv[1:]
    {"cosy": main_cosy, "codec": main_codec, "q4": main_q4}.get(mode[0] if mode else "", main)()
