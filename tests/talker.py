"""Helpers of the full-size talker tests: the device model (vox_amd.synth.Decoder) restated for the oracle, and the
reference's quantized-model criterion (`vox verify --quant`, cli/main.cpp:764-790)."""
import numpy as np


def to_oracle(oracle, hip, dec, seqs=None, kv_len=None, cap=None):
    """The decoder's stored weights (with their biases), norms and the f16 caches of `seqs` (default: the decoder's
    own sequence) as oracle objects: (Xfmr, [KV per sequence], head Mat). cap: the oracle caches' capacity (default
    kv_len + 8)."""
    c = dec.cfg
    L = []
    for li in range(c["layers"]):
        d = {}
        for n in ("q", "k", "v", "o", "gate", "up", "down"):
            h = dec.mats[li][n]
            rows, cols = hip.mat_shape(h)
            data, scale, bias = hip.mat_download(h, c["wtype"])
            has_bias = c.get("qkv_bias", False) and n in ("q", "k", "v")
            d[n] = oracle.Mat(c["wtype"], data, rows, cols, scale, bias if has_bias else None)
        d.update(dec.layers[li])
        L.append(d)
    X = oracle.Xfmr(L, dec.final_norm, c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["inter"], c["eps"], dec.inv_freq)
    kd = c["kv_heads"] * c["head_dim"]
    n = kv_len or c["kv_len"]
    kvs = []
    for s in (seqs or [dec.seq]):
        kv = oracle.KV(c["layers"], cap or n + 8, kd, kv_f16=1)
        for li in range(c["layers"]):
            k, v = hip.seq_download(s, li, n, kd)
            kv.k[li, :n] = k
            kv.v[li, :n] = v
        kv.c.len = n
        kvs.append(kv)
    hd, hs, hb = hip.mat_download(dec.head, c["head_type"])
    head = oracle.Mat(c["head_type"], hd, c["head_rows"], c["hidden"], hs, hb if c.get("head_bias", False) else None)
    return X, kvs, head


def kl_top5(ours, ref):
    """KL(ref || ours) of softmax(logits) and whether the reference argmax is in our top-5 (cli/main.cpp:769-787)."""
    a, b = np.asarray(ours, np.float64), np.asarray(ref, np.float64)
    la = a.max() + np.log(np.exp(a - a.max()).sum())
    lb = b.max() + np.log(np.exp(b - b.max()).sum())
    lp, lq = b - lb, a - la
    kl = float(np.sum(np.exp(lp) * (lp - lq)))
    ib = int(np.argmax(b))
    return kl, int(np.sum(a > a[ib])) < 5
