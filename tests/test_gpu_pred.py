"""The code predictor's frame loop on the device (gpu_pred_frame, gpu_vulkan.cpp:968-1045; the CPU loop it replaces
is engine.cpp:676-683 around backend_qwen3.cpp:398-424).

Pass 1 takes the talker's hidden state and the first code's embedding as two rows at positions 0 and 1; pass cb >= 2
takes the embedding of the code pass cb - 1 sampled at position cb; each pass runs in_proj (or none), the layers,
the final norm and head cb - 1 on its last row, then sample_logits with the draw (frame, cb).

Two checks:
- the whole frame in one device graph gives exactly the codes of the same loop run pass by pass through the
  host-pointer forward path (same kernels, so the same logits bit for bit), with every pass sampled by the oracle
  sampler on the device logits and the next input gathered by the oracle's mat_row;
- every pass's state and logits match the oracle transformer within the north star's 1e-3, teacher-forced on the
  device's codes and on the device's cache of the earlier positions (f16 KV model): the int8 requantization at every
  GEMV input turns ulp-level differences into whole quanta, so two caches left to run apart for 16 positions drift
  by more than one pass's error, which is what the bar is about (as the full-size talker tests do per layer).
"""
import numpy as np
import pytest

from conftest import rel_err
from models import Model, make_mat

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4
TOL = 1e-3


def predictor(hip, oracle, seed, G, V, din, wt_emb, with_proj):
    mdl = Model(seed, 2, 128, 4, 2, 64, 256, wtype=Q8)
    xf = hip.xfmr_create(mdl.hx, "pred")
    rng = np.random.default_rng(seed)
    heads, oheads, embs, oembs = [], [], [], []
    for _ in range(G - 1):
        d, s, b = make_mat(rng, Q8, V, 128, std=0.05)
        heads.append(hip.upload(hip.HostMat(Q8, d, V, 128, s, b)))
        oheads.append(oracle.Mat(Q8, d, V, 128, s, b))
    for _ in range(G - 2):
        d, s, b = make_mat(rng, wt_emb, V, din, std=1.0)
        embs.append(hip.upload(hip.HostMat(wt_emb, d, V, din, s, b)))
        oembs.append(oracle.Mat(wt_emb, d, V, din, s, b))
    ip, oip = -1, None
    if with_proj:
        d, s, b = make_mat(rng, Q8, 128, din, bias=True)
        ip = hip.upload(hip.HostMat(Q8, d, 128, din, s, b))
        oip = oracle.Mat(Q8, d, 128, din, s, b)
    return mdl, xf, heads, oheads, embs, oembs, ip, oip


@pytest.mark.parametrize("G,V,with_proj,wt_emb", [(8, 64, False, F32), (16, 200, True, BF16), (4, 96, True, Q8)])
def test_pred_frame(hip, oracle, G, V, with_proj, wt_emb):
    din = 96 if with_proj else 128
    mdl, xf, heads, oheads, embs, oembs, ip, oip = predictor(hip, oracle, 900 + G, G, V, din, wt_emb, with_proj)
    rng = np.random.default_rng(G)
    T, top_p, top_k, seed = 0.9, 0.95, 20, 4321
    for frame in (0, 7):
        in2 = rng.standard_normal((2, din)).astype(np.float32)
        cfg = hip.sample_cfg(T, top_p, top_k, seed=seed, frame=frame)
        seq = hip.seq_create(xf, G + 2)
        codes = hip.pred_frame(xf, seq, in2, ip, heads, embs, cfg)
        assert codes.shape == (G,) and codes[0] == 0
        # the same loop pass by pass on the host-pointer path, sampled by the oracle on the device logits
        seq2 = hip.seq_create(xf, G + 2)
        kv = mdl.oracle_kv(G + 2, kv_f16=1)
        x, pos, want = in2, 0, [0]
        for cb in range(1, G):
            out, logits = hip.forward(xf, seq2, pos, x, 128, in_proj=ip, head=heads[cb - 1])
            u = oracle.uniform(seed, frame, cb, 0)
            want.append(oracle.sample_logits(logits, T, top_p, top_k, 1.0, None, u))
            # oracle: the same pass on the device's cache of positions < pos, fed the device's codes
            kd = mdl.kv_heads * mdl.head_dim
            for li in range(mdl.n_layers):
                if pos:
                    k, v = hip.seq_download(seq2, li, pos, kd)
                    kv.k[li, :pos] = k
                    kv.v[li, :pos] = v
            kv.c.len = pos
            h = oracle.matmul(oip, x) if with_proj else x
            ref = oracle.transformer_forward(mdl.ox, kv, h)
            assert rel_err(out, ref) < TOL, (frame, cb, rel_err(out, ref))
            ref_logits = oracle.matmul(oheads[cb - 1], np.asarray(out, np.float32)[None])[0]
            assert rel_err(logits, ref_logits) < TOL, (frame, cb)
            pos += x.shape[0]
            if cb + 1 < G:
                x = oracle.mat_row(oembs[cb - 1], int(want[cb]))[None]
        assert list(codes) == want, (frame, list(codes), want)
        hip.seq_free(seq)
        hip.seq_free(seq2)


def test_pred_frame_replays_and_rejects(hip, oracle):
    # the captured frame replays with new inputs and sampler settings; bad shapes are errors, not faults
    G, V, din = 6, 64, 128
    mdl, xf, heads, oheads, embs, oembs, ip, oip = predictor(hip, oracle, 950, G, V, din, F16, False)
    rng = np.random.default_rng(3)
    seq = hip.seq_create(xf, G + 2)
    results = []
    for rep in range(3):
        in2 = rng.standard_normal((2, din)).astype(np.float32)
        cfg = hip.sample_cfg(0.8 + 0.1 * rep, 1.0, 10 + rep, seed=rep, frame=rep)
        a = hip.pred_frame(xf, seq, in2, ip, heads, embs, cfg)
        b = hip.pred_frame(xf, seq, in2, ip, heads, embs, cfg)
        assert np.array_equal(a, b), rep
        results.append(a)
    with pytest.raises(hip.VoxHipError, match="embedding"):
        hip.pred_frame(xf, seq, rng.standard_normal((2, din)).astype(np.float32), ip, heads, embs[:-1],
                       hip.sample_cfg(0.9, 1.0, 10))
    with pytest.raises(hip.VoxHipError, match="64 codebooks"):  # the reference's bound (gpu_vulkan.cpp:977)
        hip.pred_frame(xf, seq, rng.standard_normal((2, din)).astype(np.float32), ip, heads * 13, embs * 13,
                       hip.sample_cfg(0.9, 1.0, 10))
    # the frame still runs after the rejected calls
    a = hip.pred_frame(xf, seq, in2, ip, heads, embs, cfg)
    assert np.array_equal(a, results[-1])
