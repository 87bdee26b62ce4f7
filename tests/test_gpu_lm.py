"""CosyVoice2 LM on the device (cosyvoice.cpp:564-690) against the oracle.

The sampler is checked bit-exactly: the device's step on given logits must pick the oracle's token (the same
lm_logp, the same RAS trial loop), and its log-probabilities must match lm_logp to f32 rounding. The generation
loop is checked by teacher forcing: each step's device log-probabilities against the oracle's transformer + head
+ lm_logp on the device's own token history (1e-3 with the `vox verify` metric), and each device token against
the oracle's trial loop run on the device's log-probabilities (exact).
"""
import numpy as np
import pytest

from conftest import rel_err
from models import Model, make_mat

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4
TOL = 1e-3


def dev_logits(hip, v):
    d = hip.DevBuf(v.nbytes)
    d.upload(np.ascontiguousarray(v, np.float32))
    return d


def dev_ints(hip, a):
    a = np.ascontiguousarray(a, np.int32)
    d = hip.DevBuf(max(a.nbytes, 4))
    if a.size:
        d.upload(a)
    return d


@pytest.mark.parametrize("n,speech,top_k,top_p,win,tau", [(6564, 6561, 25, 0.8, 10, 0.1), (300, 297, 1, 0.8, 10, 0.1),
                                                          (300, 290, 200, 1.0, 4, 0.5), (100, 99, 25, 0.95, 0, 0.1),
                                                          (8192, 8000, 64, 0.8, 10, 0.1)])
def test_lm_sample_parity(hip, oracle, n, speech, top_k, top_p, win, tau):
    rng = np.random.default_rng(n + top_k)
    resampled = 0
    for case in range(24):
        v = (rng.standard_normal(n) * rng.choice([0.5, 2.0, 6.0])).astype(np.float32)
        if case % 4 == 1:
            v[speech:] += 8.0                        # end tokens likely: the trial loop runs before min_len
        if case % 4 == 2:
            v[: n // 2] = np.round(v[: n // 2])      # ties: equal probabilities sort by index
        hist = rng.integers(0, speech, int(rng.integers(0, 30))).astype(np.int32)
        if case % 3 == 0 and hist.size:
            hist[-win:] = int(np.argmax(v[:speech]))  # the likely pick repeats in the window: RAS resamples
        step = int(rng.integers(0, 40))
        min_len = int(rng.choice([0, 20, 100]))
        cfg = hip.lm_cfg(top_p=top_p, top_k=top_k, win_size=win, tau_r=tau, speech_tokens=speech, min_len=min_len,
                         seed=int(rng.integers(0, 2**40)), piece=int(rng.integers(0, 8)))
        dv, dh, dl = dev_logits(hip, v), dev_ints(hip, hist), hip.DevBuf(n * 4)
        want_lp = oracle.lm_logp(v)
        want, after = oracle.lm_step(want_lp, hist, step, min_len, speech, top_p, top_k, win, tau, cfg.seed, cfg.piece)
        resampled += bool(np.isneginf(after).any() and not np.isneginf(want_lp).any())
        if want == -2:
            with pytest.raises(hip.VoxHipError, match="max_trials"):
                hip.lm_sample_dev(dv, n, cfg, step, dh, hist.size, dl)
            continue
        got = hip.lm_sample_dev(dv, n, cfg, step, dh, hist.size, dl)
        lp = dl.download(n, np.float32)
        assert np.max(np.abs(lp - want_lp)) <= 2 * np.spacing(np.float32(np.abs(want_lp).max())), case
        assert got == want, (case, got, want)
        for d in (dv, dh, dl):
            d.free()
    assert resampled > 0  # the repetition-aware draw ran in some cases


def test_lm_sample_trial_limit(hip, oracle):
    # only end tokens have probability: before min_len every trial draws an end token -> the reference's failure
    n, speech = 300, 297
    v = np.full(n, -1e30, np.float32)
    v[speech:] = 0.0
    cfg = hip.lm_cfg(speech_tokens=speech, min_len=50)
    dv = dev_logits(hip, v)
    assert oracle.lm_step(oracle.lm_logp(v), [], 3, 50, speech)[0] == -2
    with pytest.raises(hip.VoxHipError, match="max_trials"):
        hip.lm_sample_dev(dv, n, cfg, 3)
    assert hip.lm_sample_dev(dv, n, cfg, 50) >= speech  # at min_len the end token is accepted
    with pytest.raises(hip.VoxHipError):
        hip.lm_sample_dev(dv, n, hip.lm_cfg(top_k=0, speech_tokens=speech), 0)


def cosy_model(seed, wtype=Q8, V=300, speech=297, emb_type=Q8):
    # CosyVoice2-shaped (Qwen2): GQA 7:1, head_dim 64, q/k/v biases, no q/k norm; f32 head with bias
    mdl = Model(seed, 2, 128, 7, 1, 64, 256, wtype=wtype, qk_norm=False, bias=True)
    rng = np.random.default_rng(seed + 1)
    hd, hs, hb = make_mat(rng, F32, V, 128, bias=True)
    ed, es, _ = make_mat(rng, emb_type, speech + 3, 128)
    return mdl, (hd, hs, hb), (ed, es)


@pytest.mark.parametrize("wtype,n,min_len,max_len", [(Q8, 20, 6, 24), (Q8, 5, 0, 40), (F16, 12, 3, 17)])
def test_lm_generate_teacher_forced(hip, oracle, wtype, n, min_len, max_len):
    V, speech = 300, 297
    mdl, (hd, hs, hb), (ed, es) = cosy_model(700 + n, wtype, V, speech)
    xf = hip.xfmr_create(mdl.hx, "llm")
    head = hip.upload(hip.HostMat(F32, hd, V, 128, hs, hb))
    emb = hip.upload(hip.HostMat(Q8, ed, speech + 3, 128, es))
    Ho = oracle.Mat(F32, hd, V, 128, hs, hb)
    Eo = oracle.Mat(Q8, ed, speech + 3, 128, es)
    seq = hip.seq_create(xf, n + max_len + 1)
    rng = np.random.default_rng(n)
    x = rng.standard_normal((n, 128)).astype(np.float32)
    cfg = hip.lm_cfg(speech_tokens=speech, min_len=min_len, max_len=max_len, seed=4321, piece=2)
    tokens, logp = hip.lm_generate(xf, seq, x, head, emb, cfg, want_logp=True)
    assert logp.shape[0] == min(tokens.size + 1, max_len)
    kv = mdl.oracle_kv(n + max_len + 1, kv_f16=1)
    h = oracle.transformer_forward(mdl.ox, kv, x)
    for i in range(logp.shape[0]):
        want_lp = oracle.lm_logp(oracle.matmul(Ho, h[None])[0])
        assert rel_err(logp[i], want_lp) < TOL, (i, rel_err(logp[i], want_lp))
        tok, _ = oracle.lm_step(logp[i], tokens[:i], i, min_len, speech, cfg.top_p, cfg.top_k, cfg.win_size, cfg.tau_r,
                                cfg.seed, cfg.piece)
        if i < tokens.size:
            assert tok == tokens[i], (i, tok, tokens[i])
            h = oracle.transformer_forward(mdl.ox, kv, oracle.mat_row(Eo, int(tokens[i]))[None])
        else:
            assert tok >= speech  # the generation ended on an end token
    if tokens.size == max_len:
        assert logp.shape[0] == max_len
    # the same generation again (cached graph, reused sequence) gives the same tokens
    tokens2, _ = hip.lm_generate(xf, seq, x, head, emb, cfg)
    assert np.array_equal(tokens, tokens2)


def test_lm_generate_rejects_short_capacity(hip):
    V, speech = 300, 297
    mdl, (hd, hs, hb), (ed, es) = cosy_model(800, Q8, V, speech)
    xf = hip.xfmr_create(mdl.hx, "llm")
    head = hip.upload(hip.HostMat(F32, hd, V, 128, hs, hb))
    emb = hip.upload(hip.HostMat(Q8, ed, speech + 3, 128, es))
    seq = hip.seq_create(xf, 30)
    x = np.zeros((10, 128), np.float32)
    with pytest.raises(hip.VoxHipError, match="capacity"):
        hip.lm_generate(xf, seq, x, head, emb, hip.lm_cfg(speech_tokens=speech, max_len=20))
    toks, _ = hip.lm_generate(xf, seq, x, head, emb, hip.lm_cfg(speech_tokens=speech, max_len=19))
    assert toks.size <= 19
