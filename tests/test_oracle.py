"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the parity checker.

Each restated function is checked against at least one of:
  - the reference's own known answers (tests/test_core.cpp of the reference: Philox KAT :35-43, sampler rules
    :45-79, Q4 bounds :461-521, noise moments :630-645);
  - the golden fixture written by the compiled reference (tests/golden/golden_ref.npz, bit-exact);
  - the compiled reference harness itself when present (oracle/_ref, bit-exact);
  - float64 / closed-form / brute-force checks that do not restate the oracle's code path.
"""
import os

import numpy as np
import pytest

import pyoracle as po

GOLD = os.path.join(os.path.dirname(__file__), "golden", "golden_ref.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def philox(c, k):
    c = np.ascontiguousarray(c, np.uint32)
    k = np.ascontiguousarray(k, np.uint32)
    out = np.empty(4, np.uint32)
    po.lib().vo_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
    return out


# ------------------------------------------------------------------ Philox / DetRng
def test_philox_random123_kat(oracle):
    # Random123 known-answer vectors, as the reference checks them (test_core.cpp:35-43)
    assert list(philox([0, 0, 0, 0], [0, 0])) == [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]
    assert list(philox([0xffffffff] * 4, [0xffffffff] * 2)) == [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]
    assert list(philox([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0])) == \
        [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]


def test_philox_golden(oracle, gold):
    for c, k, o in zip(gold["philox_ctr"], gold["philox_key"], gold["philox_out"]):
        assert list(philox(c, k)) == list(o)


def test_uniform_closed_form_and_golden(oracle, gold):
    # u = (r0 >> 8) / 2^24 with counter (frame lo, frame hi, codebook, draw) under key (seed lo, seed hi):
    # KAT vector 1 is the counter/key (0,0,0,0)/(0,0)
    assert po.uniform(0, 0, 0, 0) == np.float32((0x6627e8d5 >> 8) / 16777216.0)
    for a, o in zip(gold["uniform_args"], gold["uniform_out"]):
        assert np.float32(po.uniform(int(a[0]), int(a[1]), int(a[2]) & 0xFFFFFFFF, int(a[3]) & 0xFFFFFFFF)) == o
    assert po.uniform(42, 5, 3) == po.uniform(42, 5, 3)
    assert po.uniform(42, 5, 3) != po.uniform(43, 5, 3)
    assert po.uniform(42, 5, 3) != po.uniform(42, 5, 4)
    assert 0.0 <= po.uniform(42, 0, 0) < 1.0


# ------------------------------------------------------------------ sampler
def test_sampler_rules(oracle):
    # test_core.cpp:45-79
    l = [0.1, 3.0, 0.2, 3.0]
    assert po.sample_logits(l, temperature=0.0) == 1  # tie -> lower index
    for u in (0.0, 0.3, 0.99):
        assert po.sample_logits(l, top_k=1, u=u) == 1
    assert po.sample_logits(l, temperature=0.0, rep=10.0, history=[1]) == 3
    two = [0.0, float(np.log(3.0))]
    ones = sum(po.sample_logits(two, temperature=1.0, top_k=0, u=po.uniform(42, i, 0)) == 1 for i in range(20000))
    assert abs(ones / 20000.0 - 0.75) < 0.02


def test_sampler_inverse_cdf_brute_force(oracle):
    # With u on a fine grid, the share of draws picking token i equals its probability after top-k / top-p,
    # computed here independently in float64.
    rng = np.random.default_rng(1)
    for T, k, p in ((1.0, 0, 1.0), (0.7, 5, 1.0), (1.3, 8, 0.6)):
        l = rng.standard_normal(12).astype(np.float32) * 2
        order = sorted(range(12), key=lambda i: (-l[i], i))
        kk = k if 0 < k < 12 else 12
        sel = order[:kk]
        w = np.exp((l[sel].astype(np.float64) - l[sel[0]]) / T)
        w /= w.sum()
        keep = kk
        if 0 < p < 1:
            keep = int(np.searchsorted(np.cumsum(w), p) + 1)
        w = w[:keep] / w[:keep].sum()
        N = 20000
        counts = np.zeros(12)
        for j in range(N):
            counts[po.sample_logits(l, temperature=T, top_k=k, top_p=p, u=(j + 0.5) / N)] += 1
        exp = np.zeros(12)
        exp[sel[:keep]] = w
        assert np.max(np.abs(counts / N - exp)) < 2.0 / N + 1e-9


def test_sampler_golden(oracle, gold):
    off = hoff = 0
    for i in range(len(gold["sample_idx"])):
        n, hn = int(gold["sample_n"][i]), int(gold["sample_hist_n"][i])
        l = gold["sample_logits"][off:off + n]
        h = gold["sample_hist"][hoff:hoff + hn]
        off += n
        hoff += hn
        T, top_p, top_k, rep, u = gold["sample_params"][i]
        got = po.sample_logits(l, float(T), float(top_p), int(top_k), float(rep), h if hn else None, float(u))
        assert got == gold["sample_idx"][i], i


def test_sampler_vs_ref(ref):
    rng = np.random.default_rng(5)
    for i in range(300):
        n = int(rng.choice([3, 64, 3072, 6564]))
        l = (rng.standard_normal(n) * 3).astype(np.float32)
        if i % 3 == 0:
            l = np.round(l * 2).astype(np.float32)
        T = float(rng.choice([0.0, 0.9, 1.0]))
        k = int(rng.choice([0, 1, 25, 50]))
        p = float(rng.choice([1.0, 0.8]))
        u = float(np.float32(rng.uniform()))
        assert po.sample_logits(l, T, p, k, 1.0, None, u) == po.sample_logits(l, T, p, k, 1.0, None, u, use_ref=True)


def test_ras_sample_properties(oracle):
    # cosyvoice.cpp:617-664: nucleus by probability, then a repetition-aware resample from the full distribution
    rng = np.random.default_rng(3)
    n = 40
    lp = rng.standard_normal(n).astype(np.float32)
    pr = np.exp(lp.astype(np.float64) - lp.max())
    pr /= pr.sum()
    order = np.argsort(-pr, kind="stable")
    f = po.lib().vo_ras_sample

    def ras(decoded, u0, u1, top_p=0.8, top_k=25, win=10, tau=0.1):
        l = lp.copy()
        d = np.ascontiguousarray(decoded, np.int32)
        return f(l.ctypes.data, n, d.ctypes.data if d.size else None, d.size, top_p, top_k, win, tau, u0, u1)

    # top_k = 1 -> the most probable token, whatever u
    assert all(ras([], u, 0.5, top_k=1) == order[0] for u in (0.0, 0.5, 0.999))
    # no history: the nucleus (cum < top_p, at most top_k) is sampled by inverse CDF
    keep, cum = [], 0.0
    for i in order:
        if cum < 0.8 and len(keep) < 25:
            keep.append(i)
            cum += pr[i]
        else:
            break
    w = pr[keep] / pr[keep].sum()
    N = 4000
    counts = np.zeros(n)
    for j in range(N):
        counts[ras([], (j + 0.5) / N, 0.5)] += 1
    exp = np.zeros(n)
    exp[keep] = w
    assert np.max(np.abs(counts / N - exp)) < 2.0 / N + 1e-9
    # the top token repeated in the window -> never returned; the resample follows the rest of the distribution
    top = order[0]
    got = [ras([top] * 10, 0.0, (j + 0.5) / 400) for j in range(400)]
    assert top not in got
    rest = pr.copy()
    rest[top] = 0
    rest /= rest.sum()
    c = np.bincount(got, minlength=n) / 400
    assert np.max(np.abs(c - rest)) < 2.0 / 400 + 1e-9


def test_lm_logp_closed_form(oracle):
    # cosyvoice.cpp:602-606: logp = v - (mx + float(log(sum exp(double(v - mx))))): a float64 log-softmax to f32 ulps
    rng = np.random.default_rng(11)
    for n in (2, 300, 6564):
        v = (rng.standard_normal(n) * 4).astype(np.float32)
        v[rng.integers(0, n)] += 30  # a dominant entry
        got = po.lm_logp(v)
        v64 = v.astype(np.float64)
        want = v64 - (v64.max() + np.log(np.exp(v64 - v64.max()).sum()))
        assert np.max(np.abs(got - want)) <= 4 * np.spacing(np.float32(np.abs(want).max()))
        assert abs(np.log(np.exp(got.astype(np.float64)).sum())) < 1e-5  # normalized
        assert np.argmax(got) == np.argmax(v)


def test_lm_step_trial_loop(oracle):
    # lm_generate (cosyvoice.cpp:674-683): u0, u1 = DetRng(seed).uniform(step, 0x43560000 + piece, 2 trial (+1));
    # no end token before min_len; failure after trial 101
    rng = np.random.default_rng(12)
    n, speech = 64, 60
    lp = po.lm_logp(rng.standard_normal(n).astype(np.float32))
    f = po.lib().vo_ras_sample
    def ras(l, decoded, u0, u1):
        l = l.copy()
        d = np.ascontiguousarray(decoded, np.int32)
        return f(l.ctypes.data, n, d.ctypes.data if d.size else None, d.size, 0.8, 25, 10, 0.1, u0, u1), l
    # at or past min_len: one ras_sample draw with the trial-0 counters
    for step in (0, 5, 17):
        u0 = po.uniform(99, step, 0x43560000 + 7, 0)
        u1 = po.uniform(99, step, 0x43560000 + 7, 1)
        tok, _ = po.lm_step(lp, [], step, 0, speech, seed=99, piece=7)
        assert tok == ras(lp, [], u0, u1)[0]
    # only end tokens can be picked: every trial draws one, the reference fails after trial 101 (102 draws)
    only_end = np.full(n, -np.inf, np.float32)
    only_end[speech:] = np.log(0.25)
    assert po.lm_step(only_end, [], 3, 10, speech)[0] == -2
    assert po.lm_step(only_end, [], 10, 10, speech)[0] >= speech  # at min_len the end is accepted
    # half end token, half speech token (same probability: the lower index sorts first): the loop ends at the
    # first trial whose u0 falls in the speech token's half
    two = np.full(n, -np.inf, np.float32)
    two[[5, speech]] = np.log(0.5)
    tok, _ = po.lm_step(two, [], 2, 10, speech, seed=5)
    first = next(t for t in range(102) if po.uniform(5, 2, 0x43560000, 2 * t) * 1.0 < 0.5)
    assert tok == 5 and first < 101
    # the resampled pick keeps logp = -inf across trials: a token repeated twice in the window is never returned
    rep = int(np.argmax(lp[:speech]))
    tok, l2 = po.lm_step(lp, [rep, rep, 1, 2], 0, 5, speech)
    assert tok != rep and tok < speech


def test_f5_activations_closed_form(oracle):
    # f5.cpp:93-100 against float64 formulas
    xs = np.concatenate([np.linspace(-12, 25, 2001), [-0.0, 1e-8, 19.999, 20.0, 20.001]]).astype(np.float32)
    x64 = xs.astype(np.float64)
    gel = 0.5 * x64 * (1 + np.tanh(np.sqrt(2 / np.pi) * (x64 + 0.044715 * x64 ** 3)))
    mis = x64 * np.tanh(np.where(x64 > 20, x64, np.log1p(np.exp(x64))))
    g = np.array([po.lib().vo_gelu_tanh(float(v)) for v in xs])
    mm = np.array([po.lib().vo_mish(float(v)) for v in xs])
    assert np.max(np.abs(g - gel) / np.maximum(1, np.abs(gel))) < 2e-6
    assert np.max(np.abs(mm - mis) / np.maximum(1, np.abs(mis))) < 2e-6


def test_conv1d_matches_reference_and_brute_force(oracle):
    # Conv1d (f5_ops.cpp:86-147): grouped "same" convolution; bit-exact against the compiled reference, and a float64
    # brute force of y[t][o] = b[o] + sum_{k,i} w[o][i][k] x[t + k - K/2][g cig + i]
    rng = np.random.default_rng(21)
    for cin, K, groups, T in ((64, 31, 16, 45), (48, 7, 4, 9), (32, 5, 32, 20), (16, 3, 1, 2)):
        w = (rng.standard_normal((cin, cin // groups, K)) * 0.1).astype(np.float32)
        b = (rng.standard_normal(cin) * 0.1).astype(np.float32)
        x = rng.standard_normal((T, cin)).astype(np.float32)
        cv = po.Conv.from_torch(w, b, groups)
        y = po.conv1d(cv, x)
        if po.ref() is not None:
            assert np.array_equal(y, po.conv1d(cv, x, use_ref=True, w_pt=w))
        cig, cog, pad = cin // groups, cin // groups, K // 2
        xp = np.zeros((T + 2 * pad, cin))
        xp[pad:pad + T] = x
        want = np.tile(b.astype(np.float64), (T, 1))
        for o in range(cin):
            g = o // cog
            for k in range(K):
                want[:, o] += xp[k:k + T, g * cig:(g + 1) * cig] @ w[o, :, k].astype(np.float64)
        assert np.max(np.abs(y - want)) < 1e-5


def convt_brute(w, b, x, s, pad, out_pad):
    """ConvTranspose1d in float64 from its definition: y[t s + k - pad][o] += sum_i x[t][i] w[i][o][k], kept where
    0 <= t s + k - pad < To, plus the bias."""
    cin, cout, K = w.shape
    T = x.shape[0]
    To = (T - 1) * s - 2 * pad + K + out_pad
    y = np.zeros((To, cout)) + (0 if b is None else b.astype(np.float64))
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    for t in range(T):
        for k in range(K):
            r = t * s + k - pad
            if 0 <= r < To:
                y[r] += x64[t] @ w64[:, :, k]
    return y


# (cin, cout, K, stride, pad, out_pad, T, bias): HiFT's and Kokoro's upsample stages (pad (K - stride) / 2), output
# padding, K < stride (frames that no tap reaches carry only the bias), pad >= K / 2, one frame, and 300 frames at
# K cout = 14336 (the reference's 292-frame product blocks, so two blocks)
CONVT_CASES = [(64, 32, 16, 8, 4, 0, 12, True), (48, 24, 11, 5, 3, 0, 9, True), (40, 20, 20, 10, 5, 0, 6, True),
               (24, 16, 5, 2, 2, 1, 13, False), (16, 8, 4, 3, 1, 2, 7, True), (16, 8, 3, 5, 0, 0, 9, True),
               (8, 8, 4, 1, 3, 0, 12, True), (20, 12, 6, 3, 1, 0, 1, True), (12, 1024, 14, 7, 3, 0, 300, True)]


@pytest.mark.parametrize("cin,cout,K,s,pad,op,T,bias", CONVT_CASES)
def test_convt_matches_reference_and_brute_force(oracle, cin, cout, K, s, pad, op, T, bias):
    # nn::ConvT (nn.cpp:205-245): bit-exact against the compiled reference's ConvT::forward, and within float rounding
    # of the float64 definition
    rng = np.random.default_rng(cin * 31 + K * 7 + T)
    w = (rng.standard_normal((cin, cout, K)) * 0.2).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32) if bias else None
    x = rng.standard_normal((T, cin)).astype(np.float32)
    y = po.convt(w, b, x, s, pad, op)
    want = convt_brute(w, b, x, s, pad, op)
    assert y.shape == want.shape
    assert np.max(np.abs(y - want)) < 1e-5 * max(1.0, np.abs(want).max())
    if po.ref() is not None:
        assert np.array_equal(y.view(np.uint32), po.convt(w, b, x, s, pad, op, use_ref=True).view(np.uint32))
    with pytest.raises(ValueError):
        po.convt(w, b, x[:1], 1, K + 1, 0)  # no output frames


def test_f5_modulate_closed_form(oracle):
    # f5.cpp:608-625: LayerNorm without parameters (double statistics, eps 1e-6) then x * (1 + scale) + shift
    rng = np.random.default_rng(22)
    x = (rng.standard_normal((7, 96)) * 3 + 1).astype(np.float32)
    sc, sh = rng.standard_normal(96).astype(np.float32), rng.standard_normal(96).astype(np.float32)
    y = po.f5_modulate(x, sc, sh)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-6) * (1 + sc) + sh
    assert np.max(np.abs(y - want)) < 1e-5


def test_gelu_erf_pinned(oracle):
    # kernels.hpp:106: 0.5 x (1 + erf(x / sqrt 2)); bit-exact against the compiled reference, within float rounding of the
    # float64 closed form (absolute: the formula's own cancellation near x = -5.5, where the value is ~1e-7), and the
    # identity gelu(x) - gelu(-x) = x
    import math
    xs = np.concatenate([np.linspace(-9, 9, 3001), np.random.default_rng(5).standard_normal(500) * 3]).astype(np.float32)
    for x in xs:
        g = po.gelu_erf(float(x))
        if po.ref() is not None:
            assert np.float32(g) == np.float32(po.gelu_erf(float(x), use_ref=True))
        want = 0.5 * float(x) * (1 + math.erf(float(x) / math.sqrt(2)))
        assert abs(g - want) <= 3e-7 * max(1.0, abs(float(x))), (x, g, want)
        assert abs((g - po.gelu_erf(float(-x))) - float(x)) <= 4e-7 * max(1.0, abs(float(x)))
    assert po.gelu_erf(0.0) == 0.0


def vocos_numpy(v, mel):
    """F5Model::vocode up to the head in float64 numpy, written from the Vocos equations (ConvNeXt blocks), for pinning
    vo_vocos_head."""
    from scipy.special import erf

    def conv(c, x):
        w, b, cin, cout, K, groups = c
        if groups == cin and w.ndim == 2:  # depthwise [C][K]
            w = w.reshape(groups, 1, K, 1)
        cig, pad = cin // groups, K // 2
        cog = cout // groups
        xp = np.zeros((x.shape[0] + 2 * pad, cin))
        xp[pad:pad + x.shape[0]] = x
        y = np.tile(b.astype(np.float64), (x.shape[0], 1))
        for g in range(groups):
            for k in range(K):
                y[:, g * cog:(g + 1) * cog] += xp[k:k + x.shape[0], g * cig:(g + 1) * cig] @ w[g, :, k, :].T.astype(np.float64)
        return y

    def ln(x, w, b):
        return (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-6) * w + b

    def lin(t, x):
        typ, d, r, c, s, b = t
        W = np.stack([po.mat_row(po.Mat(typ, d, r, c, s, b), i) for i in range(r)]).astype(np.float64)
        return x @ W.T + (b.astype(np.float64) if b is not None else 0)
    x = ln(conv(v["embed"], mel.astype(np.float64)), v["ln_w"], v["ln_b"])
    for blk in v["blocks"]:
        y = ln(conv(blk["dw"], x), blk["ln_w"], blk["ln_b"])
        h = lin(blk["pw1"], y)
        h = 0.5 * h * (1 + erf(h / np.sqrt(2)))
        x = x + blk["gamma"] * lin(blk["pw2"], h)
    return lin(v["head"], ln(x, v["fln_w"], v["fln_b"]))


@pytest.mark.parametrize("wt", [0, 1, 2])
def test_vocos_head_against_numpy(oracle, wt):
    import models
    m = models.F5Model(40 + wt, 32, 1, 2, dim_head=16, mel=12, text=8, K=5, groups=4, wtype=wt,
                       vocos=dict(dim=48, inter=96, layers=2, out=18))
    mel = np.random.default_rng(wt).standard_normal((37, 12)).astype(np.float32)
    got = po.vocos_head(m.vox, mel)
    want = vocos_numpy(m.vocos, mel)
    assert np.max(np.abs(got - want)) / max(1.0, np.max(np.abs(want))) < 1e-5


def f5_numpy(m, B, N, cat, ts, rope):
    """dit_forward in float64 numpy, written from the model's equations (F5-TTS DiT), for pinning vo_f5_step."""
    D, H, HD, mel = m.dim, m.heads, m.hd, m.mel
    INNER, HH = H * HD, HD // 2

    def lin(name_or_tuple, x):
        t, d, r, c, s, b = name_or_tuple
        w = po.Mat(t, d, r, c, s, b)
        W = np.stack([po.mat_row(w, i) for i in range(r)]).astype(np.float64)
        return x @ W.T + (b.astype(np.float64) if b is not None else 0)

    def conv(c, x):
        w, b, cin, cout, K, groups = c
        cig, pad = cin // groups, K // 2
        xp = np.zeros((x.shape[0] + 2 * pad, cin))
        xp[pad:pad + x.shape[0]] = x
        y = np.tile(b.astype(np.float64), (x.shape[0], 1))
        for g in range(groups):
            for k in range(K):
                y[:, g * cig:(g + 1) * cig] += xp[k:k + x.shape[0], g * cig:(g + 1) * cig] @ w[g, :, k, :].T.astype(np.float64)
        return y

    def mish(v):
        return v * np.tanh(np.where(v > 20, v, np.log1p(np.exp(np.minimum(v, 20)))))

    def modulate(x, sc, sh):
        return (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-6) * (1 + sc) + sh

    ts = ts.astype(np.float64)
    h = lin(m.mats["in_proj"], cat.astype(np.float64))
    for s in range(B):
        hs = h[s * N:(s + 1) * N]
        hs += mish(conv(m.pos[1], mish(conv(m.pos[0], hs))))
    cos, sin = rope[..., 0].astype(np.float64), rope[..., 1].astype(np.float64)
    for blk in m.blocks:
        ada = lin(blk["ada"], ts[None])[0]
        sh1, sc1, g1, sh2, sc2, g2 = (ada[i * D:(i + 1) * D] for i in range(6))
        nrm = modulate(h, sc1, sh1)
        q, k, v = lin(blk["q"], nrm), lin(blk["k"], nrm), lin(blk["v"], nrm)
        for t in (q, k):
            for hh in range(H):
                if m.pe > 0 and hh >= m.pe:
                    continue
                pos = np.arange(B * N) % N
                x0 = t[:, hh * HD:(hh + 1) * HD:2].copy()
                x1 = t[:, hh * HD + 1:(hh + 1) * HD:2].copy()
                t[:, hh * HD:(hh + 1) * HD:2] = x0 * cos[pos] - x1 * sin[pos]
                t[:, hh * HD + 1:(hh + 1) * HD:2] = x1 * cos[pos] + x0 * sin[pos]
        at = np.zeros((B * N, INNER))
        for s in range(B):
            for hh in range(H):
                rows, cols = slice(s * N, (s + 1) * N), slice(hh * HD, (hh + 1) * HD)
                sc = q[rows, cols] @ k[rows, cols].T / np.sqrt(HD)
                p = np.exp(sc - sc.max(1, keepdims=True))
                at[rows, cols] = (p / p.sum(1, keepdims=True)) @ v[rows, cols]
        h = h + g1 * lin(blk["o"], at)
        f = lin(blk["ff1"], modulate(h, sc2, sh2))
        f = 0.5 * f * (1 + np.tanh(np.sqrt(2 / np.pi) * (f + 0.044715 * f ** 3)))
        h = h + g2 * lin(blk["ff2"], f)
    fin = lin(m.mats["norm_out"], ts[None])[0]
    return lin(m.mats["proj_out"], modulate(h, fin[:D], fin[D:]))


@pytest.mark.parametrize("pe", [0, 1])
def test_f5_step_against_numpy(oracle, pe):
    import models
    m = models.F5Model(30 + pe, 64, 2, 2, dim_head=16, mel=12, text=8, K=5, groups=4, pe_attn_head=pe, wtype=models.F16)
    rng = np.random.default_rng(31)
    B, N = 2, 23
    cat0, x, ts, rope = m.inputs(rng, B, N)
    cat = m.with_x(cat0, x, B)
    got = po.f5_step(m.ox, B, N, cat, ts, rope)
    want = f5_numpy(m, B, N, cat, ts, rope)
    assert np.max(np.abs(got - want)) / max(1.0, np.max(np.abs(want))) < 2e-5


def test_noise_moments(oracle):
    # test_core.cpp:630-645
    a = po.noise(42, 0xF5000000 + 3, 100001)
    b = po.noise(42, 0xF5000000 + 3, 100001)
    c = po.noise(42, 0xF5000000 + 4, 100001)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    m = a.astype(np.float64).mean()
    v = ((a - m) ** 2).mean()
    assert abs(m) < 0.02 and abs(v - 1.0) < 0.03


# ------------------------------------------------------------------ formats
def test_f16_conversions_exhaustive(oracle):
    L = po.lib()
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.vo_f16_to_f32(int(x)) for x in h], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin], ref[fin]) and np.all(np.isnan(got[~fin]) == np.isnan(ref[~fin]))
    rng = np.random.default_rng(2)
    f = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-3, 1, 1e3, 7e4)])
    f = np.concatenate([f, np.float32([0, -0.0, 65504, 65519, 65520, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08, 2.98e-08])])
    got = np.array([L.vo_f32_to_f16(float(x)) for x in f], np.uint16)
    assert np.array_equal(got, f.astype(np.float16).view(np.uint16))


def test_quantize_q8_golden_and_bounds(oracle, gold):
    q, s = po.quantize_q8(gold["quant_w"])
    assert np.array_equal(q, gold["q8_q"]) and np.array_equal(s.view(np.uint32), gold["q8_s"].view(np.uint32))
    w = gold["quant_w"]
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    deq = q.astype(np.float32).reshape(37, 5, 32) * s[:, :, None]
    err = np.abs(deq - w.reshape(37, 5, 32))
    assert np.all(err <= s[:, :, None] * 0.5 * (1 + 1e-6) + 1e-30)


def test_quantize_q4_golden_and_bounds(oracle, gold):
    q, s = po.quantize_q4(gold["quant_w"])
    assert np.array_equal(q, gold["q4_q"]) and np.array_equal(s.view(np.uint32), gold["q4_s"].view(np.uint32))
    # test_core.cpp:461-500: error within two quantization steps per element
    M = po.Mat(po.Q4, q, 37, 160, s)
    deq = np.stack([po.mat_row(M, r) for r in range(37)])
    step = np.repeat(np.abs(s), 32, axis=1)
    assert np.all(np.abs(deq - gold["quant_w"]) <= step * 2.001)


GOLD_Q4 = os.path.join(os.path.dirname(__file__), "golden", "golden_q4.npz")


def test_quantize_q4_float_rounding_golden(oracle):
    # blocks whose best candidate error and a rival lie within float rounding of each other: the reference keeps
    # best_err as a float (kernels.cpp:616, :629, :638), which decides these blocks (tests/golden/make_golden.py q4)
    g = np.load(GOLD_Q4, allow_pickle=False)
    q, s = po.quantize_q4(g["w"])
    assert g["w"].shape[0] >= 2000
    assert np.array_equal(s.view(np.uint32), g["s"].view(np.uint32))
    assert np.array_equal(q, g["q"])


def _random_quant_matrices(rng):
    """N(0, 0.02), U(-1, 1), near-grid and wide-range 4096 x 1024 matrices (131,072 blocks each)."""
    yield (rng.standard_normal((4096, 1024)) * 0.02).astype(np.float32)
    yield rng.uniform(-1, 1, (4096, 1024)).astype(np.float32)
    yield (rng.integers(-8, 8, (4096, 1024)) * 0.01 + rng.standard_normal((4096, 1024)) * 1e-6).astype(np.float32)
    yield (rng.standard_normal((4096, 1024)) * np.geomspace(1e-6, 1e3, 1024)).astype(np.float32)


@pytest.mark.ref
def test_quantizers_vs_ref_random(ref):
    # >= 1M random blocks per quantizer against the compiled reference (kernels.cpp:606-645, :918-929); the
    # seed-0 N(0, 0.02) matrix held 77 blocks a double best_err got wrong
    rng = np.random.default_rng(0)
    n = 0
    for _ in range(2):
        for w in _random_quant_matrices(rng):
            q, s = po.quantize_q4(w)
            rq, rs = po.quantize_q4(w, use_ref=True)
            assert np.array_equal(s.view(np.uint32), rs.view(np.uint32)) and np.array_equal(q, rq)
            q, s = po.quantize_q8(w)
            rq, rs = po.quantize_q8(w, use_ref=True)
            assert np.array_equal(s.view(np.uint32), rs.view(np.uint32)) and np.array_equal(q, rq)
            n += w.size // 32
    assert n >= 1 << 20


@pytest.mark.ref
@pytest.mark.parametrize("wt", [po.Q8, po.Q4, po.F32, po.F16, po.BF16])
def test_mat_row_vs_ref_random(ref, wt):
    # mat_row / mat_gather (kernels.cpp:432-471) on every type, f16 subnormals and infinities included
    rng = np.random.default_rng(40 + wt)
    rows, cols = 2048, 1024
    w = (rng.standard_normal((rows, cols)) * np.geomspace(1e-7, 1e4, cols)).astype(np.float32)
    if wt == po.Q8:
        data, s = po.quantize_q8(w)
    elif wt == po.Q4:
        data, s = po.quantize_q4(w)
    elif wt == po.F16:
        data, s = rng.integers(0, 1 << 16, (rows, cols)).astype(np.uint16), None
        data[:, :4] = [0x7c00, 0xfc00, 0x0001, 0x83ff]
    elif wt == po.BF16:
        data, s = (w.view(np.uint32) >> 16).astype(np.uint16), None
    else:
        data, s = w, None
    M = po.Mat(wt, data, rows, cols, s)
    for r in range(rows):
        a, b = po.mat_row(M, r), po.mat_row(M, r, use_ref=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), r


def test_q4_unpack_closed_form(oracle):
    # byte j of a block = w[j] | w[j+16] << 4, value (u - 8) * scale (kernels.hpp:44-47)
    rng = np.random.default_rng(4)
    u = rng.integers(0, 16, size=(3, 64)).astype(np.uint8)
    packed = np.empty((3, 32), np.uint8)
    for b in range(2):
        packed[:, b * 16:(b + 1) * 16] = u[:, b * 32:b * 32 + 16] | (u[:, b * 32 + 16:b * 32 + 32] << 4)
    s = rng.uniform(0.1, 1, size=(3, 2)).astype(np.float32)
    M = po.Mat(po.Q4, packed, 3, 64, s)
    for r in range(3):
        exp = (u[r].astype(np.float32) - 8) * np.repeat(s[r], 32)
        assert np.array_equal(po.mat_row(M, r), exp)


# ------------------------------------------------------------------ matmul
@pytest.mark.parametrize("name,wt", [("q8", po.Q8), ("q4", po.Q4), ("f32", po.F32), ("f16", po.F16)])
@pytest.mark.parametrize("m", [1, 3, 8, 12])
def test_matmul_golden(oracle, gold, name, wt, m):
    w = gold["quant_w"]
    data = {"q8": gold["q8_q"], "q4": gold["q4_q"], "f32": w, "f16": w.astype(np.float16).view(np.uint16)}[name]
    scale = {"q8": gold["q8_s"], "q4": gold["q4_s"]}.get(name)
    M = po.Mat(wt, data, 37, 160, scale, gold["mm_bias"])
    got = po.matmul(M, gold["mm_x"][:m])
    assert np.array_equal(got.view(np.uint32), gold[f"mm_{name}_m{m}"].view(np.uint32))


def test_matmul_int_path_vs_float64(oracle):
    # q8 m <= 8: exact int32 block dots on int8 activations; compare with a float64 sum over the same
    # quantized operands (an independent evaluation order)
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    q, s = po.quantize_q8(w)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    M = po.Mat(po.Q8, q, 64, 1024, s)
    y = po.matmul(M, x)
    for i in range(4):
        xq, xs = po.quantize_act(x[i])
        d = (q.reshape(64, 32, 32).astype(np.int64) * xq.reshape(32, 32).astype(np.int64)).sum(-1).astype(np.float64)
        ref = (d * (s.astype(np.float64) * xs.astype(np.float64))).sum(-1)
        assert np.max(np.abs(y[i] - ref)) <= 1e-5 * np.max(np.abs(ref))
    # the activation quantizer itself: |x - xq * xs| <= xs / 2 and max |xq| == 127 per non-zero block
    xq, xs = po.quantize_act(x[0])
    assert np.all(np.abs(x[0] - xq.astype(np.float32) * np.repeat(xs, 32)) <= np.repeat(xs, 32) * 0.5001)
    assert np.all(np.abs(xq.reshape(32, 32)).max(-1) == 127)


def test_matmul_vs_ref_random(ref):
    rng = np.random.default_rng(11)
    for wt in (po.Q8, po.Q4, po.F32, po.F16, po.BF16):
        for rows, cols in ((5, 32), (33, 96), (256, 1024)):
            w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
            if wt == po.Q8:
                data, s = po.quantize_q8(w)
            elif wt == po.Q4:
                data, s = po.quantize_q4(w)
            elif wt == po.F16:
                data, s = w.astype(np.float16).view(np.uint16), None
            elif wt == po.BF16:
                data, s = (w.view(np.uint32) >> 16).astype(np.uint16), None
            else:
                data, s = w, None
            b = rng.standard_normal(rows).astype(np.float32)
            M = po.Mat(wt, data, rows, cols, s, b)
            for m in (1, 2, 8, 9, 20):
                x = rng.standard_normal((m, cols)).astype(np.float32)
                a, r = po.matmul(M, x), po.matmul(M, x, use_ref=True)
                assert np.array_equal(a.view(np.uint32), r.view(np.uint32)), (wt, rows, cols, m)


# ------------------------------------------------------------------ elementwise
def test_norms_rope_softmax_golden(oracle, gold):
    L = po.lib()
    out = np.empty(1024, np.float32)
    x, w = gold["rms_x"], gold["rms_w"]
    L.vo_rmsnorm(x.ctypes.data, w.ctypes.data, 1024, np.float32(1e-6), out.ctypes.data)
    assert np.array_equal(out, gold["rms_out"])
    L.vo_layernorm(x.ctypes.data, w.ctypes.data, None, 1024, np.float32(1e-6), out.ctypes.data)
    assert np.array_equal(out, gold["ln_out"])
    s = x[:513].copy()
    L.vo_softmax(s.ctypes.data, 513)
    assert np.array_equal(s, gold["softmax_out"])
    inv = np.empty(64, np.float32)
    L.vo_rope_inv_freq(128, 1e6, inv.ctypes.data)
    assert np.array_equal(inv, gold["rope_inv"])
    q = gold["rope_x"].copy()
    L.vo_rope_apply(q.ctypes.data, 16, 128, inv.ctypes.data, 512)
    assert np.array_equal(q, gold["rope_out"])


def test_norms_rope_float64(oracle):
    # textbook formulas in float64 (independent evaluation): RMSNorm, LayerNorm, softmax, rotate-half RoPE
    L = po.lib()
    rng = np.random.default_rng(12)
    x = rng.standard_normal(1024).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    out = np.empty(1024, np.float32)
    L.vo_rmsnorm(x.ctypes.data, w.ctypes.data, 1024, np.float32(1e-6), out.ctypes.data)
    x64 = x.astype(np.float64)
    assert np.allclose(out, w * x64 / np.sqrt((x64 ** 2).mean() + 1e-6), rtol=2e-6, atol=1e-7)
    L.vo_layernorm(x.ctypes.data, w.ctypes.data, None, 1024, np.float32(1e-6), out.ctypes.data)
    assert np.allclose(out, (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-6) * w, rtol=2e-6, atol=1e-6)
    s = x[:100].copy()
    L.vo_softmax(s.ctypes.data, 100)
    e = np.exp(x64[:100] - x64[:100].max())
    assert np.allclose(s, e / e.sum(), rtol=1e-5, atol=1e-9)
    inv = np.empty(64, np.float32)
    L.vo_rope_inv_freq(128, 1e6, inv.ctypes.data)
    assert np.allclose(inv, 1.0 / 1e6 ** (np.arange(64) * 2 / 128.0), rtol=1e-7)
    q = rng.standard_normal(128).astype(np.float32)
    r = q.copy()
    L.vo_rope_apply(r.ctypes.data, 1, 128, inv.ctypes.data, 37)
    ang = inv.astype(np.float64) * 37
    a, b = q[:64].astype(np.float64), q[64:].astype(np.float64)
    assert np.allclose(r, np.concatenate([a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)]), atol=1e-5)
    assert abs(L.vo_silu(np.float32(1.5)) - 1.5 / (1 + np.exp(-1.5))) < 1e-6


# ------------------------------------------------------------------ transformer
def test_transformer_golden(oracle, gold):
    from models import Model
    mdl = Model(7, 2, 64, 4, 2, 32, 96, wtype=po.Q8)
    kv = mdl.oracle_kv(16, kv_f16=0)
    xs = gold["xf_x"]
    _, oa = po.transformer_forward(mdl.ox, kv, xs[:5], want_all=True)
    assert np.array_equal(oa, gold["xf_out_all5"])
    assert np.array_equal(po.transformer_forward(mdl.ox, kv, xs[5:6]), gold["xf_out6"])
    assert np.array_equal(po.transformer_forward(mdl.ox, kv, xs[6:7]), gold["xf_out7"])


def test_transformer_vs_ref(ref):
    from models import Model
    rng = np.random.default_rng(13)
    for wt, m in ((po.Q8, 1), (po.Q8, 4), (po.Q8, 11), (po.Q4, 3), (po.BF16, 2), (po.F16, 1)):
        mdl = Model(21 + m, 2, 128, 4, 2, 64, 256, wtype=wt)
        ka, kb = mdl.oracle_kv(64, 0), mdl.oracle_kv(64, 0)
        for step in range(3):
            x = rng.standard_normal((m, 128)).astype(np.float32)
            a = po.transformer_forward(mdl.ox, ka, x)
            b = po.transformer_forward(mdl.ox, kb, x, use_ref=True)
            assert np.array_equal(a, b), (wt, m, step)
        assert np.array_equal(ka.k[:, :ka.len], kb.k[:, :kb.len])
    # B sessions in one pass (transformer_forward_steps)
    mdl = Model(5, 2, 128, 4, 2, 64, 256, wtype=po.Q8)
    kvs_a = [mdl.oracle_kv(16, 0) for _ in range(3)]
    kvs_b = [mdl.oracle_kv(16, 0) for _ in range(3)]
    for b in range(3):  # different lengths per session
        pre = rng.standard_normal((b + 1, 128)).astype(np.float32)
        po.transformer_forward(mdl.ox, kvs_a[b], pre)
        po.transformer_forward(mdl.ox, kvs_b[b], pre, use_ref=True)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    assert np.array_equal(po.transformer_forward_steps(mdl.ox, kvs_a, x), po.transformer_forward_steps(mdl.ox, kvs_b, x, use_ref=True))


def test_transformer_steps_equal_single_calls(oracle):
    # transformer_forward_steps == B calls of transformer_forward with m = 1 (kernels.hpp:144-146)
    from models import Model
    rng = np.random.default_rng(14)
    mdl = Model(6, 2, 128, 4, 2, 64, 256, wtype=po.Q8)
    kv1 = [mdl.oracle_kv(16, 1) for _ in range(2)]
    kv2 = [mdl.oracle_kv(16, 1) for _ in range(2)]
    x = rng.standard_normal((2, 128)).astype(np.float32)
    a = po.transformer_forward_steps(mdl.ox, kv1, x)
    b = np.stack([po.transformer_forward(mdl.ox, kv2[i], x[i:i + 1]) for i in range(2)])
    assert np.array_equal(a, b)


def test_transformer_kv_f16_mode(oracle):
    # kv_f16 = 1 stores exactly the f16 rounding of what kv_f16 = 0 stores
    from models import Model
    rng = np.random.default_rng(15)
    mdl = Model(8, 1, 128, 4, 2, 64, 256, wtype=po.Q8)
    k0, k1 = mdl.oracle_kv(8, 0), mdl.oracle_kv(8, 1)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    po.transformer_forward(mdl.ox, k0, x)
    po.transformer_forward(mdl.ox, k1, x)
    assert np.array_equal(k1.k[:, :3], k0.k[:, :3].astype(np.float16).astype(np.float32))


def test_transformer_layers_compose(oracle):
    # layers [0, a) then [a, L) == layers [0, L); final norm of that == transformer_forward (bit-exact)
    from models import Model
    rng = np.random.default_rng(16)
    mdl = Model(9, 3, 128, 4, 2, 64, 256, wtype=po.Q8)
    x = rng.standard_normal((2, 128)).astype(np.float32)
    k1, k2, k3 = mdl.oracle_kv(8, 1), mdl.oracle_kv(8, 1), mdl.oracle_kv(8, 1)
    full = po.transformer_layers(mdl.ox, k1, x, 0, 3)
    part = po.transformer_layers(mdl.ox, k2, po.transformer_layers(mdl.ox, k2, x, 0, 1), 1, 2)
    assert np.array_equal(full, part)
    out = po.transformer_forward(mdl.ox, k3, x)
    nrm = np.empty(128, np.float32)
    po.lib().vo_rmsnorm(full[1].ctypes.data, mdl.final_norm.ctypes.data, 128, np.float32(1e-6), nrm.ctypes.data)
    assert np.array_equal(nrm, out)


# ------------------------------------------------------------------ CosyVoice2 / Chatterbox flow estimator
COSY_GOLD = os.path.join(os.path.dirname(__file__), "golden", "golden_cosy.npz")


@pytest.fixture(scope="module")
def cgold():
    return np.load(COSY_GOLD, allow_pickle=False)


def test_cosy_layers_golden(oracle, cgold):
    # nn.cpp's layers against the compiled reference's outputs, bit for bit: gelu_inplace (vector and scalar paths),
    # mish, layer_norm, attention, Conv::forward on a causally padded input
    x = cgold["act_x"]
    assert np.array_equal(po.gelu_poly(x), cgold["gelu_out"])
    assert np.array_equal(np.array([po.mish_nn(float(v)) for v in x], np.float32), cgold["mish_out"])
    assert np.array_equal(po.layer_norm_nn(cgold["ln_x"], cgold["ln_w"], cgold["ln_b"], 1e-5), cgold["ln_out"])
    assert np.array_equal(po.attention_nn(cgold["attn_q"], cgold["attn_k"], cgold["attn_v"], 3, 16, 0.25), cgold["attn_out"])
    cv = po.Conv(cgold["conv_w"], cgold["conv_b"], 8, 6, 3, 1)
    assert np.array_equal(po.causal_conv(cv, cgold["conv_x"]), cgold["conv_out"])


def test_cosy_step_golden(oracle, cgold):
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_golden
    import models
    # the weights come back from the fixture's seed; the inputs are checked against the stored ones
    T = make_golden.COSY_T
    m = models.CosyModel(make_golden.COSY_SEED, n_mid=1, n_x=1)
    in0, x, tb = m.inputs(np.random.default_rng(make_golden.COSY_SEED), T)
    assert np.array_equal(m.with_x(in0, x), cgold["cosy_in"]) and np.array_equal(tb, cgold["cosy_tb"])
    assert np.array_equal(po.cosy_step(m.ox, T, cgold["cosy_in"], tb), cgold["cosy_out"])


def test_cosy_layers_closed_forms(oracle):
    # what the mathematics fixes, independent of the restated code: gelu_poly is the erf GELU within its erfc fit
    # (1.2e-7 relative), mish is x tanh(softplus x), the causal conv never reads later rows, attention is
    # softmax(q k^T s) v
    import math
    rng = np.random.default_rng(8)
    xs = np.concatenate([np.linspace(-10, 10, 2001), rng.standard_normal(300) * 4]).astype(np.float32)
    g = po.gelu_poly(xs)
    for x, y in zip(xs.astype(np.float64), g):
        want = 0.5 * x * (1 + math.erf(x / math.sqrt(2)))
        assert abs(y - want) <= 2e-7 * max(1.0, abs(x)), (x, y, want)
    for x in xs.astype(np.float64):
        want = x if x > 20 else x * math.tanh(math.log1p(math.exp(x)))
        assert abs(po.mish_nn(float(x)) - want) <= 1e-6 * max(1.0, abs(x)), x
    w = (rng.standard_normal((5, 3, 8)) * 0.3).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    cv = po.Conv(w, b, 8, 5, 3, 1)
    x = rng.standard_normal((9, 8)).astype(np.float32)
    y = po.causal_conv(cv, x)
    xp = np.concatenate([np.zeros((2, 8)), x]).astype(np.float64)
    want = np.stack([sum(w[:, k, :].astype(np.float64) @ xp[t + k] for k in range(3)) + b for t in range(9)])
    assert np.max(np.abs(y - want)) < 1e-5
    x2 = x.copy()
    x2[6:] += 1.0  # later rows change, earlier outputs do not
    assert np.array_equal(po.causal_conv(cv, x2)[:6], y[:6])
    q, k, v = (rng.standard_normal((7, 2 * 16)).astype(np.float32) for _ in range(3))
    out = po.attention_nn(q, k, v, 2, 16, 0.25)
    for h in range(2):
        sl = slice(16 * h, 16 * h + 16)
        s = q[:, sl].astype(np.float64) @ k[:, sl].T.astype(np.float64) * 0.25
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert np.max(np.abs(out[:, sl] - p @ v[:, sl])) < 1e-5


@pytest.mark.parametrize("wt", [0, 1, 3])
def test_cosy_step_against_reference(ref, wt):
    # the whole estimator call, restated, against the same call composed from the compiled reference's own layers
    # (ref_cosy_step: nn.cpp's Conv, layer_norm, mish, Linear, attention and gelu_inplace in cosyvoice.cpp's order)
    import models
    m = models.CosyModel(60 + wt, M=8, C=64, heads=2, head_dim=32, n_mid=2, n_x=2, ff=96, wtype=wt)
    rng = np.random.default_rng(wt)
    for T in (1, 5, 16):
        in0, x, tb = m.inputs(rng, T)
        inp = m.with_x(in0, x)
        assert np.array_equal(po.cosy_step(m.ox, T, inp, tb), po.cosy_step(m.ox, T, inp, tb, use_ref=True)), T


# ------------------------------------------------------------------ Qwen3-TTS codec decoder
def test_codec_golden(oracle):
    # the whole codec_forward (quantizer, pre_conv, windowed transformer with layer scales, upsampling ConvNeXt,
    # decoder blocks, clamp) against the compiled reference's Qwen3Weights::codec_forward, bit for bit, two calls
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_golden
    import models
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_codec.npz"), allow_pickle=False)
    m = models.CodecModel(make_golden.CODEC_SEED)
    assert np.array_equal(m.codes(np.random.default_rng(make_golden.CODEC_SEED), make_golden.CODEC_F), g["codes"])
    st = po.CodecState(m.ox)
    z = po.codec_quantize(m.ox, g["codes"])
    pcm = np.concatenate([po.codec_forward(st, z[:4]), po.codec_forward(st, z[4:])])
    assert np.array_equal(pcm, g["pcm"])


def test_codec_streaming_and_clone(oracle):
    # a causal streaming decoder: any split of the frames into calls gives the same samples (the histories, tails
    # and cache carry exactly), and a cloned state continues like the original
    import models
    m = models.CodecModel(8)
    z = po.codec_quantize(m.ox, m.codes(np.random.default_rng(1), 11))
    whole = po.codec_forward(po.CodecState(m.ox), z)
    st = po.CodecState(m.ox)
    parts = [po.codec_forward(st, z[a:b]) for a, b in ((0, 1), (1, 4), (4, 5), (5, 11))]
    assert np.array_equal(np.concatenate(parts), whole)
    st = po.CodecState(m.ox)
    po.codec_forward(st, z[:6])
    cl = st.clone()
    assert np.array_equal(po.codec_forward(st, z[6:]), po.codec_forward(cl, z[6:]))
    assert np.array_equal(po.codec_forward(po.CodecState(m.ox), z[:6]), whole[:6 * m.spf])
    assert np.max(np.abs(whole)) < 1.0  # the model stays inside the clamp, so the comparisons see the signal


def test_codec_window_and_scale_pins(oracle):
    # the transformer's sliding window and layer scales against float64 brute force on one layer: window 3 at
    # positions 0..5 (rows see at most 3 keys), scales applied to the o and down outputs before the residual add
    import models
    rng = np.random.default_rng(4)
    H, heads, hd, I, W = 16, 2, 8, 24, 3
    mk = lambda r, c: (rng.standard_normal((r, c)) / np.sqrt(c)).astype(np.float32)
    mats = {n: mk(*s) for n, s in (("q", (16, H)), ("k", (16, H)), ("v", (16, H)), ("o", (H, 16)), ("gate", (I, H)),
                                   ("up", (I, H)), ("down", (H, I)))}
    ln1, ln2, fn = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32), np.ones(H, np.float32), np.ones(H, np.float32)
    sa, sm = (0.5 + 0.1 * rng.standard_normal(H)).astype(np.float32), (0.5 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    om = {n: po.Mat(po.F32, a, a.shape[0], a.shape[1]) for n, a in mats.items()}
    lay = (po.VoLayer * 1)()
    for n in mats:
        setattr(lay[0], n, om[n].c)
    lay[0].ln1, lay[0].ln2, lay[0].attn_scale, lay[0].mlp_scale = ln1.ctypes.data, ln2.ctypes.data, sa.ctypes.data, sm.ctypes.data
    inv = np.empty(hd // 2, np.float32)
    po.lib().vo_rope_inv_freq(hd, 1e4, inv.ctypes.data)
    xf = po.VoXfmr(1, lay, fn.ctypes.data, H, heads, heads, hd, I, 1e-5, inv.ctypes.data, W)
    x = rng.standard_normal((6, H)).astype(np.float32)
    k = np.zeros((1, 8, 16), np.float32)
    v = np.zeros_like(k)
    kv = po.VoKV(k.ctypes.data, v.ctypes.data, 8, 0, 0, 0)
    h = np.empty_like(x)
    assert po.lib().vo_transformer_layers(po.C.byref(xf), po.C.byref(kv), x.ctypes.data, 6, 0, 1, h.ctypes.data) == 0
    X = x.astype(np.float64)
    rms = lambda a, w: a / np.sqrt((a * a).mean(-1, keepdims=True) + 1e-5) * w
    xn = rms(X, ln1)
    q, kk, vv = xn @ mats["q"].T, xn @ mats["k"].T, xn @ mats["v"].T
    def rope(a, pos):
        a = a.reshape(heads, hd).copy()
        ang = np.float32(inv * np.float32(pos)).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = a[:, :hd // 2].copy(), a[:, hd // 2:].copy()  # rotate-half pairs (i, i + hd / 2)
        a[:, :hd // 2], a[:, hd // 2:] = x0 * c - x1 * s, x1 * c + x0 * s
        return a
    Qr = np.stack([rope(q[i], i) for i in range(6)])
    Kr = np.stack([rope(kk[i], i) for i in range(6)])
    ao = np.zeros((6, heads, hd))
    for i in range(6):
        f = max(0, i - W + 1)
        for hh in range(heads):
            sc = Kr[f:i + 1, hh] @ Qr[i, hh] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            ao[i, hh] = (p / p.sum()) @ vv[f:i + 1].reshape(-1, heads, hd)[:, hh]
    X = X + (ao.reshape(6, -1) @ mats["o"].T) * sa
    xn = rms(X, ln2)
    g_ = xn @ mats["gate"].T
    X = X + (((g_ / (1 + np.exp(-g_))) * (xn @ mats["up"].T)) @ mats["down"].T) * sm
    assert np.max(np.abs(h - X)) < 1e-4
