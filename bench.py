#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X: the Qwen3-TTS-0.6B-shaped q8 talker decode step (BASELINE.json
configs[1]): 28 layers, hidden 1024, 16 q / 8 kv heads x 128, SwiGLU FFN 3072, RoPE theta 1e6, q8 weights
~N(0, 0.02) generated on the device, a 512-token f16 KV cache ~N(0, 1), a 3072-entry q8 head and Philox top-k 50
sampling at T 0.9, batch 1.

A step is one device-resident decode at position 512 (x already in HBM -> 28 layers -> final norm -> head ->
sampled token in HBM), replayed as one captured HIP graph. Each step rewrites the same KV slot, so every step
is the same work. Prints one JSON line:
  value      tokens per second (one GPU, the whole job);
  roofline   the dominant kernel, k_gemv_int (the step's q8 GEMVs, 113 of its 142 launches): algorithmic bytes per
             launch / average launch duration, summed over those launches, with durations stamped by HIP events at
             each kernel's start and end (hipExtLaunchKernel) on its stream; traffic from profiles/traffic.json;
  cpu_baseline  the reference's own CPU step (oracle/_ref, compiled from its sources) or the C restatement,
             timed on this host for a bounded number of steps.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "talker decode tok/s (0.6B q8, batch 1); GEMV HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 matrix peak
POS = 512


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(vh, dec, seconds, x):
    """Times the reference CPU decode step (transformer_forward + head matmul + sample_logits) on this host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    c = dec.cfg
    threads = max(1, min(16, os.cpu_count() or 1))
    layers = []
    for li in range(c["layers"]):
        d = {}
        for n in ("q", "k", "v", "o", "gate", "up", "down"):
            h = dec.mats[li][n]
            rows, cols = vh.mat_shape(h)
            data, scale, _ = vh.mat_download(h, c["wtype"])
            d[n] = po.Mat(c["wtype"], data, rows, cols, scale)
        d.update(dec.layers[li])
        layers.append(d)
    X = po.Xfmr(layers, dec.final_norm, c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["inter"], c["eps"], dec.inv_freq)
    kd = c["kv_heads"] * c["head_dim"]
    kv = po.KV(c["layers"], POS + 4, kd, kv_f16=1)
    for li in range(c["layers"]):
        k, v = vh.seq_download(dec.seq, li, POS, kd)
        kv.k[li, :POS], kv.v[li, :POS] = k, v
    kv.c.len = POS
    hd, hs, _ = vh.mat_download(dec.head, c["head_type"])
    head = po.Mat(c["head_type"], hd, c["head_rows"], c["hidden"], hs)
    out = np.empty(c["hidden"], np.float32)
    u = po.uniform(0, 0, 0, 0)
    import ctypes
    tok = ctypes.c_int32()
    R = po.ref()
    times = []
    if R is not None:
        kind = "reference"
        R.ref_set_threads(threads)
        sess = R.ref_session_new(ctypes.byref(X.c), ctypes.byref(kv.c), ctypes.byref(head.c))
        if not sess:
            raise RuntimeError("reference session setup failed")
        R.ref_session_step(sess, x.ctypes.data, out.ctypes.data, 0.9, 50, u, ctypes.byref(tok))  # warm
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end and len(times) < 2000:
            t0 = time.perf_counter()
            R.ref_session_step(sess, x.ctypes.data, out.ctypes.data, 0.9, 50, u, ctypes.byref(tok))
            times.append(time.perf_counter() - t0)
        R.ref_session_free(sess)
    else:
        kind = "port"
        po.lib().vo_set_threads(threads)
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end and len(times) < 2000:
            t0 = time.perf_counter()
            kv.c.len = POS
            o = po.transformer_forward(X, kv, x[None])
            lg = po.matmul(head, o[None])[0]
            po.sample_logits(lg, 0.9, 1.0, 50, 1.0, None, u)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    model, simd = host_cpu()
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads, "kind": kind, "cpu_model": model,
            "simd": simd, "nproc": os.cpu_count(),
            "sample": f"{len(times)} decode steps at position {POS} (28-layer q8 talker + 3072-row q8 head + top-k 50 "
                      f"sampling, {threads} threads, median of the steps, {sum(times):.1f} s of CPU work)"}


def classes_of(vh, r):
    """The per-class table of a bench_decode / bench_decode_steps result: launches per step, event-stamped us per
    launch, algorithmic bytes per launch and GB/s, for every class the step launches."""
    out = {}
    for i, name in enumerate(vh.KERNEL_CLASSES):
        n = r.class_launches[i]
        if not n:
            continue
        ms, b = r.class_ms[i], r.class_bytes[i]
        out[name] = {"launches_per_step": n, "us_per_launch": round(ms * 1000, 3), "bytes_per_launch": int(b),
                     "GBps": round(b / (ms * 1e-3) / 1e9, 1) if ms > 0 else None}
    return out


def bench_cfg1(vh):
    """BASELINE configs[0] on the device: one q8 FFN block (H 1024, FFN 3072), rotating over 40 weight sets
    (425 MB, above the 256 MB Infinity Cache)."""
    us = vh.bench_ffn_q8(1024, 3072, 40, 3, 20)
    nbytes = 10_616_832  # gate|up + down q8 weights and scales
    return {"workload": "q8 FFN block 1024->3072->1024 (BASELINE configs[0]), 40 rotating weight sets",
            "us_per_block": round(us, 3), "bytes_per_block": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_cfg3(vh, synth, steps, warmup):
    """the 1.7B-shaped q4 talker (f16 block scales, q8 head) at KV length 1024, batch 1 and
    8 independent sessions, device-resident graph replays."""
    dec = synth.Decoder(synth.TALKER_1_7B_Q4, seed=0)
    c = dec.cfg
    pos, H = c["kv_len"], c["hidden"]
    rng = np.random.default_rng(1)
    out = {"workload": "qwen3-tts-1.7b-talker-decode-q4 f16 scales (BASELINE configs[2]), KV 1024"}
    for B in (1, 8):
        seqs = [dec.seq] + [dec.extra_seq(0xC0DE + 17 * b) for b in range(1, B)]
        x = rng.standard_normal((B, H)).astype(np.float32)
        dx, dtok = vh.DevBuf(x.nbytes), vh.DevBuf(4 * B)
        dx.upload(x)
        cfgs = [vh.sample_cfg(0.9, 1.0, 50, seed=0, frame=b) for b in range(B)]

        def step():
            if B == 1:
                vh.decode_dev(dec.xfmr, dec.seq, pos, dx, 1, None, dec.head, None, cfgs[0], dtok)
            else:
                vh.decode_steps_dev(dec.xfmr, seqs, [pos] * B, dx, None, dec.head, None, cfgs, dtok)
        for _ in range(warmup):
            step()
        vh.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        vh.sync()
        ms = (time.perf_counter() - t0) * 1000.0 / steps
        kv = c["layers"] * 2 * (pos + 1) * c["kv_heads"] * c["head_dim"] * 2 * B
        nbytes = dec.weight_bytes() + kv
        out[f"b{B}"] = {"tok_s": round(B * 1000.0 / ms, 2), "ms_per_step": round(ms, 5), "bytes_per_step": nbytes,
                        "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        # the same step's kernels launched one by one, event-stamped (the per-class evidence of this leg)
        if B == 1:
            r = vh.bench_decode(dec.xfmr, dec.seq, pos, dx, dec.head, cfgs[0], dtok, 3, 20)
        else:
            r = vh.bench_decode_steps(dec.xfmr, seqs, [pos] * B, dx, dec.head, cfgs, dtok, 3, 20)
        out[f"b{B}"]["kernels"] = classes_of(vh, r)
        out[f"b{B}"]["kernel_us_per_step"] = round(r.kernel_ms_per_step * 1000, 2)
        out[f"b{B}"]["kernels_per_step"] = r.kernels_per_step
        dx.free()
        dtok.free()
    return out


def bench_cfg4(vh, synth, reps=3):
    """one F5-TTS DiT step (22 blocks, dim 1024, 16 x 64 heads, N = 1000 frames, f16 weights) on
    the device, B = 2 (classifier-free guidance, the reference default) and B = 1. The f16 linears run on the f16
    matrix cores with the f32 activations split in two f16 halves (two MFMAs per product), the attention tiles on
    the f16 matrix cores with both operands split (three MFMAs per product), the grouped position convolutions on
    f32 MFMA. frac_f16_mfma is against the dense f16 peak, counting each product once (the split costs two or
    three MFMAs per product, so 0.5 of it is the practical ceiling of the linears). Host wall-clock around
    gpu_f5_step (median of reps), x / ts upload and the [B][N][100] download included."""
    dit = synth.DiT(synth.F5_DIT, seed=0)
    c = dit.cfg
    N = c["frames"]
    out = {"workload": "f5-tts DiT step, 22 x 1024, N 1000, f16 weights (BASELINE configs[3])"}
    for B in (2, 1):
        rng = np.random.default_rng(B)
        W = 2 * c["mel"] + c["text"]
        cat0 = rng.standard_normal((B * N, W)).astype(np.float32)
        cat0[:, :c["mel"]] = 0.0
        HH = c["dim_head"] // 2
        inv = np.array([np.float32(1.0 / 10000.0 ** (2 * j / c["dim_head"])) for j in range(HH)], np.float32)
        ang = (np.arange(N, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
        rope = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
        x = rng.standard_normal((N, c["mel"])).astype(np.float32)
        ts = rng.standard_normal(c["dim"]).astype(np.float32)
        vh.f5_begin(dit.f5, B, N, cat0, rope)
        vh.f5_step(dit.f5, x, ts, B, N, c["mel"])
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            y = vh.f5_step(dit.f5, x, ts, B, N, c["mel"])
            times.append((time.perf_counter() - t0) * 1000.0)
        vh.f5_end(dit.f5)
        assert np.isfinite(y).all()
        ms = float(np.median(times))
        fl = dit.flops(B, N)
        tot = sum(fl.values())
        out[f"b{B}"] = {"ms_per_step": round(ms, 3), "gflop": round(tot / 1e9, 1),
                        "gflop_parts": {k: round(v / 1e9, 1) for k, v in fl.items()},
                        "tflops": round(tot / (ms * 1e-3) / 1e12, 2),
                        "frac_f16_mfma": round(tot / (ms * 1e-3) / 1e12 / F16_MFMA_PEAK_TFLOPS, 4)}
    return out


def bench_cfg5(vh, synth, reps=3):
    """the CosyVoice2-0.5B-shaped LM on the device. Prefill: 512 prompt rows (q8 weights on the
    f32-activation GEMM, as matmul's path above 8 rows: int8 values exact in f16, activations split in two f16
    halves on the f16 matrix cores; attention on the matrix cores in 64-row query tiles). Generation: 256 steps of q8 int8 GEMVs, f32 head + bias,
    log-softmax, the RAS sampler with lm_generate's trial loop (top-p 0.8, top-k 25, window 10, tau 0.1, Philox seed
    1234) and the speech-token embedding, all device-resident (min_len = max_len = 256: exactly 256 steps).
    Times are host wall-clock around the entry points (median of reps), prompt upload included."""
    c = synth.COSY_LM_0_5B
    P, S = c["prefill"], c["decode_steps"]
    dec = synth.Decoder(c, seed=0, capacity=P + S + 8)
    emb = vh.mat_synthetic(vh.F32, c["head_rows"], c["hidden"], 0, 0xE4B, 0.0, 0.02)
    x = np.random.default_rng(5).standard_normal((P, c["hidden"])).astype(np.float32)
    pre = vh.lm_cfg(speech_tokens=c["speech_tokens"], min_len=0, max_len=0, seed=1234)
    gen = vh.lm_cfg(speech_tokens=c["speech_tokens"], min_len=S, max_len=S, seed=1234)

    def timed(cfg):
        vh.sync()
        t0 = time.perf_counter()
        toks, _ = vh.lm_generate(dec.xfmr, dec.seq, x, dec.head, emb, cfg)
        return (time.perf_counter() - t0) * 1000.0, toks
    timed(pre)
    timed(gen)
    t_pre = float(np.median([timed(pre)[0] for _ in range(reps)]))
    runs = [timed(gen) for _ in range(reps)]
    t_all = float(np.median([r[0] for r in runs]))
    ntok = int(runs[0][1].size)
    assert all(np.array_equal(r[1], runs[0][1]) for r in runs) and ntok == S
    flops = dec.linear_flops(P) + dec.attention_flops(P)
    dec_ms = t_all - t_pre
    kv_avg = c["layers"] * 2 * (P + (S + 1) / 2) * c["kv_heads"] * c["head_dim"] * 2
    step_bytes = dec.weight_bytes() + kv_avg
    # one generation step's layers and head launched one by one, event-stamped, at the middle of the generation (the
    # RAS sampler and the embedding gather, which lm_generate adds, are not in this pass)
    dx = vh.DevBuf(c["hidden"] * 4)
    dx.upload(x[0])
    r = vh.bench_decode(dec.xfmr, dec.seq, P + S // 2, dx, dec.head, None, None, 3, 20)
    dx.free()
    vh.mat_free(emb)
    return {"workload": "cosyvoice2-0.5b LM q8: prefill 512 + 256 RAS-sampled steps (BASELINE configs[4])",
            "prefill_ms": round(t_pre, 3), "prefill_gflop": round(flops / 1e9, 1),
            "prefill_tflops": round(flops / (t_pre * 1e-3) / 1e12, 2),
            "prefill_frac_f16_mfma": round(flops / (t_pre * 1e-3) / 1e12 / F16_MFMA_PEAK_TFLOPS, 4),
            "decode_ms": round(dec_ms, 3), "decode_tok_s": round(S / (dec_ms * 1e-3), 1),
            "decode_bytes_per_step": int(step_bytes),
            "decode_GBps": round(step_bytes * S / (dec_ms * 1e-3) / 1e9, 1),
            "decode_frac": round(step_bytes * S / (dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "total_ms": round(t_all, 3), "tokens": ntok,
            "decode_kernels": classes_of(vh, r), "decode_kernel_us_per_step": round(r.kernel_ms_per_step * 1000, 2)}


def bench_cfg5_prefill(vh, synth, reps=10):
    """The 512-row prefill of BASELINE configs[4]'s LM alone, through voxhip_xfmr_forward_layers over the 24 layers
    (the same layer passes as lm_generate's prefill: one 512-row pass per layer, its GEMMs on f16 halves of their
    inputs, q8 weights as widened int8 values with the block-scale step). Host wall-clock (median of reps, after
    the pass has been captured as a graph), the 512 x 896 upload and download included; per_layer_us is the slope
    between 24 and 1 layers, which cancels the copies."""
    c = synth.COSY_LM_0_5B
    P = c["prefill"]
    dec = synth.Decoder(c, seed=0, capacity=P + 8)
    x = np.random.default_rng(5).standard_normal((P, c["hidden"])).astype(np.float32)

    def timed(count):
        for _ in range(3):
            vh.forward_layers(dec.xfmr, dec.seq, 0, x, 0, count)
        ts = []
        for _ in range(reps):
            vh.sync()
            t0 = time.perf_counter()
            vh.forward_layers(dec.xfmr, dec.seq, 0, x, 0, count)
            ts.append((time.perf_counter() - t0) * 1000.0)
        return float(np.median(ts))
    t_all, t_one = timed(c["layers"]), timed(1)
    flops = dec.linear_flops(P) + dec.attention_flops(P)
    return {"workload": "cosyvoice2-0.5b LM q8: the 512-row prefill's 24 layers (BASELINE configs[4])",
            "ms": round(t_all, 3), "per_layer_us": round((t_all - t_one) / (c["layers"] - 1) * 1000.0, 1),
            "gflop": round(flops / 1e9, 1), "tflops": round(flops / (t_all * 1e-3) / 1e12, 2)}


def bench_vocos(vh, synth, reps=5):
    """F5-TTS's Vocos backbone + head (gpu_f5_vocos; the iSTFT stays on the host as in the reference) on 938 mel frames
    (10 s of 24 kHz audio), f16 linears. Host wall-clock (median), the mel upload and the [T][1026] download included."""
    dit = synth.DiT(dict(synth.F5_DIT, depth=1), seed=0, vocos=synth.F5_VOCOS)
    T = synth.F5_VOCOS["frames"]
    mel = np.random.default_rng(3).standard_normal((T, synth.F5_DIT["mel"])).astype(np.float32)
    vh.f5_vocos(dit.f5, mel)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        out = vh.f5_vocos(dit.f5, mel)
        times.append((time.perf_counter() - t0) * 1000.0)
    assert np.isfinite(out).all()
    ms = float(np.median(times))
    fl = dit.vocos_flops(T)
    return {"workload": "f5-tts vocos backbone + head (gpu_f5_vocos): 938 frames, dim 512, 8 ConvNeXt blocks, f16 linears",
            "ms": round(ms, 3), "gflop": round(fl / 1e9, 2), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
            "audio_s_per_s": round(T * 256 / 24000 / (ms * 1e-3), 1)}


def bench_cosy(vh, synth, reps=5):
    """CosyVoice2's flow estimator (gpu_cosy_step; cosyvoice.cpp:822-863): one Euler step = the conditional and the
    unconditional pass over 512 mel frames (the 256 speech tokens of configs[4]), f16 linears, f32 causal
    convolutions. Host wall-clock per step (median), the x / time-bias upload and the [2][512][80] download included."""
    c = synth.COSY_FLOW
    flow = synth.CosyFlow(c, seed=0)
    T, M, C = c["frames"], c["M"], c["C"]
    rng = np.random.default_rng(4)
    in0 = np.zeros((2 * T, 4 * M), np.float32)
    in0[:T, M:] = rng.standard_normal((T, 3 * M)).astype(np.float32)
    vh.cosy_begin(flow.est, T, in0)
    x = rng.standard_normal((T, M)).astype(np.float32)
    tb = (rng.standard_normal((2 + c["n_mid"], C)) * 0.1).astype(np.float32)
    vh.cosy_step(flow.est, x, tb, T, M)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        out = vh.cosy_step(flow.est, x, tb, T, M)
        times.append((time.perf_counter() - t0) * 1000.0)
    vh.cosy_end(flow.est)  # the estimator keeps its matrices (mat_free refuses a matrix an estimator uses)
    assert np.isfinite(out).all()
    ms = float(np.median(times))
    fl = flow.flops(T)
    return {"workload": "cosyvoice2 flow estimator step (gpu_cosy_step): 2 x 512 frames, 256 ch, 14 causal resnets, "
                        "56 transformer blocks (8 x 64 heads, FFN 1024), f16 linears",
            "ms_per_step": round(ms, 3), "gflop": round(fl / 1e9, 2), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
            "flow_ms_10_steps": round(10 * ms, 2)}


def bench_codec(vh, synth, reps=10):
    """Qwen3-TTS's codec decoder (gpu_codec_forward; qwen3.cpp:390-480 on the CPU) at its full widths with synthetic f32
    weights: chunks of 16 frames (1.28 s of 24 kHz audio per call) and single frames (streaming). Host wall-clock per
    call (median), the z upload and the PCM download included; the ring wraps during the run."""
    c = synth.QWEN3_CODEC
    dec = synth.CodecDec(c, seed=0)
    rng = np.random.default_rng(9)
    st = vh.codec_state_new(dec.codec)
    out = {}
    for F in (16, 1):
        z = (rng.standard_normal((F, c["codebook_dim"])) * 0.5).astype(np.float32)
        for _ in range(3):
            vh.codec_forward(dec.codec, st, z)
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            pcm = vh.codec_forward(dec.codec, st, z)
            times.append((time.perf_counter() - t0) * 1000.0)
        assert pcm.size == F * dec.spf and np.isfinite(pcm).all()
        ms = float(np.median(times))
        fl = F * dec.flops_per_frame()
        out[f"f{F}"] = {"ms_per_call": round(ms, 3), "gflop": round(fl / 1e9, 2), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                        "audio_s_per_s": round(F * dec.spf / 24000 / (ms * 1e-3), 1)}
    vh.codec_state_free(st)  # the decoder keeps its matrices (mat_free refuses a matrix a decoder uses)
    return {"workload": "qwen3-tts codec decoder (gpu_codec_forward): 8-layer windowed transformer + 2 upsample + 4 "
                        "decoder blocks (1536 ch, 1920 samples per frame), f32 weights", **out}


def bench_pred(vh, synth, frames=20):
    """The code predictor's frame on the device (gpu_pred_frame; the loop engine.cpp:676-683 runs on the CPU in the
    reference when the device does not provide it): 15 passes of the 5-layer q8 predictor (2 rows at positions 0-1,
    then one row per codebook), each with its codebook's q8 head, the sampler (top-k 50, T 0.9, draw (frame, cb))
    and the next code's bf16 embedding gathered on the device, in one graph. Host wall-clock per frame (median),
    the [2][1024] input upload and the codes download included."""
    c = synth.PRED_0_6B
    dec = synth.Decoder(c, seed=0, capacity=32)
    G, V, H = c["groups"], c["vocab"], c["hidden"]
    heads = [vh.mat_synthetic(c["head_type"], V, H, 0, 0x5000 + i, 0.0, 0.02) for i in range(G - 1)]
    embs = [vh.mat_synthetic(c["emb_type"], V, H, 0, 0x6000 + i, 0.0, 1.0) for i in range(G - 2)]
    rng = np.random.default_rng(11)
    times, codes = [], None
    for f in range(frames + 3):
        in2 = rng.standard_normal((2, H)).astype(np.float32)
        cfg = vh.sample_cfg(0.9, 1.0, 50, seed=1, frame=f)
        t0 = time.perf_counter()
        codes = vh.pred_frame(dec.xfmr, dec.seq, in2, -1, heads, embs, cfg)
        if f >= 3:
            times.append((time.perf_counter() - t0) * 1000.0)
    ms = float(np.median(times))
    layer_bytes = dec.weight_bytes()  # the 5 layers (no head in this config)
    head_bytes = V * H + V * (H // 32) * 4
    kd = c["kv_heads"] * c["head_dim"]
    kv = sum(c["layers"] * 2 * (p + 1) * kd * 2 for p in range(1, G))  # keys/values read per pass (f16)
    frame_bytes = (G - 1) * (layer_bytes + head_bytes) + (G - 2) * H * 2 + kv
    for h in heads + embs:
        vh.mat_free(h)
    assert codes is not None and codes.shape == (G,)
    return {"workload": "qwen3-tts-0.6b code-predictor frame (gpu_pred_frame): 15 passes x 5 q8 layers + q8 head "
                        "2048 + sampler, bf16 code embeddings",
            "ms_per_frame": round(ms, 3), "bytes_per_frame": int(frame_bytes),
            "GBps": round(frame_bytes / (ms * 1e-3) / 1e9, 1), "frac": round(frame_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "passes_per_s": round((G - 1) / (ms * 1e-3), 1)}


def load_traffic(kernel_classes, launches):
    """Calibrated HBM bytes (FETCH_SIZE + WRITE_SIZE) per launch, averaged over the launches of kernel_classes in one
    step, from profiles/traffic.json (the counter passes of the same benchmark); None when a class is missing."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        t = json.load(open(p))
    except (OSError, ValueError):
        return None
    if any(k not in t for k in kernel_classes):
        return None
    n = sum(launches[k] for k in kernel_classes)
    return int(round(sum(t[k] * launches[k] for k in kernel_classes) / n)) if n else None


def write_classes(path, classes, gemv, gemv_bytes, gemv_us, achieved, ms_per_step, step_bytes, r):
    """The per-class pass behind `roofline` as markdown: each class's launches per step, average event-stamped
    duration, algorithmic bytes per launch and GB/s, then the GEMV sums that `roofline.achieved` divides."""
    rows = ["| class | launches per step | us per launch | algorithmic bytes per launch | GB/s |", "|---|---|---|---|---|"]
    for name, c in classes.items():
        rows.append(f"| {name} | {c['launches_per_step']} | {c['us_per_launch']:.3f} | {c['bytes_per_launch']:,} | "
                    f"{c['GBps'] if c['GBps'] is not None else '-'} |")
    timing = "hipExtLaunchKernel start/stop events" if r.kernel_stamped else "stream events around each launch"
    text = "\n".join([
        "# Decode-step kernel classes, event-stamped (`bench.py` per-class pass)",
        "",
        f"Every kernel of one decode step launched on its own stream, timed by {timing}, averaged over the timed",
        f"steps; the same enqueue path as the captured graph. Graph replay: {ms_per_step * 1000:.1f} us per step; the",
        f"kernels summed: {r.kernel_ms_per_step * 1000:.1f} us per step ({r.kernels_per_step} launches).",
        "",
        *rows,
        "",
        f"GEMV classes ({', '.join(gemv)}): {gemv_bytes:,.0f} algorithmic bytes in {gemv_us:.2f} us per step = "
        f"{achieved} GB/s, {achieved / HBM_PEAK_GBS:.4f} of {HBM_PEAK_GBS:.0f} GB/s (`roofline.achieved`, `frac`).",
        f"Whole step: {step_bytes:,.0f} bytes in {ms_per_step * 1000:.1f} us = "
        f"{step_bytes / (ms_per_step * 1e-3) / 1e9:.1f} GB/s.",
        ""])
    with open(path, "w") as f:
        f.write(text)


def host_cpu():
    """CPU model and the SIMD extensions the reference's kernels can use, from /proc/cpuinfo."""
    model, flags = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    simd = [f for f in ("sse4_2", "avx", "avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512_vnni", "avx_vnni") if f in flags]
    return model, simd


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-other", action="store_true",
                    help="skip the configs[0] / [2] / [3] / [4] and code-predictor measurements")
    ap.add_argument("--only", choices=["configs[0]", "configs[2]", "configs[3]", "configs[4]", "cfg5_prefill", "pred_frame",
                                       "f5_vocos", "cosy_flow", "codec"],
                    help="run one of the other BASELINE configurations (or the code-predictor frame) alone and print "
                         "its JSON object (for profiling)")
    ap.add_argument("--classes-out", metavar="PATH",
                    help="also write the event-stamped per-class pass (launches, us, algorithmic bytes, GB/s) and the "
                         "roofline figures it gives as a markdown table to PATH")
    ap.add_argument("--no-breakdown", action="store_true",
                    help="skip the event-timed per-kernel pass (for runs under rocprofv3, whose tracer does not survive "
                         "HIP events recorded around graph launches); rocprof then times the graph's kernels itself")
    args = ap.parse_args()
    if args.gpus != 1:
        log("bench.py runs on one GPU only: this build's hot path (the batch-1 talker decode step) lives on a single "
            "MI355X, and no figure at several GPUs is produced.")
        sys.exit(2)
    from vox_amd import synth
    from vox_amd import voxhip as vh

    vh.init("hip:0")
    log("device:", vh.device_name())
    if args.only:
        legs = {"configs[0]": lambda: bench_cfg1(vh), "configs[2]": lambda: bench_cfg3(vh, synth, 100, 10),
                "configs[3]": lambda: bench_cfg4(vh, synth), "configs[4]": lambda: bench_cfg5(vh, synth),
                "pred_frame": lambda: bench_pred(vh, synth), "f5_vocos": lambda: bench_vocos(vh, synth),
                "cfg5_prefill": lambda: bench_cfg5_prefill(vh, synth),
                "cosy_flow": lambda: bench_cosy(vh, synth), "codec": lambda: bench_codec(vh, synth)}
        print(json.dumps({args.only: legs[args.only]()}))
        return
    t0 = time.perf_counter()
    dec = synth.Decoder(synth.TALKER_0_6B, seed=0)
    c = dec.cfg
    log(f"synthetic talker built in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(0)
    x = rng.standard_normal(c["hidden"]).astype(np.float32)
    dx, dtok = vh.DevBuf(x.nbytes), vh.DevBuf(4)
    dx.upload(x)
    cfg = vh.sample_cfg(0.9, 1.0, 50, seed=0, frame=0)

    def step():
        vh.decode_dev(dec.xfmr, dec.seq, POS, dx, 1, None, dec.head, None, cfg, dtok)

    for _ in range(args.warmup):
        step()
    vh.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    vh.sync()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1000.0 / args.steps
    tok = int(dtok.download(1, np.int32)[0])
    log(f"timed {args.steps} steps: {ms_per_step * 1000:.1f} us/step, token {tok}")

    # STREAM copy of 256 MiB (the measured HBM ceiling next to the 8 TB/s spec; also the kernel that calibrates
    # the FETCH_SIZE / WRITE_SIZE counters in profiling runs)
    copy_bytes = 256 << 20
    copy_ms = vh.bench_copy(copy_bytes, 3, 10)
    stream = {"kernel": "k_copy16", "bytes_read": copy_bytes, "bytes_written": copy_bytes,
              "us": round(copy_ms * 1000, 2), "GBps": round(2 * copy_bytes / (copy_ms * 1e-3) / 1e9, 1)}
    log(f"stream copy: {stream}")
    if args.no_breakdown:
        print(json.dumps({"metric": METRIC, "value": round(1000.0 / ms_per_step, 2), "unit": "tok/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
                          "stream": stream, "note": "--no-breakdown: graph replay only"}), flush=True)
        return
    r = vh.bench_decode(dec.xfmr, dec.seq, POS, dx, dec.head, cfg, dtok, max(3, args.warmup // 5), args.steps)
    classes = classes_of(vh, r)
    # the dominant kernel: k_gemv_int, the int8 GEMV that makes 113 of the step's 142 launches (q|k|v, o, gate|up and
    # down of every layer, and the head); its algorithmic bytes and durations are summed over those launches
    gemv = [k for k in classes if k.endswith("_gemv")]
    gemv_launches = sum(classes[k]["launches_per_step"] for k in gemv)
    gemv_bytes = sum(classes[k]["bytes_per_launch"] * classes[k]["launches_per_step"] for k in gemv)
    gemv_us = sum(classes[k]["us_per_launch"] * classes[k]["launches_per_step"] for k in gemv)
    achieved = round(gemv_bytes / (gemv_us * 1e-6) / 1e9, 1)
    step_bytes = dec.step_bytes(POS)
    log(json.dumps(classes))
    if args.classes_out:
        write_classes(args.classes_out, classes, gemv, gemv_bytes, gemv_us, achieved, ms_per_step, step_bytes, r)

    other = None
    if not args.no_other:
        t0 = time.perf_counter()
        other = {"configs[0]": bench_cfg1(vh), "configs[2]": bench_cfg3(vh, synth, 100, 10),
                 "configs[3]": bench_cfg4(vh, synth), "configs[4]": bench_cfg5(vh, synth),
                 "pred_frame": bench_pred(vh, synth), "f5_vocos": bench_vocos(vh, synth),
                 "cosy_flow": bench_cosy(vh, synth), "codec": bench_codec(vh, synth)}
        log(f"other configs: {json.dumps(other)} ({time.perf_counter() - t0:.1f} s)")

    cpu = None
    if not args.no_cpu:
        t0 = time.perf_counter()
        cpu = cpu_baseline(vh, dec, args.cpu_seconds, x)
        log(f"cpu baseline: {cpu} ({time.perf_counter() - t0:.1f} s incl. setup)")

    line = {
        "metric": METRIC,
        "value": round(1000.0 / ms_per_step, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x int8 -> int32 GEMV dots, f32 activations, f16 KV",
        "data": "synthetic (device-generated Philox N(0,0.02) weights quantized to q8, f16 KV ~N(0,1))",
        "config": {"workload": "qwen3-tts-0.6b-talker-decode-q8 (BASELINE configs[1])", "layers": c["layers"],
                   "hidden": c["hidden"], "heads": c["heads"], "kv_heads": c["kv_heads"], "head_dim": c["head_dim"],
                   "ffn": c["inter"], "kv_len": POS, "head_rows": c["head_rows"], "batch": 1, "top_k": 50,
                   "temperature": 0.9, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "k_gemv_int (the step's q8 GEMVs: q|k|v, o, gate|up, down x 28, head)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(gemv, {k: classes[k]["launches_per_step"] for k in gemv}),
                     "launches_per_step": gemv_launches, "bytes_per_launch": int(gemv_bytes / gemv_launches),
                     "us_per_launch": round(gemv_us / gemv_launches, 3),
                     "source": "per-class pass (bench.py --classes-out), committed as profiles/decode_q8_0p6b_event_classes.md; "
                               "traffic: profiles/decode_q8_0p6b_hbm_traffic.md"},
        "gemv": {"GBps": round(gemv_bytes / (gemv_us * 1e-6) / 1e9, 1), "frac": round(gemv_bytes / (gemv_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                 "bytes_per_step": gemv_bytes, "us_per_step": round(gemv_us, 2)},
        "step": {"bytes": step_bytes, "GBps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                 "frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "kernel_us_per_step": round(r.kernel_ms_per_step * 1000, 2), "graph_us_per_step": round(r.ms_per_step * 1000, 2),
                 "host_launch_us_per_step": round(r.launch_ms_per_step * 1000, 2),
                 "kernels_per_step": r.kernels_per_step},
        "stream": stream,
        "other_configs": other,
        "kernels": classes,
        "kernel_timing": "hipExtLaunchKernel start/stop events" if r.kernel_stamped else "stream events around each launch",
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
