"""BASELINE configs[1] at full size: the Qwen3-TTS-0.6B-shaped q8 talker decode step (28 layers, hidden 1024,
16 q / 8 kv heads x 128, FFN 3072, theta 1e6, KV 512 prior tokens f16 ~N(0,1), 3072-entry head, Philox top-k 50,
T 0.9) on the device, checked against the oracle on the same stored weights and cache.

Bars:
- every layer, teacher-forced (the device layer runs on the oracle's residual stream): within 1e-3 (`vox verify`
  metric, cli/main.cpp:796-803);
- the whole 28-layer step: the reference's own criterion for quantized models (`vox verify --quant`,
  cli/main.cpp:764-790, :826-827): KL(ref || ours) of the logits <= 0.02 and the reference argmax in our top-5.
  A 1e-3 bar end to end is not meaningful for this path: the int8 activation requantization at every GEMV input
  makes the reference's own output move by ~0.5% under 1e-7 relative input noise at this depth;
- the device sampler's token bit-exact with the oracle sampler on the device's logits.
"""
import numpy as np
import pytest

from conftest import rel_err
from talker import kl_top5, to_oracle

pytestmark = pytest.mark.gpu


def test_talker_0_6b_decode_step(hip, oracle):
    from vox_amd import synth
    oracle.lib().vo_set_threads(8)
    dec = synth.Decoder(synth.TALKER_0_6B, seed=0)
    c = dec.cfg
    X, (kv,), head = to_oracle(oracle, hip, dec)
    rng = np.random.default_rng(0)
    pos = c["kv_len"]
    # per layer, teacher-forced, at the full shape (both sides write this step's K/V of the layer at `pos`)
    h = rng.standard_normal((1, c["hidden"])).astype(np.float32)
    worst = 0.0
    for li in range(c["layers"]):
        hg = hip.forward_layers(dec.xfmr, dec.seq, pos, h, li, 1)
        hr = oracle.transformer_layers(X, kv, h, li, 1)
        e = rel_err(hg, hr)
        worst = max(worst, e)
        assert e < 1e-3, (li, e)
        h = hr
    print("worst per-layer rel err", worst)
    for step in range(2):
        x = rng.standard_normal((1, c["hidden"])).astype(np.float32)
        # device-resident step with the device sampler (the benchmark's path)
        dx, dout, dlog, dtok = hip.DevBuf(x.nbytes), hip.DevBuf(x.nbytes), hip.DevBuf(c["head_rows"] * 4), hip.DevBuf(4)
        dx.upload(x)
        cfg = hip.sample_cfg(0.9, 1.0, 50, seed=0, frame=step)
        hip.decode_dev(dec.xfmr, dec.seq, pos + step, dx, 1, dout, dec.head, dlog, cfg, dtok)
        hip.sync()
        out = dout.download(c["hidden"], np.float32)
        logits = dlog.download(c["head_rows"], np.float32)
        tok = int(dtok.download(1, np.int32)[0])
        for b in (dx, dout, dlog, dtok):
            b.free()
        ref = oracle.transformer_forward(X, kv, x)
        ref_logits = oracle.matmul(head, ref[None])[0]
        kl, top5 = kl_top5(logits, ref_logits)
        print(f"step {step}: hidden rel err {rel_err(out, ref):.3e}, logits KL {kl:.2e}, ref argmax in top-5 {top5}")
        assert kl <= 0.02 and top5
        # the head itself on the device's own normed state: 1e-3 (teacher-forced)
        assert rel_err(logits, oracle.matmul(head, out[None])[0]) < 1e-3
        u = oracle.uniform(0, step, 0, 0)
        assert tok == oracle.sample_logits(logits, 0.9, 1.0, 50, 1.0, None, u)
