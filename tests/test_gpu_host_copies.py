"""Every copy between host and device memory the library makes goes through one pair of helpers, which with
VOXHIP_CHECK_HOST=1 check (hipPointerGetAttributes) that the host side is not device memory and the device side is.
This runs the paths of the two legs that once ended in a host segmentation fault at a device address under
rocprofv3 (the configs[2] talker steps through voxhip_decode_dev / voxhip_decode_steps_dev, and the CosyVoice2-shaped
LM through voxhip_lm_generate), plus the host-pointer entry points, with the check on: no copy may hand the runtime a
device address as host memory. A deliberate violation through voxhip_memcpy_h2d shows that the check is live (it
fails the call before any copy is issued)."""
import os

import numpy as np
import pytest

from vox_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def checked(hip):
    os.environ["VOXHIP_CHECK_HOST"] = "1"
    hip.init("hip:0")  # re-reads the switch
    try:
        yield hip
    finally:
        os.environ.pop("VOXHIP_CHECK_HOST", None)
        hip.init("hip:0")


def _small(cfg, **kw):
    c = dict(cfg, layers=2, kv_len=64)
    c.update(kw)
    return c


def test_check_is_live(checked):
    hip = checked
    a, b = hip.DevBuf(256), hip.DevBuf(256)
    try:
        a.upload(np.arange(64, dtype=np.float32))
        with pytest.raises(hip.VoxHipError, match="host-to-device copy: the source is device memory"):
            hip._check(hip.lib().voxhip_memcpy_h2d(b.ptr, a.ptr, 256), "memcpy_h2d")
        with pytest.raises(hip.VoxHipError, match="device-to-host copy: the destination is device memory"):
            hip._check(hip.lib().voxhip_memcpy_d2h(b.ptr, a.ptr, 256), "memcpy_d2h")
        assert np.array_equal(a.download(64, np.float32), np.arange(64, dtype=np.float32))
    finally:
        a.free()
        b.free()


def test_talker_steps_copy_host_memory_only(checked):
    hip = checked
    dec = synth.Decoder(_small(synth.TALKER_1_7B_Q4, hidden=512, inter=1536, head_rows=512), seed=3)
    c = dec.cfg
    pos, H, B = c["kv_len"], c["hidden"], 8
    seqs = [dec.seq] + [dec.extra_seq(0xC0DE + 17 * b) for b in range(1, B)]
    x = np.random.default_rng(2).standard_normal((B, H)).astype(np.float32)
    dx, dtok = hip.DevBuf(x.nbytes), hip.DevBuf(4 * B)
    try:
        dx.upload(x)
        cfgs = [hip.sample_cfg(0.9, 1.0, 50, seed=0, frame=b) for b in range(B)]
        for step in range(3):  # the first call captures the graph, the later ones replay it at new positions
            hip.decode_dev(dec.xfmr, dec.seq, pos + step, dx, 1, None, dec.head, None, cfgs[0], dtok)
            hip.decode_steps_dev(dec.xfmr, seqs, [pos + 3 + step] * B, dx, None, dec.head, None, cfgs, dtok)
        hip.sync()
        toks = dtok.download(B, np.int32)
        assert np.all((toks >= 0) & (toks < c["head_rows"]))
        # the host-pointer paths: a prefill pass, a matmul, the sampler
        out, _ = hip.forward(dec.xfmr, hip.seq_create(dec.xfmr, 128), 0, x[:5], H)
        assert np.all(np.isfinite(out))
        y = hip.matmul(dec.head, x[:3])
        assert y.shape == (3, c["head_rows"])
        assert 0 <= hip.sample_logits(y[0], hip.sample_cfg(0.9, 1.0, 50, seed=0)) < c["head_rows"]
    finally:
        dx.free()
        dtok.free()


def test_lm_generate_copies_host_memory_only(checked):
    hip = checked
    c = _small(synth.COSY_LM_0_5B, kv_len=0, head_rows=300, speech_tokens=290)
    dec = synth.Decoder(c, seed=5, capacity=64 + 40)
    emb = hip.mat_synthetic(hip.F32, c["head_rows"], c["hidden"], 0, 0xE4B, 0.0, 0.02)
    try:
        x = np.random.default_rng(5).standard_normal((20, c["hidden"])).astype(np.float32)
        cfg = hip.lm_cfg(speech_tokens=c["speech_tokens"], min_len=12, max_len=12, seed=1234)
        toks, logp = hip.lm_generate(dec.xfmr, dec.seq, x, dec.head, emb, cfg, want_logp=True)
        assert toks.size == 12 and np.all(np.isfinite(logp))
    finally:
        hip.mat_free(emb)
