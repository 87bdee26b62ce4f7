"""Long contexts through the decode paths: keys far past the attention's short first batch (512 keys), split
over the 8 interleaved key ranges, one row and 8 sessions at different positions in one step. The reference
(transformer_forward, kernels.cpp:797-826) attends over keys 0 .. pos of the row's cache; the oracle runs it on the
same stored weights and f16 cache. Bar: 1e-3 (`vox verify` metric), the per-layer check teacher-forced; the
B-session rows also agree with their own batch-1 steps to 1e-3 (other GEMV tiles, so another summation order)."""
import numpy as np
import pytest

from conftest import rel_err
from talker import to_oracle
from vox_amd import synth

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, hidden=512, heads=8, kv_heads=4, head_dim=128, inter=1536, theta=1e6, eps=1e-6, kv_len=8192,
           head_rows=512, wtype=synth.vh.Q8, head_type=synth.vh.Q8)


@pytest.fixture(scope="module")
def dec(hip):
    return synth.Decoder(CFG, seed=11, capacity=CFG["kv_len"] + 16)


def test_one_row_at_8191(hip, oracle, dec):
    c = dec.cfg
    pos = c["kv_len"] - 1
    X, (kv,), _ = to_oracle(oracle, hip, dec, kv_len=pos, cap=pos + 8)
    rng = np.random.default_rng(3)
    h = rng.standard_normal((1, c["hidden"])).astype(np.float32)
    for li in range(c["layers"]):  # teacher-forced: both sides append this step's K/V of the layer at pos
        hg = hip.forward_layers(dec.xfmr, dec.seq, pos, h, li, 1)
        hr = oracle.transformer_layers(X, kv, h, li, 1)
        assert rel_err(hg, hr) < 1e-3, (li, rel_err(hg, hr))
        h = hr
    # the fused one-row step (speculative batch + 15 more key batches per split) and its graph replay at pos + 1
    X, (kv,), _ = to_oracle(oracle, hip, dec, kv_len=pos, cap=pos + 8)
    for step in range(2):
        x = rng.standard_normal((1, c["hidden"])).astype(np.float32)
        out, _ = hip.forward(dec.xfmr, dec.seq, pos + step, x, c["hidden"])
        ref = oracle.transformer_forward(X, kv, x)
        assert rel_err(out, ref) < 1e-3, (step, rel_err(out, ref))


def test_sessions_at_long_positions(hip, oracle, dec):
    c = dec.cfg
    H, B = c["hidden"], 8
    positions = [8191, 5000, 3071, 2047, 513, 100, 1, 0]
    seqs = [dec.extra_seq(0xD00D + 31 * b) for b in range(B)]
    rng = np.random.default_rng(4)
    x = rng.standard_normal((B, H)).astype(np.float32)
    # oracle copies of each session's cache before the step
    kvs = [to_oracle(oracle, hip, dec, seqs=[s], kv_len=max(p, 1), cap=p + 8)[1][0] for s, p in zip(seqs, positions)]
    X = to_oracle(oracle, hip, dec, kv_len=1, cap=8)[0]
    for kv, p in zip(kvs, positions):
        kv.c.len = p
    dx, dout = hip.DevBuf(x.nbytes), hip.DevBuf(x.nbytes)
    try:
        dx.upload(x)
        hip.decode_steps_dev(dec.xfmr, seqs, positions, dx, dout, -1, None, None, None)
        hip.sync()
        outs = dout.download((B, H), np.float32)
    finally:
        dx.free()
        dout.free()
    for b in range(B):
        ref = oracle.transformer_forward(X, kvs[b], x[b:b + 1])
        assert rel_err(outs[b], ref) < 1e-3, (b, positions[b], rel_err(outs[b], ref))
    # each row again alone at the same position (its key at that position is rewritten from the same input)
    for b in (0, 2, 6):
        o1, _ = hip.forward(dec.xfmr, seqs[b], positions[b], x[b:b + 1], H)
        assert rel_err(o1, outs[b]) < 1e-3, (b, rel_err(o1, outs[b]))


def test_prefill_rows_after_long_context(hip, oracle, dec):
    # 300 rows at positions 7800 .. 8099 in one pass: the prefill attention's key runs span ~8K keys per query tile
    c = dec.cfg
    oracle.lib().vo_set_threads(8)
    pos0, m = 7800, 300
    s = dec.extra_seq(0xBEEF)
    X, (kv,), _ = to_oracle(oracle, hip, dec, seqs=[s], kv_len=pos0, cap=pos0 + m + 8)
    x = np.random.default_rng(6).standard_normal((m, c["hidden"])).astype(np.float32)
    out, _ = hip.forward(dec.xfmr, s, pos0, x, c["hidden"])
    ref = oracle.transformer_forward(X, kv, x)
    assert rel_err(out, ref) < 1e-3, rel_err(out, ref)


def test_one_row_steps_across_512(hip, oracle, dec):
    # device-resident one-row steps at positions 508 .. 517: below 513 the attention's first batch is 512 keys, past
    # it a full batch; the captured step is keyed by that, so the graph from before the crossing is not replayed after
    c = dec.cfg
    H = c["hidden"]
    s = dec.extra_seq(0xFACE)
    X, (kv,), _ = to_oracle(oracle, hip, dec, seqs=[s], kv_len=508, cap=528)
    rng = np.random.default_rng(8)
    dx, dout = hip.DevBuf(H * 4), hip.DevBuf(H * 4)
    try:
        for pos in range(508, 518):
            x = rng.standard_normal((1, H)).astype(np.float32)
            dx.upload(x)
            hip.decode_dev(dec.xfmr, s, pos, dx, 1, dout)
            hip.sync()
            out = dout.download(H, np.float32)
            ref = oracle.transformer_forward(X, kv, x)
            assert rel_err(out, ref) < 1e-3, (pos, rel_err(out, ref))
    finally:
        dx.free()
        dout.free()
