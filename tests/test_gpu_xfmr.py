"""Transformer parity: the device decode/prefill path against the oracle's transformer_forward.

The oracle runs with an f16 KV cache model (kv_f16 = 1: appended keys/values rounded to f16, as the device
stores them), so differences come only from float summation order and libm ulps; the bar is the north star's
1e-3 for f32 activations with the `vox verify` metric. Against the reference's own f32 cache (kv_f16 = 0) the
bar is the f16 class, 1e-2.
"""
import numpy as np
import pytest

from conftest import rel_err
from models import Model

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4
TOL = 1e-3


def build(hip, mdl):
    x = hip.xfmr_create(mdl.hx, "t")
    head = hip.upload(mdl.head[1]) if mdl.head else -1
    return x, head


def oracle_head(oracle, mdl, out_last):
    """The head on a given normed state. Tests pass the device's own state (teacher forcing): the head's int8
    activation quantization turns ulp-level input differences into whole-quantum steps, so comparing it on the
    oracle's state would test the cascade, not the head."""
    return oracle.matmul(mdl.head[0], np.asarray(out_last, np.float32)[None])[0]


@pytest.mark.parametrize("wt", [Q8, Q4, BF16, F16, F32])
def test_decode_steps(hip, oracle, wt):
    mdl = Model(100 + wt, 2, 256, 4, 2, 128, 512, wtype=wt, head_rows=300)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 64)
    kv = mdl.oracle_kv(64, kv_f16=1)
    kv32 = mdl.oracle_kv(64, kv_f16=0)
    rng = np.random.default_rng(wt)
    for step in range(6):
        x = rng.standard_normal((1, 256)).astype(np.float32)
        out, logits = hip.forward(xf, seq, step, x, 256, head=head)
        ref = oracle.transformer_forward(mdl.ox, kv, x)
        ref32 = oracle.transformer_forward(mdl.ox, kv32, x)
        assert rel_err(out, ref) < TOL, (step, rel_err(out, ref))
        assert rel_err(out, ref32) < 1e-2
        assert rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
    k, v = hip.seq_download(seq, 1, 6, 256)
    assert np.array_equal(k, kv.k[1, :6]) or rel_err(k, kv.k[1, :6]) < 2e-3


@pytest.mark.parametrize("m", [3, 8, 12])
def test_prefill_then_decode(hip, oracle, m):
    # m <= 8 keeps int8 activations; m > 8 switches q8 to f32 activations (kernels.cpp:660-679)
    mdl = Model(200 + m, 2, 256, 4, 2, 128, 512, wtype=Q8, head_rows=64)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 64)
    kv = mdl.oracle_kv(64, kv_f16=1)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, 256)).astype(np.float32)
    out, logits = hip.forward(xf, seq, 0, x, 256, head=head)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    assert rel_err(out, ref) < TOL
    assert rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
    for step in range(3):
        x = rng.standard_normal((1, 256)).astype(np.float32)
        out, _ = hip.forward(xf, seq, m + step, x, 256, head=head)
        assert rel_err(out, oracle.transformer_forward(mdl.ox, kv, x)) < TOL


@pytest.mark.parametrize("wt,m", [(F16, 70), (BF16, 130), (F32, 37), (Q8, 520)])
def test_prefill_gemm(hip, oracle, wt, m):
    # f32-activation prefill: the matrices run on the MFMA GEMM with the RMSNorm / attention-merge prologues as
    # their own kernels; 520 rows take two passes (512 + 8). Biased q/k/v.
    mdl = Model(500 + m, 2, 256, 4, 2, 128, 512, wtype=wt, bias=True, head_rows=96)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 1024)
    kv = mdl.oracle_kv(1024, kv_f16=1)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, 256)).astype(np.float32)
    out, logits = hip.forward(xf, seq, 0, x, 256, head=head)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    assert rel_err(out, ref) < TOL, rel_err(out, ref)
    assert rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
    for step in range(2):
        x = rng.standard_normal((1, 256)).astype(np.float32)
        out, _ = hip.forward(xf, seq, m + step, x, 256, head=head)
        assert rel_err(out, oracle.transformer_forward(mdl.ox, kv, x)) < TOL


@pytest.mark.parametrize("qkn", [False, True])
def test_gqa7_bias_hd64(hip, oracle, qkn):
    # CosyVoice2-shaped attention: 7 query heads per kv head, head_dim 64, q/k/v biases, no q/k norm; and the same
    # with q/k norms (the prefill's q/k pass sums each head's squares over its 32 lanes of a wave)
    mdl = Model(300 + qkn, 2, 128, 7, 1, 64, 256, wtype=Q8, qk_norm=qkn, bias=True, head_rows=100, head_type=F32)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 32)
    kv = mdl.oracle_kv(32, 1)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    out, logits = hip.forward(xf, seq, 0, x, 128, head=head)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    assert rel_err(out, ref) < TOL and rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
    for step in range(4):
        x = rng.standard_normal((1, 128)).astype(np.float32)
        out, logits = hip.forward(xf, seq, 5 + step, x, 128, head=head)
        ref = oracle.transformer_forward(mdl.ox, kv, x)
        assert rel_err(out, ref) < TOL and rel_err(logits, oracle_head(oracle, mdl, out)) < TOL


def test_long_context_splits(hip, oracle):
    # 700 keys: the split-K attention uses many splits; one kv head per 2 query heads
    mdl = Model(400, 1, 256, 4, 2, 128, 256, wtype=Q8)
    xf, _ = build(hip, mdl)
    seq = hip.seq_create(xf, 1024)
    kv = mdl.oracle_kv(1024, 1)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((699, 256)).astype(np.float32)
    out, _ = hip.forward(xf, seq, 0, x, 256)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    assert rel_err(out, ref) < TOL
    x = rng.standard_normal((1, 256)).astype(np.float32)
    out, _ = hip.forward(xf, seq, 699, x, 256)
    assert rel_err(out, oracle.transformer_forward(mdl.ox, kv, x)) < TOL


def test_forward_hidden_and_in_proj(hip, oracle):
    mdl = Model(500, 2, 128, 4, 2, 64, 256, wtype=Q8)
    xf, _ = build(hip, mdl)
    rng = np.random.default_rng(7)
    # hidden states of all rows, no final norm (gpu_xfmr_forward_hidden)
    seq = hip.seq_create(xf, 16)
    kv = mdl.oracle_kv(16, 1)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    hid = hip.forward_hidden(xf, seq, 0, x, 128)
    _, all_ref = oracle.transformer_forward(mdl.ox, kv, x, want_all=True)
    L = oracle.lib()
    for i in range(3):
        nrm = np.empty(128, np.float32)
        L.vo_rmsnorm(hid[i].ctypes.data, mdl.final_norm.ctypes.data, 128, np.float32(1e-6), nrm.ctypes.data)
        assert rel_err(nrm, all_ref[i]) < TOL
    # input projection inside the step (transformer_step_fused with in_proj)
    from models import make_mat
    d, s, b = make_mat(rng, Q8, 128, 96, bias=True)
    ip = hip.upload(hip.HostMat(Q8, d, 128, 96, s, b))
    seq2 = hip.seq_create(xf, 16)
    kv2 = mdl.oracle_kv(16, 1)
    xi = rng.standard_normal((2, 96)).astype(np.float32)
    out, _ = hip.forward(xf, seq2, 0, xi, 128, in_proj=ip)
    h = oracle.matmul(oracle.Mat(Q8, d, 128, 96, s, b), xi)
    assert rel_err(out, oracle.transformer_forward(mdl.ox, kv2, h)) < TOL


def test_pair_and_steps(hip, oracle):
    mdl = Model(600, 2, 256, 4, 2, 128, 512, wtype=Q8, head_rows=80)
    xf, head = build(hip, mdl)
    rng = np.random.default_rng(9)
    seqs = [hip.seq_create(xf, 32) for _ in range(3)]
    kvs = [mdl.oracle_kv(32, 1) for _ in range(3)]
    lens = [4, 4, 7]
    for s, k, n in zip(seqs, kvs, lens):
        pre = rng.standard_normal((n, 256)).astype(np.float32)
        hip.forward(xf, s, 0, pre, 256)
        oracle.transformer_forward(mdl.ox, k, pre)
    # pair: sequences 0 and 1 at the same position (gpu_xfmr_forward_pair)
    x2 = rng.standard_normal((2, 256)).astype(np.float32)
    out2, log2 = hip.forward_pair(xf, seqs[0], seqs[1], 4, x2, 256, head=head)
    for i in range(2):
        r = oracle.transformer_forward(mdl.ox, kvs[i], x2[i:i + 1])
        assert rel_err(out2[i], r) < TOL and rel_err(log2[i], oracle_head(oracle, mdl, out2[i])) < TOL
    # B independent sessions at their own positions (transformer_forward_steps)
    x3 = rng.standard_normal((3, 256)).astype(np.float32)
    out3, log3 = hip.forward_steps(xf, seqs, [5, 5, 7], x3, 256, head=head)
    ref3 = oracle.transformer_forward_steps(mdl.ox, kvs, x3)
    assert rel_err(out3, ref3) < TOL
    for i in range(3):
        assert rel_err(log3[i], oracle_head(oracle, mdl, out3[i])) < TOL


def test_decode_steps_dev(hip, oracle):
    # B sessions at their own positions in one device-resident graph: same states and logits as the host-pointer
    # forward_steps, each row's token from the oracle sampler on the device logits with that row's counter.
    mdl = Model(710, 2, 256, 4, 2, 128, 512, wtype=Q4, head_rows=200)
    xf, head = build(hip, mdl)
    rng = np.random.default_rng(12)
    B = 5
    seqs_a = [hip.seq_create(xf, 32) for _ in range(B)]
    seqs_b = [hip.seq_create(xf, 32) for _ in range(B)]
    lens = [3, 7, 1, 5, 9]
    for sa, sb, n in zip(seqs_a, seqs_b, lens):
        pre = rng.standard_normal((n, 256)).astype(np.float32)
        hip.forward(xf, sa, 0, pre, 256)
        hip.forward(xf, sb, 0, pre, 256)
    x = rng.standard_normal((B, 256)).astype(np.float32)
    out_ref, log_ref = hip.forward_steps(xf, seqs_a, lens, x, 256, head=head)
    dx, dout, dlog, dtok = hip.DevBuf(x.nbytes), hip.DevBuf(x.nbytes), hip.DevBuf(B * 200 * 4), hip.DevBuf(B * 4)
    dx.upload(x)
    cfgs = [hip.sample_cfg(0.9, 0.8, 25, seed=77, frame=10 + b, codebook=b) for b in range(B)]
    for rep in range(3):
        hip.decode_steps_dev(xf, seqs_b, lens, dx, dout, head, dlog, cfgs, dtok)
        hip.sync()
        out = dout.download(B * 256, np.float32).reshape(B, 256)
        lg = dlog.download(B * 200, np.float32).reshape(B, 200)
        assert np.array_equal(out, out_ref) and np.array_equal(lg, log_ref), rep
        toks = dtok.download(B, np.int32)
        for b in range(B):
            u = oracle.uniform(77, 10 + b, b, 0)
            assert toks[b] == oracle.sample_logits(lg[b], 0.9, 0.8, 25, 1.0, None, u), (rep, b)
    for bf in (dx, dout, dlog, dtok):
        bf.free()


def test_decode_graph_replays(hip, oracle):
    # The captured decode step replays to the same result as the host-pointer forward, every replay.
    mdl = Model(700, 2, 256, 4, 2, 128, 512, wtype=Q8, head_rows=256)
    xf, head = build(hip, mdl)
    seq_a, seq_b = hip.seq_create(xf, 32), hip.seq_create(xf, 32)
    rng = np.random.default_rng(10)
    pre = rng.standard_normal((5, 256)).astype(np.float32)
    hip.forward(xf, seq_a, 0, pre, 256)
    hip.forward(xf, seq_b, 0, pre, 256)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    out_ref, log_ref = hip.forward(xf, seq_a, 5, x, 256, head=head)
    dx, dout, dlog, dtok = hip.DevBuf(256 * 4), hip.DevBuf(256 * 4), hip.DevBuf(256 * 4), hip.DevBuf(4)
    dx.upload(x)
    cfg = hip.sample_cfg(0.9, 1.0, 50, seed=1234, frame=3)
    toks = []
    for rep in range(4):
        hip.decode_dev(xf, seq_b, 5, dx, 1, dout, head, dlog, cfg, dtok)
        hip.sync()
        out = dout.download(256, np.float32)
        lg = dlog.download(256, np.float32)
        assert np.array_equal(out, out_ref) and np.array_equal(lg, log_ref), rep
        toks.append(int(dtok.download(1, np.int32)[0]))
    assert len(set(toks)) == 1
    u = oracle.uniform(1234, 3, 0, 0)
    assert toks[0] == oracle.sample_logits(log_ref, 0.9, 1.0, 50, 1.0, None, u)
    for b in (dx, dout, dlog, dtok):
        b.free()


@pytest.mark.parametrize("wt", [F16, Q8])
def test_decode_dev_rows_new_position(hip, oracle, wt):
    # m = 6 rows of one sequence per captured step, replayed at a later position: F16 takes the prefill attention
    # kernel (q8 the int path), which must take the pass's first position from the device row table, not from the
    # capture. Both replays against the oracle continuing the same sequence.
    mdl = Model(720 + wt, 2, 256, 4, 2, 128, 512, wtype=wt, head_rows=128)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 32)
    kv = mdl.oracle_kv(32, kv_f16=1)
    rng = np.random.default_rng(20 + wt)
    pre = rng.standard_normal((3, 256)).astype(np.float32)
    hip.forward(xf, seq, 0, pre, 256)
    oracle.transformer_forward(mdl.ox, kv, pre)
    dx, dout, dlog = hip.DevBuf(6 * 256 * 4), hip.DevBuf(256 * 4), hip.DevBuf(128 * 4)
    for pos0 in (3, 9, 15):
        x = rng.standard_normal((6, 256)).astype(np.float32)
        dx.upload(x)
        hip.decode_dev(xf, seq, pos0, dx, 6, dout, head, dlog)
        hip.sync()
        out = dout.download(256, np.float32)
        lg = dlog.download(128, np.float32)
        ref = oracle.transformer_forward(mdl.ox, kv, x)
        assert rel_err(out, ref) < TOL, (pos0, rel_err(out, ref))
        assert rel_err(lg, oracle_head(oracle, mdl, out)) < TOL, pos0
    for b in (dx, dout, dlog):
        b.free()


@pytest.mark.parametrize("wt,m", [(F16, 70), (Q8, 6), (Q8, 1)])
def test_layer_pass_graph_replays(hip, oracle, wt, m):
    # forward_rows runs a layer pass eagerly the first time its shape is seen, captures it the second time and replays
    # the graph after: three identical passes over the same positions of one sequence, with other work (a pass of
    # another shape on another sequence) between them, give identical results, equal to the oracle.
    mdl = Model(730 + m, 2, 256, 4, 2, 128, 512, wtype=wt, head_rows=64)
    xf, head = build(hip, mdl)
    seq, other = hip.seq_create(xf, 128), hip.seq_create(xf, 128)
    rng = np.random.default_rng(40 + m)
    pre = rng.standard_normal((3, 256)).astype(np.float32)
    hip.forward(xf, seq, 0, pre, 256)
    kv = mdl.oracle_kv(128, kv_f16=1)
    oracle.transformer_forward(mdl.ox, kv, pre)
    x = rng.standard_normal((m, 256)).astype(np.float32)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    outs = []
    for rep in range(3):
        out, logits = hip.forward(xf, seq, 3, x, 256, head=head)
        outs.append((out, logits))
        hip.forward(xf, other, rep, rng.standard_normal((2, 256)).astype(np.float32), 256)
    for out, logits in outs:
        assert np.array_equal(out, outs[0][0]) and np.array_equal(logits, outs[0][1])
    assert rel_err(outs[0][0], ref) < TOL, rel_err(outs[0][0], ref)


def test_prefill_planes_under_vram_limit(hip, oracle):
    # a Q8 prefill of more than 8 rows takes the planes path, which widens every matrix to f16 once (26 MB here);
    # with a VRAM limit just above the weights those copies cannot be made, and the pass must still run (on the
    # f32-activation GEMM) with the same results
    warm = Model(840, 1, 256, 4, 2, 64, 512, wtype=Q8)  # allocates the library's pass scratch first
    wx, _ = build(hip, warm)
    hip.forward(wx, hip.seq_create(wx, 64), 0, np.ones((9, 256), np.float32), 256)
    mdl = Model(841, 2, 512, 8, 2, 64, 4096, wtype=Q8, head_rows=64)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 64)
    kv = mdl.oracle_kv(64, kv_f16=1)
    used = hip.mem_info().used
    hip.lib().voxhip_set_vram_limit(used + (4 << 20))
    try:
        rng = np.random.default_rng(17)
        x = rng.standard_normal((9, 512)).astype(np.float32)
        out, logits = hip.forward(xf, seq, 0, x, 512, head=head)
        assert hip.mem_info().used < used + (4 << 20)
        ref = oracle.transformer_forward(mdl.ox, kv, x)
        assert rel_err(out, ref) < TOL, rel_err(out, ref)
        assert rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
        x = rng.standard_normal((1, 512)).astype(np.float32)
        out, _ = hip.forward(xf, seq, 9, x, 512, head=head)
        assert rel_err(out, oracle.transformer_forward(mdl.ox, kv, x)) < TOL
    finally:
        hip.lib().voxhip_set_vram_limit(0)


@pytest.mark.parametrize("wt,hd", [(F16, 128), (Q8, 128), (F16, 64), (Q8, 64)])
def test_prefill_key_splits(hip, oracle, wt, hd):
    # prefill passes whose grid of 64-row query tiles leaves CUs idle split each tile's keys into runs merged by
    # k_pattn_merge, at both head dims of the kernel: 300 rows from position 0 (8 runs, the last ones empty for the
    # early tiles), then 100 rows at position 300 (7 non-empty runs and an empty one), then the same 100-row pass
    # again: captured, then replayed
    mdl = Model(760 + wt + hd, 2, 256, 256 // hd * 2, 2, hd, 512, wtype=wt, head_rows=64)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 512)
    kv = mdl.oracle_kv(512, kv_f16=1)
    rng = np.random.default_rng(61 + wt)
    x = rng.standard_normal((300, 256)).astype(np.float32)
    out, _ = hip.forward(xf, seq, 0, x, 256, head=head)
    assert rel_err(out, oracle.transformer_forward(mdl.ox, kv, x)) < TOL
    x2 = rng.standard_normal((100, 256)).astype(np.float32)
    ref = oracle.transformer_forward(mdl.ox, kv, x2)
    outs = [hip.forward(xf, seq, 300, x2, 256, head=head) for _ in range(3)]
    assert rel_err(outs[0][0], ref) < TOL, rel_err(outs[0][0], ref)
    for out, logits in outs[1:]:
        assert np.array_equal(out, outs[0][0]) and np.array_equal(logits, outs[0][1])


@pytest.mark.parametrize("wt", [F16, Q8])
def test_prefill_down_reduce_norms(hip, oracle, wt):
    # planes prefill of 3 layers whose down projection (K 2048, 8 tiles) splits K: the split-K reduce of layers 0 and
    # 1 also writes the next layer's first RMSNorm; the last layer's reduce does not. Against the oracle, then the
    # same pass captured and replayed (bit-identical).
    mdl = Model(820 + wt, 3, 256, 4, 2, 64, 2048, wtype=wt, bias=True, head_rows=64)
    xf, head = build(hip, mdl)
    seq = hip.seq_create(xf, 512)
    kv = mdl.oracle_kv(512, kv_f16=1)
    rng = np.random.default_rng(83 + wt)
    x = rng.standard_normal((128, 256)).astype(np.float32)
    out, logits = hip.forward(xf, seq, 0, x, 256, head=head)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    assert rel_err(out, ref) < TOL, rel_err(out, ref)
    assert rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
    x2 = rng.standard_normal((96, 256)).astype(np.float32)
    ref2 = oracle.transformer_forward(mdl.ox, kv, x2)
    outs = [hip.forward(xf, seq, 128, x2, 256, head=head) for _ in range(3)]
    assert rel_err(outs[0][0], ref2) < TOL, rel_err(outs[0][0], ref2)
    for o, lg in outs[1:]:
        assert np.array_equal(o, outs[0][0]) and np.array_equal(lg, outs[0][1])


# head_dim other than 64 / 128 (the reference's device path takes any even head_dim <= 128, gpu_vulkan.cpp:770):
# (wtype, heads, kv_heads, head_dim, qk_norm); the q|k|v and o widths satisfy the matrix column rules
@pytest.mark.parametrize("wt,heads,kvh,hd,qkn", [(Q8, 4, 2, 96, True), (BF16, 4, 1, 80, True), (F16, 4, 2, 34, False),
                                                  (F32, 4, 4, 2, True), (Q8, 8, 2, 32, True)])
def test_any_head_dim(hip, oracle, wt, heads, kvh, hd, qkn):
    # prefill of 9 rows, host-pointer decode steps, a captured device decode step replayed at new positions, and two
    # sessions in one step, all against the oracle continuing the same sequences
    mdl = Model(740 + hd, 2, 256, heads, kvh, hd, 512, wtype=wt, qk_norm=qkn, head_rows=96)
    xf, head = build(hip, mdl)
    seq, seq2 = hip.seq_create(xf, 64), hip.seq_create(xf, 64)
    kv, kv2 = mdl.oracle_kv(64, 1), mdl.oracle_kv(64, 1)
    rng = np.random.default_rng(hd)
    x = rng.standard_normal((9, 256)).astype(np.float32)
    out, logits = hip.forward(xf, seq, 0, x, 256, head=head)
    ref = oracle.transformer_forward(mdl.ox, kv, x)
    assert rel_err(out, ref) < TOL, rel_err(out, ref)
    assert rel_err(logits, oracle_head(oracle, mdl, out)) < TOL
    for step in range(2):
        x = rng.standard_normal((1, 256)).astype(np.float32)
        out, _ = hip.forward(xf, seq, 9 + step, x, 256, head=head)
        assert rel_err(out, oracle.transformer_forward(mdl.ox, kv, x)) < TOL, step
    dx, dout, dlog = hip.DevBuf(256 * 4), hip.DevBuf(256 * 4), hip.DevBuf(96 * 4)
    for pos in (11, 12, 13):
        x = rng.standard_normal((1, 256)).astype(np.float32)
        dx.upload(x)
        hip.decode_dev(xf, seq, pos, dx, 1, dout, head, dlog)
        hip.sync()
        out = dout.download(256, np.float32)
        ref = oracle.transformer_forward(mdl.ox, kv, x)
        assert rel_err(out, ref) < TOL, (pos, rel_err(out, ref))
        assert rel_err(dlog.download(96, np.float32), oracle_head(oracle, mdl, out)) < TOL, pos
    for b in (dx, dout, dlog):
        b.free()
    pre = rng.standard_normal((5, 256)).astype(np.float32)
    hip.forward(xf, seq2, 0, pre, 256)
    oracle.transformer_forward(mdl.ox, kv2, pre)
    x2 = rng.standard_normal((2, 256)).astype(np.float32)
    out2, _ = hip.forward_steps(xf, [seq, seq2], [14, 5], x2, 256, head=head)
    assert rel_err(out2, oracle.transformer_forward_steps(mdl.ox, [kv, kv2], x2)) < TOL


def test_layer_ranges_compose(hip, oracle):
    # forward_layers over [0, 1) then [1, 2) equals the oracle's layers, teacher-forced per layer
    mdl = Model(900, 2, 256, 4, 2, 128, 512, wtype=Q8)
    xf, _ = build(hip, mdl)
    seq = hip.seq_create(xf, 16)
    kv = mdl.oracle_kv(16, 1)
    rng = np.random.default_rng(11)
    h = rng.standard_normal((2, 256)).astype(np.float32)
    for li in range(2):
        hg = hip.forward_layers(xf, seq, 0, h, li, 1)
        hr = oracle.transformer_layers(mdl.ox, kv, h, li, 1)
        assert rel_err(hg, hr) < TOL
        h = hr


def test_errors_are_reported(hip):
    mdl = Model(800, 1, 128, 4, 2, 64, 256, wtype=Q8)
    xf, _ = build(hip, mdl)
    seq = hip.seq_create(xf, 8)
    with pytest.raises(hip.VoxHipError, match="capacity"):
        hip.forward(xf, seq, 7, np.zeros((2, 128), np.float32), 128)
    with pytest.raises(hip.VoxHipError):
        hip.seq_create(xf, 0)
    with pytest.raises(hip.VoxHipError):
        hip.forward(xf, 999, 0, np.zeros((1, 128), np.float32), 128)


def test_pair_graph_replayed_with_another_second_row(hip, oracle):
    # a pair pass is captured as a graph the second time its shape is seen, keyed by the first row's cache: the same
    # graph replayed with another second sequence must read that sequence's keys (its attention takes every row's
    # cache view from the device row table), so both rows agree with the oracle
    mdl = Model(601, 2, 256, 4, 2, 128, 512, wtype=Q8)
    xf, _ = build(hip, mdl)
    rng = np.random.default_rng(10)
    seqs = [hip.seq_create(xf, 32) for _ in range(3)]
    kvs = [mdl.oracle_kv(32, 1) for _ in range(3)]
    for s, k in zip(seqs, kvs):
        pre = rng.standard_normal((6, 256)).astype(np.float32)
        hip.forward(xf, s, 0, pre, 256)
        oracle.transformer_forward(mdl.ox, k, pre)
    for pos, (a, b) in zip((6, 7, 8, 9), ((0, 1), (0, 1), (0, 2), (0, 2))):
        x2 = rng.standard_normal((2, 256)).astype(np.float32)
        out2, _ = hip.forward_pair(xf, seqs[a], seqs[b], pos, x2, 256)
        for row, sq in enumerate((a, b)):
            kv = kvs[sq]
            kv.c.len = pos  # the oracle appends at pos, as the device did
            r = oracle.transformer_forward(mdl.ox, kv, x2[row:row + 1])
            assert rel_err(out2[row], r) < TOL, (pos, a, b, row, rel_err(out2[row], r))
