"""Parity of the gfx950 kernels with the oracle, through the C ABI (libvoxhip.so).

Bars: bit-exact for quantization, unpacking and sampled token ids; the GEMVs are
f32 activations, compared with the reference's `vox verify` metric max|a-b| / max(1, max|b|) at 1e-5 (they
differ from the CPU only in float summation order).
"""
import numpy as np
import pytest

from conftest import rel_err
from models import make_mat

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4
GEMV_TOL = 1e-5


def test_device_is_gfx950(hip):
    assert "gfx950" in hip.device_name()
    assert hip.lib().voxhip_active() == 1


def test_packed_f16_split_bit_exact(hip):
    # the attention's P split (v_cvt_pk_f16_f32, v_fma_mix{lo,hi}_f16) against hi = f16(x), lo = f16(x - hi) on 2^27
    # pseudo-random pairs, half of them spread over the f16 subnormal, normal and overflow ranges
    assert hip.selftest_split_f16(1 << 27) == 0


def test_quantizers_bit_exact(hip, oracle):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 256)) * np.geomspace(1e-4, 10, 256)).astype(np.float32)
    w[0, :32] = 0.0                       # all-zero block
    w[1, :32] = 0.25                      # equal magnitudes
    w[2, :32] = np.linspace(-1, 1, 32)    # exact ties at .5 steps
    w[3, 32:64] = -w[3, 32:64]
    q, s = hip.quantize_q8_dev(w)
    oq, os_ = oracle.quantize_q8(w)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    q, s = hip.quantize_q4_dev(w)
    oq, os_ = oracle.quantize_q4(w)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    x = rng.standard_normal(4096).astype(np.float32) * 3
    x[:32] = 0
    x[32:64] = np.arange(32) - 15.5  # x * inv lands on .5 for some elements
    xq, xs = hip.quantize_act_dev(x)
    oq, os_ = oracle.quantize_act(x)
    assert np.array_equal(xq, oq) and np.array_equal(xs.view(np.uint32), os_.view(np.uint32))


def test_quantizers_bit_exact_large(hip, oracle):
    # 4 x 131,072 random blocks, then the blocks where kernels.cpp:616's float best_err decides the q4 scale
    # (tests/golden/golden_q4.npz holds the compiled reference's output for them)
    import os
    rng = np.random.default_rng(5)
    mats = [(rng.standard_normal((4096, 1024)) * 0.02).astype(np.float32),
            rng.uniform(-1, 1, (4096, 1024)).astype(np.float32),
            (rng.integers(-8, 8, (4096, 1024)) * 0.01 + rng.standard_normal((4096, 1024)) * 1e-6).astype(np.float32),
            (rng.standard_normal((4096, 1024)) * np.geomspace(1e-6, 1e3, 1024)).astype(np.float32)]
    for w in mats:
        q, s = hip.quantize_q4_dev(w)
        oq, os_ = oracle.quantize_q4(w)
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32)) and np.array_equal(q, oq)
        q, s = hip.quantize_q8_dev(w)
        oq, os_ = oracle.quantize_q8(w)
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32)) and np.array_equal(q, oq)
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_q4.npz"), allow_pickle=False)
    q, s = hip.quantize_q4_dev(g["w"])
    assert np.array_equal(s.view(np.uint32), g["s"].view(np.uint32)) and np.array_equal(q, g["q"])


@pytest.mark.parametrize("wt", [Q8, Q4, F32, F16, BF16, "q4h"])
def test_mat_gather_bit_exact(hip, oracle, wt):
    # mat_row / mat_gather (kernels.cpp:432-471): the device unpack of every weight type, the one the LM and code
    # predictor embedding gathers use, equals the oracle's row bit for bit (q4h: Q4 whose scales are all exact in
    # f16, stored in 2 bytes on the device)
    rng = np.random.default_rng(31 + (wt if isinstance(wt, int) else 9))
    t = Q4 if wt == "q4h" else wt
    rows, cols = 300, 896
    data, scale, _ = make_mat(rng, t, rows, cols, std=0.5)
    if wt == "q4h":
        scale = scale.astype(np.float16).astype(np.float32)
    M = oracle.Mat(t, data, rows, cols, scale, None)
    h = hip.upload(hip.HostMat(t, data, rows, cols, scale, None))
    ids = np.concatenate([[0, rows - 1, 7, 7], rng.integers(0, rows, 60)]).astype(np.int32)
    got = hip.mat_gather(h, ids, cols)
    want = np.stack([oracle.mat_row(M, int(r)) for r in ids])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(hip.VoxHipError, match="outside"):
        hip.mat_gather(h, np.array([0, rows], np.int32), cols)


@pytest.mark.parametrize("wt", [Q8, Q4, F32, F16, BF16])
# tiles: (37,160) R1; (4096,1024) R4; (1024,3072) IT3; (3072,1024) R3; (5,4864) IT4 over two passes; (6144,1024) R6;
# (8192,256) R8; (2048,2048) IT2 (R2 for m > 1)
@pytest.mark.parametrize("rows,cols", [(37, 160), (4096, 1024), (1024, 3072), (3072, 1024), (5, 4864), (6144, 1024),
                                       (8192, 256), (2048, 2048)])
def test_matmul_parity(hip, oracle, wt, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols + wt)
    data, scale, bias = make_mat(rng, wt, rows, cols, bias=True)
    M = oracle.Mat(wt, data, rows, cols, scale, bias)
    h = hip.upload(hip.HostMat(wt, data, rows, cols, scale, bias))
    for m in (1, 2, 3, 5, 8, 9, 13):
        x = rng.standard_normal((m, cols)).astype(np.float32)
        y = hip.matmul(h, x)
        r = oracle.matmul(M, x)
        assert y.shape == r.shape
        assert rel_err(y, r) < GEMV_TOL, (wt, rows, cols, m, rel_err(y, r))


@pytest.mark.parametrize("wt", [Q8, F32, F16, BF16])
@pytest.mark.parametrize("rows,cols", [(37, 160), (1000, 1024), (2048, 896)])
def test_matmul_gemm_rows(hip, oracle, wt, rows, cols):
    # f32-activation passes of more than 4 rows run on the MFMA GEMM: ragged row/column tiles, bias, and 600 rows
    # over two passes (512 + 88)
    rng = np.random.default_rng(rows + cols * 3 + wt)
    data, scale, bias = make_mat(rng, wt, rows, cols, bias=True)
    M = oracle.Mat(wt, data, rows, cols, scale, bias)
    h = hip.upload(hip.HostMat(wt, data, rows, cols, scale, bias))
    for m in (6, 64, 65, 200, 600):
        x = rng.standard_normal((m, cols)).astype(np.float32)
        y = hip.matmul(h, x)
        r = oracle.matmul(M, x)
        assert rel_err(y, r) < GEMV_TOL, (wt, rows, cols, m, rel_err(y, r))


# (cin, cout, K, stride, pad, out_pad, T, bias): HiFT's three upsample stages (CosyVoice2: rates 8 / 5 / 3, kernels
# 16 / 11 / 7, channels 512 -> 64) at 640 and 1200 frames (the GEMM over two and three 512-frame passes), Kokoro's
# first stage (rate 10, kernel 20), output padding, K < stride, pad >= K / 2, one frame and a GEMV-sized product
CONVT_GPU_CASES = [(512, 256, 16, 8, 4, 0, 80, True), (256, 128, 11, 5, 3, 0, 640, True), (128, 64, 7, 3, 2, 0, 1200, True),
                   (512, 256, 20, 10, 5, 0, 50, True), (64, 48, 5, 2, 2, 1, 33, False), (32, 16, 4, 3, 1, 2, 17, True),
                   (16, 8, 3, 5, 0, 0, 9, True), (8, 8, 4, 1, 3, 0, 12, True), (40, 24, 6, 3, 1, 0, 1, True),
                   (96, 64, 8, 4, 2, 0, 3, True)]


@pytest.mark.parametrize("cin,cout,K,s,pad,op,T,bias", CONVT_GPU_CASES)
def test_convt_parity(hip, oracle, cin, cout, K, s, pad, op, T, bias):
    # nn::ConvT (nn.cpp:205-245): the F32 product on the device (GEMV up to 4 frames, MFMA GEMM above) and the padded
    # overlap-add in the reference's order, against the oracle's restatement at the GEMV bar
    rng = np.random.default_rng(cin + 3 * K + 11 * T)
    w = (rng.standard_normal((cin, cout, K)) * (1.0 / np.sqrt(cin))).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32) if bias else None
    x = rng.standard_normal((T, cin)).astype(np.float32)
    ct = hip.ConvT().load(w, b, s, pad, op)
    try:
        y = ct.forward(x)
        want = oracle.convt(w, b, x, s, pad, op)
        assert y.shape == want.shape == (ct.out_len(T), cout)
        assert rel_err(y, want) < GEMV_TOL, rel_err(y, want)
    finally:
        hip.mat_free(ct.mat)


def test_convt_rejects_bad_calls(hip):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((8, 4, 3)).astype(np.float32)
    ct = hip.ConvT().load(w, None, 2, 0)
    try:
        x = rng.standard_normal((1, 8)).astype(np.float32)
        with pytest.raises(hip.VoxHipError, match="no output frames"):
            hip.convt(ct.mat, 3, 1, 3, 0, None, x)
        with pytest.raises(hip.VoxHipError, match="K cout"):
            hip.convt(ct.mat, 5, 2, 0, 0, None, x)
    finally:
        hip.mat_free(ct.mat)
    withb = hip.upload(hip.HostMat(F32, rng.standard_normal((12, 8)).astype(np.float32), 12, 8, None,
                                   np.ones(12, np.float32)))
    try:
        with pytest.raises(hip.VoxHipError, match="bias"):
            hip.convt(withb, 3, 2, 0, 0, None, rng.standard_normal((4, 8)).astype(np.float32))
    finally:
        hip.mat_free(withb)


@pytest.mark.parametrize("rows,cols", [(4096, 2048), (2048, 6144), (37, 160)])
def test_q4_f16_scales(hip, oracle, rows, cols):
    # Q4 scales that are exact in f16 are stored in 2 bytes on the device (the cfg 3 "4-bit + f16 scale" format):
    # same products as the f32 scales, and the download widens them back bit-exactly.
    rng = np.random.default_rng(rows + cols)
    data, scale, _ = make_mat(rng, Q4, rows, cols)
    scale = scale.astype(np.float16).astype(np.float32)
    h = hip.upload(hip.HostMat(Q4, data, rows, cols, scale))
    d2, s2, _ = hip.mat_download(h, Q4)
    assert np.array_equal(d2, data) and np.array_equal(s2.view(np.uint32), scale.view(np.uint32))
    M = oracle.Mat(Q4, data, rows, cols, scale)
    for m in (1, 3, 8):
        x = rng.standard_normal((m, cols)).astype(np.float32)
        assert rel_err(hip.matmul(h, x), oracle.matmul(M, x)) < GEMV_TOL
    # one scale that is not exact in f16 keeps the whole matrix on f32 scales, with the same results
    scale2 = scale.copy()
    scale2.flat[7] = np.float32(scale2.flat[7] * (1 + 2**-20))
    h2 = hip.upload(hip.HostMat(Q4, data, rows, cols, scale2))
    x = rng.standard_normal((2, cols)).astype(np.float32)
    assert rel_err(hip.matmul(h2, x), oracle.matmul(oracle.Mat(Q4, data, rows, cols, scale2), x)) < GEMV_TOL
    _, s3, _ = hip.mat_download(h2, Q4)
    assert np.array_equal(s3.view(np.uint32), scale2.view(np.uint32))


def test_matmul_stacked_upload(hip, oracle):
    # n_parts > 1 stacks rows like upload_parts (gpu_vulkan.cpp:476-536)
    rng = np.random.default_rng(3)
    parts = [make_mat(rng, Q8, r, 256, bias=True) for r in (64, 32, 32)]
    h = hip.upload(*[hip.HostMat(Q8, d, d.shape[0], 256, s, b) for d, s, b in parts])
    assert hip.mat_shape(h) == (128, 256)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    y = hip.matmul(h, x)
    r = np.concatenate([oracle.matmul(oracle.Mat(Q8, d, d.shape[0], 256, s, b), x) for d, s, b in parts], axis=1)
    assert rel_err(y, r) < GEMV_TOL


def test_matmul_rejects_bad_shapes(hip):
    bad = hip.HostMat(Q8, np.zeros((4, 40), np.int8), 4, 40, np.zeros((4, 1), np.float32))
    with pytest.raises(hip.VoxHipError):
        hip.upload(bad)  # Q8 needs cols % 32 == 0 (kernels.cpp:655)
    with pytest.raises(hip.VoxHipError):
        hip.matmul(12345, np.zeros(32, np.float32))


def masked(l, cfg):
    """engine.cpp:664-668 applied on the host for the oracle."""
    l = l.copy()
    for i in range(max(0, cfg.suppress_from), min(len(l), cfg.suppress_to)):
        if i != cfg.eos_code:
            l[i] = -np.inf
    if cfg.block_eos and 0 <= cfg.eos_code < len(l):
        l[cfg.eos_code] = -np.inf
    return l


def test_sampler_parity(hip, oracle):
    rng = np.random.default_rng(8)
    for i in range(400):
        n = int(rng.choice([2, 3, 50, 64, 65, 257, 3072, 6564, 16384]))
        l = (rng.standard_normal(n) * rng.uniform(0.3, 5)).astype(np.float32)
        if i % 4 == 0:
            l = np.round(l).astype(np.float32)  # ties
        if i % 5 == 0:
            l[rng.integers(0, n, max(1, n // 3))] = -np.inf
        T = float(rng.choice([0.0, 0.7, 0.9, 1.0, 1.5]))
        k = int(rng.choice([0, 1, 25, 50, 64, 65, 4096]))
        p = float(rng.choice([1.0, 0.8, 0.3]))
        rep = float(rng.choice([1.0, 1.3]))
        hist = rng.integers(0, n, int(rng.integers(0, 30))).astype(np.int32) if rep != 1.0 else None
        seed = int(rng.integers(0, 2**63))
        cfg = hip.sample_cfg(T, p, k, rep, seed=seed, frame=int(rng.integers(0, 1 << 40)), codebook=int(rng.integers(0, 16)))
        if i % 3 == 0 and n > 40:
            cfg.suppress_from, cfg.suppress_to, cfg.eos_code, cfg.block_eos = n - 20, n, n - 5, int(i % 2)
        u = oracle.uniform(seed, cfg.frame, cfg.codebook, 0)
        want = oracle.sample_logits(masked(l, cfg), T, p, k, rep, hist, u)
        assert hip.sample_logits(l, cfg, hist) == want, (i, n, T, k, p, rep)


@pytest.mark.parametrize("n,k", [(3072, 50), (16384, 64), (2048, 17)])
def test_sampler_skewed_blocks(hip, oracle, n, k):
    # the sampler instance for each vocabulary size (1, 2, 4, 8 or 16 logits per thread), with the logits of one
    # wave (indices i with i % 1024 < 64) pushed far down in half the cases, so the radix select's first buckets
    # are split unevenly across waves
    rng = np.random.default_rng(n + k)
    for case in range(12):
        l = (rng.standard_normal(n) * 2).astype(np.float32)
        if case % 2 == 0:
            idx = np.arange(n)
            l[idx % 1024 < 64] -= 50.0
        cfg = hip.sample_cfg(0.9, 1.0 if case % 3 else 0.8, k, seed=case, frame=case)
        u = oracle.uniform(case, case, 0, 0)
        assert hip.sample_logits(l, cfg) == oracle.sample_logits(l, 0.9, cfg.top_p, k, 1.0, None, u), case


def test_sampler_limits(hip):
    with pytest.raises(hip.VoxHipError):
        hip.sample_logits(np.zeros(16385, np.float32), hip.sample_cfg())
    with pytest.raises(hip.VoxHipError):
        hip.sample_logits(np.zeros(0, np.float32), hip.sample_cfg())


def test_sampler_reference_rules(hip):
    # test_core.cpp:53-78 on the device
    l = np.float32([0.1, 3.0, 0.2, 3.0])
    assert hip.sample_logits(l, hip.sample_cfg(temperature=0.0)) == 1
    for fr in range(5):
        assert hip.sample_logits(l, hip.sample_cfg(top_k=1, frame=fr)) == 1
    assert hip.sample_logits(l, hip.sample_cfg(temperature=0.0, repetition_penalty=10.0), [1]) == 3
    two = np.float32([0.0, np.log(3.0)])
    ones = sum(hip.sample_logits(two, hip.sample_cfg(temperature=1.0, top_k=0, seed=42, frame=i)) == 1 for i in range(3000))
    assert abs(ones / 3000.0 - 0.75) < 0.03
