"""The split-f16 MFMA GEMM of the multi-row passes on its own, through voxhip_bench_gemm_hh: every block tile of the
shape policy gives the same bits (each output is the same MFMA sequence whatever the tile), and the product matches a
float64 evaluation of the same f16 operands (A = A_hi + A_lo, W as f16, or q8 as float(q) * scale per 32-block, the
reference's dequantized matmul, kernels.cpp:661-679). The inputs are rebuilt with voxhip_mat_synthetic, which draws
from the same generator with the same seeds."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F16, Q8 = 1, 3


def _operands(hip, m, n, K, q8):
    ah = hip.mat_synthetic(F16, m, K, 11, 0x90, 0.0, 1.0)
    al = hip.mat_synthetic(F16, m, K, 12, 0x91, 0.0, 1e-3)
    wm = hip.mat_synthetic(Q8 if q8 else F16, n, K, 13, 0x92, 0.0, 0.02)
    try:
        a = hip.mat_download(ah, F16)[0].view(np.float16).astype(np.float64)
        a += hip.mat_download(al, F16)[0].view(np.float16).astype(np.float64)
        if q8:
            q, sc, _ = hip.mat_download(wm, Q8)
            w = (q.astype(np.float64).reshape(n, K // 32, 32) * sc.astype(np.float64)[:, :, None]).reshape(n, K)
        else:
            w = hip.mat_download(wm, F16)[0].view(np.float16).astype(np.float64)
    finally:
        for h in (ah, al, wm):
            hip.mat_free(h)
    return a, w


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("shape", [(300, 272, 320), (97, 1152, 896), (512, 96, 2048)])
def test_tiles_bit_identical_and_exact(hip, shape, q8):
    m, n, K = shape
    a, w = _operands(hip, m, n, K, q8)
    want = a @ w.T
    outs = {t: hip.bench_gemm_hh(m, n, K, q8=q8, tile=t, warmup=0, iters=1, out=True)[1] for t in range(5)}
    for t in range(1, 5):
        assert np.array_equal(outs[t], outs[0]), (shape, q8, t)
    err = np.max(np.abs(outs[0] - want)) / np.max(np.abs(want))
    assert err < 1e-5, (shape, q8, err)  # f32 accumulation over K; a dropped lo plane would give ~1e-3


def test_bad_arguments_rejected(hip):
    with pytest.raises(hip.VoxHipError):
        hip.bench_gemm_hh(64, 64, 96, tile=0, iters=1)  # K not a multiple of 64
    with pytest.raises(hip.VoxHipError):
        hip.bench_gemm_hh(64, 64, 128, tile=5, iters=1)
