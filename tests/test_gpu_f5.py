"""F5-TTS DiT step on the device (gpu_f5_create / begin / step / end, f5.cpp:586-725) against the oracle's vo_f5_step.

Both sides consume the same stored f16 / bf16 / f32 weights and f32 position convolutions. The device runs f16
linears on the split-f16 matrix cores (activations as f16 hi + lo halves, products exact in the f32 accumulator;
the models here with all widths multiples of 64 take the pre-split path, the others the f32-row path), bf16 / f32
linears and the convolutions on f32 MFMA, and attention on split-f16 MFMA tiles with an online softmax, so the
outputs differ only by summation order, the dropped lo x lo terms (below 2^-22) and libm ulps: the north star's
1e-3 for f32 activations with the `vox verify` metric.
"""
import numpy as np
import pytest

from conftest import rel_err
from models import F5Model, F16, BF16, F32

pytestmark = pytest.mark.gpu
TOL = 1e-3


def run(hip, oracle, m, B, N, seed, steps=1):
    f5 = m.create(hip)
    rng = np.random.default_rng(seed)
    cat0, x, ts, rope = m.inputs(rng, B, N)
    hip.f5_begin(f5, B, N, cat0, rope)
    for _ in range(steps):
        got = hip.f5_step(f5, x, ts, B, N, m.mel)
        want = oracle.f5_step(m.ox, B, N, m.with_x(cat0, x, B), ts, rope)
        assert rel_err(got, want) < TOL, rel_err(got, want)
        x = rng.standard_normal(x.shape).astype(np.float32)  # the next Euler step's x; cat0 stays
        ts = rng.standard_normal(ts.shape).astype(np.float32)
    hip.f5_end(f5)
    return f5


@pytest.mark.parametrize("wtype,pe,B,N", [(F16, 0, 2, 70), (F16, 1, 1, 130), (BF16, 0, 2, 64), (F32, 2, 2, 33)])
def test_f5_step_small(hip, oracle, wtype, pe, B, N):
    m = F5Model(40 + wtype + pe, 128, 2, 4, mel=20, text=32, K=7, groups=4, pe_attn_head=pe, wtype=wtype)
    run(hip, oracle, m, B, N, seed=N, steps=2)


def test_f5_step_f16_row_path(hip, oracle):
    # dim 96 is not a multiple of 64: f16 linears take the f32-row GEMM (k_gemm_h16) with the same epilogues
    m = F5Model(47, 96, 2, 2, mel=20, text=32, K=7, groups=4, wtype=F16)
    run(hip, oracle, m, 2, 68, seed=5, steps=2)


def test_f5_step_full_width(hip, oracle):
    # the configs[3] widths (dim 1024, 16 x 64 heads, FFN 2048, mel 100, text 512, position conv K 31 / 16 groups)
    # with one block and 200 frames, so the oracle finishes in seconds
    m = F5Model(50, 1024, 1, 16, mel=100, text=512, K=31, groups=16, wtype=F16, std=0.02)
    run(hip, oracle, m, 2, 200, seed=3)


@pytest.mark.parametrize("B", [2, 1])
def test_f5_step_cfg4_shape(hip, oracle, B):
    # configs[3]'s benchmarked step shape: N = 1000 frames (the attention's last key tile holds 40 keys), B = 2 (CFG)
    # and B = 1, at the full widths; two of the 22 blocks (every block takes the same kernels and tiles, which depend
    # on the rows B N, not on the depth), so the 16-thread oracle finishes in about 10 s
    oracle.lib().vo_set_threads(16)
    m = F5Model(51, 1024, 2, 16, mel=100, text=512, K=31, groups=16, wtype=F16, std=0.02)
    run(hip, oracle, m, B, 1000, seed=4 + B)


def test_f5_step_wide_tiles_partial(hip, oracle):
    # dim 320 (5 x 64 heads) at B = 2, N = 1000: the q|k|v product (n 960) runs 64 x 128 tiles of 8 waves, 8 x 32 = 256
    # blocks, whose last column tile is half past n and whose tiles straddle the q|k / v boundary of the RoPE epilogue;
    # o (n 320) and the FFN (n 640) keep 64 x 64 tiles
    oracle.lib().vo_set_threads(16)
    m = F5Model(52, 320, 1, 5, mel=100, text=512, K=31, groups=16, wtype=F16, std=0.02)
    run(hip, oracle, m, 2, 1000, seed=9)


@pytest.mark.parametrize("wtype,hd,pe,B,N", [(F16, 32, 1, 2, 70), (F16, 48, 0, 1, 130), (BF16, 34, 2, 2, 33),
                                             (F32, 16, 0, 1, 64)])
def test_f5_step_head_dim_below_64(hip, oracle, wtype, hd, pe, B, N):
    # any even dim_head <= 64, as gpu_f5.cpp:211: q|k|v and to_out are padded per head to the attention tiles' 64
    # dims with zero rows / columns at create; RoPE rotates the model's own dims from its [N][hd/2] table
    m = F5Model(90 + hd, 128, 2, 4, dim_head=hd, mel=20, text=32, K=7, groups=4, pe_attn_head=pe, wtype=wtype)
    run(hip, oracle, m, B, N, seed=hd, steps=2)


def test_f5_rejects_bad_shapes(hip):
    for heads, hd in ((2, 80), (8, 33)):  # above 64, odd (gpu_f5.cpp:211)
        m = F5Model(60, 128, 1, heads, dim_head=hd, wtype=F16)
        with pytest.raises(hip.VoxHipError, match="head_dim"):
            m.create(hip)
    m = F5Model(61, 128, 1, 2, wtype=F16)
    f5 = m.create(hip)
    with pytest.raises(hip.VoxHipError, match="before begin"):
        hip.f5_step(f5, np.zeros((10, 20), np.float32), np.zeros(128, np.float32), 1, 10, 20)


@pytest.mark.parametrize("wtype", [F16, BF16, F32])
def test_f5_vocos(hip, oracle, wtype):
    # gpu_f5_vocos (gpu_f5.cpp:334-373): the Vocos backbone and head on the device against the oracle's restatement of
    # F5Model::vocode (f5.cpp:792-806); the embed conv's rows (K 7 x mel 20 = 140) are zero-padded to 144 on the device
    m = F5Model(70 + wtype, 128, 1, 2, mel=20, text=32, K=7, groups=4, wtype=wtype,
                vocos=dict(dim=64, inter=192, layers=2, out=34))
    f5 = m.create(hip)
    rng = np.random.default_rng(wtype)
    for T in (57, 9):
        mel = rng.standard_normal((T, 20)).astype(np.float32)
        got = hip.f5_vocos(f5, mel)
        want = oracle.vocos_head(m.vox, mel)
        assert got.shape == want.shape and rel_err(got, want) < TOL, (T, rel_err(got, want))


def test_f5_vocos_full_width(hip, oracle):
    # F5-TTS's Vocos widths (mel 100, dim 512, intermediate 1536, 8 blocks, head 2 x 513) on 100 frames
    m = F5Model(80, 128, 1, 2, mel=100, text=32, K=7, groups=4, wtype=F16,
                vocos=dict(dim=512, inter=1536, layers=8, out=1026))
    f5 = m.create(hip)
    mel = np.random.default_rng(8).standard_normal((100, 100)).astype(np.float32)
    got = hip.f5_vocos(f5, mel)
    want = oracle.vocos_head(m.vox, mel)
    assert rel_err(got, want) < TOL, rel_err(got, want)
    # a model created without Vocos reports it instead of running
    plain = F5Model(81, 128, 1, 2, wtype=F16).create(hip)
    with pytest.raises(hip.VoxHipError, match="Vocos"):
        hip.f5_vocos(plain, mel[:, :20])
