"""The CosyVoice2 / Chatterbox flow estimator on the device (gpu_cosy_create / begin / step / end, gpu.hpp:100-119;
the CPU estimator cosyvoice.cpp:126-221, :839-863) against the oracle's vo_cosy_step.

Both sides consume the same stored weights: f32 convolutions in Conv::w layout, f16 / bf16 / q8 / f32 linears. The
device runs the causal convolutions on f32 MFMA (implicit im2col with K - 1 zero rows in front of each pass), the
LayerNorms in double like nn.cpp, f16 linears on the split-f16 matrix cores (all widths multiples of 64: the
pre-split path; otherwise the f32-row path), q8 / bf16 / f32 linears on the f32-activation GEMMs and attention on
split-f16 MFMA tiles, so the outputs differ from the oracle's by summation order, the dropped lo x lo terms (below
2^-22), libm ulps and the erf GELU against nn.cpp's erfc fit of it (1.2e-7 relative): the north star's 1e-3 for f32
activations with the `vox verify` metric.
"""
import numpy as np
import pytest

from conftest import rel_err
from models import CosyModel, F16, BF16, F32, Q8

pytestmark = pytest.mark.gpu
TOL = 1e-3


def run(hip, oracle, m, T, seed, steps=3):  # step 1 captures the graph, the rest replay it
    est = m.create(hip)
    rng = np.random.default_rng(seed)
    in0, x, tb = m.inputs(rng, T)
    hip.cosy_begin(est, T, in0)
    for _ in range(steps):
        got = hip.cosy_step(est, x, tb, T, m.M)
        want = oracle.cosy_step(m.ox, T, m.with_x(in0, x), tb)
        assert rel_err(got, want) < TOL, (T, rel_err(got, want))
        x = rng.standard_normal(x.shape).astype(np.float32)  # the next Euler step's x and time biases; in0 stays
        tb = (rng.standard_normal(tb.shape) * 0.5).astype(np.float32)
    hip.cosy_end(est)
    return est


@pytest.mark.parametrize("wtype,T", [(F16, 40), (F16, 97), (Q8, 64), (BF16, 33), (F32, 7)])
def test_cosy_step_small(hip, oracle, wtype, T):
    m = CosyModel(70 + wtype, M=8, C=64, heads=2, head_dim=64, n_mid=1, n_x=1, ff=128, wtype=wtype)
    run(hip, oracle, m, T, seed=T)


@pytest.mark.parametrize("wtype,hd,T", [(F16, 32, 40), (Q8, 32, 64), (F32, 48, 9), (BF16, 22, 33)])
def test_cosy_step_head_dim_below_64(hip, oracle, wtype, hd, T):
    # any even head_dim <= 64, as gpu_f5.cpp:425 (Chatterbox's estimator has 8 x 64, other checkpoints fewer dims):
    # the attention runs on heads padded with zero dims to 64 (q8 needs whole 32-column scale blocks)
    m = CosyModel(80 + hd, M=8, C=64, heads=4, head_dim=hd, n_mid=1, n_x=1, ff=128, wtype=wtype)
    run(hip, oracle, m, T, seed=hd)


def test_cosy_step_f16_row_path(hip, oracle):
    # ff 96 is not a multiple of 64: the f16 linears take the f32-row GEMM with the same epilogues
    m = CosyModel(75, M=8, C=64, heads=1, head_dim=64, n_mid=2, n_x=1, ff=96, wtype=F16)
    run(hip, oracle, m, 50, seed=2)


def test_cosy_step_one_frame(hip, oracle):
    # T = 1: every causal tap but the last reads the zero padding; attention over one key
    m = CosyModel(76, M=8, C=64, heads=2, head_dim=64, n_mid=1, n_x=1, ff=128, wtype=F16)
    run(hip, oracle, m, 1, seed=1)


def test_cosy_step_full_width(hip, oracle):
    # CosyVoice2's widths (mel 80, 256 channels, 8 x 64 heads, FFN 1024) with 2 mid blocks and 2 transformers per
    # level, 150 frames, so the oracle finishes in seconds
    m = CosyModel(77, M=80, C=256, heads=8, head_dim=64, n_mid=2, n_x=2, ff=1024, wtype=F16)
    run(hip, oracle, m, 150, seed=3, steps=1)


def test_cosy_begin_again_and_rejects(hip, oracle):
    m = CosyModel(78, M=8, C=64, heads=2, head_dim=96, n_mid=1, n_x=1, ff=128, wtype=F16)  # above 64 (gpu_f5.cpp:425)
    with pytest.raises(hip.VoxHipError, match="head_dim"):
        m.create(hip)
    m = CosyModel(78, M=8, C=64, heads=2, head_dim=48, n_mid=1, n_x=1, ff=128, wtype=Q8)  # q8 padding: 32-column blocks
    with pytest.raises(hip.VoxHipError, match="multiple of 32"):
        m.create(hip)
    m = CosyModel(79, M=8, C=64, heads=2, head_dim=64, n_mid=1, n_x=1, ff=128, wtype=F16)
    est = m.create(hip)
    with pytest.raises(hip.VoxHipError, match="before begin"):
        hip.cosy_step(est, np.zeros((4, 8), np.float32), np.zeros((3, 64), np.float32), 4, 8)
    rng = np.random.default_rng(9)
    for T in (70, 20):  # begin again with another length: the buffers follow
        in0, x, tb = m.inputs(rng, T)
        hip.cosy_begin(est, T, in0)
        got = hip.cosy_step(est, x, tb, T, m.M)
        assert rel_err(got, oracle.cosy_step(m.ox, T, m.with_x(in0, x), tb)) < TOL
    hip.cosy_end(est)
    with pytest.raises(hip.VoxHipError, match="before begin"):
        hip.cosy_step(est, x, tb, 20, 8)
