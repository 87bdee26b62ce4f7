"""The Qwen3-TTS codec decoder on the device (gpu_codec_create / state_new / state_clone / state_free / forward,
gpu.hpp:53-60; the chain of gpu_codec.cpp:400-556 and the CPU codec_forward, qwen3.cpp:390-480) against the oracle's
vo_codec_forward, which is bit-exact with the reference's own Qwen3Weights::codec_forward.

z comes from the oracle's quantizer, as the reference's GPU path takes it from the CPU. The device runs the streaming
and transposed convolutions and the linears on the f32 MFMA GEMM (f32 / f16 / bf16 weights, the oracle holding the
same rounded values), the pre-transformer's projections on the GEMV / GEMM paths of matmul, its attention over an
f32 ring of the window, so the samples differ by summation order and libm ulps: the north star's 1e-3 for f32
activations (`vox verify`'s metric; the samples lie in [-1, 1]).
"""
import numpy as np
import pytest

from conftest import rel_err
from models import CodecModel, F16, BF16, F32

pytestmark = pytest.mark.gpu
TOL = 1e-3


def decode(hip, oracle, m, codec, chunks, seed):
    rng = np.random.default_rng(seed)
    z = oracle.codec_quantize(m.ox, m.codes(rng, sum(chunks)))
    st = hip.codec_state_new(codec)
    ost = oracle.CodecState(m.ox)
    f0 = 0
    for n in chunks:
        got = hip.codec_forward(codec, st, z[f0:f0 + n])
        want = oracle.codec_forward(ost, z[f0:f0 + n])
        assert got.shape == want.shape and rel_err(got, want) < TOL, (f0, n, rel_err(got, want))
        f0 += n
    return st, ost, z


@pytest.mark.parametrize("wtype", [F32, F16, BF16])
def test_codec_stream(hip, oracle, wtype):
    # 48 frames in calls of 1..16: the histories, tails and the ring (21 slots for window 5) wrap several times; a call
    # is a graph per (frame count, buffer parity), so the repeated (3, even) and (1, odd) calls replay one
    m = CodecModel(30 + wtype, wround=wtype)
    codec = m.create(hip, wtype)
    assert hip.codec_spf(codec) == m.spf
    st, _, _ = decode(hip, oracle, m, codec, [3, 1, 16, 5, 7, 8, 3, 3, 1, 1], seed=wtype)
    hip.codec_state_free(st)


def test_codec_clone_and_states(hip, oracle):
    # a cloned state continues like the original (cloned after an odd number of calls, so from the second buffers);
    # two states decode independently
    m = CodecModel(40)
    codec = m.create(hip)
    st, ost, _ = decode(hip, oracle, m, codec, [6, 4, 2], seed=1)
    z = oracle.codec_quantize(m.ox, m.codes(np.random.default_rng(2), 9))
    cl = hip.codec_state_clone(st)
    ocl = ost.clone()
    a = hip.codec_forward(codec, st, z)
    b = hip.codec_forward(codec, cl, z)
    assert np.array_equal(a, b)
    assert rel_err(a, oracle.codec_forward(ocl, z)) < TOL
    fresh = hip.codec_state_new(codec)
    assert rel_err(hip.codec_forward(codec, fresh, z[:5]), oracle.codec_forward(oracle.CodecState(m.ox), z[:5])) < TOL
    for s in (st, cl, fresh):
        hip.codec_state_free(s)
    with pytest.raises(hip.VoxHipError, match="bad codec state"):
        hip.codec_forward(codec, st, z[:1])
    with pytest.raises(hip.VoxHipError, match="16 frames"):
        hip.codec_forward(codec, hip.codec_state_new(codec), np.zeros((17, m.cc["codebook_dim"]), np.float32))


def test_codec_wider(hip, oracle):
    # Qwen3-TTS's structure at reduced widths: upsample ratios [2, 2], decoder rates [8, 5, 4, 3] (1920 samples per
    # frame), window 72 (ring 88), 4 x 64 heads; 100 frames in calls of 16 and 4 wrap the ring
    cc = dict(codebook_size=64, hidden_size=256, latent_dim=128, num_attention_heads=4, num_key_value_heads=4, head_dim=64,
              sliding_window=72, intermediate_size=512, layer_scale_initial_scale=0.01, rms_norm_eps=1e-5,
              num_hidden_layers=2, num_quantizers=4, upsample_rates=[8, 5, 4, 3], upsampling_ratios=[2, 2],
              decoder_dim=256, codebook_dim=64, rope_theta=10000.0)
    m = CodecModel(50, cc)
    codec = m.create(hip)
    assert m.spf == 1920
    decode(hip, oracle, m, codec, [16] * 6 + [4], seed=3)
