"""Range guards of the device arithmetic, through the C ABI.

The split-f16 matrix products keep an f32 activation as two f16 halves (hi = f16(a), lo = f16(a - hi)), which cannot
hold |a| >= 65520; the f32-weight product scales the weights by 2^10 before the same split, so it cannot hold
|w| >= 64; the fused one-row FFN sums its down product in fixed point (+-2^18 per term). The reference computes all
of these in f32 (kernels.cpp:337-412, :515-538), so the device must not return a different value where it cannot
represent one:
- f32 weights with max |w| >= 63 are routed at upload to the f32 matrix cores, with the reference's results;
- an activation or a down term outside its range fails the call (the reference backend's convention: false / -1,
  the reason in last_error, and the engine computes that call on the CPU), and the next call runs normally.
"""
import numpy as np
import pytest

from conftest import rel_err
from models import Model

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4


def test_wide_f32_weights_take_f32_products(hip, oracle):
    # 16 rows on the MFMA GEMM over f32 weights up to ~250 in magnitude (and one exactly 64): the split kernel's
    # 2^10-scaled halves would overflow to inf; the f32 kernel gives the reference's products
    rng = np.random.default_rng(7)
    rows, cols = 192, 256
    w = (rng.standard_normal((rows, cols)) * 50).astype(np.float32)
    w[3, 5] = 64.0
    b = rng.standard_normal(rows).astype(np.float32)
    h = hip.upload(hip.HostMat(F32, w, rows, cols, None, b))
    x = rng.standard_normal((16, cols)).astype(np.float32)
    y = hip.matmul(h, x)
    want = oracle.matmul(oracle.Mat(F32, w, rows, cols, None, b), x)
    assert np.all(np.isfinite(y))
    assert rel_err(y, want) < 1e-5, rel_err(y, want)
    # the same matrix scaled into range stays on the split-f16 kernel and agrees too
    h2 = hip.upload(hip.HostMat(F32, w / 8, rows, cols, None, b))
    assert rel_err(hip.matmul(h2, x), oracle.matmul(oracle.Mat(F32, w / 8, rows, cols, None, b), x)) < 1e-5


def test_activation_beyond_f16_fails_the_call(hip, oracle):
    rng = np.random.default_rng(8)
    rows, cols = 128, 256
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    h = hip.upload(hip.HostMat(F16, w.astype(np.float16).view(np.uint16), rows, cols, None, None))
    x = rng.standard_normal((16, cols)).astype(np.float32)
    M = oracle.Mat(F16, w.astype(np.float16).view(np.uint16), rows, cols, None, None)
    assert rel_err(hip.matmul(h, x), oracle.matmul(M, x)) < 1e-5
    big = x.copy()
    big[5, 17] = 1e5  # beyond f16: the split product would give inf - inf
    with pytest.raises(hip.VoxHipError, match="outside the device arithmetic's range"):
        hip.matmul(h, big)
    edge = x.copy()
    edge[5, 17] = 65504.0  # the largest f16 still splits exactly
    assert rel_err(hip.matmul(h, edge), oracle.matmul(M, edge)) < 1e-5
    # the word is cleared: the next call runs normally
    assert rel_err(hip.matmul(h, x), oracle.matmul(M, x)) < 1e-5


def test_fused_ffn_term_beyond_fixed_point_fails_the_call(hip, oracle):
    # FFN 4x hidden takes the fused one-row FFN, whose down terms are summed in fixed point (+-2^18 per term). With
    # the down block scales raised 1e7-fold the terms reach ~1e6: the step fails instead of returning clamped sums,
    # and the same model with the two-GEMV FFN (f32 sums, as the reference) matches the oracle. (A NaN input does not
    # get there: the reference's int8 activation quantizer, and the device's, turn it into 0, kernels.cpp:515-523.)
    import os
    mdl = Model(61, 2, 256, 4, 2, 64, 1024, wtype=Q8)
    for L in mdl.hx.layers:
        L["down"].scale *= np.float32(1e7)  # shared with the oracle's matrices (the same arrays)
    assert all(np.shares_memory(L["down"].scale, oL["down"].scale) for L, oL in zip(mdl.hx.layers, mdl.ox.layers))
    x = np.random.default_rng(9).standard_normal((1, 256)).astype(np.float32)
    ref = oracle.transformer_forward(mdl.ox, mdl.oracle_kv(8, kv_f16=1), x)
    assert np.all(np.isfinite(ref))
    xf = hip.xfmr_create(mdl.hx, "range_ffn")
    with pytest.raises(hip.VoxHipError, match="fused-FFN term"):
        hip.forward(xf, hip.seq_create(xf, 8), 0, x, 256)
    os.environ["VOXHIP_FFN_FUSED"] = "0"
    try:
        xf2 = hip.xfmr_create(mdl.hx, "range_ffn_two_gemv")
    finally:
        os.environ.pop("VOXHIP_FFN_FUSED", None)
    out, _ = hip.forward(xf2, hip.seq_create(xf2, 8), 0, x, 256)
    assert rel_err(out, ref) < 1e-3, rel_err(out, ref)
