"""The constants of the device range guards, read from the kernel sources and checked against the limits they
guard (IEEE f16 through numpy, int64 through exact integers). No GPU needed.

- split_f16 (vh_common.hpp) flags a finite value whose f16 rounds to infinity: that must be exactly |x| >= 65520,
  while 65504 (the largest f16) and everything below 65520 split into finite halves with hi + lo == x in f32;
- f32 weights take the split kernel only below kF32SplitMaxW (voxhip_runtime.hip): 2^10 w must then round to a
  finite f16, and lo must keep x to the f32 product's accuracy;
- fix_of (vh_gemv.hpp) clamps a term to +-lim units: with at most 1024 groups plus the bias term, every partial
  sum, and the sum of the kAccCopies planes, must stay inside int64.
"""
import os
import re

import numpy as np

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vox_amd", "csrc")


def _src(name):
    with open(os.path.join(CSRC, name)) as f:
        return f.read()


def _split(x):
    x = np.float32(x)
    hi = np.float16(x)
    lo = np.float16(x - np.float32(hi))
    return hi, lo


def test_f16_split_threshold():
    # the rule split_f16 applies: hi infinite while x finite
    assert "__builtin_isinf(float(hi)) && !__builtin_isinf(x)" in _src("vh_common.hpp")
    with np.errstate(over="ignore"):
        for x in (65504.0, 65519.99, -65519.99, 1.0e4, 3.14159):
            hi, lo = _split(x)
            assert np.isfinite(hi) and np.isfinite(lo)
            assert abs(np.float64(hi) + np.float64(lo) - np.float64(np.float32(x))) <= abs(np.float64(np.float32(x))) * 2.0 ** -21
        for x in (65520.0, -65520.0, 1e5, 3e38):
            assert np.isinf(np.float16(np.float32(x)))


def test_f32_weight_split_bound():
    m = re.search(r"constexpr float kF32SplitMaxW = ([0-9.]+)f;", _src("voxhip_runtime.hip"))
    wmax = float(m.group(1))
    scale = float(re.search(r"constexpr float kWs = ([0-9.]+)f", _src("vh_gemm.hpp")).group(1))
    assert scale == 1024.0
    # every |w| below the bound splits into finite halves after scaling; the bound itself is below the first
    # weight that overflows (65520 / 1024 = 63.98...)
    with np.errstate(over="ignore"):
        below = np.nextafter(np.float32(wmax), np.float32(0))
        assert np.isfinite(np.float16(np.float32(below * scale)))
        assert np.isfinite(np.float16(np.float32(wmax * scale)))
        assert np.isinf(np.float16(np.float32(64.0 * scale)))
    assert wmax * scale < 65520.0


def test_fixed_point_sum_bound():
    src = _src("vh_gemv.hpp")
    lim = float(re.search(r"const float lim = ([0-9.]+)f;", src).group(1))
    one = float(re.search(r"constexpr float kFixOne = ([0-9.]+)f;", src).group(1))
    copies = int(re.search(r"constexpr int kAccCopies = (\d+);", _src("vh_types.hpp")).group(1))
    assert one == 2.0 ** 32 and lim == 2.0 ** 50
    # the most terms one accumulator row receives: I / 32 <= 1024 groups (ffn_shape_ok) plus one bias term, each
    # of either sign; the planes are then added in int64 too
    max_terms = 1024 + 1
    assert "I <= 32 * 1024" in _src("vh_ffn.hip")
    assert max_terms * int(lim) < 2 ** 63
    assert max_terms * int(lim) * 1 < 2 ** 63 // copies * copies  # any split of the terms over the planes
    # float(t) of the clamp is exact, so the clamp is the integer the bound assumes
    assert float(np.float32(lim)) == lim
