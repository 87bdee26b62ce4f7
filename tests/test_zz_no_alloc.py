"""voxhip_matmul_dev_noalloc, the entry point that allocates nothing: its split-K partial sums and once-quantized
input rows live in the library's fixed device array instead of buffers it allocates. Checked against voxhip_matmul
(the existing entry point, same kernels) on the same weights and rows, two calls in a row with the second smaller,
and against the library's allocation count (unchanged by the calls)."""
import numpy as np
import pytest

from conftest import rel_err
from models import make_mat

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4


# (type, rows, cols, first m, second m): Q8 int path with the quantized rows in the scratch (5..8 rows per pass); Q4
# in passes of 8 rows; F16 on the MFMA GEMM with K split into the scratch (16 output tiles, K 1024); BF16 on the GEMM
# then (3 rows) the f32 GEMV; F32 split K with a second call of one row
CASES = [(Q8, 4096, 1024, 8, 5), (Q4, 2048, 2048, 13, 6), (F16, 1000, 1024, 64, 9), (BF16, 300, 896, 200, 3),
         (F32, 512, 2048, 32, 1)]


@pytest.mark.parametrize("wt,rows,cols,m1,m2", CASES)
def test_matmul_dev_noalloc_matches_matmul(hip, wt, rows, cols, m1, m2):
    rng = np.random.default_rng(rows + cols + wt)
    data, scale, bias = make_mat(rng, wt, rows, cols, bias=True)
    h = hip.upload(hip.HostMat(wt, data, rows, cols, scale, bias))
    dx, dy = hip.DevBuf(m1 * cols * 4), hip.DevBuf(m1 * rows * 4)
    for m in (m1, m2):
        x = rng.standard_normal((m, cols)).astype(np.float32)
        want = hip.matmul(h, x)
        dx.upload(x)
        used = hip.mem_info().used
        hip.matmul_dev_noalloc(h, dx, m, dy)
        hip.sync()
        assert hip.mem_info().used == used  # the call allocated nothing
        got = dy.download((m, rows), np.float32)
        e = rel_err(got, want)
        print(f"type {wt} {rows}x{cols} m {m}: rel err {e:.2e}, identical {np.array_equal(got, want)}")
        assert e < 1e-5, (wt, m, e)
    dx.free()
    dy.free()
    hip.mat_free(h)


def test_matmul_dev_noalloc_rejects_bad_arguments(hip):
    rng = np.random.default_rng(3)
    data, scale, _ = make_mat(rng, Q8, 64, 256)
    h = hip.upload(hip.HostMat(Q8, data, 64, 256, scale, None))
    with pytest.raises(hip.VoxHipError, match="missing argument"):
        hip._check(hip.lib().voxhip_matmul_dev_noalloc(h, None, 2, None), "matmul_dev_noalloc")
    with pytest.raises(hip.VoxHipError, match="bad matrix handle"):
        hip._check(hip.lib().voxhip_matmul_dev_noalloc(10 ** 6, None, 1, None), "matmul_dev_noalloc")
    hip.mat_free(h)
