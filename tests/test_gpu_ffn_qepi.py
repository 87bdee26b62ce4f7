"""The FFN of 5-8 rows on the int path with the SwiGLU output quantized in the gate|up GEMV's epilogue
(EPI_SWIGLU_Q: one block of 16 waves holds the 64 interleaved gate|up rows of 32 outputs and quantizes them as
k_quant_rows would for the down pass) against the same passes with the separate k_quant_rows launch
(VOXHIP_FFN_QEPI=0). Both quantize the same floats with the same per-32-block arithmetic (kernels.cpp:515-523),
so prefill passes, B-session steps and the device-resident step give bit-identical states, caches and logits;
the oracle checks the states to the `vox verify` bar of 1e-3 (cli/main.cpp:796-803)."""
import os

import numpy as np
import pytest

from conftest import rel_err
from models import Model

pytestmark = pytest.mark.gpu

Q8, Q4 = 3, 4


def _run(hip, mdl, qepi, B, lens, pre_rows, x):
    os.environ["VOXHIP_FFN_QEPI"] = "1" if qepi else "0"
    try:
        xf = hip.xfmr_create(mdl.hx, "qepi%d" % qepi)
        head = hip.upload(mdl.head[1])
        seqs = [hip.seq_create(xf, 32) for _ in range(B)]
        for s, pre in zip(seqs, pre_rows):
            hip.forward(xf, s, 0, pre, 256)
        out, logits = hip.forward_steps(xf, seqs, lens, x, 256, head=head)
        dx, dout, dlog = hip.DevBuf(x.nbytes), hip.DevBuf(x.nbytes), hip.DevBuf(B * 300 * 4)
        try:
            dx.upload(x)
            for _ in range(2):  # the first call captures the step's graph, the second replays it
                hip.decode_steps_dev(xf, seqs, [n + 1 for n in lens], dx, dout, head, dlog, None, None)
            hip.sync()
            out_dev = dout.download(B * 256, np.float32).reshape(B, 256)
            log_dev = dlog.download(B * 300, np.float32).reshape(B, 300)
        finally:
            for bf in (dx, dout, dlog):
                bf.free()
        caches = [hip.seq_download(s, 1, n, 256) for s, n in zip(seqs, lens)]
        return out, logits, out_dev, log_dev, caches
    finally:
        os.environ.pop("VOXHIP_FFN_QEPI", None)


@pytest.mark.parametrize("wt", [Q8, Q4])
@pytest.mark.parametrize("B", [5, 8])
def test_swiglu_quant_epilogue_matches_quant_rows(hip, oracle, wt, B):
    mdl = Model(820 + wt, 2, 256, 4, 2, 128, 512, wtype=wt, head_rows=300)
    rng = np.random.default_rng(B)
    lens = [5, 8, 6, 7, 5, 8, 6, 7][:B]  # prefill passes of 5-8 rows take the same paths
    pre_rows = [rng.standard_normal((n, 256)).astype(np.float32) for n in lens]
    x = rng.standard_normal((B, 256)).astype(np.float32)
    fused = _run(hip, mdl, True, B, lens, pre_rows, x)
    apart = _run(hip, mdl, False, B, lens, pre_rows, x)
    for a, b in zip(fused[:4], apart[:4]):
        assert np.array_equal(a, b)
    for (ka, va), (kb, vb) in zip(fused[4], apart[4]):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # the B-session step against the oracle on each row's own cache
    out = fused[0]
    for b in range(B):
        kv = mdl.oracle_kv(32, kv_f16=1)
        oracle.transformer_forward(mdl.ox, kv, pre_rows[b])
        ref = oracle.transformer_forward(mdl.ox, kv, x[b:b + 1])
        assert rel_err(out[b], ref) < 1e-3, (b, rel_err(out[b], ref))
