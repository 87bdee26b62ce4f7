"""VOX_PROFILE=gpu: the per-launch GPU profile of the reference's Vulkan backend (gpu_vulkan.cpp:62-87, :312-326),
on HIP events. Run in a child process, since the variable is read when the library initialises the device."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r'''
import sys, numpy as np
sys.path[:0] = [ROOT, ROOT + "/oracle", ROOT + "/tests"]
from vox_amd import voxhip as hip
from models import Model
from conftest import rel_err
import pyoracle as po
hip.init("hip:0")
mdl = Model(5, 2, 256, 4, 2, 64, 512, wtype=hip.Q8, head_rows=64)
xf = hip.xfmr_create(mdl.hx, "talker")
seq = hip.seq_create(xf, 16)
kv = mdl.oracle_kv(16, kv_f16=1)
x = np.random.default_rng(1).standard_normal((3, 256)).astype(np.float32)
out, _ = hip.forward(xf, seq, 0, x, 256)                       # eager launches, results unchanged
assert rel_err(out, po.transformer_forward(mdl.ox, kv, x)) < 1e-3
for p in range(3, 6):                                          # device-resident steps: booked at sync
    d = hip.DevBuf(256 * 4); d.upload(x[0]); hip.decode_dev(xf, seq, p, d, 1); hip.sync(); d.free()
h = hip.upload(hip.HostMat(hip.F32, np.ones((64, 256), np.float32), 64, 256))
hip.matmul(h, np.ones((16, 256), np.float32))
print(hip.profile_report(), flush=True)
'''.replace("ROOT", repr(ROOT))


def test_vox_profile_gpu_table():
    env = dict(os.environ, VOX_PROFILE="gpu")
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-3000:]
    rep = r.stdout
    print(rep)
    assert rep.startswith("[vox gpu profile]") and "GPU busy" in rep and "stage/kernel" in rep
    rows = [l.split() for l in rep.splitlines()[2:] if l.strip()]
    labels = {row[0]: row for row in rows}
    # the transformer's launches under its name, the GEMM under matmul; calls and times positive, shares add up
    assert any(k.startswith("talker/k_gemv_int<") for k in labels), list(labels)[:10]
    assert any(k.startswith("talker/k_attn") for k in labels), list(labels)[:10]
    assert any(k.startswith("matmul/k_gemm_") for k in labels), list(labels)[:10]
    assert all(int(row[-4]) > 0 and float(row[-3]) > 0 for row in rows)
    assert abs(sum(float(row[-1].rstrip("%")) for row in rows) - 100.0) < 1.0
    # and the same table on stderr at exit
    assert "[vox gpu profile]" in r.stderr
