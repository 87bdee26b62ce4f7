"""The reference's planner selects this backend: vox::make_plan (resources.cpp:496-586) runs on the GpuDeviceInfo
that gpu_enumerate (vox_amd/csrc/gpu_hip.cpp, libvox_gpu_hip.so) builds from a recorded MI355X property set
(tests/golden/mi355x_props.json), and must place the Qwen3-TTS stages on the GPU. The checker (oracle/_ref/plan_check,
tests/cpp/plan_check.cpp) links the reference's resources.cpp, so it exists only where the reference sources do."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "oracle", "_ref", "plan_check")


@pytest.mark.skipif(not os.path.exists(CHECK), reason="oracle/_ref/plan_check is built only where /root/reference exists")
def test_make_plan_selects_the_mi355x():
    d = json.load(open(os.path.join(ROOT, "tests", "golden", "mi355x_props.json")))
    major, minor = d["major"], d["minor"]
    runtime = int(d["hip_version"].replace(".", "0", 1).replace(".", ""))  # "7.0.51831" -> 70051831 (hipRuntimeGetVersion)
    args = [CHECK, d["hip_name"], d["gcnArchName"], str(d["totalGlobalMem"]), str(d["free"]), str(d["integrated"]),
            str(major), str(minor), str(runtime)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all passed" in r.stdout
    assert "device: vulkan:0 (AMD Instinct MI350 series (MI350X / MI355X) (gfx950" in r.stdout
