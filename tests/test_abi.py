"""The C-ABI library loads and exports every entry point include/voxhip.h declares (no GPU needed)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "voxhip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(voxhip_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("voxhip_init", "voxhip_upload", "voxhip_matmul", "voxhip_xfmr_create", "voxhip_seq_create",
                 "voxhip_xfmr_forward", "voxhip_xfmr_forward_pair", "voxhip_sample_logits", "voxhip_decode_dev"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from vox_amd import voxhip
    lib = ctypes.CDLL(voxhip.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares a signature for each of them too
    assert not [n for n in declared() if n not in voxhip.SIGNATURES]


def test_no_device_means_a_clean_error():
    # Without a GPU (this container) init fails with a message instead of crashing, and every call after it
    # reports failure; the product has no CPU fallback to hide behind.
    from vox_amd import voxhip
    if voxhip.device_count() > 0:
        import pytest
        pytest.skip("a HIP device is present")
    try:
        voxhip.init("hip:0")
        raise AssertionError("init succeeded without a device")
    except voxhip.VoxHipError as e:
        assert "HIP" in str(e) or "device" in str(e)
    assert voxhip.lib().voxhip_active() == 0
    assert voxhip.lib().voxhip_upload(None, 0) == -1


def test_dropin_library_exports_gpu_interface():
    # libvox_gpu_hip.so implements the reference's vox::gpu_* C++ interface (gpu.hpp:10-119, kernels.hpp:89-100)
    path = os.path.join(ROOT, "vox_amd", "libvox_gpu_hip.so")
    syms = os.popen(f"nm -DC --defined-only {path}").read().replace("[abi:cxx11]", "")
    for fn in ("vox::gpu_init(", "vox::gpu_upload(", "vox::gpu_matmul(", "vox::gpu_xfmr_create(", "vox::gpu_seq_create(",
               "vox::gpu_seq_free(", "vox::gpu_xfmr_forward(", "vox::gpu_xfmr_forward_hidden(", "vox::gpu_xfmr_forward_pair(",
               "vox::gpu_pred_frame(", "vox::gpu_enumerate(", "vox::gpu_mem_info(", "vox::gpu_stats(", "vox::gpu_list_devices(",
               "vox::gpu_set_vram_limit(", "vox::gpu_codec_create(", "vox::gpu_f5_create(", "vox::gpu_cosy_create(",
               "vox::gpu_gemm_choice(", "vox::gpu_active(", "vox::gpu_device_name("):
        assert fn in syms, fn
