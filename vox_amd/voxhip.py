"""ctypes binding of libvoxhip.so (the C ABI declared in include/voxhip.h).

The names and argument meaning mirror the reference's device interface (src/gpu.hpp, src/kernels.hpp:88-100):
upload -> gpu_upload, matmul -> gpu_matmul, xfmr_create -> gpu_xfmr_create, seq_create -> gpu_seq_create,
forward -> gpu_xfmr_forward, ... Failures raise VoxHipError with the library's last error (the reference
returns false and keeps the reason in gpu_stats().last_error).

There is no CPU fallback here: if the library is not built, or no gfx950 device is present, every call
raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvoxhip.so")

F32, F16, BF16, Q8, Q4 = 0, 1, 2, 3, 4


class VoxHipError(RuntimeError):
    pass


class Mat(C.Structure):
    _fields_ = [("type", C.c_int32), ("data", C.c_void_p), ("scale", C.c_void_p), ("rows", C.c_int64),
                ("cols", C.c_int64), ("bias", C.c_void_p)]


class DeviceInfo(C.Structure):
    _fields_ = [("index", C.c_int32), ("name", C.c_char * 256), ("type", C.c_char * 16), ("software", C.c_int32),
                ("unified_memory", C.c_int32), ("vram_total", C.c_uint64), ("vram_free", C.c_uint64),
                ("max_storage_range", C.c_uint64), ("subgroup_arith", C.c_int32), ("coop_matrix", C.c_int32),
                ("memory_budget", C.c_int32), ("api_version", C.c_uint32), ("vendor_id", C.c_uint32),
                ("driver_version", C.c_uint32)]


class Stats(C.Structure):
    _fields_ = [("mats_ok", C.c_int64), ("mats_failed", C.c_int64), ("bytes", C.c_uint64), ("bytes_failed", C.c_uint64)]


class MemInfo(C.Structure):
    _fields_ = [("used", C.c_uint64), ("limit", C.c_uint64), ("device_free", C.c_uint64), ("device_total", C.c_uint64),
                ("device_index", C.c_int32)]


class Layer(C.Structure):
    _fields_ = [(n, Mat) for n in ("q", "k", "v", "o", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("qn", "kn", "ln1", "ln2", "attn_scale", "mlp_scale")]


class XfmrDesc(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("layers", C.POINTER(Layer)), ("final_norm", C.c_void_p), ("hidden", C.c_int32),
                ("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32), ("inter", C.c_int32),
                ("eps", C.c_float), ("theta", C.c_double), ("window", C.c_int32), ("inv_freq", C.c_void_p)]


class SampleCfg(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32), ("repetition_penalty", C.c_float),
                ("key0", C.c_uint32), ("key1", C.c_uint32), ("frame", C.c_uint64), ("codebook", C.c_uint32),
                ("draw", C.c_uint32), ("suppress_from", C.c_int32), ("suppress_to", C.c_int32), ("eos_code", C.c_int32),
                ("block_eos", C.c_int32)]


class LmCfg(C.Structure):
    """voxhip_lm_cfg: CosyVoice2 LM sampling (CosyCfg top_p / top_k / win_size / tau_r, lm_generate bounds)."""
    _fields_ = [("top_p", C.c_float), ("top_k", C.c_int32), ("win_size", C.c_int32), ("tau_r", C.c_float),
                ("speech_tokens", C.c_int32), ("min_len", C.c_int32), ("max_len", C.c_int32), ("piece", C.c_uint32),
                ("seed", C.c_uint64)]


class F5Conv(C.Structure):
    _fields_ = [("w", C.c_void_p), ("b", C.c_void_p), ("cin", C.c_int32), ("cout", C.c_int32), ("K", C.c_int32),
                ("groups", C.c_int32)]


class F5Block(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("ada", "q", "k", "v", "o", "ff1", "ff2")]


class F5VBlock(C.Structure):
    _fields_ = [("dw", F5Conv), ("ln_w", C.c_void_p), ("ln_b", C.c_void_p), ("gamma", C.c_void_p), ("pw1", C.c_int32),
                ("pw2", C.c_int32)]


class F5Desc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "depth", "heads", "dim_head", "ff_mult", "mel_dim", "text_dim",
                                         "pe_attn_head", "in_proj", "norm_out", "proj_out")] + \
               [("blocks", C.POINTER(F5Block)), ("pos1", F5Conv), ("pos2", F5Conv)] + \
               [(n, C.c_int32) for n in ("vocos_dim", "vocos_inter", "vocos_out")] + [("v_embed", F5Conv)] + \
               [(n, C.c_void_p) for n in ("v_ln_w", "v_ln_b", "v_fln_w", "v_fln_b")] + \
               [("v_blocks", C.POINTER(F5VBlock)), ("n_vblocks", C.c_int32), ("v_head", C.c_int32)]


class CosyRes(C.Structure):
    _fields_ = [("c1", F5Conv), ("c2", F5Conv), ("res", F5Conv)] + [(n, C.c_void_p) for n in ("n1w", "n1b", "n2w", "n2b")]


class CosyX(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("n1w", "n1b", "n3w", "n3b")] + \
               [(n, C.c_int32) for n in ("q", "k", "v", "o", "ff1", "ff2", "ff_dim")]


class CosyDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("M", "C", "heads", "head_dim")] + \
               [("down_res", CosyRes), ("up_res", CosyRes), ("mid_res", C.POINTER(CosyRes)), ("n_mid", C.c_int32),
                ("down_x", C.POINTER(CosyX)), ("up_x", C.POINTER(CosyX)), ("mid_x", C.POINTER(CosyX)),
                ("n_down_x", C.c_int32), ("n_up_x", C.c_int32), ("mid_x_count", C.c_void_p)] + \
               [(n, F5Conv) for n in ("down_conv", "up_out", "final_conv", "final_proj")] + \
               [("fn_w", C.c_void_p), ("fn_b", C.c_void_p)]


class CodecConv(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("mat", "K", "cin", "cout", "dil")]


class CodecSnake(C.Structure):
    _fields_ = [("a", C.c_void_p), ("inv_b", C.c_void_p)]


class CodecUp(C.Structure):
    _fields_ = [("tr", C.c_int32), ("K", C.c_int32), ("tr_b", C.c_void_p), ("dw_w", C.c_void_p), ("dw_b", C.c_void_p),
                ("dw_K", C.c_int32), ("ln_w", C.c_void_p), ("ln_b", C.c_void_p), ("gamma", C.c_void_p), ("pw1", C.c_int32),
                ("pw2", C.c_int32)]


class CodecBlock(C.Structure):
    _fields_ = [("act", CodecSnake)] + [(n, C.c_int32) for n in ("tr", "K", "stride", "cin", "cout")] + \
               [("tr_b", C.c_void_p), ("a1", CodecSnake * 3), ("a2", CodecSnake * 3), ("c1", CodecConv * 3),
                ("c2", CodecConv * 3)]


class CodecDesc(C.Structure):
    _fields_ = [("codebook_dim", C.c_int32), ("latent", C.c_int32), ("pre_conv", CodecConv), ("pt_in", C.c_int32),
                ("pt_out", C.c_int32), ("pt", XfmrDesc), ("pt_mats", C.c_void_p), ("ups", C.POINTER(CodecUp)),
                ("n_ups", C.c_int32), ("conv0", CodecConv), ("blocks", C.POINTER(CodecBlock)), ("n_blocks", C.c_int32),
                ("final_act", CodecSnake), ("final_conv", CodecConv)]


KERNEL_CLASSES = ("qkv_gemv", "o_gemv", "gateup_gemv", "down_gemv", "head_gemv", "attention", "attn_combine", "qk_post", "sampler",
                  "ffn", "acc_fold", "quant_rows")


class BenchResult(C.Structure):
    _fields_ = [("ms_per_step", C.c_double), ("launch_ms_per_step", C.c_double), ("kernel_ms_per_step", C.c_double),
                ("step_bytes", C.c_double),
                ("kernels_per_step", C.c_int32), ("n_classes", C.c_int32), ("kernel_stamped", C.c_int32),
                ("class_ms", C.c_double * len(KERNEL_CLASSES)), ("class_bytes", C.c_double * len(KERNEL_CLASSES)),
                ("class_launches", C.c_int32 * len(KERNEL_CLASSES))]


UPLOADED_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int32, C.c_int32)

# every symbol include/voxhip.h declares, with (restype, argtypes)
_P, _I, _I32, _I64, _F, _D, _U32, _U64, _S = (C.c_void_p, C.c_int, C.c_int32, C.c_int64, C.c_float, C.c_double, C.c_uint32,
                                            C.c_uint64, C.c_size_t)
SIGNATURES = {
    "voxhip_device_count": (_I, []),
    "voxhip_device_info_get": (_I, [_I, C.POINTER(DeviceInfo)]),
    "voxhip_init": (_I, [C.c_char_p, C.c_char_p, _S]),
    "voxhip_active": (_I, []),
    "voxhip_profile_report": (C.c_char_p, []),
    "voxhip_device_name": (C.c_char_p, []),
    "voxhip_stats_get": (None, [C.POINTER(Stats)]),
    "voxhip_last_error": (C.c_char_p, []),
    "voxhip_set_vram_limit": (None, [_U64]),
    "voxhip_mem_info_get": (None, [C.POINTER(MemInfo)]),
    "voxhip_upload": (_I, [C.POINTER(Mat), _I]),
    "voxhip_matmul": (_I, [_I, _P, _I64, _P]),
    "voxhip_mat_shape": (_I, [_I, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "voxhip_xfmr_create": (_I, [C.POINTER(XfmrDesc), C.c_char_p, _I, UPLOADED_FN, _P]),
    "voxhip_seq_create": (_I, [_I, _I64]),
    "voxhip_seq_free": (None, [_I]),
    "voxhip_xfmr_forward": (_I, [_I, _I, _I64, _P, _I64, _P, _I, _I, _P]),
    "voxhip_xfmr_forward_hidden": (_I, [_I, _I, _I64, _P, _I64, _P]),
    "voxhip_xfmr_forward_layers": (_I, [_I, _I, _I64, _P, _I64, _I32, _I32, _P]),
    "voxhip_xfmr_forward_pair": (_I, [_I, _I, _I, _I64, _P, _I, _P, _P]),
    "voxhip_xfmr_forward_steps": (_I, [_I, _P, _P, _I64, _P, _P, _I, _P]),
    "voxhip_sample_logits": (_I, [_P, _I32, C.POINTER(SampleCfg), _P, _I32, C.POINTER(C.c_int32)]),
    "voxhip_dev_alloc": (_P, [_S]),
    "voxhip_dev_free": (None, [_P]),
    "voxhip_memcpy_h2d": (_I, [_P, _P, _S]),
    "voxhip_memcpy_d2h": (_I, [_P, _P, _S]),
    "voxhip_sync": (_I, []),
    "voxhip_decode_dev": (_I, [_I, _I, _I64, _P, _I64, _P, _I, _P, C.POINTER(SampleCfg), _P]),
    "voxhip_decode_steps_dev": (_I, [_I, _P, _P, _I64, _P, _P, _I, _P, C.POINTER(SampleCfg), _P]),
    "voxhip_f5_create": (_I, [C.POINTER(F5Desc)]),
    "voxhip_f5_begin": (_I, [_I, _I, _I, _P, _P]),
    "voxhip_f5_step": (_I, [_I, _P, _P, _P]),
    "voxhip_f5_end": (_I, [_I]),
    "voxhip_f5_vocos": (_I, [_I, _P, _I, _P]),
    "voxhip_f5_vocos_out": (_I, [_I, _P]),
    "voxhip_cosy_create": (_I, [C.POINTER(CosyDesc)]),
    "voxhip_codec_create": (_I, [C.POINTER(CodecDesc)]),
    "voxhip_codec_state_new": (_I, [_I]),
    "voxhip_codec_state_clone": (_I, [_I]),
    "voxhip_codec_state_free": (_I, [_I]),
    "voxhip_codec_forward": (_I, [_I, _I, _P, _I, _P, _P]),
    "voxhip_codec_spf": (_I, [_I, _P]),
    "voxhip_cosy_begin": (_I, [_I, _I, _P]),
    "voxhip_cosy_step": (_I, [_I, _P, _P, _P]),
    "voxhip_cosy_end": (_I, [_I]),
    "voxhip_lm_sample_dev": (_I, [_P, C.c_int32, C.POINTER(LmCfg), _I64, _P, C.c_int32, _P, _P]),
    "voxhip_lm_generate": (_I, [_I, _I, _P, _I64, _I, _I, C.POINTER(LmCfg), _P, _P, _P]),
    "voxhip_pred_frame": (_I, [_I, _I, _P, _I, _P, _I, _P, _I, C.POINTER(SampleCfg), _P]),
    "voxhip_mat_synthetic": (_I, [_I32, _I64, _I64, _U64, _U32, _F, _F, _I]),
    "voxhip_mat_download": (_I, [_I, _P, _P, _P]),
    "voxhip_mat_free": (_I, [_I]),
    "voxhip_mat_gather": (_I, [_I, _P, C.c_int64, _P]),
    "voxhip_matmul_dev_noalloc": (_I, [_I, _P, C.c_int64, _P]),
    "voxhip_convt": (_I, [_I, _I32, _I32, _I32, _I32, _P, _P, _I32, _P]),
    "voxhip_xfmr_create_from_mats": (_I, [C.POINTER(XfmrDesc), _P, C.c_char_p]),
    "voxhip_seq_fill_synthetic": (_I, [_I, _I64, _U64, _U32, _F, _F]),
    "voxhip_seq_download": (_I, [_I, _I32, _I64, _P, _P]),
    "voxhip_quantize_q8_dev": (_I, [_P, _I64, _I64, _P, _P]),
    "voxhip_quantize_q4_dev": (_I, [_P, _I64, _I64, _P, _P]),
    "voxhip_quantize_act_dev": (_I, [_P, _I64, _P, _P]),
    "voxhip_bench_decode": (_I, [_I, _I, _I64, _P, _I, C.POINTER(SampleCfg), _P, _I, _I, C.POINTER(BenchResult)]),
    "voxhip_bench_decode_steps": (_I, [_I, _P, _P, _I64, _P, _I, _P, _P, _I, _I, C.POINTER(BenchResult)]),
    "voxhip_bench_gemv_q8": (_I, [_I64, _I64, _I, _I, _I, C.POINTER(C.c_double)]),
    "voxhip_bench_copy": (_I, [_I64, _I, _I, C.POINTER(C.c_double)]),
    "voxhip_selftest_split_f16": (_I, [_I64, C.POINTER(C.c_int64)]),
    "voxhip_bench_gemm_hh": (_I, [_I64, _I64, _I64, _I, _I, _I, _I, C.POINTER(C.c_double), _P]),
    "voxhip_bench_ffn_q8": (_I, [_I64, _I64, _I, _I, _I, C.POINTER(C.c_double), _P]),
}

_lib = None


def lib():
    """Loads libvoxhip.so; raises when it is not built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VoxHipError(f"{LIB_PATH} is not built: run __graft_entry__.build() or python -m vox_amd.build")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _err(what):
    raise VoxHipError(f"{what}: {lib().voxhip_last_error().decode(errors='replace')}")


def _check(rc, what):
    if not rc:
        _err(what)
    return rc


def _handle(h, what):
    if h < 0:
        _err(what)
    return h


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- device, init
def device_count():
    return lib().voxhip_device_count()


def init(device="hip:0"):
    err = C.create_string_buffer(512)
    if not lib().voxhip_init(device.encode(), err, 512):
        raise VoxHipError(err.value.decode(errors="replace"))


def device_name():
    return lib().voxhip_device_name().decode()


def mem_info():
    m = MemInfo()
    lib().voxhip_mem_info_get(C.byref(m))
    return m


def profile_report():
    """The VOX_PROFILE=gpu table of the launches booked so far (empty when the profile is off)."""
    return lib().voxhip_profile_report().decode()


def stats():
    s = Stats()
    lib().voxhip_stats_get(C.byref(s))
    return s


# ---------------------------------------------------------------- matrices
class HostMat:
    """A weight matrix in the reference layout (vox::Mat): keeps its arrays alive for the ctypes view."""

    def __init__(self, wtype, data, rows, cols, scale=None, bias=None):
        self.type, self.rows, self.cols = wtype, int(rows), int(cols)
        self.data = np.ascontiguousarray(data)
        self.scale = None if scale is None else f32(scale)
        self.bias = None if bias is None else f32(bias)
        self.c = Mat(wtype, self.data.ctypes.data, None if self.scale is None else self.scale.ctypes.data, self.rows, self.cols,
                     None if self.bias is None else self.bias.ctypes.data)


def upload(*parts):
    arr = (Mat * len(parts))(*[p.c for p in parts])
    return _handle(lib().voxhip_upload(arr, len(parts)), "upload")


def matmul(mat, x):
    x = f32(x)
    m = 1 if x.ndim == 1 else x.shape[0]
    rows, cols = C.c_int64(), C.c_int64()
    _check(lib().voxhip_mat_shape(mat, C.byref(rows), C.byref(cols)), "mat_shape")
    y = np.empty((m, rows.value), np.float32)
    _check(lib().voxhip_matmul(mat, _p(x), m, _p(y)), "matmul")
    return y


def mat_shape(mat):
    rows, cols = C.c_int64(), C.c_int64()
    _check(lib().voxhip_mat_shape(mat, C.byref(rows), C.byref(cols)), "mat_shape")
    return rows.value, cols.value


SYN_BIAS, SYN_F16_SCALES = 1, 2


def mat_synthetic(wtype, rows, cols, seed, stream, mean=0.0, std=0.02, bias=False, f16_scales=False):
    flags = (SYN_BIAS if bias else 0) | (SYN_F16_SCALES if f16_scales else 0)
    return _handle(lib().voxhip_mat_synthetic(wtype, rows, cols, seed, stream, mean, std, flags), "mat_synthetic")


def mat_download(mat, wtype):
    rows, cols = mat_shape(mat)
    if wtype == Q8:
        data = np.empty((rows, cols), np.int8)
    elif wtype == Q4:
        data = np.empty((rows, cols // 2), np.uint8)
    elif wtype == F32:
        data = np.empty((rows, cols), np.float32)
    else:
        data = np.empty((rows, cols), np.uint16)
    scale = np.empty((rows, cols // 32), np.float32) if wtype in (Q8, Q4) else None
    bias = np.zeros(rows, np.float32)  # stays zero for a matrix without bias
    _check(lib().voxhip_mat_download(mat, _p(data), _p(scale), _p(bias)), "mat_download")
    return data, scale, bias


def matmul_dev_noalloc(mat, d_x, m, d_y):
    """matmul on device rows d_x [m][cols] -> d_y [m][rows] with the library's fixed scratch (no allocation)."""
    _check(lib().voxhip_matmul_dev_noalloc(mat, d_x.ptr, m, d_y.ptr), "matmul_dev_noalloc")


def mat_gather(mat, ids, cols):
    """mat_gather of rows ids on the device -> f32 [len(ids)][cols]."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, cols), np.float32)
    _check(lib().voxhip_mat_gather(mat, _p(ids), ids.size, _p(out)), "mat_gather")
    return out


def mat_free(mat):
    _check(lib().voxhip_mat_free(mat), "mat_free")


class ConvT:
    """nn::ConvT (nn.hpp:64-71; ConvTranspose1d, groups 1) with its weights on the device. load() takes PyTorch's
    weight [cin][cout][K] and lays it out as ConvT::load does (nn.cpp:205-215): K cout rows of cin, row k cout + o;
    forward(x [T][cin]) returns y [(T - 1) stride - 2 pad + K + out_pad][cout] (nn.cpp:217-245)."""

    def __init__(self):
        self.cin = self.cout = 0
        self.K = self.stride = 1
        self.pad = self.out_pad = 0
        self.b = None
        self.mat = -1

    def load(self, weight, bias, stride, pad, out_pad=0):
        w = np.asarray(weight, np.float32)
        self.cin, self.cout, self.K = (int(d) for d in w.shape)
        self.stride, self.pad, self.out_pad = int(stride), int(pad), int(out_pad)
        self.b = None if bias is None else f32(bias)
        rows = np.ascontiguousarray(w.transpose(2, 1, 0).reshape(self.K * self.cout, self.cin))
        self.mat = upload(HostMat(F32, rows, self.K * self.cout, self.cin))
        return self

    def out_len(self, T):
        return (T - 1) * self.stride - 2 * self.pad + self.K + self.out_pad

    def forward(self, x):
        return convt(self.mat, self.K, self.stride, self.pad, self.out_pad, self.b, x)


def convt(mat, K, stride, pad, out_pad, bias, x):
    """voxhip_convt: the transposed conv of x [T][cin] with the matrix `mat` (K cout rows of cin) -> y [To][cout]."""
    x = f32(x)
    T = x.shape[0]
    rows, _ = mat_shape(mat)
    cout = rows // K
    To = (T - 1) * stride - 2 * pad + K + out_pad
    y = np.empty((max(To, 1), cout), np.float32)
    b = None if bias is None else f32(bias)
    _check(lib().voxhip_convt(mat, K, stride, pad, out_pad, _p(b), _p(x), T, _p(y)), "convt")
    return y


# ---------------------------------------------------------------- transformer
class XfmrHost:
    """Host description of a Qwen3-shaped transformer (vox::TransformerW) for xfmr_create."""

    def __init__(self, layers, final_norm, hidden, heads, kv_heads, head_dim, inter, eps, theta, inv_freq):
        self.layers = layers  # list of dicts: q,k,v,o,gate,up,down -> HostMat (or None for *_from_mats), qn,kn,ln1,ln2 -> arrays
        self.final_norm = f32(final_norm)
        self.inv_freq = f32(inv_freq)
        arr = (Layer * len(layers))()
        for i, L in enumerate(layers):
            for n in ("q", "k", "v", "o", "gate", "up", "down"):
                if L.get(n) is not None:
                    setattr(arr[i], n, L[n].c)
            for n in ("qn", "kn", "ln1", "ln2"):
                v = L.get(n)
                setattr(arr[i], n, None if v is None else v.ctypes.data)
        self._arr = arr
        self.c = XfmrDesc(len(layers), arr, self.final_norm.ctypes.data, hidden, heads, kv_heads, head_dim, inter, eps, theta, 0,
                          self.inv_freq.ctypes.data)
        self.hidden, self.heads, self.kv_heads, self.head_dim, self.inter = hidden, heads, kv_heads, head_dim, inter


def xfmr_create(desc, name="xfmr", n_layers=-1, uploaded=None):
    cb = UPLOADED_FN(uploaded) if uploaded else UPLOADED_FN()
    h = lib().voxhip_xfmr_create(C.byref(desc.c), name.encode(), n_layers, cb, None)
    return _handle(h, "xfmr_create")


def xfmr_create_from_mats(desc, mats, name="xfmr"):
    ids = np.ascontiguousarray(mats, dtype=np.int32)
    return _handle(lib().voxhip_xfmr_create_from_mats(C.byref(desc.c), _p(ids), name.encode()), "xfmr_create_from_mats")


def seq_create(xfmr, capacity):
    return _handle(lib().voxhip_seq_create(xfmr, capacity), "seq_create")


def seq_free(seq):
    lib().voxhip_seq_free(seq)


def seq_fill_synthetic(seq, length, seed, stream, mean=0.0, std=1.0):
    _check(lib().voxhip_seq_fill_synthetic(seq, length, seed, stream, mean, std), "seq_fill_synthetic")


def seq_download(seq, layer, length, kd):
    k = np.empty((length, kd), np.float32)
    v = np.empty((length, kd), np.float32)
    _check(lib().voxhip_seq_download(seq, layer, length, _p(k), _p(v)), "seq_download")
    return k, v


def forward(xfmr, seq, pos0, x, hidden, in_proj=-1, head=-1):
    x = f32(x)
    m = x.shape[0]
    out = np.empty(hidden, np.float32)
    head_out = None
    if head >= 0:
        head_out = np.empty(mat_shape(head)[0], np.float32)
    _check(lib().voxhip_xfmr_forward(xfmr, seq, pos0, _p(x), m, _p(out), in_proj, head, _p(head_out)), "xfmr_forward")
    return out, head_out


def forward_hidden(xfmr, seq, pos0, x, hidden):
    x = f32(x)
    out = np.empty((x.shape[0], hidden), np.float32)
    _check(lib().voxhip_xfmr_forward_hidden(xfmr, seq, pos0, _p(x), x.shape[0], _p(out)), "xfmr_forward_hidden")
    return out


def forward_layers(xfmr, seq, pos0, x, first, count):
    x = f32(x)
    out = np.empty_like(x)
    _check(lib().voxhip_xfmr_forward_layers(xfmr, seq, pos0, _p(x), x.shape[0], first, count, _p(out)), "xfmr_forward_layers")
    return out


def forward_pair(xfmr, seq0, seq1, pos, x2, hidden, head=-1):
    x2 = f32(x2)
    out = np.empty((2, hidden), np.float32)
    head_out = np.empty((2, mat_shape(head)[0]), np.float32) if head >= 0 else None
    _check(lib().voxhip_xfmr_forward_pair(xfmr, seq0, seq1, pos, _p(x2), head, _p(out), _p(head_out)), "xfmr_forward_pair")
    return out, head_out


def forward_steps(xfmr, seqs, pos, x, hidden, head=-1):
    x = f32(x)
    B = x.shape[0]
    s = np.ascontiguousarray(seqs, dtype=np.int32)
    p = np.ascontiguousarray(pos, dtype=np.int64)
    out = np.empty((B, hidden), np.float32)
    head_out = np.empty((B, mat_shape(head)[0]), np.float32) if head >= 0 else None
    _check(lib().voxhip_xfmr_forward_steps(xfmr, _p(s), _p(p), B, _p(x), _p(out), head, _p(head_out)), "xfmr_forward_steps")
    return out, head_out


# ---------------------------------------------------------------- sampling
def sample_cfg(temperature=0.9, top_p=1.0, top_k=50, repetition_penalty=1.0, seed=0, frame=0, codebook=0, draw=0,
               suppress_from=0, suppress_to=0, eos_code=-1, block_eos=0):
    return SampleCfg(temperature, top_p, top_k, repetition_penalty, seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF, frame, codebook,
                     draw, suppress_from, suppress_to, eos_code, block_eos)


def sample_logits(logits, cfg, history=None):
    l = f32(logits)
    h = None if history is None else np.ascontiguousarray(history, dtype=np.int32)
    out = C.c_int32(-1)
    _check(lib().voxhip_sample_logits(_p(l), l.size, C.byref(cfg), _p(h), 0 if h is None else h.size, C.byref(out)),
           "sample_logits")
    return out.value


# ---------------------------------------------------------------- device-resident
class DevBuf:
    def __init__(self, nbytes):
        self.nbytes = nbytes
        self.ptr = lib().voxhip_dev_alloc(nbytes)
        if not self.ptr:
            _err("dev_alloc")

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        _check(lib().voxhip_memcpy_h2d(self.ptr, _p(arr), arr.nbytes), "memcpy_h2d")

    def download(self, shape, dtype):
        out = np.empty(shape, dtype)
        _check(lib().voxhip_memcpy_d2h(_p(out), self.ptr, out.nbytes), "memcpy_d2h")
        return out

    def free(self):
        if self.ptr:
            lib().voxhip_dev_free(self.ptr)
            self.ptr = None


def decode_dev(xfmr, seq, pos0, d_x, m=1, d_out=None, head=-1, d_logits=None, cfg=None, d_token=None):
    _check(lib().voxhip_decode_dev(xfmr, seq, pos0, d_x.ptr, m, None if d_out is None else d_out.ptr, head,
                                   None if d_logits is None else d_logits.ptr, None if cfg is None else C.byref(cfg),
                                   None if d_token is None else d_token.ptr), "decode_dev")


def decode_steps_dev(xfmr, seqs, pos, d_x, d_out=None, head=-1, d_logits=None, cfgs=None, d_tokens=None):
    """One token for each of B sequences at its own position (device-resident, one captured graph)."""
    sq = np.ascontiguousarray(seqs, dtype=np.int32)
    ps = np.ascontiguousarray(pos, dtype=np.int64)
    carr = None
    if cfgs is not None:
        carr = (SampleCfg * len(cfgs))(*cfgs)
    _check(lib().voxhip_decode_steps_dev(xfmr, _p(sq), _p(ps), sq.size, d_x.ptr, None if d_out is None else d_out.ptr, head,
                                         None if d_logits is None else d_logits.ptr, carr,
                                         None if d_tokens is None else d_tokens.ptr), "decode_steps_dev")


def lm_cfg(top_p=0.8, top_k=25, win_size=10, tau_r=0.1, speech_tokens=6561, min_len=0, max_len=256, piece=0, seed=1234):
    return LmCfg(top_p, top_k, win_size, tau_r, speech_tokens, min_len, max_len, piece, seed)


def lm_sample_dev(d_logits, n, cfg, step, d_decoded=None, n_decoded=0, d_logp=None):
    """lm_logp + the RAS trial loop of one step on device logits [n]; returns the token."""
    tok = C.c_int32()
    _check(lib().voxhip_lm_sample_dev(d_logits.ptr, n, C.byref(cfg), step, None if d_decoded is None else d_decoded.ptr,
                                      n_decoded, None if d_logp is None else d_logp.ptr, C.byref(tok)), "lm_sample_dev")
    return tok.value


def lm_generate(xfmr, seq, x, head, speech_emb, cfg, want_logp=False):
    """lm_begin's prefill of x [n][hidden] + lm_generate on the device: (tokens, logp [steps][V] or None)."""
    x = f32(x)
    tokens = np.zeros(max(cfg.max_len, 1), np.int32)
    V = mat_shape(head)[0]
    logp = np.zeros((max(cfg.max_len, 1), V), np.float32) if want_logp else None
    nt = C.c_int32()
    _check(lib().voxhip_lm_generate(xfmr, seq, _p(x), x.shape[0], head, speech_emb, C.byref(cfg), _p(tokens),
                                    None if logp is None else _p(logp), C.byref(nt)), "lm_generate")
    n = nt.value
    if logp is not None:
        rows = min(n + 1, cfg.max_len)
        logp = logp[:rows]
    return tokens[:n], logp


def pred_frame(xfmr, seq, in2, in_proj, heads, embs, cfg):
    """gpu_pred_frame: the code predictor's frame on the device. in2 [2][din]; heads / embs lists of matrix handles
    (in_proj -1 for none); cfg a SampleCfg (temperature, top_k, top_p, seed, frame). Returns codes [len(heads) + 1]
    with codes[0] = 0 (the talker's code is the caller's)."""
    in2 = f32(in2)
    h = np.ascontiguousarray(heads, dtype=np.int32)
    e = np.ascontiguousarray(embs, dtype=np.int32) if len(embs) else np.zeros(1, np.int32)
    codes = np.zeros(len(heads) + 1, np.int32)
    _check(lib().voxhip_pred_frame(xfmr, seq, _p(in2), in_proj, _p(h), h.size, _p(e), len(embs), C.byref(cfg), _p(codes)),
           "pred_frame")
    return codes


def f5_create(dim, depth, heads, dim_head, ff_mult, mel_dim, text_dim, pe_attn_head, in_proj, norm_out, proj_out, blocks,
              pos1, pos2, vocos=None):
    """gpu_f5_create: blocks = list of dicts ada,q,k,v,o,ff1,ff2 -> matrix handles; pos1/pos2 = (w [groups][cout/groups]
    [K][cin/groups] f32, bias or None, cin, cout, K, groups). vocos: dict dim, inter, out, embed (a conv tuple), ln_w,
    ln_b, fln_w, fln_b (arrays), head (handle), blocks = list of dicts dw (conv tuple, w [C][K]), ln_w, ln_b, gamma,
    pw1, pw2 (handles)."""
    arr = (F5Block * len(blocks))(*[F5Block(*[b[n] for n in ("ada", "q", "k", "v", "o", "ff1", "ff2")]) for b in blocks])
    keep = []

    def conv(c):
        w, b, cin, cout, K, groups = c
        w = f32(w)
        b = None if b is None else f32(b)
        keep.extend([w, b])
        return F5Conv(_p(w), _p(b), cin, cout, K, groups)

    def vec(a):
        a = None if a is None else f32(a)
        keep.append(a)
        return _p(a)
    d = F5Desc(dim, depth, heads, dim_head, ff_mult, mel_dim, text_dim, pe_attn_head, in_proj, norm_out, proj_out, arr,
               conv(pos1), conv(pos2))
    if vocos:
        vb = (F5VBlock * max(1, len(vocos["blocks"])))()
        for i, b in enumerate(vocos["blocks"]):
            vb[i] = F5VBlock(conv(b["dw"]), vec(b["ln_w"]), vec(b["ln_b"]), vec(b["gamma"]), b["pw1"], b["pw2"])
        keep.append(vb)
        d.vocos_dim, d.vocos_inter, d.vocos_out = vocos["dim"], vocos["inter"], vocos["out"]
        d.v_embed = conv(vocos["embed"])
        d.v_ln_w, d.v_ln_b, d.v_fln_w, d.v_fln_b = (vec(vocos[n]) for n in ("ln_w", "ln_b", "fln_w", "fln_b"))
        d.v_blocks, d.n_vblocks, d.v_head = vb, len(vocos["blocks"]), vocos["head"]
    return _handle(lib().voxhip_f5_create(C.byref(d)), "f5_create")


def f5_vocos(f5, mel):
    """gpu_f5_vocos: mel [T][mel_dim] -> the Vocos head output [T][vocos_out]."""
    mel = f32(mel)
    vout = C.c_int32()
    _check(lib().voxhip_f5_vocos_out(f5, C.byref(vout)), "f5_vocos_out")
    out = np.empty((mel.shape[0], vout.value), np.float32)
    _check(lib().voxhip_f5_vocos(f5, _p(mel), mel.shape[0], _p(out)), "f5_vocos")
    return out


def f5_begin(f5, B, N, cat0, rope):
    _check(lib().voxhip_f5_begin(f5, B, N, _p(f32(cat0)), _p(f32(rope))), "f5_begin")


def f5_step(f5, x, ts, B, N, mel):
    out = np.empty((B * N, mel), np.float32)
    _check(lib().voxhip_f5_step(f5, _p(f32(x)), _p(f32(ts)), _p(out)), "f5_step")
    return out


def f5_end(f5):
    _check(lib().voxhip_f5_end(f5), "f5_end")


def cosy_create(M, C_, heads, head_dim, down_res, up_res, mid_res, down_x, up_x, mid_x, down_conv, up_out, final_conv,
                final_proj, fn_w, fn_b):
    """gpu_cosy_create: resnets = dicts c1, c2, res (conv tuples (w [cout][K][cin] f32, bias or None, cin, cout, K, 1)),
    n1w, n1b, n2w, n2b; transformer blocks = dicts n1w, n1b, n3w, n3b, q, k, v, o, ff1, ff2 (handles), ff_dim;
    mid_x a list of such lists, one per mid resnet."""
    keep = []

    def vec(a):
        a = f32(a)
        keep.append(a)
        return _p(a)

    def conv(c):
        w, b, cin, cout, K, groups = c
        return F5Conv(vec(w), None if b is None else vec(b), cin, cout, K, groups)

    def res(r):
        return CosyRes(conv(r["c1"]), conv(r["c2"]), conv(r["res"]), *[vec(r[n]) for n in ("n1w", "n1b", "n2w", "n2b")])

    def xs(lst):
        arr = (CosyX * max(1, len(lst)))()
        for i, x in enumerate(lst):
            arr[i] = CosyX(*[vec(x[n]) for n in ("n1w", "n1b", "n3w", "n3b")],
                           *[x[n] for n in ("q", "k", "v", "o", "ff1", "ff2", "ff_dim")])
        keep.append(arr)
        return arr
    mids = (CosyRes * max(1, len(mid_res)))(*[res(r) for r in mid_res])
    counts = np.array([len(v) for v in mid_x] or [0], np.int32)
    keep += [mids, counts]
    d = CosyDesc(M, C_, heads, head_dim, res(down_res), res(up_res), mids, len(mid_res), xs(down_x), xs(up_x),
                 xs([x for v in mid_x for x in v]), len(down_x), len(up_x), _p(counts), conv(down_conv), conv(up_out),
                 conv(final_conv), conv(final_proj), vec(fn_w), vec(fn_b))
    return _handle(lib().voxhip_cosy_create(C.byref(d)), "cosy_create")


def cosy_begin(cosy, T, in0):
    """gpu_cosy_begin: in0 [2 T][4 M], the x columns zero."""
    _check(lib().voxhip_cosy_begin(cosy, T, _p(f32(in0))), "cosy_begin")


def cosy_step(cosy, x, tb, T, M):
    """gpu_cosy_step: x [T][M], tb [2 + n_mid][C] -> [2 T][M] (conditional pass, then unconditional)."""
    out = np.empty((2 * T, M), np.float32)
    _check(lib().voxhip_cosy_step(cosy, _p(f32(x)), _p(f32(tb)), _p(out)), "cosy_step")
    return out


def cosy_end(cosy):
    _check(lib().voxhip_cosy_end(cosy), "cosy_end")


def codec_create(codebook_dim, latent, pre_conv, pt_in, pt_out, pt, pt_mats, ups, conv0, blocks, final_act, final_conv):
    """gpu_codec_create: convs = (handle, K, cin, cout, dil); snakes = (a, inv_b) arrays; pt = dict of the pre-
    transformer (hidden, heads, kv_heads, head_dim, inter, eps, theta, window, inv_freq, final_norm, layers = list of
    dicts ln1, ln2, attn_scale, mlp_scale); pt_mats [layers][7] handles; ups = dicts tr, K, tr_b, dw_w, dw_b, dw_K, ln_w,
    ln_b, gamma, pw1, pw2; blocks = dicts act, tr, K, stride, cin, cout, tr_b, a1, a2 (3 snakes), c1, c2 (3 convs)."""
    keep = []

    def vec(a):
        a = f32(a)
        keep.append(a)
        return _p(a)

    def snake(sn):
        return CodecSnake(vec(sn[0]), vec(sn[1]))
    lay = (Layer * len(pt["layers"]))()
    for i, L in enumerate(pt["layers"]):
        for n in ("ln1", "ln2", "attn_scale", "mlp_scale"):
            if L.get(n) is not None:
                setattr(lay[i], n, vec(L[n]))
    keep.append(lay)
    xd = XfmrDesc(len(pt["layers"]), lay, vec(pt["final_norm"]), pt["hidden"], pt["heads"], pt["kv_heads"], pt["head_dim"],
                  pt["inter"], pt["eps"], pt["theta"], pt["window"], vec(pt["inv_freq"]))
    ids = np.ascontiguousarray(pt_mats, np.int32)
    keep.append(ids)
    ua = (CodecUp * max(1, len(ups)))()
    for i, u in enumerate(ups):
        ua[i] = CodecUp(u["tr"], u["K"], vec(u["tr_b"]), vec(u["dw_w"]), vec(u["dw_b"]), u["dw_K"], vec(u["ln_w"]),
                        vec(u["ln_b"]), vec(u["gamma"]), u["pw1"], u["pw2"])
    ba = (CodecBlock * max(1, len(blocks)))()
    for i, b in enumerate(blocks):
        blk = ba[i]
        blk.act = snake(b["act"])
        blk.tr, blk.K, blk.stride, blk.cin, blk.cout, blk.tr_b = b["tr"], b["K"], b["stride"], b["cin"], b["cout"], vec(b["tr_b"])
        for u in range(3):
            blk.a1[u], blk.a2[u] = snake(b["a1"][u]), snake(b["a2"][u])
            blk.c1[u], blk.c2[u] = CodecConv(*b["c1"][u]), CodecConv(*b["c2"][u])
    keep += [ua, ba]
    d = CodecDesc(codebook_dim, latent, CodecConv(*pre_conv), pt_in, pt_out, xd, _p(ids), ua, len(ups), CodecConv(*conv0), ba,
                  len(blocks), snake(final_act), CodecConv(*final_conv))
    return _handle(lib().voxhip_codec_create(C.byref(d)), "codec_create")


def codec_spf(codec):
    v = C.c_int32()
    _check(lib().voxhip_codec_spf(codec, C.byref(v)), "codec_spf")
    return v.value


def codec_state_new(codec):
    return _handle(lib().voxhip_codec_state_new(codec), "codec_state_new")


def codec_state_clone(state):
    return _handle(lib().voxhip_codec_state_clone(state), "codec_state_clone")


def codec_state_free(state):
    _check(lib().voxhip_codec_state_free(state), "codec_state_free")


def codec_forward(codec, state, z):
    """gpu_codec_forward: z [F][codebook_dim] (F <= 16) -> pcm [F spf]."""
    z = f32(z)
    out = np.empty(z.shape[0] * codec_spf(codec), np.float32)
    n = C.c_int64()
    _check(lib().voxhip_codec_forward(codec, state, _p(z), z.shape[0], _p(out), C.byref(n)), "codec_forward")
    return out[:n.value]


def sync():
    _check(lib().voxhip_sync(), "sync")


def quantize_q8_dev(w):
    w = f32(w)
    rows, cols = w.shape
    dw, dq, ds = DevBuf(w.nbytes), DevBuf(rows * cols), DevBuf(rows * cols // 32 * 4)
    try:
        dw.upload(w)
        _check(lib().voxhip_quantize_q8_dev(dw.ptr, rows, cols, dq.ptr, ds.ptr), "quantize_q8_dev")
        return dq.download((rows, cols), np.int8), ds.download((rows, cols // 32), np.float32)
    finally:
        for b in (dw, dq, ds):
            b.free()


def quantize_q4_dev(w):
    w = f32(w)
    rows, cols = w.shape
    dw, dq, ds = DevBuf(w.nbytes), DevBuf(rows * cols // 2), DevBuf(rows * cols // 32 * 4)
    try:
        dw.upload(w)
        _check(lib().voxhip_quantize_q4_dev(dw.ptr, rows, cols, dq.ptr, ds.ptr), "quantize_q4_dev")
        return dq.download((rows, cols // 2), np.uint8), ds.download((rows, cols // 32), np.float32)
    finally:
        for b in (dw, dq, ds):
            b.free()


def quantize_act_dev(x):
    x = f32(x).ravel()
    n = x.size
    dx, dq, ds = DevBuf(x.nbytes), DevBuf(n), DevBuf(n // 32 * 4)
    try:
        dx.upload(x)
        _check(lib().voxhip_quantize_act_dev(dx.ptr, n, dq.ptr, ds.ptr), "quantize_act_dev")
        return dq.download(n, np.int8), ds.download(n // 32, np.float32)
    finally:
        for b in (dx, dq, ds):
            b.free()


def bench_decode(xfmr, seq, pos0, d_x, head, cfg, d_token, warmup, steps):
    r = BenchResult()
    _check(lib().voxhip_bench_decode(xfmr, seq, pos0, d_x.ptr, head, None if cfg is None else C.byref(cfg),
                                     None if d_token is None else d_token.ptr, warmup, steps, C.byref(r)), "bench_decode")
    return r


def bench_decode_steps(xfmr, seqs, pos, d_x, head, cfgs, d_tokens, warmup, steps):
    """voxhip_bench_decode for a step of len(seqs) sessions (decode_steps_dev)."""
    B = len(seqs)
    s = np.ascontiguousarray(seqs, np.int32)
    p = np.ascontiguousarray(pos, np.int64)
    arr = (SampleCfg * B)(*cfgs) if cfgs is not None else None
    r = BenchResult()
    _check(lib().voxhip_bench_decode_steps(xfmr, _p(s), _p(p), B, d_x.ptr, head, arr,
                                           None if d_tokens is None else d_tokens.ptr, warmup, steps, C.byref(r)),
           "bench_decode_steps")
    return r


def bench_gemv_q8(rows, cols, copies, warmup, iters):
    ms = C.c_double()
    _check(lib().voxhip_bench_gemv_q8(rows, cols, copies, warmup, iters, C.byref(ms)), "bench_gemv_q8")
    return ms.value


def bench_gemm_hh(m, n, K, q8=False, tile=0, warmup=3, iters=20, out=False):
    """Average microseconds of one split-f16 MFMA GEMM launch on an (m, n, K) product (tile 0: the library's policy,
    1..4 a forced block tile); with out, also y [m][n] of the last launch."""
    us = C.c_double()
    y = np.empty((m, n), np.float32) if out else None
    _check(lib().voxhip_bench_gemm_hh(m, n, K, int(bool(q8)), tile, warmup, iters, C.byref(us),
                                      y.ctypes.data if out else None), "bench_gemm_hh")
    return (us.value, y) if out else us.value


def selftest_split_f16(pairs):
    """Pairs (of `pairs` pseudo-random f32 pairs) whose packed f16 split differs from hi = f16(x), lo = f16(x - hi)."""
    n = C.c_int64()
    _check(lib().voxhip_selftest_split_f16(pairs, C.byref(n)), "selftest_split_f16")
    return n.value


def bench_copy(nbytes, warmup, iters):
    """Average ms of one device copy of nbytes (read nbytes + write nbytes)."""
    ms = C.c_double()
    _check(lib().voxhip_bench_copy(nbytes, warmup, iters, C.byref(ms)), "bench_copy")
    return ms.value


def bench_ffn_q8(hidden, inter, copies, warmup, iters, check=False):
    """Average microseconds of one q8 FFN block (two kernels) over `copies` rotating weight sets; with check, also
    (x, gamma, out) of copy 0's block applied once to x."""
    us = C.c_double()
    chk = np.zeros((3, hidden), np.float32) if check else None
    _check(lib().voxhip_bench_ffn_q8(hidden, inter, copies, warmup, iters, C.byref(us), None if chk is None else _p(chk)),
           "bench_ffn_q8")
    return (us.value, chk[0], chk[1], chk[2]) if check else us.value
