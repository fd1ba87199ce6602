"""Shared helpers for the tests: library loading, synthetic model writers, metrics.

The synthetic models are random-init bf16 safetensors directories in the
reference's on-disk layout (tensor names of iris_transformer_flux.c:5349-5497 and
iris_transformer_zimage.c:2024-2395). Values come from the seeded generator of
include/iris_synth.h, so the reference build, the oracle and the HIP library all
see identical weights.
"""
import ctypes
import hashlib
import json
import os
import struct

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libiris_ref.so")
HIP_SO = os.path.join(ROOT, "iris.c_amd", "libiris_hip.so")

FP = ctypes.POINTER(ctypes.c_float)
IP = ctypes.POINTER(ctypes.c_int)
U16P = ctypes.POINTER(ctypes.c_uint16)

_libs = {}


def oracle():
    """The oracle: CPU restatement of the reference path (test infrastructure)."""
    if "oracle" not in _libs:
        lib = ctypes.CDLL(ORACLE_SO)
        lib.orc_flux_load.restype = ctypes.c_void_p
        lib.orc_flux_create_synth.restype = ctypes.c_void_p
        lib.orc_flux_create_synth.argtypes = [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_float, ctypes.c_uint64]
        lib.orc_flux_forward.restype = ctypes.c_void_p
        lib.orc_flux_forward_refs.restype = ctypes.c_void_p
        lib.orc_zi_load.restype = ctypes.c_void_p
        lib.orc_zi_create_synth.restype = ctypes.c_void_p
        lib.orc_zi_forward.restype = ctypes.c_void_p
        lib.orc_official_schedule.restype = ctypes.c_void_p
        lib.orc_zimage_schedule.restype = ctypes.c_void_p
        lib.orc_init_noise.restype = ctypes.c_void_p
        lib.orc_blas_info.restype = ctypes.c_char_p
        lib.orc_qwen3_load.restype = ctypes.c_void_p
        lib.orc_qwen3_load.argtypes = [ctypes.c_char_p]
        lib.orc_qwen3_create_synth.restype = ctypes.c_void_p
        lib.orc_qwen3_create_synth.argtypes = [ctypes.c_int] * 6 + [ctypes.c_uint64]
        lib.orc_qwen3_free.argtypes = [ctypes.c_void_p]
        lib.orc_qwen3_set_mode.argtypes = [ctypes.c_void_p, ctypes.c_int]
        lib.orc_qwen3_forward.restype = ctypes.c_void_p
        lib.orc_qwen3_forward.argtypes = [ctypes.c_void_p, IP, IP, ctypes.c_int, ctypes.c_int]
        lib.iris_synth_seed.restype = ctypes.c_uint64
        lib.iris_synth_seed.argtypes = [ctypes.c_uint64, ctypes.c_char_p]
        lib.iris_synth_fill_bf16.argtypes = [U16P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64,
                                             ctypes.c_float, ctypes.c_float]
        lib.iris_synth_fill_f32.argtypes = [FP, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64,
                                            ctypes.c_float, ctypes.c_float]
        lib.orc_vae_load.restype = ctypes.c_void_p
        lib.orc_vae_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        lib.orc_vae_create_synth.restype = ctypes.c_void_p
        lib.orc_vae_create_synth.argtypes = [ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_uint64]
        lib.orc_vae_free.argtypes = [ctypes.c_void_p]
        lib.orc_vae_encode.argtypes = [ctypes.c_void_p, FP, ctypes.c_int, ctypes.c_int, FP]
        lib.orc_vae_decode.argtypes = [ctypes.c_void_p, FP, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, FP,
                                       ctypes.c_int]
        _libs["oracle"] = lib
        bind_blas(lib)
    return _libs["oracle"]


class GemmProblem(ctypes.Structure):
    _fields_ = [("A", ctypes.c_void_p), ("W", ctypes.c_void_p), ("out", ctypes.c_void_p), ("vec", ctypes.c_void_p),
                ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int), ("lda", ctypes.c_int),
                ("ldw", ctypes.c_int), ("ldo", ctypes.c_int), ("epi", ctypes.c_int),
                ("A2", ctypes.c_void_p), ("W2", ctypes.c_void_p), ("K2", ctypes.c_int), ("lda2", ctypes.c_int),
                ("ldw2", ctypes.c_int)]


class KernelTime(ctypes.Structure):
    """iris_kernel_time_t (include/iris_hip.h)"""
    _fields_ = [("kernel", ctypes.c_char_p), ("grid", ctypes.c_longlong), ("calls", ctypes.c_int),
                ("total_ms", ctypes.c_double), ("min_ms", ctypes.c_double), ("max_ms", ctypes.c_double)]


class NormArgs(ctypes.Structure):
    _fields_ = [("x", ctypes.c_void_p), ("ldx", ctypes.c_int), ("out", ctypes.c_void_p), ("ldo", ctypes.c_int),
                ("out_bf16", ctypes.c_int), ("rows", ctypes.c_int), ("cols", ctypes.c_int), ("mode", ctypes.c_int),
                ("eps", ctypes.c_float), ("split", ctypes.c_int), ("period", ctypes.c_int),
                ("shiftA", ctypes.c_void_p), ("scaleA", ctypes.c_void_p), ("wA", ctypes.c_void_p),
                ("shiftB", ctypes.c_void_p), ("scaleB", ctypes.c_void_p), ("wB", ctypes.c_void_p)]


class QkPrepArgs(ctypes.Structure):
    _fields_ = [("qkv", ctypes.c_void_p), ("ld_qkv", ctypes.c_int), ("col_k", ctypes.c_int), ("col_v", ctypes.c_int),
                ("q_out", ctypes.c_void_p), ("k_out", ctypes.c_void_p), ("vt_out", ctypes.c_void_p),
                ("ld_vt", ctypes.c_int), ("rows", ctypes.c_int), ("heads", ctypes.c_int),
                ("wqA", ctypes.c_void_p), ("wkA", ctypes.c_void_p), ("wqB", ctypes.c_void_p), ("wkB", ctypes.c_void_p),
                ("split", ctypes.c_int), ("cos_t", ctypes.c_void_p), ("sin_t", ctypes.c_void_p),
                ("period", ctypes.c_int), ("eps", ctypes.c_float), ("kv_heads", ctypes.c_int),
                ("kcos_t", ctypes.c_void_p), ("ksin_t", ctypes.c_void_p)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("vt", ctypes.c_void_p), ("o", ctypes.c_void_p),
                ("ld_q", ctypes.c_int), ("ld_k", ctypes.c_int), ("ld_vt", ctypes.c_int), ("ld_o", ctypes.c_int),
                ("sq", ctypes.c_int), ("sk", ctypes.c_int), ("heads", ctypes.c_int), ("batch", ctypes.c_int),
                ("q_bstride", ctypes.c_longlong), ("k_bstride", ctypes.c_longlong),
                ("vt_bstride", ctypes.c_longlong), ("o_bstride", ctypes.c_longlong),
                ("scale", ctypes.c_float), ("kv_lo0", ctypes.c_int), ("kv_hi0", ctypes.c_int),
                ("kv_lo1", ctypes.c_int), ("kv_hi1", ctypes.c_int), ("causal", ctypes.c_int),
                ("kv_group", ctypes.c_int), ("bias_from", ctypes.c_int), ("key_bias", ctypes.c_float),
                ("qn_wA", ctypes.c_void_p), ("qn_wB", ctypes.c_void_p), ("qn_split", ctypes.c_int),
                ("qn_eps", ctypes.c_float), ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
                ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_size_t), ("rope_pos", ctypes.c_void_p),
                ("rope_axis", ctypes.c_void_p), ("rope_axis_len", ctypes.c_int)]


class Conv3x3(ctypes.Structure):
    """iris_conv3x3_t (include/iris_hip.h)"""
    _fields_ = [("inp", ctypes.c_void_p), ("wt", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("H", ctypes.c_int), ("W", ctypes.c_int), ("cin", ctypes.c_int),
                ("cout", ctypes.c_int), ("up", ctypes.c_int), ("ldo", ctypes.c_int), ("epi", ctypes.c_int),
                ("splits", ctypes.c_int), ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_size_t),
                ("gn_part", ctypes.c_void_p), ("gn_groups", ctypes.c_int)]


class IrisImage(ctypes.Structure):
    """iris_image (reference iris.h:73-78, include/iris_vae.h)"""
    _fields_ = [("width", ctypes.c_int), ("height", ctypes.c_int), ("channels", ctypes.c_int),
                ("data", ctypes.POINTER(ctypes.c_uint8))]


class IrisRef(ctypes.Structure):
    _fields_ = [("latent", FP), ("h", ctypes.c_int), ("w", ctypes.c_int), ("t_offset", ctypes.c_int)]


def hip():
    """The product: the HIP build's C ABI (iris.c_amd/libiris_hip.so). Fails
    loudly when it is missing: there is no fallback path."""
    if "hip" not in _libs:
        if not os.path.exists(HIP_SO):
            raise RuntimeError(f"{HIP_SO} is not built (python -c 'import __graft_entry__ as g; g.build()')")
        lib = ctypes.CDLL(HIP_SO)
        vp = ctypes.c_void_p
        lib.iris_hip_malloc.restype = vp
        lib.iris_hip_malloc.argtypes = [ctypes.c_size_t]
        lib.iris_hip_free.argtypes = [vp]
        lib.iris_hip_memcpy_h2d.argtypes = [vp, vp, ctypes.c_size_t]
        lib.iris_hip_memcpy_d2h.argtypes = [vp, vp, ctypes.c_size_t]
        lib.iris_hip_memset.argtypes = [vp, ctypes.c_int, ctypes.c_size_t]
        lib.iris_hip_last_error.restype = ctypes.c_char_p
        lib.iris_hip_device_name.restype = ctypes.c_char_p
        lib.iris_hip_event_elapsed_ms.restype = ctypes.c_float
        lib.iris_hip_attention_workspace_bytes.restype = ctypes.c_size_t
        lib.iris_hip_gemv.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_hip_euler.argtypes = [vp, vp, vp, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_size_t]
        lib.iris_hip_nchw_to_tokens.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int]
        lib.iris_hip_patchify.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_hip_unpatchify.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_hip_rms_gated_add.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                               ctypes.c_int]
        lib.iris_hip_fill_rows.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_hip_tanh_cols.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_transformer_load_safetensors.restype = vp
        lib.iris_transformer_create_synthetic.restype = vp
        lib.iris_transformer_create_synthetic.argtypes = [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_float,
                                                                                ctypes.c_uint64]
        lib.iris_transformer_free.argtypes = [vp]
        for fn in ("iris_transformer_forward", "iris_transformer_forward_with_multi_refs",
                   "iris_transformer_forward_with_refs", "iris_sample_euler", "iris_sample_euler_cfg",
                   "iris_sample_euler_with_multi_refs", "zi_transformer_forward", "iris_official_schedule",
                   "iris_init_noise", "zi_transformer_load_safetensors", "zi_transformer_create_synthetic",
                   "iris_sample_euler_zimage", "iris_zimage_schedule"):
            if hasattr(lib, fn):
                getattr(lib, fn).restype = vp
        lib.qwen3_model_load.restype = vp
        lib.qwen3_model_load.argtypes = [ctypes.c_char_p]
        lib.qwen3_model_create_synthetic.restype = vp
        lib.qwen3_model_create_synthetic.argtypes = [ctypes.c_int] * 6 + [ctypes.c_uint64]
        lib.qwen3_model_free.argtypes = [vp]
        lib.qwen3_model_set_extraction_mode.argtypes = [vp, ctypes.c_int]
        lib.qwen3_model_text_dim.argtypes = [vp]
        lib.qwen3_forward.restype = vp
        lib.qwen3_forward.argtypes = [vp, IP, IP, ctypes.c_int]
        lib.iris_hip_embed_rows.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_hip_copy_rows.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_flux_device_buffer.restype = vp
        lib.iris_flux_device_buffer.argtypes = [vp, ctypes.c_char_p]
        for fn in ("iris_flux_prepare", "iris_flux_upload", "iris_flux_velocity", "iris_flux_step",
                   "iris_flux_download_latent", "iris_flux_download_velocity", "iris_flux_double_block_forward",
                   "iris_flux_single_block_forward"):
            getattr(lib, fn).restype = ctypes.c_int
        lib.iris_flux_prepare.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int]
        lib.iris_flux_upload.argtypes = [vp, vp, vp, vp]
        lib.iris_flux_velocity.argtypes = [vp, ctypes.c_float]
        lib.iris_flux_step.argtypes = [vp, ctypes.c_float, ctypes.c_float, ctypes.c_float]
        lib.iris_flux_download_latent.argtypes = [vp, vp]
        lib.iris_flux_download_velocity.argtypes = [vp, vp]
        lib.iris_flux_double_block_forward.argtypes = [vp, ctypes.c_int]
        lib.iris_flux_single_block_forward.argtypes = [vp, ctypes.c_int]
        lib.zi_transformer_load_safetensors.argtypes = [ctypes.c_char_p] + [ctypes.c_int] * 7 + [ctypes.c_float, vp]
        lib.zi_transformer_create_synthetic.argtypes = ([ctypes.c_int] * 7 + [ctypes.c_float, vp, ctypes.c_int,
                                                        ctypes.c_int, ctypes.c_uint64])
        lib.zi_transformer_forward.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_float, vp, ctypes.c_int]
        lib.zi_transformer_free.argtypes = [vp]
        lib.iris_sample_euler_zimage.argtypes = [vp, vp] + [ctypes.c_int] * 5 + [vp, ctypes.c_int, vp, ctypes.c_int,
                                                                                 vp]
        lib.zi_device_buffer.restype = vp
        lib.zi_device_buffer.argtypes = [vp, ctypes.c_char_p]
        lib.zi_prepare.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.zi_upload.argtypes = [vp, vp, vp]
        lib.zi_velocity.argtypes = [vp, ctypes.c_float]
        lib.zi_step.argtypes = [vp, ctypes.c_float, ctypes.c_float]
        lib.zi_download_latent.argtypes = [vp, vp]
        lib.iris_vae_gpu_load.restype = vp
        lib.iris_vae_gpu_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        lib.iris_vae_gpu_load_dir.restype = vp
        lib.iris_vae_gpu_load_dir.argtypes = [ctypes.c_char_p]
        lib.iris_vae_gpu_create_synthetic.restype = vp
        lib.iris_vae_gpu_create_synthetic.argtypes = [ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_uint64]
        lib.iris_vae_gpu_free.argtypes = [vp]
        lib.iris_vae_gpu_decode_to.argtypes = [vp, FP, ctypes.c_int, ctypes.c_int, vp, FP]
        lib.iris_vae_gpu_decode_device.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, vp]
        lib.iris_vae_gpu_decode.restype = ctypes.POINTER(IrisImage)
        lib.iris_vae_gpu_decode.argtypes = [vp, FP, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_image_free.argtypes = [ctypes.POINTER(IrisImage)]
        lib.iris_vae_gpu_z_channels.argtypes = [vp]
        lib.iris_vae_gpu_encode.restype = ctypes.POINTER(ctypes.c_float)
        lib.iris_vae_gpu_encode.argtypes = [vp, FP, ctypes.c_int, ctypes.c_int, ctypes.c_int, IP, IP]
        lib.iris_vae_gpu_encode_device.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
        lib.iris_vae_gpu_has_encoder.argtypes = [vp]
        lib.iris_hip_conv3x3.argtypes = [ctypes.POINTER(Conv3x3)]
        if lib.iris_hip_init(0) != 0:
            raise RuntimeError("iris_hip_init failed: " + lib.iris_hip_last_error().decode())
        _libs["hip"] = lib
    return _libs["hip"]


class Dev:
    """A device buffer of the product library (freed on close/gc)."""

    def __init__(self, nbytes):
        self.lib = hip()
        self.n = int(nbytes)
        self.ptr = self.lib.iris_hip_malloc(max(self.n, 1))
        assert self.ptr, self.lib.iris_hip_last_error()

    @classmethod
    def of(cls, arr):
        arr = np.ascontiguousarray(arr)
        d = cls(arr.nbytes)
        d.put(arr)
        return d

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        assert self.lib.iris_hip_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes) == 0
        assert self.lib.iris_hip_sync() == 0

    def get(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert self.lib.iris_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes) == 0
        return out

    def close(self):
        if self.ptr:
            self.lib.iris_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def to_bf16(a):
    """float32 -> bf16 bits, round to nearest even (same as the device)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def d2h_f32(lib, ptr, shape):
    out = np.empty(shape, np.float32)
    assert lib.iris_hip_memcpy_d2h(out.ctypes.data, ptr, out.nbytes) == 0
    return out


def find_openblas():
    """The OpenBLAS bundled with scipy (same image on every machine)."""
    try:
        import scipy
        d = os.path.join(os.path.dirname(os.path.dirname(scipy.__file__)), "scipy.libs")
        for f in sorted(os.listdir(d)):
            if f.startswith("libscipy_openblas") and f.endswith(".so"):
                return os.path.join(d, f), "scipy_"
    except Exception:
        pass
    return None, None


def bind_blas(lib, threads=None):
    path, prefix = find_openblas()
    if path:
        n = threads or int(os.environ.get("IRIS_ORACLE_THREADS", min(os.cpu_count() or 1, 16)))
        lib.orc_set_blas(path.encode(), prefix.encode(), n)


def ref():
    """The reference build (only where the reference tree exists)."""
    if "ref" not in _libs:
        lib = ctypes.CDLL(REF_SO)
        lib.iris_transformer_load_safetensors.restype = ctypes.c_void_p
        lib.iris_transformer_forward.restype = ctypes.c_void_p
        lib.iris_transformer_forward_with_multi_refs.restype = ctypes.c_void_p
        lib.zi_transformer_load_safetensors.restype = ctypes.c_void_p
        lib.zi_transformer_forward.restype = ctypes.c_void_p
        lib.iris_official_schedule.restype = ctypes.c_void_p
        lib.iris_zimage_schedule.restype = ctypes.c_void_p
        lib.iris_init_noise.restype = ctypes.c_void_p
        lib.iris_sample_euler.restype = ctypes.c_void_p
        lib.qwen3_model_load.restype = ctypes.c_void_p
        lib.qwen3_model_load.argtypes = [ctypes.c_char_p]
        lib.qwen3_model_free.argtypes = [ctypes.c_void_p]
        lib.qwen3_forward.restype = ctypes.c_void_p
        lib.qwen3_forward.argtypes = [ctypes.c_void_p, IP, IP, ctypes.c_int]
        lib.qwen3_set_extraction_mode.argtypes = [ctypes.c_void_p, ctypes.c_int]
        lib.safetensors_open.restype = ctypes.c_void_p
        lib.safetensors_open.argtypes = [ctypes.c_char_p]
        lib.safetensors_close.argtypes = [ctypes.c_void_p]
        lib.iris_vae_load_safetensors_ex.restype = ctypes.c_void_p
        lib.iris_vae_load_safetensors_ex.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        lib.iris_vae_decode.restype = ctypes.POINTER(IrisImage)
        lib.iris_vae_decode.argtypes = [ctypes.c_void_p, FP, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.iris_vae_free.argtypes = [ctypes.c_void_p]
        lib.iris_vae_encode.restype = ctypes.POINTER(ctypes.c_float)
        lib.iris_vae_encode.argtypes = [ctypes.c_void_p, FP, ctypes.c_int, ctypes.c_int, ctypes.c_int, IP, IP]
        lib.iris_image_free.argtypes = [ctypes.POINTER(IrisImage)]
        _libs["ref"] = lib
    return _libs["ref"]


def fptr(a):
    return a.ctypes.data_as(FP)


def take_f32(lib, ptr, n):
    """Copies a malloc'd float array returned by a C library and frees it."""
    out = np.ctypeslib.as_array(ctypes.cast(ptr, FP), shape=(n,)).copy()
    lib_free = getattr(lib, "orc_free", None)
    if lib_free is not None:
        lib_free(ctypes.c_void_p(ptr))
    else:
        ctypes.CDLL(None).free(ctypes.c_void_p(ptr))
    return out


def synth_f32(shape, seed, mean=0.0, std=1.0):
    n = int(np.prod(shape))
    a = np.empty(n, np.float32)
    oracle().iris_synth_fill_f32(fptr(a), n, seed, 0, mean, std)
    return a.reshape(shape)


def synth_bf16(name, shape, model_seed, mean=0.0, std=0.02):
    lib = oracle()
    n = int(np.prod(shape))
    a = np.empty(n, np.uint16)
    lib.iris_synth_fill_bf16(a.ctypes.data_as(U16P), n, lib.iris_synth_seed(model_seed, name.encode()), 0,
                             mean, std)
    return a.reshape(shape)


def bf16_to_f32(a):
    return (a.astype(np.uint32) << 16).view(np.float32)


def write_safetensors(path, tensors):
    """tensors: list of (name, array): uint16 arrays are written as BF16,
    float32 arrays as F32."""
    header, off, blobs = {}, 0, []
    for name, arr in tensors:
        b = np.ascontiguousarray(arr).tobytes()
        dt = "F32" if arr.dtype == np.float32 else "BF16"
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def flux_tensor_list(cfg):
    """(name, shape, is_norm) of a Flux.2-Klein transformer, reference naming."""
    h = cfg["heads"] * 128
    mlp = int(h * cfg.get("mlp_ratio", 3.0))
    C, td = cfg.get("latent_ch", 128), cfg["text_dim"]
    t = [("x_embedder.weight", (h, C), 0), ("context_embedder.weight", (h, td), 0),
         ("time_guidance_embed.timestep_embedder.linear_1.weight", (h, 256), 0),
         ("time_guidance_embed.timestep_embedder.linear_2.weight", (h, h), 0),
         ("double_stream_modulation_img.linear.weight", (6 * h, h), 0),
         ("double_stream_modulation_txt.linear.weight", (6 * h, h), 0),
         ("single_stream_modulation.linear.weight", (3 * h, h), 0)]
    for i in range(cfg["n_double"]):
        p = f"transformer_blocks.{i}."
        t += [(p + "attn.norm_q.weight", (128,), 1), (p + "attn.norm_k.weight", (128,), 1),
              (p + "attn.to_q.weight", (h, h), 0), (p + "attn.to_k.weight", (h, h), 0),
              (p + "attn.to_v.weight", (h, h), 0), (p + "attn.to_out.0.weight", (h, h), 0),
              (p + "ff.linear_in.weight", (2 * mlp, h), 0), (p + "ff.linear_out.weight", (h, mlp), 0),
              (p + "attn.norm_added_q.weight", (128,), 1), (p + "attn.norm_added_k.weight", (128,), 1),
              (p + "attn.add_q_proj.weight", (h, h), 0), (p + "attn.add_k_proj.weight", (h, h), 0),
              (p + "attn.add_v_proj.weight", (h, h), 0), (p + "attn.to_add_out.weight", (h, h), 0),
              (p + "ff_context.linear_in.weight", (2 * mlp, h), 0),
              (p + "ff_context.linear_out.weight", (h, mlp), 0)]
    for i in range(cfg["n_single"]):
        p = f"single_transformer_blocks.{i}."
        t += [(p + "attn.norm_q.weight", (128,), 1), (p + "attn.norm_k.weight", (128,), 1),
              (p + "attn.to_qkv_mlp_proj.weight", (3 * h + 2 * mlp, h), 0),
              (p + "attn.to_out.weight", (h, h + mlp), 0)]
    t += [("norm_out.linear.weight", (2 * h, h), 0), ("proj_out.weight", (C, h), 0)]
    return t


def write_flux_model(d, cfg, seed):
    os.makedirs(os.path.join(d, "transformer"), exist_ok=True)
    conf = {"num_attention_heads": cfg["heads"], "attention_head_dim": 128,
            "num_layers": cfg["n_double"], "num_single_layers": cfg["n_single"],
            "joint_attention_dim": cfg["text_dim"], "in_channels": cfg.get("latent_ch", 128),
            "mlp_ratio": cfg.get("mlp_ratio", 3.0), "rope_theta": cfg.get("theta", 2000.0)}
    with open(os.path.join(d, "transformer", "config.json"), "w") as f:
        json.dump(conf, f)
    tensors = [(n, synth_bf16(n, s, seed, 1.0 if norm else 0.0, 0.02))
               for n, s, norm in flux_tensor_list(cfg)]
    write_safetensors(os.path.join(d, "transformer", "diffusion_pytorch_model.safetensors"), tensors)


def zimage_tensor_list(cfg):
    """(name, shape, mean, std) of a Z-Image transformer, reference naming."""
    d, hd, ps, C = cfg["dim"], 128, cfg.get("ps", 2), cfg.get("in_ch", 16)
    ffn, tmid, cap = cfg["ffn"], cfg["t_mid"], cfg["cap_dim"]
    ad = min(d, 256)
    pf = ps * ps * C
    t = [("t_embedder.mlp.0.weight", (tmid, 256), 0.0, 0.02), ("t_embedder.mlp.0.bias", (tmid,), 0.0, 0.02),
         ("t_embedder.mlp.2.weight", (ad, tmid), 0.0, 0.02), ("t_embedder.mlp.2.bias", (ad,), 0.0, 0.02),
         ("cap_embedder.0.weight", (cap,), 1.0, 0.02), ("cap_embedder.1.weight", (d, cap), 0.0, 0.02),
         ("cap_embedder.1.bias", (d,), 0.0, 0.02),
         (f"all_x_embedder.{ps}-1.weight", (d, pf), 0.0, 0.02), (f"all_x_embedder.{ps}-1.bias", (d,), 0.0, 0.02),
         ("x_pad_token", (d,), 0.0, 1.0), ("cap_pad_token", (d,), 0.0, 1.0)]

    def block(pre, mod):
        b = [(pre + ".attention.to_q.weight", (d, d), 0.0, 0.02), (pre + ".attention.to_k.weight", (d, d), 0.0, 0.02),
             (pre + ".attention.to_v.weight", (d, d), 0.0, 0.02),
             (pre + ".attention.to_out.0.weight", (d, d), 0.0, 0.02),
             (pre + ".attention.norm_q.weight", (hd,), 1.0, 0.02), (pre + ".attention.norm_k.weight", (hd,), 1.0, 0.02),
             (pre + ".attention_norm1.weight", (d,), 1.0, 0.02), (pre + ".attention_norm2.weight", (d,), 1.0, 0.02),
             (pre + ".feed_forward.w1.weight", (ffn, d), 0.0, 0.02),
             (pre + ".feed_forward.w2.weight", (d, ffn), 0.0, 0.02),
             (pre + ".feed_forward.w3.weight", (ffn, d), 0.0, 0.02),
             (pre + ".ffn_norm1.weight", (d,), 1.0, 0.02), (pre + ".ffn_norm2.weight", (d,), 1.0, 0.02)]
        if mod:
            b += [(pre + ".adaLN_modulation.0.weight", (4 * d, ad), 0.0, 0.02),
                  (pre + ".adaLN_modulation.0.bias", (4 * d,), 0.0, 0.02)]
        return b
    for i in range(cfg["refiners"]):
        t += block(f"noise_refiner.{i}", True)
        t += block(f"context_refiner.{i}", False)
    for i in range(cfg["layers"]):
        t += block(f"layers.{i}", True)
    t += [(f"all_final_layer.{ps}-1.adaLN_modulation.1.weight", (d, ad), 0.0, 0.02),
          (f"all_final_layer.{ps}-1.adaLN_modulation.1.bias", (d,), 0.0, 0.02),
          (f"all_final_layer.{ps}-1.linear.weight", (pf, d), 0.0, 0.02),
          (f"all_final_layer.{ps}-1.linear.bias", (pf,), 0.0, 0.02)]
    return t


def write_zimage_model(d, cfg, seed, triu_out=False):
    """triu_out: every attention output projection W[n][k] is zeroed for k < n.
    Then an in-place product row <- row . W^T taken column by column in
    increasing n reads only inputs it has not yet overwritten, so it equals
    the out-of-place product (pins the out-of-place oracle on the reference's
    in-place CPU path)."""
    os.makedirs(os.path.join(d, "transformer"), exist_ok=True)
    tensors = []
    for n, s, m, sd in zimage_tensor_list(cfg):
        a = synth_bf16(n, s, seed, m, sd)
        if triu_out and n.endswith("attention.to_out.0.weight"):
            a = np.triu(a)
        tensors.append((n, a))
    write_safetensors(os.path.join(d, "transformer", "diffusion_pytorch_model.safetensors"), tensors)


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-30))


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def fingerprint(x, stride=97):
    """Compact golden of a large array: strided subsample plus moments."""
    x = np.asarray(x, np.float32).ravel()
    return {"sub": x[::stride].copy(), "sum": np.float64(x.astype(np.float64).sum()),
            "sumsq": np.float64((x.astype(np.float64) ** 2).sum())}


# ---------------------------------------------------------------- Qwen3 files

def write_qwen3_dir(d, hidden=256, inter=512, heads=4, kv_heads=2, layers=28, vocab=300, seed=0):
    """A random-init Qwen3 directory in the HuggingFace layout the reference
    loads (config.json, model.safetensors.index.json, one bf16 shard)."""
    os.makedirs(d, exist_ok=True)
    rng = np.random.default_rng(seed)
    hd = 128
    cfg = {"hidden_size": hidden, "intermediate_size": inter, "num_attention_heads": heads,
           "num_key_value_heads": kv_heads, "head_dim": hd, "vocab_size": vocab, "num_hidden_layers": layers,
           "rope_theta": 1000000.0}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)

    def w(*shape, scale=0.02):
        return to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))

    def nrm(n):
        return to_bf16((1.0 + rng.standard_normal(n) * 0.1).astype(np.float32))

    t = {"model.embed_tokens.weight": w(vocab, hidden, scale=0.5), "model.norm.weight": nrm(hidden)}
    for i in range(layers):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = nrm(hidden)
        t[p + "post_attention_layernorm.weight"] = nrm(hidden)
        t[p + "self_attn.q_proj.weight"] = w(heads * hd, hidden, scale=0.05)
        t[p + "self_attn.k_proj.weight"] = w(kv_heads * hd, hidden, scale=0.05)
        t[p + "self_attn.v_proj.weight"] = w(kv_heads * hd, hidden, scale=0.05)
        t[p + "self_attn.o_proj.weight"] = w(hidden, heads * hd)
        t[p + "self_attn.q_norm.weight"] = nrm(hd)
        t[p + "self_attn.k_norm.weight"] = nrm(hd)
        t[p + "mlp.gate_proj.weight"] = w(inter, hidden, scale=0.05)
        t[p + "mlp.up_proj.weight"] = w(inter, hidden, scale=0.05)
        t[p + "mlp.down_proj.weight"] = w(hidden, inter)
    shard = "model-00001-of-00001.safetensors"
    write_safetensors(os.path.join(d, shard), list(t.items()))
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": {k: shard for k in t}}, f)
    return cfg


class Qwen3Encoder(ctypes.Structure):
    """The reference's qwen3_encoder_t (tokenizer, model) for its mode setter."""
    _fields_ = [("tokenizer", ctypes.c_void_p), ("model", ctypes.c_void_p)]


def vae_tensor_list(z, flux=True, encoder=False):
    """(name, shape) of the VAE decoder (and encoder) tensors in the diffusers
    layout the reference loads (iris_vae.c:1227-1386); Flux adds bn,
    post_quant_conv and quant_conv."""
    t = [("decoder.conv_in.weight", (512, z, 3, 3)), ("decoder.conv_in.bias", (512,))]

    def res(p, cin, cout):
        r = [(p + ".norm1.weight", (cin,)), (p + ".norm1.bias", (cin,)), (p + ".conv1.weight", (cout, cin, 3, 3)),
             (p + ".conv1.bias", (cout,)), (p + ".norm2.weight", (cout,)), (p + ".norm2.bias", (cout,)),
             (p + ".conv2.weight", (cout, cout, 3, 3)), (p + ".conv2.bias", (cout,))]
        if cin != cout:
            r += [(p + ".conv_shortcut.weight", (cout, cin, 1, 1)), (p + ".conv_shortcut.bias", (cout,))]
        return r

    t += res("decoder.mid_block.resnets.0", 512, 512) + res("decoder.mid_block.resnets.1", 512, 512)
    a = "decoder.mid_block.attentions.0."
    t += [(a + "group_norm.weight", (512,)), (a + "group_norm.bias", (512,))]
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        t += [(a + n + ".weight", (512, 512)), (a + n + ".bias", (512,))]
    mult = [1, 2, 4, 4]
    for i in range(4):
        level = 3 - i
        ch = 128 * mult[level]
        prev = 512 if level == 3 else 128 * mult[level + 1]
        for r in range(3):
            t += res(f"decoder.up_blocks.{i}.resnets.{r}", prev if r == 0 else ch, ch)
        if i < 3:
            t += [(f"decoder.up_blocks.{i}.upsamplers.0.conv.weight", (ch, ch, 3, 3)),
                  (f"decoder.up_blocks.{i}.upsamplers.0.conv.bias", (ch,))]
    t += [("decoder.conv_norm_out.weight", (128,)), ("decoder.conv_norm_out.bias", (128,)),
          ("decoder.conv_out.weight", (3, 128, 3, 3)), ("decoder.conv_out.bias", (3,))]
    if flux:
        t += [("bn.running_mean", (4 * z,)), ("bn.running_var", (4 * z,)),
              ("post_quant_conv.weight", (z, z, 1, 1)), ("post_quant_conv.bias", (z,))]
    if encoder:
        t += [("encoder.conv_in.weight", (128, 3, 3, 3)), ("encoder.conv_in.bias", (128,))]
        for level in range(4):
            ch, prev = 128 * mult[level], 128 * mult[level - 1] if level else 128
            for r in range(2):
                t += res(f"encoder.down_blocks.{level}.resnets.{r}", prev if r == 0 and level else ch, ch)
            if level < 3:
                t += [(f"encoder.down_blocks.{level}.downsamplers.0.conv.weight", (ch, ch, 3, 3)),
                      (f"encoder.down_blocks.{level}.downsamplers.0.conv.bias", (ch,))]
        t += res("encoder.mid_block.resnets.0", 512, 512) + res("encoder.mid_block.resnets.1", 512, 512)
        a = "encoder.mid_block.attentions.0."
        t += [(a + "group_norm.weight", (512,)), (a + "group_norm.bias", (512,))]
        for n in ("to_q", "to_k", "to_v", "to_out.0"):
            t += [(a + n + ".weight", (512, 512)), (a + n + ".bias", (512,))]
        t += [("encoder.conv_norm_out.weight", (512,)), ("encoder.conv_norm_out.bias", (512,)),
              ("encoder.conv_out.weight", (2 * z, 512, 3, 3)), ("encoder.conv_out.bias", (2 * z,))]
        if flux:
            t += [("quant_conv.weight", (2 * z, 2 * z, 1, 1)), ("quant_conv.bias", (2 * z,))]
    return t


def write_vae_file(path, z=32, flux=True, seed=0, bf16=False, encoder=False):
    """A random-init VAE decoder file: norm scales ~1, biases small, conv
    weights 1/sqrt(fan_in) (conv_out half that), batch-norm variances ~1."""
    rng = np.random.default_rng(seed)
    out = []
    for name, shape in vae_tensor_list(z, flux, encoder):
        n = int(np.prod(shape))
        fan = n // shape[0] if len(shape) > 1 else 1
        if name.endswith("running_var"):
            a = 1.0 + 0.1 * rng.standard_normal(n)
        elif name.endswith("running_mean"):
            a = 0.1 * rng.standard_normal(n)
        elif name.endswith(".bias"):
            a = 0.05 * rng.standard_normal(n)
        elif "norm" in name:
            a = 1.0 + 0.1 * rng.standard_normal(n)
        else:
            a = (0.5 if name == "decoder.conv_out.weight" else 1.0) / np.sqrt(fan) * rng.standard_normal(n)
        a = a.astype(np.float32).reshape(shape)
        out.append((name, to_bf16(a) if bf16 else a))
    write_safetensors(path, out)


class LoraAdapter(ctypes.Structure):
    """lora_adapter_t (reference iris_lora.h:22-28)"""
    _fields_ = [("lora_A", FP), ("lora_B", FP), ("rank", ctypes.c_int), ("in_dim", ctypes.c_int),
                ("out_dim", ctypes.c_int)]


class LoraState(ctypes.Structure):
    """lora_state_t (reference iris_lora.h:30-51)"""
    _fields_ = ([("scale", ctypes.c_float), ("num_double_blocks", ctypes.c_int)] +
                [(n, ctypes.POINTER(LoraAdapter)) for n in ("double_img_q", "double_img_k", "double_img_v",
                                                            "double_img_proj", "double_txt_q", "double_txt_k",
                                                            "double_txt_v", "double_txt_proj")] +
                [("num_single_blocks", ctypes.c_int), ("single_linear1", ctypes.POINTER(LoraAdapter)),
                 ("single_linear2", ctypes.POINTER(LoraAdapter)), ("scratch", FP), ("scratch_len", ctypes.c_int),
                 ("max_rank", ctypes.c_int)])


def make_lora(cfg, seed, rank=8, scale=1.0, std=0.05, max_seq=4096):
    """A LoRA state for a Flux-shaped model with every adapter filled from the
    seeded generator, all memory from the C allocator (the reference's
    lora_free releases it)."""
    libc = ctypes.CDLL(None)
    libc.malloc.restype = ctypes.c_void_p
    libc.malloc.argtypes = [ctypes.c_size_t]
    h = cfg["heads"] * 128
    mlp = int(h * cfg.get("mlp_ratio", 3.0))

    def carr(a):
        a = np.ascontiguousarray(a, np.float32)
        p = libc.malloc(a.nbytes)
        ctypes.memmove(p, a.ctypes.data, a.nbytes)
        return ctypes.cast(p, FP)

    def adapters(n, in_dim, out_dim, tag):
        p = ctypes.cast(libc.malloc(n * ctypes.sizeof(LoraAdapter)), ctypes.POINTER(LoraAdapter))
        for i in range(n):
            s = seed * 1000 + tag * 50 + i
            p[i] = LoraAdapter(carr(synth_f32((rank, in_dim), 2 * s, 0.0, std)),
                               carr(synth_f32((out_dim, rank), 2 * s + 1, 0.0, std)), rank, in_dim, out_dim)
        return p

    st = ctypes.cast(libc.malloc(ctypes.sizeof(LoraState)), ctypes.POINTER(LoraState))
    nd, ns = cfg["n_double"], cfg["n_single"]
    f = st.contents
    f.scale, f.num_double_blocks, f.num_single_blocks = scale, nd, ns
    for k, name in enumerate(("double_img_q", "double_img_k", "double_img_v", "double_img_proj",
                              "double_txt_q", "double_txt_k", "double_txt_v", "double_txt_proj")):
        setattr(f, name, adapters(nd, h, h, k))
    f.single_linear1 = adapters(ns, h, 3 * h + 2 * mlp, 8)
    f.single_linear2 = adapters(ns, h + mlp, h, 9)
    f.scratch = ctypes.cast(libc.malloc(rank * max_seq * 4), FP)
    f.scratch_len, f.max_rank = max_seq, rank
    return st


def c_floats(a):
    """A copy of a float32 array in memory from the C allocator (for setters
    that take ownership and release it with free())."""
    libc = ctypes.CDLL(None)
    libc.malloc.restype = ctypes.c_void_p
    libc.malloc.argtypes = [ctypes.c_size_t]
    a = np.ascontiguousarray(a, np.float32)
    p = libc.malloc(a.nbytes)
    ctypes.memmove(p, a.ctypes.data, a.nbytes)
    return p
