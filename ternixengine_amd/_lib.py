"""Loader of libternix_hip.so (built in-tree by ternixengine_amd/csrc/Makefile).

The library is the product: if it is missing the import fails loudly; nothing here falls back to a
CPU implementation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libternix_hip.so")

_lib = None


class LibraryNotBuilt(ImportError):
    pass


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryNotBuilt(
            f"{LIB_PATH} is missing: build it with `make -C ternixengine_amd/csrc` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    lib = ctypes.CDLL(LIB_PATH)
    i8p = ctypes.c_void_p
    i64 = ctypes.c_int64
    for name in ("ternix_hip_mul_mat_ternary", "ternix_hip_mul_mat_ternary_gemv", "ternix_hip_mul_mat_ternary_gemm",
                 "ternix_hip_mul_mat_ternary_tiled", "ternix_hip_mul_mat_ternary_naive",
                 "ternix_hip_mul_mat_ternary_tile64"):
        f = getattr(lib, name)
        f.argtypes = [i8p, i8p, i8p, i64, i64, i64, ctypes.c_void_p]
        f.restype = ctypes.c_int
    lib.ternix_hip_mul_mat_ternary_host.argtypes = [i8p, i8p, i8p, i64, i64, i64, ctypes.c_int]
    lib.ternix_hip_mul_mat_ternary_host.restype = ctypes.c_int
    lib.ternix_hip_error_string.argtypes = [ctypes.c_int]
    lib.ternix_hip_error_string.restype = ctypes.c_char_p
    lib.ternix_hip_version.restype = ctypes.c_int
    lib.ternix_hip_debug_set.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.ternix_hip_debug_set.restype = ctypes.c_int
    lib.ternix_hip_debug_reset.argtypes = []
    lib.ternix_hip_debug_reset.restype = None
    lib.ternix_hip_debug_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.ternix_hip_debug_stream_read.restype = ctypes.c_int
    lib.ternix_hip_debug_alloc_count.argtypes = []
    lib.ternix_hip_debug_alloc_count.restype = ctypes.c_longlong
    lib.ternix_hip_take_faults.argtypes = [ctypes.c_void_p]
    lib.ternix_hip_take_faults.restype = ctypes.c_int
    lib.ternix_hip_mul_mat_ternary_workspace_size.argtypes = [i64, i64, i64]
    lib.ternix_hip_mul_mat_ternary_workspace_size.restype = ctypes.c_size_t
    lib.ternix_hip_mul_mat_ternary_workspace_size_for.argtypes = [i8p, i8p, i64, i64, i64]
    lib.ternix_hip_mul_mat_ternary_workspace_size_for.restype = ctypes.c_size_t
    lib.ternix_hip_mul_mat_ternary_ws.argtypes = [i8p, i8p, i8p, i64, i64, i64, ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p]
    lib.ternix_hip_mul_mat_ternary_ws.restype = ctypes.c_int
    lib.ternix_hip_mul_mat_ternary_noalloc.argtypes = [i8p, i8p, i8p, i64, i64, i64, ctypes.c_void_p]
    lib.ternix_hip_mul_mat_ternary_noalloc.restype = ctypes.c_int
    lib.ternix_hip_noalloc_scratch_bytes.argtypes = []
    lib.ternix_hip_noalloc_scratch_bytes.restype = ctypes.c_size_t
    lib.ternix_hip_release_stream.argtypes = [ctypes.c_void_p]
    lib.ternix_hip_release_stream.restype = ctypes.c_int
    lib.ternix_hip_plan_describe.argtypes = [i8p, i8p, i64, i64, i64, ctypes.c_char_p, ctypes.c_size_t]
    lib.ternix_hip_plan_describe.restype = ctypes.c_int
    for name in ("ternix_pack_ternary_weights", "ternix_unpack_ternary_weights", "ternix_interleave_weights_offline"):
        f = getattr(lib, name)
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        f.restype = None
    for name in ("ternix_hip_pack_ternary_weights", "ternix_hip_unpack_ternary_weights",
                 "ternix_hip_interleave_weights_offline"):
        f = getattr(lib, name)
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        f.restype = ctypes.c_int
    vp = ctypes.c_void_p
    lib.ternix_interleave_weights_tile64.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_size_t]
    lib.ternix_interleave_weights_tile64.restype = ctypes.c_int
    lib.ternix_hip_interleave_weights_tile64.argtypes = [vp, vp, i64, i64, vp]
    lib.ternix_hip_interleave_weights_tile64.restype = ctypes.c_int
    lib.ternix_hip_quantize_activations.argtypes = [vp, vp, vp, i64, i64, vp]
    lib.ternix_hip_quantize_activations.restype = ctypes.c_int
    lib.ternix_hip_mul_mat_ternary_dequant.argtypes = [vp, vp, vp, i64, i64, i64, vp, ctypes.c_float, vp]
    lib.ternix_hip_mul_mat_ternary_dequant.restype = ctypes.c_int
    lib.ternix_hip_mul_mat_ternary_tile64_dequant.argtypes = [vp, vp, vp, i64, i64, i64, vp, ctypes.c_float, vp]
    lib.ternix_hip_mul_mat_ternary_tile64_dequant.restype = ctypes.c_int
    lib.ternix_quantize_weights_absmean.argtypes = [vp, vp, vp, ctypes.c_size_t]
    lib.ternix_quantize_weights_absmean.restype = ctypes.c_int
    f32 = ctypes.c_float
    lib.ternix_hip_rms_norm.argtypes = [vp, vp, vp, i64, i64, f32, vp]
    lib.ternix_hip_rms_norm_quantize.argtypes = [vp, vp, vp, vp, i64, i64, f32, vp]
    lib.ternix_hip_swiglu.argtypes = [vp, vp, i64, vp]
    lib.ternix_hip_mul_mat_ternary_swiglu.argtypes = [vp, vp, vp, i64, i64, i64, vp, f32, vp, vp]
    lib.ternix_hip_ffn_workspace_size.argtypes = [i64, i64, i64]
    lib.ternix_hip_ffn_workspace_size.restype = ctypes.c_size_t
    lib.ternix_hip_ffn_forward.argtypes = [vp, vp, vp, f32, vp, f32, vp, f32, i64, i64, i64, vp, ctypes.c_size_t, vp]
    lib.ternix_hip_ffn_forward_tile64.argtypes = lib.ternix_hip_ffn_forward.argtypes
    lib.ternix_hip_ffn_forward_tile64.restype = ctypes.c_int
    for name in ("ternix_hip_rms_norm", "ternix_hip_rms_norm_quantize", "ternix_hip_swiglu",
                 "ternix_hip_mul_mat_ternary_swiglu", "ternix_hip_ffn_forward"):
        getattr(lib, name).restype = ctypes.c_int
    u64 = ctypes.c_uint64
    lib.ternix_synth_u64.argtypes = [u64, u64, u64]
    lib.ternix_synth_u64.restype = u64
    lib.ternix_synth_act_uniform.argtypes = [ctypes.c_void_p, ctypes.c_size_t, u64, u64]
    lib.ternix_synth_act_gauss.argtypes = [ctypes.c_void_p, ctypes.c_size_t, u64, u64, ctypes.c_int]
    lib.ternix_synth_ternary.argtypes = [ctypes.c_void_p, ctypes.c_size_t, u64, u64, u64, u64]
    lib.ternix_synth_ternary_packed.argtypes = [ctypes.c_void_p, ctypes.c_size_t, u64, u64, u64, u64]
    for name in ("ternix_synth_act_uniform", "ternix_synth_act_gauss", "ternix_synth_ternary",
                 "ternix_synth_ternary_packed"):
        getattr(lib, name).restype = None
    _lib = lib
    return lib
