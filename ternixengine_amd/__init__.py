"""ternixengine_amd -- MI355X (gfx950) ternary matmul: C[M,N] int32 = A[M,K] int8 x W[K,N] ternary.

Python face of libternix_hip.so, shaped like the reference's `ternix_engine` module
(bindings/python/pybind11_wrapper.cpp:21-90):

  pack_ternary(w)                 (K, N) int8 in {-1,0,1}  -> (K, N/4) uint8     (:21-31)
  unpack_ternary(packed)          (K, N/4) uint8           -> (K, N) int8        (:33-39)
  ternary_matmul(a, b_packed, impl="hip") -> (M, N) int32                         (:41-71)
  has_cuda (False), has_hip

`impl` names the GPU kernel: "hip" (automatic choice), "hip_gemv" (skinny split-K, M <= 32),
"hip_gemm" (LDS-tiled MFMA), "hip_tiled" (the reference tiled kernel's M,N,K % 64 contract) and
"hip_naive".  Errors follow the reference: ValueError for bad shapes, weights or impl names;
RuntimeError("HIP error: ...") for device errors.  The GIL is released during device work (ctypes).

Device-pointer access (no copies) is `mul_mat_ternary(dA, dB, dC, M, K, N, stream=None, path="auto")`
with integer device addresses, mirroring the C-ABI in include/ternix/ternix_hip.h; the weight format
on device memory is `pack_ternary_device` / `unpack_ternary_device`.

Opt-in pre-permuted weights: `interleave_tile64(packed)` (host) / `interleave_tile64_device` rewrite the
(K, N/4) packed matrix as 1 KB blocks of 64 k-rows x 16 bytes, which `ternary_matmul_tile64` and
`mul_mat_ternary(..., path="tile64")` consume (same results, faster decode-shaped calls).
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import LibraryNotBuilt, load as _load  # noqa: F401

__all__ = ["pack_ternary", "unpack_ternary", "ternary_matmul", "mul_mat_ternary", "pack_ternary_device",
           "unpack_ternary_device", "quantize_weights_absmean", "quantize_activations", "ternary_matmul_dequant", "rms_norm", "swiglu",
           "ffn_forward", "interleave_tile64", "interleave_tile64_device", "ternary_matmul_tile64",
           "ternary_matmul_tile64_dequant", "ffn_forward_tile64",
           "has_cuda", "has_hip", "HIP_IMPLS", "ternix_error"]

has_cuda = False
HIP_IMPLS = {"hip": 0, "hip_naive": 1, "hip_gemv": 2, "hip_gemm": 3, "hip_tiled": 4}
_PATHS = {"auto": "ternix_hip_mul_mat_ternary", "gemv": "ternix_hip_mul_mat_ternary_gemv",
          "gemm": "ternix_hip_mul_mat_ternary_gemm", "tiled": "ternix_hip_mul_mat_ternary_tiled",
          "naive": "ternix_hip_mul_mat_ternary_naive", "tile64": "ternix_hip_mul_mat_ternary_tile64"}


def _has_hip():
    try:
        from . import hip_runtime
        return hip_runtime.device_count() > 0
    except OSError:
        return False


has_hip = _has_hip()


def ternix_error(status):
    return _load().ternix_hip_error_string(int(status)).decode(errors="replace")


def _ptr(arr):
    return arr.ctypes.data_as(ctypes.c_void_p)


def pack_ternary(w):
    """Pack a (K, N) int8 array with values in {-1, 0, +1} into the (K, N/4) uint8 layout."""
    w = np.ascontiguousarray(np.asarray(w).astype(np.int8, copy=False))
    if w.ndim != 2:
        raise ValueError("pack_ternary expects a 2-D (K, N) array")
    k, n = w.shape
    if n % 4 != 0:
        raise ValueError("N must be a multiple of 4")
    if w.size and (w.min() < -1 or w.max() > 1):
        raise ValueError("weights must be in {-1, 0, +1}")
    out = np.empty((k, n // 4), dtype=np.uint8)
    _load().ternix_pack_ternary_weights(_ptr(out), _ptr(w), w.size)
    return out


def unpack_ternary(packed):
    """Inverse of pack_ternary: (K, N/4) uint8 -> (K, N) int8."""
    p = np.ascontiguousarray(np.asarray(packed).astype(np.uint8, copy=False))
    if p.ndim != 2:
        raise ValueError("unpack_ternary expects a 2-D (K, N/4) array")
    k, n4 = p.shape
    out = np.empty((k, n4 * 4), dtype=np.int8)
    _load().ternix_unpack_ternary_weights(_ptr(out), _ptr(p), out.size)
    return out


def ternary_matmul(a, b_packed, impl="hip"):
    """C = A (M,K int8) @ W (K,N ternary, packed (K, N/4) uint8) -> (M,N) int32, computed on the GPU."""
    a = np.ascontiguousarray(np.asarray(a).astype(np.int8, copy=False))
    b = np.ascontiguousarray(np.asarray(b_packed).astype(np.uint8, copy=False))
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("A must be (M, K) and B_packed (K, N/4)")
    m, k = a.shape
    n = b.shape[1] * 4
    if b.shape[0] != k:
        raise ValueError("inner dimensions do not match")
    if impl not in HIP_IMPLS:
        raise ValueError(f"unknown impl '{impl}'")
    c = np.empty((m, n), dtype=np.int32)
    status = _load().ternix_hip_mul_mat_ternary_host(_ptr(a), _ptr(b), _ptr(c), m, k, n, HIP_IMPLS[impl])
    if status != 0:  # device-side rejection included, as the reference binding reports it
        raise RuntimeError(f"HIP error: {ternix_error(status)} (impl '{impl}', M={m} K={k} N={n})")
    return c


def pack_ternary_device(d_packed, d_w, size, stream=None):
    """Device-memory pack_ternary_weights: `size` int8 weights at address d_w -> size//4 bytes at
    d_packed, asynchronously on `stream`.  Returns the hipError_t status as an int."""
    return _load().ternix_hip_pack_ternary_weights(d_packed, d_w, int(size), stream)


def unpack_ternary_device(d_w, d_packed, size, stream=None):
    """Device-memory unpack_ternary_weights: size//4 bytes at d_packed -> 4*(size//4) int8 at d_w."""
    return _load().ternix_hip_unpack_ternary_weights(d_w, d_packed, int(size), stream)


def quantize_weights_absmean(w):
    """Offline absmean ternary quantisation of fp32 weights (K, N) -> ((K, N/4) uint8 packed, w_scale):
    gamma = max(mean|W|, 1e-5), w = clamp(rint(W / gamma), -1, 1) (host C code in the library)."""
    w = np.ascontiguousarray(np.asarray(w, dtype=np.float32))
    if w.ndim != 2 or w.shape[1] % 4 != 0:
        raise ValueError("quantize_weights_absmean expects a 2-D (K, N) array with N % 4 == 0")
    out = np.empty((w.shape[0], w.shape[1] // 4), dtype=np.uint8)
    scale = np.zeros(1, dtype=np.float32)
    if _load().ternix_quantize_weights_absmean(_ptr(out), _ptr(scale), _ptr(w), w.size) != 0:
        raise ValueError("quantize_weights_absmean rejected its arguments")
    return out, float(scale[0])


def quantize_activations(x):
    """Per-row absmax int8 quantisation of fp32 activations (M, K) on the GPU -> (q int8 (M, K),
    row_scale float32 (M,)) with q = clamp(rint(x * 127 / a), -128, 127), row_scale = a / 127,
    a = max(max|x_row|, 1e-5)."""
    from . import hip_runtime as hr
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    if x.ndim != 2:
        raise ValueError("quantize_activations expects a 2-D (M, K) array")
    m, k = x.shape
    dx, dq, ds = hr.DeviceBuffer.from_array(x), hr.DeviceBuffer(max(m * k, 1)), hr.DeviceBuffer(max(4 * m, 4))
    status = _load().ternix_hip_quantize_activations(dx.value, dq.value, ds.value, m, k, None)
    if status != 0:
        raise RuntimeError(f"HIP error: {ternix_error(status)}")
    hr.synchronize()
    return dq.download(np.int8, (m, k)), ds.download(np.float32, (m,))


def ternary_matmul_dequant(a, b_packed, row_scale, w_scale):
    """Y = (A @ W) * row_scale[:, None] * w_scale as fp32 on the GPU, the scaling fused into the
    matmul's output (see ternix_hip_mul_mat_ternary_dequant)."""
    from . import hip_runtime as hr
    a = np.ascontiguousarray(np.asarray(a).astype(np.int8, copy=False))
    b = np.ascontiguousarray(np.asarray(b_packed).astype(np.uint8, copy=False))
    rs = np.ascontiguousarray(np.asarray(row_scale, dtype=np.float32).reshape(-1))
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("A must be (M, K) and B_packed (K, N/4)")
    m, k = a.shape
    n = b.shape[1] * 4
    if b.shape[0] != k:
        raise ValueError("inner dimensions do not match")
    if rs.shape[0] != m:
        raise ValueError("row_scale must have M entries")
    da, db, drs = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(b), hr.DeviceBuffer.from_array(rs)
    dy = hr.DeviceBuffer(max(4 * m * n, 4))
    status = _load().ternix_hip_mul_mat_ternary_dequant(da.value, db.value, dy.value, m, k, n, drs.value,
                                                        float(w_scale), None)
    if status != 0:
        raise RuntimeError(f"HIP error: {ternix_error(status)}")
    hr.synchronize()
    return dy.download(np.float32, (m, n))


def interleave_tile64(packed):
    """(K, N/4) packed weights -> the same bytes in the tile-64 layout (flat uint8, K*N/4 bytes):
    block (strip c, k-step s) of 64 rows x 16 bytes at (c * K/64 + s) * 1024, row r of the step at
    16-byte position r ^ (8 * ((r / 16) % 2)).  Needs K % 64 == 0 and (N/4) % 16 == 0."""
    p = np.ascontiguousarray(np.asarray(packed).astype(np.uint8, copy=False))
    if p.ndim != 2:
        raise ValueError("interleave_tile64 expects a 2-D (K, N/4) array")
    k, nb = p.shape
    out = np.empty(k * nb, dtype=np.uint8)
    if _load().ternix_interleave_weights_tile64(_ptr(out), _ptr(p), k, nb * 4) != 0:
        raise ValueError("interleave_tile64 needs K % 64 == 0 and (N/4) % 16 == 0")
    return out


def interleave_tile64_device(d_out, d_packed, K, N, stream=None):
    """Device-memory tile-64 conversion (asynchronous on `stream`); returns the hipError_t status."""
    return _load().ternix_hip_interleave_weights_tile64(d_out, d_packed, int(K), int(N), stream)


def ternary_matmul_tile64(a, w_tile64, n):
    """C = A (M,K int8) @ W on the GPU, W given in the tile-64 layout (interleave_tile64) with N
    columns -> (M, N) int32.  Needs K % 128 == 0 and N % 256 == 0."""
    from . import hip_runtime as hr
    a = np.ascontiguousarray(np.asarray(a).astype(np.int8, copy=False))
    wt = np.ascontiguousarray(np.asarray(w_tile64).astype(np.uint8, copy=False)).reshape(-1)
    if a.ndim != 2:
        raise ValueError("A must be (M, K)")
    m, k = a.shape
    n = int(n)
    if n % 4 != 0 or wt.size != k * (n // 4):
        raise ValueError("w_tile64 must hold K * N/4 bytes")
    da, dw = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wt)
    dc = hr.DeviceBuffer(max(4 * m * n, 4))
    _check(_load().ternix_hip_mul_mat_ternary_tile64(da.value, dw.value, dc.value, m, k, n, None))
    hr.synchronize()
    return dc.download(np.int32, (m, n))


def ternary_matmul_tile64_dequant(a, w_tile64, n, row_scale, w_scale):
    """ternary_matmul_dequant on tile-64 weights: (A @ W) * row_scale[:, None] * w_scale as fp32, W in
    the tile-64 layout with N columns (K % 128 == 0, N % 256 == 0)."""
    from . import hip_runtime as hr
    a = np.ascontiguousarray(np.asarray(a).astype(np.int8, copy=False))
    wt = np.ascontiguousarray(np.asarray(w_tile64).astype(np.uint8, copy=False)).reshape(-1)
    rs = np.ascontiguousarray(np.asarray(row_scale, dtype=np.float32).reshape(-1))
    if a.ndim != 2:
        raise ValueError("A must be (M, K)")
    m, k = a.shape
    n = int(n)
    if n % 4 != 0 or wt.size != k * (n // 4):
        raise ValueError("w_tile64 must hold K * N/4 bytes")
    if rs.shape[0] != m:
        raise ValueError("row_scale must have M entries")
    da, dw, drs = hr.DeviceBuffer.from_array(a), hr.DeviceBuffer.from_array(wt), hr.DeviceBuffer.from_array(rs)
    dy = hr.DeviceBuffer(max(4 * m * n, 4))
    _check(_load().ternix_hip_mul_mat_ternary_tile64_dequant(da.value, dw.value, dy.value, m, k, n, drs.value,
                                                             float(w_scale), None))
    hr.synchronize()
    return dy.download(np.float32, (m, n))


def _check(status):
    if status != 0:
        if status == 1:
            raise ValueError("arguments rejected (hipErrorInvalidValue)")
        raise RuntimeError(f"HIP error: {ternix_error(status)}")


def rms_norm(x, weight, eps=1e-5):
    """Row-wise RMSNorm of fp32 (rows, size) on the GPU (reference rms_norm_avx2 per row)."""
    from . import hip_runtime as hr
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    x2 = x.reshape(1, -1) if x.ndim == 1 else x
    w = np.ascontiguousarray(np.asarray(weight, dtype=np.float32).reshape(-1))
    rows, size = x2.shape
    if w.shape[0] != size:
        raise ValueError("weight must have one entry per column")
    dx, dw, do = hr.DeviceBuffer.from_array(x2), hr.DeviceBuffer.from_array(w), hr.DeviceBuffer(max(x2.nbytes, 4))
    _check(_load().ternix_hip_rms_norm(do.value, dx.value, dw.value, rows, size, float(eps), None))
    hr.synchronize()
    return do.download(np.float32, x2.shape).reshape(x.shape)


def swiglu(x):
    """Reference swiglu on the GPU: interleaved (gate, up) pairs of a flat fp32 array -> size//2 outputs."""
    from . import hip_runtime as hr
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
    dx, do = hr.DeviceBuffer.from_array(x), hr.DeviceBuffer(max(4 * (x.size // 2), 4))
    _check(_load().ternix_hip_swiglu(do.value, dx.value, x.size, None))
    hr.synchronize()
    return do.download(np.float32, (x.size // 2,))


def ffn_forward(x, norm_weight, eps, w_gateup_packed, ws_gateup, w_down_packed, ws_down):
    """One feed-forward block on the GPU (see ternix_hip_ffn_forward): x (M, H) fp32 -> (M, H) fp32,
    w_gateup_packed (H, 2F/4) with interleaved gate/up columns, w_down_packed (F, H/4)."""
    from . import hip_runtime as hr
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    g = np.ascontiguousarray(np.asarray(norm_weight, dtype=np.float32).reshape(-1))
    wgu = np.ascontiguousarray(np.asarray(w_gateup_packed, dtype=np.uint8))
    wd = np.ascontiguousarray(np.asarray(w_down_packed, dtype=np.uint8))
    m, h = x.shape
    f = wgu.shape[1] * 2
    if wgu.shape[0] != h or wd.shape != (f, h // 4) or g.shape[0] != h:
        raise ValueError("inconsistent FFN shapes")
    lib = _load()
    nws = lib.ternix_hip_ffn_workspace_size(m, h, f)
    dx, dg, dgu, dd = (hr.DeviceBuffer.from_array(a) for a in (x, g, wgu, wd))
    dy, dws = hr.DeviceBuffer(max(x.nbytes, 4)), hr.DeviceBuffer(max(nws, 256))
    _check(lib.ternix_hip_ffn_forward(dy.value, dx.value, dg.value, float(eps), dgu.value, float(ws_gateup),
                                      dd.value, float(ws_down), m, h, f, dws.value, nws, None))
    hr.synchronize()
    return dy.download(np.float32, (m, h))


def ffn_forward_tile64(x, norm_weight, eps, w_gateup_packed, ws_gateup, w_down_packed, ws_down):
    """ffn_forward with the weights in the tile-64 layout (ternix_hip_ffn_forward_tile64).  Takes the
    same (K, N/4) packed matrices as ffn_forward and converts them on the host here (a caller keeps the
    converted copies and calls the C-ABI instead); the result equals ffn_forward's bit for bit."""
    from . import hip_runtime as hr
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    g = np.ascontiguousarray(np.asarray(norm_weight, dtype=np.float32).reshape(-1))
    wgu = np.ascontiguousarray(np.asarray(w_gateup_packed, dtype=np.uint8))
    wd = np.ascontiguousarray(np.asarray(w_down_packed, dtype=np.uint8))
    m, h = x.shape
    f = wgu.shape[1] * 2
    if wgu.shape[0] != h or wd.shape != (f, h // 4) or g.shape[0] != h:
        raise ValueError("inconsistent FFN shapes")
    lib = _load()
    nws = lib.ternix_hip_ffn_workspace_size(m, h, f)
    dx, dg = hr.DeviceBuffer.from_array(x), hr.DeviceBuffer.from_array(g)
    dgu, dd = hr.DeviceBuffer.from_array(interleave_tile64(wgu)), hr.DeviceBuffer.from_array(interleave_tile64(wd))
    dy, dws = hr.DeviceBuffer(max(x.nbytes, 4)), hr.DeviceBuffer(max(nws, 256))
    _check(lib.ternix_hip_ffn_forward_tile64(dy.value, dx.value, dg.value, float(eps), dgu.value, float(ws_gateup),
                                             dd.value, float(ws_down), m, h, f, dws.value, nws, None))
    hr.synchronize()
    return dy.download(np.float32, (m, h))


def mul_mat_ternary(dA, dB, dC, M, K, N, stream=None, path="auto"):
    """Asynchronous device-pointer call of the C-ABI; returns the hipError_t status as an int."""
    fn = getattr(_load(), _PATHS[path])
    return fn(dA, dB, dC, int(M), int(K), int(N), stream)
