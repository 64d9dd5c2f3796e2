"""Loader for libturboquant_hip.so (the gfx950 kernels) and small host-side helpers.

The library exposes a plain C ABI (include/turboquant_hip.h); it is bound here with ctypes
in the same way the reference binds its hipcc-built FP4 kernels
(turboquant/integration/tq_fp4_backend.py:58-76, 272-295): device pointers come from torch
tensors and the stream is torch's current stream.  There is no CPU fallback: every entry point
raises when the library is missing or a tensor is not on the GPU.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libturboquant_hip.so"
LIB_PATH = Path(__file__).resolve().parent / "lib" / LIB_NAME
ABI_VERSION = 4
HEAD_DIM = 128

TQ_F32, TQ_F16, TQ_BF16, TQ_I32, TQ_I64 = 0, 1, 2, 3, 4
_DTYPE_CODE = {
    torch.float32: TQ_F32,
    torch.float16: TQ_F16,
    torch.bfloat16: TQ_BF16,
    torch.int32: TQ_I32,
    torch.int64: TQ_I64,
}


class TurboQuantError(RuntimeError):
    """Raised when a tq_* entry point returns a nonzero status."""


class TQRegion(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("stride_block", ctypes.c_int64),
        ("stride_head", ctypes.c_int64),
        ("stride_seq", ctypes.c_int64),
        ("stride_row", ctypes.c_int64),
    ]


class TQKVView(ctypes.Structure):
    _fields_ = [
        ("idx", TQRegion),
        ("signs", TQRegion),
        ("norm", TQRegion),
        ("rnorm", TQRegion),
        ("centroids", ctypes.c_void_p),
        ("bits", ctypes.c_int32),
        ("qjl", ctypes.c_int32),
        ("signs_permuted", ctypes.c_int32),
        ("centroid_scale", ctypes.c_float),
        ("layout", ctypes.c_int32),
    ]


class TQPagedTarget(ctypes.Structure):
    """tq_paged_target: one tensor of a K + V cache update."""
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_stride_token", ctypes.c_int64),
        ("x_stride_head", ctypes.c_int64),
        ("cache", ctypes.c_void_p),
        ("cache_stride_block", ctypes.c_int64),
        ("cache_stride_head", ctypes.c_int64),
        ("bits", ctypes.c_int32),
        ("use_qjl", ctypes.c_int32),
        ("tile_layout", ctypes.c_int32),
        ("centroids", ctypes.c_void_p),
        ("boundaries", ctypes.c_void_p),
    ]


TILE_ROWS, TILE_KEYS, TILE_VALUES = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 64 << 20  # TQ_NOALLOC_SCRATCH_BYTES


_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/turboquant_hip.h
SIGNATURES = {
    "tq_abi_version": (_i32, []),
    "tq_status_string": (ctypes.c_char_p, [_i32]),
    "tq_polarquant_compress": (
        _i32,
        [_vp, _i32, _i64, _i64, _i32, _i32, _f32, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "tq_compress_paged": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _i32, _vp, _i64, _i64, _i64, _i32,
         _i32, _i32, _i32, _i32, _f32, _vp, _vp, _vp],
    ),
    "tq_compress_paged_kv": (
        _i32,
        [ctypes.POINTER(TQPagedTarget), ctypes.POINTER(TQPagedTarget), _i32, _i64, _i32, _i32, _vp, _i32, _i64, _i32,
         _i32, _f32, _vp],
    ),
    "tq_compress_regions": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _i32, ctypes.POINTER(TQKVView), _vp, _i64, _i32, _i32, _f32,
         _vp],
    ),
    "tq_tile_bytes": (_i64, [_i32, _i32, _i32]),
    "tq_tile_offsets": (
        _i32,
        [_i32, _i32, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    ),
    "tq_decode": (
        _i32,
        [_vp, _i32, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _i32,
         ctypes.POINTER(TQKVView), ctypes.POINTER(TQKVView), _i32, _i64, _vp, _i64, _i32, _vp, _i32,
         _f32, _f32, _f32, _i32, _vp, _sz, _vp, _i32, _i64, _i64, _vp, _vp],
    ),
    "tq_decode_rotated": (
        _i32,
        [_vp, _i32, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _i32,
         ctypes.POINTER(TQKVView), ctypes.POINTER(TQKVView), _i32, _i64, _vp, _i64, _i32, _vp, _i32,
         _f32, _f32, _f32, _i32, _vp, _sz, _vp, _i32, _i64, _i64, _vp, _vp],
    ),
    "tq_wht_rows": (_i32, [_vp, _i32, _i64, _i64, _i32, _i32, _i32, _vp, _i32, _i64, _i64, _vp]),
    "tq_prefill": (
        _i32,
        [_vp, _i32, _i64, _i64, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _i32, _i32,
         ctypes.POINTER(TQKVView), ctypes.POINTER(TQKVView), _i32, _i64, _vp, _i64, _i32, _vp,
         _f32, _f32, _i32, _vp, _i32, _i64, _i64, _vp],
    ),
    "tq_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "tq_decode_noalloc": (
        _i32,
        [_vp, _i32, _i64, _i64, _vp, _i64, _i64, _i32, _i32, _i32, _i32,
         ctypes.POINTER(TQKVView), ctypes.POINTER(TQKVView), _i32, _i64, _vp, _i64, _i32, _vp, _i32,
         _f32, _f32, _f32, _i32, _vp, _i32, _i64, _i64, _vp, _vp],
    ),
    "tq_decode_concurrent_units": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_int)]),
    "tq_decode_workgroup_waves": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_int)]),
    "tq_packed_attention": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                   ctypes.c_float, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp, _i32, _vp]),
    "tq_packed_attention_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32]),
    "tq_polarquant_compress_matrix": (
        _i32, [_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tq_compress_packed": (
        _i32, [_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "tq_permute_signs": (_i32, [_vp, _vp, _i64, _i32, _vp]),
    "tq_unpack_bits": (_i32, [_vp, _vp, _i64, _i32, _i32, _vp]),
}

_lock = threading.Lock()
_lib = None


def library_path() -> Path:
    override = os.environ.get("TQ_HIP_LIB")
    return Path(override) if override else LIB_PATH


def lib() -> ctypes.CDLL:
    """Load the HIP library once (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise TurboQuantError(
                f"{path} is missing: build it with `python turboquant-amd_amd/build.py` "
                "(or __graft_entry__.build()); turboquant has no CPU fallback"
            )
        handle = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.tq_abi_version()
        if ver != ABI_VERSION:
            raise TurboQuantError(f"{path}: ABI version {ver}, expected {ABI_VERSION}; rebuild the library")
        _lib = handle
        return _lib


def status_string(code: int) -> str:
    return lib().tq_status_string(code).decode()


def check(code: int, what: str) -> None:
    if code != 0:
        raise TurboQuantError(f"{what} failed: {status_string(code)} (status {code})")


def dtype_code(t: torch.Tensor | torch.dtype) -> int:
    dt = t if isinstance(t, torch.dtype) else t.dtype
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def require_gpu(what: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device; returns it."""
    first = None
    idx = -1
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                f"{what}: tensors must be on a GPU (turboquant computes with HIP kernels only); "
                f"got a {t.device} tensor"
            )
        if first is None:
            first, idx = t, t.get_device()
        elif t.get_device() != idx:
            raise ValueError(f"{what}: tensors on different devices ({first.device}, {t.device})")
    if first is None:
        raise ValueError(f"{what}: no tensor arguments")
    return first.device


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of the device's current stream (torch's direct accessor where the
    build has it: a fraction of the cost of building a Stream object per call)."""
    if _RAW_STREAM is None:
        return torch.cuda.current_stream(device).cuda_stream
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _RAW_STREAM(idx)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_scale_cache: dict = {}


def centroid_scale(centroids: torch.Tensor) -> float:
    """Scale s in [1, 2) minimizing the worst relative fp16 rounding error of s * centroids.

    The decode kernels keep fp16 centroid tables; tabulating s * c and dividing s back out in
    fp32 makes the table nearly exact (3-bit: 1.8e-4 -> 1.8e-5).  Cached per tensor version, so a
    device-resident codebook is read back once."""
    key = (centroids.data_ptr(), centroids._version, centroids.numel(), str(centroids.device))
    hit = _scale_cache.get(key)
    if hit is not None:
        return hit
    import numpy as np

    c = centroids.detach().double().cpu().numpy().reshape(-1)
    c = c[c != 0]
    if c.size == 0 or np.abs(c).max() * 2 > 65504:
        best = 1.0
    else:
        s = 1.0 + np.arange(1 << 16, dtype=np.float64) / (1 << 16)
        best, best_err = 1.0, np.inf
        for lo in range(0, s.size, 1 << 12):
            v = s[lo:lo + (1 << 12), None] * c[None, :]
            err = (np.abs(v.astype(np.float16).astype(np.float64) - v) / np.abs(v)).max(axis=1)
            i = int(err.argmin())
            if err[i] < best_err:
                best, best_err = float(s[lo + i]), float(err[i])
    if len(_scale_cache) > 256:
        _scale_cache.clear()
    _scale_cache[key] = best
    return best
