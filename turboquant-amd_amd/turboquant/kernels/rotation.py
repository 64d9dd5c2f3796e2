"""Stand-alone Walsh-Hadamard rotation of 128-element rows on the GPU.

wht_rows(x) = x @ make_wht_matrix(128) (the matrix is symmetric and its own inverse), computed
with fp32 butterflies by tq_wht_rows.  It is the operation of the reference backend's
TurboQuantFP8State.rotate_query / rotate_output (integration/vllm_backend.py:158-177) for
callers that rotate outside the decode call; decode_paged(..., rotate=True) fuses both
rotations into the decode kernels instead.
"""

from __future__ import annotations

from typing import Optional

import torch

from turboquant import _lib


def wht_rows(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x @ make_wht_matrix(128) over the last dimension (f32 / f16 / bf16 GPU tensors).

    out: optional destination of x's shape (any of the three dtypes); it may be x itself.
    """
    _lib.require_gpu("wht_rows", x)
    if x.dim() < 1 or x.shape[-1] != 128:
        raise ValueError("the last dimension must be 128")
    if out is None:
        out = torch.empty_like(x)
    if out.shape != x.shape or out.device != x.device:
        raise ValueError("out must have x's shape and device")

    def rows3(t: torch.Tensor) -> torch.Tensor:
        if t.dim() == 3 and t.stride(2) == 1:
            return t
        if t.dim() == 2 and t.stride(1) == 1:
            return t.unsqueeze(1)
        return t.reshape(-1, 1, 128) if t.is_contiguous() else None

    xs = rows3(x)
    if xs is None:
        xs = rows3(x.contiguous())
    os_ = rows3(out)
    target = out
    if os_ is None:  # a non-contiguous destination of another shape: write a copy back
        target = torch.empty_like(x, memory_format=torch.contiguous_format)
        os_ = rows3(target)
    if xs.shape[0] * xs.shape[1] == 0:
        return out
    rc = _lib.lib().tq_wht_rows(
        xs.data_ptr(), _lib.dtype_code(xs), xs.stride(0), xs.stride(1), xs.shape[0], xs.shape[1], 128,
        os_.data_ptr(), _lib.dtype_code(os_), os_.stride(0), os_.stride(1), _lib.stream_handle(x.device))
    _lib.check(rc, "tq_wht_rows")
    if target is not out:
        out.copy_(target)
    return out
