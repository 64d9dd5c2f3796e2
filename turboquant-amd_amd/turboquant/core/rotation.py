"""Walsh-Hadamard rotation (host-side setup) and weight fusion.

The GPU kernels never multiply by a dense H: they run the 7-stage butterfly in registers and
scale by H's single magnitude h.  This module builds the dense matrix for the API and for
the host-side checks that a caller's rotation matrix is this WHT.

make_wht_matrix follows core/rotation.py:28-44: Sylvester doubling [[H, H], [H, -H]] with
a division by sqrt(2) at every level, so every entry is +-h with h the float32 result of
those successive divisions (h == float32(1/sqrt(d)) for d = 128), H symmetric and H @ H = I.
"""

from __future__ import annotations

import functools
import math
import weakref

import torch


def make_wht_matrix(d: int, device: torch.device = None) -> torch.Tensor:
    """Normalized Walsh-Hadamard matrix [d, d] (d a power of 2), H @ H = I."""
    if d <= 0 or d & (d - 1):
        raise ValueError(f"d must be a power of 2, got {d}")
    H = torch.tensor([[1.0]], device=device)
    while H.shape[0] < d:
        H = torch.cat([torch.cat([H, H], dim=1), torch.cat([H, -H], dim=1)], dim=0) / math.sqrt(2)
    return H[:d, :d]


@functools.lru_cache(maxsize=None)
def wht_scale(d: int = 128) -> float:
    """The magnitude h shared by all entries of make_wht_matrix(d), as the kernels use it.

    Computed once per d (building the matrix costs ~60 us of host time per call)."""
    return float(make_wht_matrix(d)[0, 0].item())


def _sylvester_signs(d: int) -> torch.Tensor:
    i = torch.arange(d).unsqueeze(1)
    j = torch.arange(d).unsqueeze(0)
    x = i & j
    parity = torch.zeros_like(x)
    while bool(x.any()):
        parity ^= x & 1
        x = x >> 1
    return 1 - 2 * parity  # (-1)^popcount(i & j)


# id(tensor) -> (weak reference, version counter, answer): a hit needs the same live tensor
# object at the same version, so a new tensor at a reused address is never mistaken for it.
_wht_cache: dict = {}


def wht_magnitude(rotation_matrix: torch.Tensor) -> float | None:
    """h if rotation_matrix == (-1)^popcount(i&j) * h exactly for one float h, else None.

    make_wht_matrix on different devices can round h differently; the kernels take the
    caller's own h, so any such matrix is accepted.  The answer is cached per tensor object and
    version (in-place writes bump it), so a device-resident matrix passed on every call is read
    back to the host once, not per call."""
    if rotation_matrix.dim() != 2 or rotation_matrix.shape[0] != rotation_matrix.shape[1]:
        return None
    d = rotation_matrix.shape[0]
    if d == 0 or d & (d - 1):
        return None
    hit = _wht_cache.get(id(rotation_matrix))
    if hit is not None and hit[0]() is rotation_matrix and hit[1] == rotation_matrix._version:
        return hit[2]
    m = rotation_matrix.detach().float().cpu()
    h = m[0, 0]
    res = float(h) if bool(h > 0) and bool(torch.equal(m, _sylvester_signs(d).float() * h)) else None
    if len(_wht_cache) > 256:
        _wht_cache.clear()
    _wht_cache[id(rotation_matrix)] = (weakref.ref(rotation_matrix), rotation_matrix._version, res)
    return res


def is_wht_matrix(rotation_matrix: torch.Tensor) -> bool:
    """True when rotation_matrix is a normalized Walsh-Hadamard matrix (sign pattern of
    make_wht_matrix, one magnitude)."""
    return wht_magnitude(rotation_matrix) is not None


def fuse_rotation_into_qkv_proj(
    qkv_weight: torch.Tensor,
    num_heads: int,
    num_kv_heads: int,
    head_size: int,
) -> torch.Tensor:
    """Fold the rotation into a packed [Q | K | V] projection weight [(nh + 2*nkv)*D, hidden].

    Each head's output rows are left-multiplied by H^T, so Q, K and V come out pre-rotated
    (core/rotation.py:47-91).  One-time weight preprocessing.
    """
    PiT = make_wht_matrix(head_size, device=qkv_weight.device).to(qkv_weight.dtype)
    q_size = num_heads * head_size
    k_size = num_kv_heads * head_size
    expected = q_size + 2 * k_size
    if qkv_weight.shape[0] != expected:
        raise ValueError(f"qkv_weight has {qkv_weight.shape[0]} rows, expected {expected}")
    heads = qkv_weight.reshape(num_heads + 2 * num_kv_heads, head_size, -1)
    fused = torch.matmul(PiT.T.contiguous(), heads)
    return fused.reshape(expected, -1)


def fuse_rotation_into_o_proj(o_weight: torch.Tensor, num_heads: int, head_size: int) -> torch.Tensor:
    """Fold the de-rotation into the output projection [hidden, nh*D] (core/rotation.py:94-111)."""
    Pi = make_wht_matrix(head_size, device=o_weight.device).to(o_weight.dtype)
    hidden = o_weight.shape[0]
    per_head = o_weight.reshape(hidden, num_heads, head_size)
    fused = torch.matmul(per_head, Pi.T.contiguous())
    return fused.reshape(hidden, num_heads * head_size)


def apply_weight_fusion(model_state_dict: dict, num_heads: int, num_kv_heads: int, head_size: int) -> dict:
    """Fuse the rotation into every qkv_proj / o_proj weight of a state dict, in place
    (core/rotation.py:114-140)."""
    for key in list(model_state_dict.keys()):
        if "qkv_proj.weight" in key:
            model_state_dict[key] = fuse_rotation_into_qkv_proj(
                model_state_dict[key], num_heads, num_kv_heads, head_size
            )
        elif "o_proj.weight" in key:
            model_state_dict[key] = fuse_rotation_into_o_proj(model_state_dict[key], num_heads, head_size)
    return model_state_dict
