"""PolarQuant configuration and the compression entry point.

PolarQuant splits each vector into its norm and a direction quantized coordinate-wise with a
Lloyd-Max codebook in the rotated space; keys add 1-bit QJL residual signs.  polarquant_compress
runs on the GPU (tq_polarquant_compress, a gfx950 kernel); PolarQuantConfig is host-side.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from turboquant import _lib
from turboquant.core.rotation import wht_magnitude


@dataclass
class PolarQuantConfig:
    """Compression settings (same fields and properties as core/quantizer.py:26-108).

    bits is the key index width (2^bits centroids); v_bits the value width (None: same as K);
    use_qjl adds residual sign bits to keys; the boundary-layer fields select layers that stay
    uncompressed.
    """

    head_dim: int = 128
    bits: int = 3
    v_bits: Optional[int] = None
    use_qjl: bool = True
    protect_boundary_layers: bool = True
    num_protected_layers: int = 2
    num_layers: int = 0

    @property
    def k_bits(self) -> int:
        return self.bits

    @property
    def effective_v_bits(self) -> int:
        return self.v_bits if self.v_bits is not None else self.bits

    @property
    def is_asymmetric(self) -> bool:
        return self.v_bits is not None and self.v_bits != self.bits

    def should_compress(self, layer_idx: int) -> bool:
        """False for the first and last num_protected_layers layers when protection is on."""
        if not self.protect_boundary_layers or self.num_layers == 0:
            return True
        if layer_idx < self.num_protected_layers:
            return False
        if layer_idx >= self.num_layers - self.num_protected_layers:
            return False
        return True

    @property
    def n_centroids(self) -> int:
        return 2 ** self.bits

    @property
    def compression_ratio(self) -> float:
        return self._compression_ratio_for_bits(self.bits)

    @property
    def k_compression_ratio(self) -> float:
        return self._compression_ratio_for_bits(self.k_bits)

    @property
    def v_compression_ratio(self) -> float:
        return self._compression_ratio_for_bits(self.effective_v_bits)

    @property
    def combined_compression_ratio(self) -> float:
        return 2.0 / (1.0 / self.k_compression_ratio + 1.0 / self.v_compression_ratio)

    def _compression_ratio_for_bits(self, bits: int) -> float:
        # fp16 bits over (index bits + one sign bit per dim for bits <= 3 + a 16-bit norm),
        # exactly the reference's accounting (core/quantizer.py:102-108).
        fp16_bits = 16 * self.head_dim
        if bits <= 3:
            total_bits = bits * self.head_dim + self.head_dim + 16
        else:
            total_bits = bits * self.head_dim + 16
        return fp16_bits / total_bits


def _rotation_mode(rotation_matrix: Optional[torch.Tensor], d: int) -> tuple[int, float]:
    """(1, h) for a Walsh-Hadamard matrix with entries +-h (rotated in registers), (0, 1) for
    None, (-1, 0) for any other [d, d] matrix (fp32 product kernel)."""
    if rotation_matrix is None:
        return 0, 1.0
    if tuple(rotation_matrix.shape) != (d, d):
        raise ValueError(f"rotation_matrix must be [{d}, {d}], got {tuple(rotation_matrix.shape)}")
    h = wht_magnitude(rotation_matrix)
    if h is None:
        return -1, 0.0
    return 1, h


def polarquant_compress(
    x: torch.Tensor,
    centroids: torch.Tensor,
    boundaries: torch.Tensor,
    config: PolarQuantConfig,
    rotation_matrix: Optional[torch.Tensor] = None,
) -> dict:
    """Compress vectors with PolarQuant on the GPU (core/quantizer.py:111-183).

    x: [N, D] or [B, H, D] (f32/f16/bf16, D = 128) on a GPU. rotation_matrix: None for
    pre-rotated input, the WHT matrix (rotated in registers) or any [D, D] matrix (fp32 product,
    x_rot = x @ rotation_matrix).  Returns the reference's dictionary:
      indices [*, D] int64, norms [N] f32 (flat also for 3-D input), k_mse_rot [*, D] f32 and,
      with config.use_qjl, signs [*, D] f32 (+-1) and rot_residual_norm [N] f32.
    """
    orig_shape = x.shape
    if x.dim() == 3:
        x = x.reshape(-1, x.shape[-1])
    if x.dim() != 2:
        raise ValueError(f"x must be [N, D] or [B, H, D], got {tuple(orig_shape)}")
    n, d = x.shape
    dev = _lib.require_gpu("polarquant_compress", x)
    if d != _lib.HEAD_DIM:
        raise ValueError(f"head_dim must be {_lib.HEAD_DIM}, got {d}")
    bits = config.bits
    if centroids.numel() != 2 ** bits or boundaries.numel() != 2 ** bits - 1:
        raise ValueError(f"codebook size does not match bits={bits}")
    rotate, scale = _rotation_mode(rotation_matrix, d)
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.float()
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 32:
        x = x.contiguous()
    cent = centroids.to(device=dev, dtype=torch.float32).contiguous()
    bnd = boundaries.to(device=dev, dtype=torch.float32).contiguous()

    indices = torch.empty((n, d), dtype=torch.int64, device=dev)
    norms = torch.empty((n,), dtype=torch.float32, device=dev)
    k_mse = torch.empty((n, d), dtype=torch.float32, device=dev)
    use_qjl = bool(config.use_qjl)
    signs = torch.empty((n, d), dtype=torch.float32, device=dev) if use_qjl else None
    rnorm = torch.empty((n,), dtype=torch.float32, device=dev) if use_qjl else None

    L = _lib.lib()
    if rotate < 0:
        rot = rotation_matrix.to(device=dev, dtype=torch.float32).contiguous()
        rc = L.tq_polarquant_compress_matrix(
            x.data_ptr(), _lib.dtype_code(x), x.stride(0), n, d, rot.data_ptr(),
            cent.data_ptr(), bnd.data_ptr(), bits, int(use_qjl),
            indices.data_ptr(), norms.data_ptr(), k_mse.data_ptr(), _lib.ptr(signs), _lib.ptr(rnorm),
            _lib.stream_handle(dev),
        )
        _lib.check(rc, "tq_polarquant_compress_matrix")
    else:
        rc = L.tq_polarquant_compress(
            x.data_ptr(), _lib.dtype_code(x), x.stride(0), n, d, rotate, scale,
            cent.data_ptr(), bnd.data_ptr(), bits, int(use_qjl),
            indices.data_ptr(), norms.data_ptr(), k_mse.data_ptr(), _lib.ptr(signs), _lib.ptr(rnorm),
            _lib.stream_handle(dev),
        )
        _lib.check(rc, "tq_polarquant_compress")

    result = {"indices": indices, "norms": norms, "k_mse_rot": k_mse}
    if use_qjl:
        result["signs"] = signs
        result["rot_residual_norm"] = rnorm
    if len(orig_shape) == 3:
        result["k_mse_rot"] = result["k_mse_rot"].reshape(orig_shape)
        result["indices"] = result["indices"].reshape(orig_shape)
        if "signs" in result:
            result["signs"] = result["signs"].reshape(orig_shape)
    return result


def polarquant_decompress(compressed: dict, centroids: torch.Tensor, config: PolarQuantConfig) -> torch.Tensor:
    """MSE reconstruction in the rotated space: the stored k_mse_rot (core/quantizer.py:186-201)."""
    return compressed["k_mse_rot"]


def compression_bytes_per_token(bits: int, use_qjl: bool, head_dim: int = 128) -> int:
    """Stored bytes per (token, head): index bits, fp16 norm, and signs + fp16 rnorm with QJL."""
    return head_dim * bits // 8 + 2 + ((head_dim // 8 + 2) if use_qjl else 0)

