"""Lloyd-Max codebooks for PolarQuant (host-side setup).

WHT-rotated unit vectors have roughly i.i.d. N(0, 1/d) coordinates; the codebook is the
Lloyd-Max quantizer of that Gaussian.  The iteration is the reference's
(turboquant/core/codebook.py:17-54): boundaries start uniform on [-6 sigma, 6 sigma], then 100
rounds of "centroid = conditional mean over its cell (scipy QUADPACK)" followed by
"boundary = midpoint of neighbouring centroids".  The integrand and the operation order are
kept identical so that the float values agree exactly with the reference on the same scipy.

For d = 128 (the head dimension of every kernel here) the solved codebooks of bits 1-4 are
committed in codebook_d128.json (written by make_codebook_table.py from the same solver) and
served from there, so hosts without scipy get the same floats; other d are solved on demand.
The table also holds the centroids of the kernel files' own recipe (kernels/packed_compress.py).
"""

from __future__ import annotations

import functools
import json
import math
import os
from typing import Optional

import torch

TABLE_D = 128
TABLE_BITS = (1, 2, 3, 4)
TABLE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "codebook_d128.json")


@functools.lru_cache(maxsize=None)
def _table() -> dict:
    with open(TABLE_PATH) as f:
        t = json.load(f)
    if t.get("d") != TABLE_D:
        raise ValueError(f"{TABLE_PATH}: expected d = {TABLE_D}")
    return {int(b): (tuple(v["centroids"]), tuple(v["boundaries"])) for b, v in t["bits"].items()}


@functools.lru_cache(maxsize=None)
def kernel_table() -> dict:
    """bits -> centroids of the kernel files' own codebook recipe for d = 128 (the variant that
    turboquant.kernels.packed_compress.solve_codebook computes), from the committed table."""
    with open(TABLE_PATH) as f:
        t = json.load(f)
    return {int(b): tuple(c) for b, c in t["kernel_recipe_centroids"].items()}


@functools.lru_cache(maxsize=None)
def _solve(d: int, bits: int) -> tuple[tuple[float, ...], tuple[float, ...]]:
    from scipy import integrate

    n_levels = 2 ** bits
    sigma = 1.0 / math.sqrt(d)

    def pdf(x):
        return (1.0 / math.sqrt(2 * math.pi * sigma**2)) * math.exp(-x * x / (2 * sigma**2))

    def first_moment(x):
        return x * pdf(x)

    lo, hi = -6 * sigma, 6 * sigma
    boundaries = [lo + (hi - lo) * i / n_levels for i in range(1, n_levels)]
    centroids = [0.0] * n_levels
    for _ in range(100):
        edges = [lo] + boundaries + [hi]
        for i in range(n_levels):
            num, _ = integrate.quad(first_moment, edges[i], edges[i + 1])
            den, _ = integrate.quad(pdf, edges[i], edges[i + 1])
            centroids[i] = num / max(den, 1e-30)
        boundaries = [(centroids[i] + centroids[i + 1]) / 2 for i in range(n_levels - 1)]
    return tuple(centroids), tuple(boundaries)


def solve_codebook(d: int, bits: int) -> tuple[list[float], list[float]]:
    """Optimal Lloyd-Max centroids (2^bits) and decision boundaries (2^bits - 1) for N(0, 1/d).

    Same contract as the reference's solve_codebook (turboquant/core/codebook.py:17).
    """
    if d <= 0 or bits <= 0:
        raise ValueError("d and bits must be positive")
    if int(d) == TABLE_D and int(bits) in TABLE_BITS:
        c, b = _table()[int(bits)]
    else:
        c, b = _solve(int(d), int(bits))
    return list(c), list(b)


def make_codebook(
    d: int = 128,
    bits: int = 3,
    device: Optional[torch.device] = None,
    dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Codebook tensors: centroids [2^bits], boundaries [2^bits - 1] (core/codebook.py:57-79)."""
    centroids, boundaries = solve_codebook(d, bits)
    return (
        torch.tensor(centroids, dtype=dtype, device=device),
        torch.tensor(boundaries, dtype=dtype, device=device),
    )
