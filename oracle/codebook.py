"""Codebook oracle (test infrastructure only).

solve_codebook_quad restates turboquant/core/codebook.py:17-54 (scipy QUADPACK, uniform
+-6 sigma initial boundaries, 100 Lloyd-Max rounds).  solve_codebook_closed_form runs the
same 100 rounds with exact Gaussian moments
    int_a^b x phi(x) dx = sigma^2 (phi(a) - phi(b)),
    int_a^b phi(x) dx   = (erf(b / (sigma sqrt 2)) - erf(a / (sigma sqrt 2))) / 2,
so any mistake in the restated iteration (initialisation, step count, sigma, update order)
shows up as a difference far above quadrature error.  kernel_codebook restates the kernel
files' variant (kernels/packed_compress.py:21-41) with closed-form moments.
"""

from __future__ import annotations

import math


def solve_codebook_quad(d: int, bits: int, iters: int = 100):
    from scipy import integrate

    n_levels = 2 ** bits
    sigma = 1.0 / math.sqrt(d)

    def pdf(x):
        return (1.0 / math.sqrt(2 * math.pi * sigma**2)) * math.exp(-x * x / (2 * sigma**2))

    lo, hi = -6 * sigma, 6 * sigma
    boundaries = [lo + (hi - lo) * i / n_levels for i in range(1, n_levels)]
    centroids = [0.0] * n_levels
    for _ in range(iters):
        edges = [lo] + boundaries + [hi]
        for i in range(n_levels):
            num, _ = integrate.quad(lambda x: x * pdf(x), edges[i], edges[i + 1])
            den, _ = integrate.quad(pdf, edges[i], edges[i + 1])
            centroids[i] = num / max(den, 1e-30)
        boundaries = [(centroids[i] + centroids[i + 1]) / 2 for i in range(n_levels - 1)]
    return centroids, boundaries


def _moments(a: float, b: float, sigma: float):
    phi = lambda x: math.exp(-x * x / (2 * sigma * sigma)) / (sigma * math.sqrt(2 * math.pi))
    num = sigma * sigma * (phi(a) - phi(b))
    s2 = sigma * math.sqrt(2.0)
    den = 0.5 * (math.erf(b / s2) - math.erf(a / s2))
    return num, den


def solve_codebook_closed_form(d: int, bits: int, iters: int = 100):
    n_levels = 2 ** bits
    sigma = 1.0 / math.sqrt(d)
    lo, hi = -6 * sigma, 6 * sigma
    boundaries = [lo + (hi - lo) * i / n_levels for i in range(1, n_levels)]
    centroids = [0.0] * n_levels
    for _ in range(iters):
        edges = [lo] + boundaries + [hi]
        for i in range(n_levels):
            num, den = _moments(edges[i], edges[i + 1], sigma)
            centroids[i] = num / max(den, 1e-30)
        boundaries = [(centroids[i] + centroids[i + 1]) / 2 for i in range(n_levels - 1)]
    return centroids, boundaries


def kernel_codebook(d: int, bits: int):
    """Centroids of kernels/packed_compress.py:21-41 (closed-form moments)."""
    n_levels = 2 ** bits
    sigma = 1.0 / math.sqrt(d)
    lo, hi = -3.5 * sigma, 3.5 * sigma
    centroids = [lo + (hi - lo) * (i + 0.5) / n_levels for i in range(n_levels)]
    for _ in range(200):
        boundaries = [(centroids[i] + centroids[i + 1]) / 2.0 for i in range(n_levels - 1)]
        edges = [lo * 3] + boundaries + [hi * 3]
        new_c = []
        for i in range(n_levels):
            num, den = _moments(edges[i], edges[i + 1], sigma)
            new_c.append(num / den if den > 1e-15 else centroids[i])
        if max(abs(new_c[i] - centroids[i]) for i in range(n_levels)) < 1e-10:
            break
        centroids = new_c
    return centroids


def lloyd_residual(centroids, boundaries, d: int) -> float:
    """Max |c_i - E[x | x in cell i]| and |b_i - (c_i + c_{i+1})/2| with closed-form moments;
    near zero at a Lloyd-Max fixed point."""
    sigma = 1.0 / math.sqrt(d)
    edges = [-12 * sigma] + list(boundaries) + [12 * sigma]
    worst = 0.0
    for i, c in enumerate(centroids):
        num, den = _moments(edges[i], edges[i + 1], sigma)
        worst = max(worst, abs(c - num / den))
    for i, b in enumerate(boundaries):
        worst = max(worst, abs(b - (centroids[i] + centroids[i + 1]) / 2))
    return worst
