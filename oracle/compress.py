"""PolarQuant compression oracle (test infrastructure only).

wht_matrix restates core/rotation.py:28-44; polarquant_compress restates
core/quantizer.py:135-183 with the same torch CPU operations in the same order, so on one
torch build its outputs equal the reference's bit for bit.

polarquant_compress_fp64 is the pinning shadow: the same math in float64 (rotation by the
exact +-h entries, no fp32 rounding), which any slip in the restated op sequence (order of
rotate / normalize, the 1e-8, tie side, clamp, sign of the residual) would contradict beyond
a few fp32 ulps.  boundary_band classifies index mismatches between two fp32 computations by
how far the value sits from the nearest boundary, in units of fp32 ulp at the coordinate
scale 1/sqrt(128) (ulp(2^-4) = 2^-27): the rotation's rounding is of that order.
"""

from __future__ import annotations

import math

import numpy as np
import torch

ULP_SIGMA = 2.0 ** -27  # fp32 ulp of values in [2^-4, 2^-3), the scale of N(0, 1/128) coordinates


def wht_matrix(d: int) -> torch.Tensor:
    H = torch.tensor([[1.0]])
    while H.shape[0] < d:
        H = torch.cat([torch.cat([H, H], dim=1), torch.cat([H, -H], dim=1)], dim=0) / math.sqrt(2)
    return H[:d, :d]


def wht_closed_form(d: int, h: float) -> np.ndarray:
    i = np.arange(d)[:, None]
    j = np.arange(d)[None, :]
    pc = np.vectorize(lambda v: bin(int(v)).count("1"))(i & j)
    return np.where(pc % 2 == 0, 1.0, -1.0) * h


def polarquant_compress(x: torch.Tensor, centroids: torch.Tensor, boundaries: torch.Tensor,
                        n_centroids: int, use_qjl: bool, rotation_matrix: torch.Tensor | None):
    """Reference op sequence on CPU tensors; returns the reference's dict."""
    x = x.cpu()
    orig_shape = x.shape
    if x.dim() == 3:
        x = x.reshape(-1, orig_shape[-1])
    N, D = x.shape
    if rotation_matrix is not None:
        x_rot = x.float() @ rotation_matrix.float().cpu()
    else:
        x_rot = x.float()
    norms = x_rot.norm(dim=-1)
    x_normalized = x_rot / (norms.unsqueeze(-1) + 1e-8)
    indices = torch.searchsorted(boundaries.float().cpu(), x_normalized.reshape(-1))
    indices = indices.clamp(0, n_centroids - 1).reshape(N, D)
    recon_normalized = centroids.cpu()[indices]
    k_mse_rot = recon_normalized * norms.unsqueeze(-1)
    result = {"indices": indices, "norms": norms, "k_mse_rot": k_mse_rot, "x_normalized": x_normalized}
    if use_qjl:
        rot_residual = (x_normalized - recon_normalized) * norms.unsqueeze(-1)
        result["rot_residual_norm"] = rot_residual.norm(dim=-1)
        signs = torch.sign(rot_residual)
        signs[signs == 0] = 1.0
        result["signs"] = signs
    if len(orig_shape) == 3:
        for k in ("k_mse_rot", "indices", "signs", "x_normalized"):
            if k in result:
                result[k] = result[k].reshape(orig_shape)
    return result


def polarquant_compress_fp64(x: torch.Tensor, centroids: torch.Tensor, boundaries: torch.Tensor,
                             use_qjl: bool, rotate: bool, matrix: torch.Tensor | None = None):
    """float64 shadow: x_n = (x @ H) / (|x @ H| + 1e-8) with H = +-h exactly (or the given
    matrix, its fp32 entries taken exactly); idx = #{b < x_n}."""
    x64 = x.detach().cpu().double().reshape(-1, x.shape[-1])
    D = x64.shape[1]
    if matrix is not None:
        x_rot = x64 @ matrix.detach().cpu().double()
    elif rotate:
        h = float(wht_matrix(D)[0, 0])
        H = torch.from_numpy(wht_closed_form(D, h))
        x_rot = x64 @ H
    else:
        x_rot = x64
    norms = x_rot.norm(dim=-1)
    xn = x_rot / (norms.unsqueeze(-1) + 1e-8)
    b = boundaries.double().cpu()
    idx = (xn.unsqueeze(-1) > b).sum(-1)
    c = centroids.double().cpu()
    out = {"indices": idx, "norms": norms, "x_normalized": xn}
    if use_qjl:
        r = (xn - c[idx]) * norms.unsqueeze(-1)
        out["rot_residual_norm"] = r.norm(dim=-1)
        out["signs"] = torch.where(r >= 0, 1.0, -1.0).double()
    return out


def boundary_band(xn: torch.Tensor, boundaries: torch.Tensor) -> torch.Tensor:
    """Distance of each value to its nearest boundary, in units of ULP_SIGMA."""
    d = (xn.double().unsqueeze(-1) - boundaries.double().cpu()).abs().min(dim=-1).values
    return d / ULP_SIGMA


def centroid_band(xn: torch.Tensor, centroids: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """Distance of each value to its own centroid (where QJL signs flip), in ULP_SIGMA units."""
    c = centroids.double().cpu()[idx.long().cpu()]
    return (xn.double().cpu() - c).abs() / ULP_SIGMA


def classify_index_mismatch(idx_test: torch.Tensor, idx_ref: torch.Tensor, xn_ref: torch.Tensor,
                            boundaries: torch.Tensor, band_ulps: float):
    """(n_mismatch, n_in_band, n_out_of_band, max_band) of index differences: a mismatch is
    'in band' when the reference value lies within band_ulps ULP_SIGMA of a boundary and the
    two indices are adjacent."""
    t = idx_test.long().cpu().reshape(-1)
    r = idx_ref.long().cpu().reshape(-1)
    mism = t != r
    n = int(mism.sum())
    if n == 0:
        return 0, 0, 0, 0.0
    band = boundary_band(xn_ref.reshape(-1)[mism], boundaries)
    adjacent = (t[mism] - r[mism]).abs() == 1
    ok = (band <= band_ulps) & adjacent
    return n, int(ok.sum()), int((~ok).sum()), float(band.max())


def compress_packed(x: np.ndarray, pit: np.ndarray, pist: np.ndarray | None, centroids: np.ndarray,
                    boundaries: np.ndarray):
    """Restates _fully_packed_k / _fully_packed_v (kernels/packed_compress.py:64-106,118-142) in
    float64 with exact products (the reference's fp16 tl.dot rounding is not a target):
        norm = |x|; x_n = x * (1 / (norm + 1e-8)); rot = x_n @ PiT; idx = #{b <= rot}  (>= rule)
        resid = (rot - c[idx]) * norm; rnorm = |resid|; proj = resid @ PiST; sign = proj >= 0.
    Returns a dict of float64 / int arrays with the decision margins the tests classify by:
    rot_margin = |rot - nearest boundary|, proj_scale = sum_d |resid_d * PiST_dj| (the size of
    the terms summed into proj_j)."""
    x = np.asarray(x, dtype=np.float64).reshape(-1, x.shape[-1])
    c = np.asarray(centroids, dtype=np.float64)
    b = np.asarray(boundaries, dtype=np.float64)
    norm = np.sqrt((x * x).sum(axis=1))
    xn = x * (1.0 / (norm + 1e-8))[:, None]
    rot = xn @ np.asarray(pit, dtype=np.float64)
    idx = (rot[..., None] >= b).sum(axis=-1)
    out = {"norm": norm, "rot": rot, "idx": idx,
           "rot_margin": np.abs(rot[..., None] - b).min(axis=-1) if b.size else np.full(rot.shape, np.inf)}
    if pist is not None:
        P = np.asarray(pist, dtype=np.float64)
        resid = (rot - c[idx]) * norm[:, None]
        proj = resid @ P
        out.update(resid=resid, rnorm=np.sqrt((resid * resid).sum(axis=1)), proj=proj,
                   sign=(proj >= 0).astype(np.uint8), proj_scale=np.abs(resid) @ np.abs(P))
    return out


def ulp32(v) -> np.ndarray:
    """Spacing of float32 at |v| (the fp32 ulp of each value), float64."""
    a = np.abs(np.asarray(v, dtype=np.float64)).astype(np.float32)
    return np.spacing(a).astype(np.float64)


def classify_strict(idx_test, idx_ref, x_ref, boundaries, idx_fp64):
    """Index mismatches of a test computation against the fp32 reference restatement, under the
    contract "bit-exact except elements within 1 ulp of a codebook boundary".

    For each mismatch, the boundary between the two indices is b[min(i, j)] (left searchsorted:
    idx = #{b < x}); its distance from the reference value is counted in fp32 ulps of
    max(|x_ref|, |b|).  A mismatch within 1 ulp is accepted; one further out is accepted only
    when the test index equals the float64 shadow's (the reference's fp32 rounding put it on the
    wrong side).  Returns a dict of counts; `failures` must be 0."""
    t = np.asarray(idx_test, dtype=np.int64).reshape(-1)
    r = np.asarray(idx_ref, dtype=np.int64).reshape(-1)
    f = np.asarray(idx_fp64, dtype=np.int64).reshape(-1)
    x = np.asarray(x_ref, dtype=np.float64).reshape(-1)
    b = np.asarray(boundaries, dtype=np.float64).reshape(-1)
    mism = np.nonzero(t != r)[0]
    out = {"elements": int(t.size), "mismatches": int(mism.size), "within_1ulp": 0, "ulp_1_to_8": 0,
           "ulp_over_8": 0, "beyond_1ulp_test_equals_fp64": 0, "failures": 0, "ref_differs_from_fp64": int((r != f).sum()),
           "test_differs_from_fp64": int((t != f).sum())}
    if mism.size == 0:
        return out
    adjacent = np.abs(t[mism] - r[mism]) == 1
    k = np.clip(np.minimum(t[mism], r[mism]), 0, max(b.size - 1, 0))
    bb = b[k] if b.size else np.zeros(mism.size)
    d = np.abs(x[mism] - bb) / np.maximum(ulp32(np.maximum(np.abs(x[mism]), np.abs(bb))), 1e-300)
    d = np.where(adjacent, d, np.inf)
    le1 = d <= 1.0
    out["within_1ulp"] = int(le1.sum())
    out["ulp_1_to_8"] = int(((d > 1.0) & (d <= 8.0)).sum())
    out["ulp_over_8"] = int((d > 8.0).sum())
    eq64 = t[mism] == f[mism]
    out["beyond_1ulp_test_equals_fp64"] = int((~le1 & eq64).sum())
    out["failures"] = int((~le1 & ~eq64).sum())
    return out


def classify_strict_fp64(idx_test, idx_fp64, x_fp64, boundaries):
    """classify_strict when the reference itself is the float64 restatement (compress_k /
    compress_v, whose fp16 tl.dot products are not a target): a mismatch is accepted only within
    1 fp32 ulp of the boundary."""
    return classify_strict(idx_test, idx_fp64, x_fp64, boundaries, idx_fp64)
