"""Decode-attention oracle (test infrastructure only), numpy float64.

Score of query head h on token t of its KV head kh = h // G (kernels/sparse_v.py:48):
    s = sm_scale * ( q . (k_cb[idx_t] * norm_t) + corr_scale * rnorm_t * (qp . sign_t) )
(attention_unpacked_ref, kernels/packed_attention.py:273-284; QJL estimator of
reference/pytorch_reference.py:123-158), out = softmax(s) . (v_cb[vidx_t] * vnorm_t).

decode_dense is the plain softmax.  decode_chunked follows the kernel's partition, which the
Sparse-V rule depends on (kernels/sparse_v.py:108-149): tokens are cut into chunks of
`chunk` tokens (or into given pieces: the kernel's balanced schedule) and each chunk is walked
in 16-token tiles with a running max m; after a tile
updates m, token t's V is dropped when max_h exp(s_h,t - m_h) <= threshold (h over the GQA
group), while exp(s - m) still enters the denominator.  Chunks are merged with the (m, l, acc)
rule of kernels/attention.py:121-140.  With threshold <= 0 it equals decode_dense.
"""

from __future__ import annotations

import numpy as np

from oracle.packing import unpack_indices, unpack_signs


def f16_to_f64(bits_u16: np.ndarray) -> np.ndarray:
    return np.asarray(bits_u16, dtype=np.uint16).view(np.float16).astype(np.float64)


def dequant_keys(payload: dict, centroids: np.ndarray, bits: int, qjl: bool, signs_permuted: bool = False):
    """(k_mse [L,128], sign +-1 [L,128] or None, rnorm [L] or None) in float64."""
    idx = unpack_indices(payload["idx"], bits)
    norm = f16_to_f64(payload["norm"])
    k = np.asarray(centroids, np.float64)[idx] * norm[:, None]
    if not qjl:
        return k, None, None
    bits01 = unpack_signs(payload["signs"])
    if signs_permuted:
        # permuted row bit 32c+k holds dim 4k+c
        nat = np.zeros_like(bits01)
        for c in range(4):
            nat[:, c::4] = bits01[:, 32 * c: 32 * (c + 1)]
        bits01 = nat
    return k, 2.0 * bits01 - 1.0, f16_to_f64(payload["rnorm"])


def dequant_values(payload: dict, centroids: np.ndarray, bits: int) -> np.ndarray:
    idx = unpack_indices(payload["idx"], bits)
    return np.asarray(centroids, np.float64)[idx] * f16_to_f64(payload["norm"])[:, None]


def scores(q: np.ndarray, qp: np.ndarray | None, k_mse, signs, rnorm, sm_scale: float, corr_scale: float):
    """q [G,128] -> scores [G, L]."""
    s = q @ k_mse.T
    if signs is not None:
        s = s + corr_scale * (qp @ signs.T) * rnorm[None, :]
    return sm_scale * s


def decode_dense(q, qp, k_mse, signs, rnorm, v, sm_scale, corr_scale):
    """q [G,128] over one KV head's L tokens -> out [G,128]."""
    if k_mse.shape[0] == 0:
        return np.zeros_like(q)
    s = scores(q, qp, k_mse, signs, rnorm, sm_scale, corr_scale)
    s = s - s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ v) / p.sum(axis=1, keepdims=True)


def _chunks(L: int, chunk):
    """(c0, c1) ranges: fixed chunks of `chunk` tokens, or, for a list of (t0, t1) pieces, those
    (the split of the kernel's balanced schedule)."""
    if isinstance(chunk, (int, np.integer)):
        return [(c0, min(c0 + int(chunk), L)) for c0 in range(0, L, int(chunk))]
    return [(int(a), min(int(b), L)) for a, b in chunk if a < L]


def decode_chunked(q, qp, k_mse, signs, rnorm, v, sm_scale, corr_scale, chunk,
                   threshold: float = 0.0, tile: int = 16):
    """Chunk/tile walk of the kernel; returns (out [G,128], skipped_tokens, total_tokens).
    chunk: tokens per chunk, or the list of (t0, t1) pieces of the sequence."""
    G = q.shape[0]
    L = k_mse.shape[0]
    if L == 0:
        return np.zeros_like(q), 0, 0
    s_all = scores(q, qp, k_mse, signs, rnorm, sm_scale, corr_scale)
    parts = []
    skipped = 0
    for c0, c1 in _chunks(L, chunk):
        m = np.full(G, -np.inf)
        lsum = np.zeros(G)
        acc = np.zeros((G, v.shape[1]))
        for t0 in range(c0, c1, tile):
            t1 = min(t0 + tile, c1)
            s = s_all[:, t0:t1]
            m_new = np.maximum(m, s.max(axis=1))
            alpha = np.exp(m - m_new)
            p = np.exp(s - m_new[:, None])
            lsum = lsum * alpha + p.sum(axis=1)
            keep = np.ones(t1 - t0, dtype=bool)
            if threshold > 0:
                keep = p.max(axis=0) > threshold
                skipped += int((~keep).sum())
            acc = acc * alpha[:, None] + (p * keep[None, :]) @ v[t0:t1]
            m = m_new
        parts.append((m, lsum, acc))
    M = np.max([pm for pm, _, _ in parts], axis=0)
    den = sum(np.exp(pm - M) * pl for pm, pl, _ in parts)
    num = sum(np.exp(pm - M)[:, None] * pa for pm, _, pa in parts)
    return num / den[:, None], skipped, L


def sparse_v_margins(q, qp, k_mse, signs, rnorm, sm_scale, corr_scale, chunk: int, tile: int = 16):
    """Per token t: max_h (s_h,t - m_h,t) in natural-log units, m_h,t being the running max of
    head h through t's tile inside t's chunk (the quantity decode_chunked compares with
    log(threshold)); [L]."""
    L = k_mse.shape[0]
    s_all = scores(q, qp, k_mse, signs, rnorm, sm_scale, corr_scale)
    out = np.empty(L)
    for c0, c1 in _chunks(L, chunk):
        m = np.full(q.shape[0], -np.inf)
        for t0 in range(c0, c1, tile):
            t1 = min(t0 + tile, c1)
            m = np.maximum(m, s_all[:, t0:t1].max(axis=1))
            out[t0:t1] = (s_all[:, t0:t1] - m[:, None]).max(axis=0)
    return out


def prefill_dense(q, qp, k_mse, signs, rnorm, v, sm_scale, corr_scale, causal: bool = True):
    """n query tokens [n, G, 128] (qp likewise, or None) over one KV head's L tokens, the new
    tokens being the last n of them -> out [n, G, 128].

    Query i sits at position L - n + i and, with causal, sees tokens 0 .. L - n + i (the limit
    of a serving extend step); without, all L tokens (the Sq > 1 kernel of
    kernels/attention.py:146-196 has no mask).  Each row is decode_dense over its visible tokens;
    a row that sees none is zero.
    """
    n, L = q.shape[0], k_mse.shape[0]
    out = np.zeros(q.shape)
    for i in range(n):
        lim = min(L, L - n + i + 1) if causal else L
        if lim <= 0:
            continue
        sg = signs[:lim] if signs is not None else None
        rn = rnorm[:lim] if rnorm is not None else None
        out[i] = decode_dense(q[i], qp[i] if qp is not None else q[i], k_mse[:lim], sg, rn, v[:lim],
                              sm_scale, corr_scale)
    return out
