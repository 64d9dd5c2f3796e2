"""The reference's PyTorch decode path in fp32 on the CPU (test infrastructure only).

This is the CPU baseline that bench.py times beside the GPU kernels, and a second restatement
of the decode oracle:
  - paged gather through the block table (integration/vllm_backend.py:223-230: block
    slot // bs, row slot % bs), then dequantisation by table gather, centroids[idx] * norm
    (core/quantizer.py:186-201, kernels/packed_attention.py:273-284);
  - scores = Q K_mse^T + corr_scale * rnorm * (Q_proj signs^T) by bmm, scaled by sm_scale
    (attention_unpacked_ref, kernels/packed_attention.py:273-284; QJL estimator of
    reference/pytorch_reference.py:123-158);
  - softmax and P V by bmm;
  - Sparse-V with the split-aware rule of the kernels (kernels/sparse_v.py:108-149): chunks of
    `chunk` tokens, a running max updated per `tile` tokens inside each chunk, token t's V
    dropped when max_h exp(s_h,t - m) <= threshold; dropped tokens stay in the denominator;
    chunks merged with the (m, l, acc) rule of kernels/attention.py:121-140.
Vectorised over whole sequences (cummax over tile maxima replaces the tile loop).

Pinned in tests/test_oracle.py against the float64 numpy oracle (oracle/decode.py), which is
itself pinned by pure-Python loops and closed forms.
"""

from __future__ import annotations

import math

import torch


def unpack_indices(packed: torch.Tensor, bits: int, d: int = 128) -> torch.Tensor:
    """uint8 [N, d*bits/8] little-endian bit stream -> int64 [N, d] (bits 2, 3, 4)."""
    p = packed.to(torch.int64)
    if bits == 4:
        return torch.stack([p & 15, p >> 4], dim=-1).reshape(p.shape[0], d)
    if bits == 2:
        return torch.stack([(p >> (2 * c)) & 3 for c in range(4)], dim=-1).reshape(p.shape[0], d)
    pos = torch.arange(d) * bits
    lo = p[:, pos >> 3]
    nxt = torch.clamp((pos >> 3) + 1, max=p.shape[1] - 1)
    hi = torch.where(((pos >> 3) + 1) < p.shape[1], p[:, nxt], torch.zeros_like(lo))
    return ((lo | (hi << 8)) >> (pos & 7)) & ((1 << bits) - 1)


def unpack_signs(packed: torch.Tensor, d: int = 128) -> torch.Tensor:
    """uint8 [N, d/8] -> float32 +-1 [N, d] (bit 1 -> +1)."""
    p = packed.to(torch.int64)
    b = torch.stack([(p >> k) & 1 for k in range(8)], dim=-1).reshape(p.shape[0], d)
    return b.to(torch.float32) * 2.0 - 1.0


def f16_bytes_to_f32(b: torch.Tensor) -> torch.Tensor:
    """uint8 [L, 2] little-endian fp16 -> float32 [L]."""
    return b.contiguous().view(torch.float16).reshape(-1).to(torch.float32)


def gather_rows(rows_cache: torch.Tensor, block_table: torch.Tensor, seq_len: int, head: int,
                block_size: int, idx_bytes: int, qjl: bool) -> dict:
    """Per-token payload of one (sequence, KV head) from tiles in the "rows" layout
    ([idx rows][sign rows][fp16 norms][fp16 rnorms]) through the block table."""
    nblk = -(-seq_len // block_size)
    tiles = rows_cache[block_table[:nblk].long(), head]               # [nblk, tile_bytes]
    off_norm = block_size * (idx_bytes + (16 if qjl else 0))
    out = {"idx": tiles[:, :block_size * idx_bytes].reshape(-1, idx_bytes)[:seq_len],
           "norm": tiles[:, off_norm:off_norm + 2 * block_size].reshape(-1, 2)[:seq_len]}
    if qjl:
        off_s = block_size * idx_bytes
        out["signs"] = tiles[:, off_s:off_s + 16 * block_size].reshape(-1, 16)[:seq_len]
        out["rnorm"] = tiles[:, off_norm + 2 * block_size:off_norm + 4 * block_size].reshape(-1, 2)[:seq_len]
    return out


def dequant(payload: dict, centroids: torch.Tensor, bits: int, qjl: bool):
    """(k_mse [L,128] f32, signs +-1 [L,128] or None, rnorm [L] or None); norms as uint8 [L, 2]."""
    idx = unpack_indices(payload["idx"], bits)
    norm = f16_bytes_to_f32(payload["norm"])
    k = centroids.to(torch.float32)[idx] * norm[:, None]
    if not qjl:
        return k, None, None
    signs = unpack_signs(payload["signs"])
    rnorm = f16_bytes_to_f32(payload["rnorm"])
    return k, signs, rnorm


def decode(q: torch.Tensor, qp: torch.Tensor | None, k_mse: torch.Tensor, signs, rnorm, v: torch.Tensor,
           sm_scale: float, corr_scale: float, chunk: int | None = None, threshold: float = 0.0,
           tile: int = 16):
    """q [G,128] over L tokens -> (out [G,128] f32, skipped tokens).  chunk None: one chunk."""
    G, L = q.shape[0], k_mse.shape[0]
    if L == 0:
        return torch.zeros_like(q), 0
    s = q @ k_mse.T
    if signs is not None:
        s = s + corr_scale * ((q if qp is None else qp) @ signs.T) * rnorm[None, :]
    s = s * sm_scale                                                   # [G, L]
    chunk = L if chunk is None else chunk
    ms, ls, accs = [], [], []
    skipped = 0
    for c0 in range(0, L, chunk):
        sc = s[:, c0:c0 + chunk]
        n = sc.shape[1]
        m = sc.max(dim=1).values
        p = torch.exp(sc - m[:, None])
        if threshold > 0:
            nt = -(-n // tile)
            pad = nt * tile - n
            tm = torch.nn.functional.pad(sc, (0, pad), value=-math.inf).reshape(G, nt, tile).max(dim=2).values
            run = torch.cummax(tm, dim=1).values                         # max through each tile
            run_t = run.repeat_interleave(tile, dim=1)[:, :n]
            keep = (torch.exp(sc - run_t) > threshold).any(dim=0)
            skipped += int((~keep).sum())
            pv = p * keep[None, :].to(p.dtype)
        else:
            pv = p
        ms.append(m)
        ls.append(p.sum(dim=1))
        accs.append(pv @ v[c0:c0 + chunk])
    M = torch.stack(ms).max(dim=0).values
    w = [torch.exp(m - M) for m in ms]
    den = sum(wi * li for wi, li in zip(w, ls))
    num = sum(wi[:, None] * ai for wi, ai in zip(w, accs))
    return num / den[:, None], skipped
