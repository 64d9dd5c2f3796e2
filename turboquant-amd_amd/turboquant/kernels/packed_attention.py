"""Packed attention on contiguous per-head arrays (drop-in for the reference's v7 API).

packed_attention keeps the signature of kernels/packed_attention.py:290-344 and reads the
same arrays: 2-bit K/V indices [BH, Sk, 32], stride-4 permuted QJL sign rows [BH, Sk, 16],
fp16 norms / residual norms [BH, Sk].  It runs the paged decode kernel (tq_decode) with a
"contiguous" view: each of the BH query heads is a sequence with its own KV (no GQA), blocks
of 16 tokens addressed by stride instead of a block table.

Differences from the reference, by design:
  - the split combine is the correct (m, l, acc) merge (kernels/attention.py:121-140), not
    the LSE-weighted average of packed_attention.py:199-227 that is off by the per-split
    softmax denominators;
  - Q_proj * corr_scale is formed in fp32 inside the kernel instead of rounding to fp16 first.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from turboquant import _lib
from turboquant.kernels.packed_compress import unpack_1bit, unpack_2bit  # noqa: F401  (API parity)
from turboquant.kernels.paged import MI355X_CUS, run_decode

BLOCK = 16


def _chunk_for(BH: int, Sk: int, num_splits: int | None) -> int:
    if num_splits is not None and num_splits > 0:
        per = math.ceil(Sk / num_splits)
    else:
        per = math.ceil(Sk * BH / (MI355X_CUS * 16))
        per = max(per, 64)
    return int(math.ceil(max(per, 1) / BLOCK) * BLOCK)


def _get_config(BH: int, Sk: int):
    """(BLOCK_SK, num_splits, waves_per_workgroup, stages) this implementation uses for (BH, Sk).

    Same tuple shape as the reference's tuning lookup (kernels/packed_attention.py:258-267);
    the values describe the HIP kernel: 16-token tiles, split count from the chunk length.
    """
    chunk = _chunk_for(BH, Sk, None)
    return BLOCK, max(1, math.ceil(Sk / chunk)), 4, 1


def _contig_region(t: torch.Tensor, row_bytes: int, Sk: int) -> _lib.TQRegion:
    return _lib.TQRegion(t.data_ptr(), BLOCK * row_bytes, 0, Sk * row_bytes, row_bytes)


def packed_attention(Q, Q_proj, k_idx_packed, k_signs_packed, k_r_norm, k_norm,
                     v_idx_packed, v_norm, centroids, corr_scale,
                     num_splits=None, block_sk=None, num_warps=None, num_stages=None):
    """Split-K decode over packed 2-bit K (+ QJL) and 2-bit V; returns fp16 [BH, D].

    Q, Q_proj: [BH, D] (any float dtype; scores are not scaled, the caller pre-scales Q).
    k_signs_packed must be in the permuted order (permute_signs_for_chunked).
    num_splits selects the split count; block_sk / num_warps / num_stages are Triton tuning
    knobs of the reference and are accepted and ignored.
    """
    dev = _lib.require_gpu("packed_attention", Q, Q_proj, k_idx_packed, k_signs_packed, k_r_norm, k_norm,
                           v_idx_packed, v_norm, centroids)
    BH, D = Q.shape
    if D != 128:
        raise ValueError("head_dim must be 128")
    Sk = k_r_norm.shape[1]
    shapes = {
        "k_idx_packed": (k_idx_packed, (BH, Sk, D // 4), torch.uint8),
        "k_signs_packed": (k_signs_packed, (BH, Sk, D // 8), torch.uint8),
        "v_idx_packed": (v_idx_packed, (BH, Sk, D // 4), torch.uint8),
        "k_r_norm": (k_r_norm, (BH, Sk), torch.float16),
        "k_norm": (k_norm, (BH, Sk), torch.float16),
        "v_norm": (v_norm, (BH, Sk), torch.float16),
    }
    ts = {}
    for name, (t, shape, dt) in shapes.items():
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must be {shape}, got {tuple(t.shape)}")
        if t.dtype == torch.int8 and dt == torch.uint8:
            t = t.view(torch.uint8)
        if t.dtype != dt:
            raise TypeError(f"{name} must be {dt}")
        ts[name] = t.contiguous()
    if centroids.numel() != 4:
        raise ValueError("packed_attention uses a 2-bit codebook (4 centroids)")
    cb = centroids.to(device=dev, dtype=torch.float32).contiguous()
    q = Q.reshape(BH, 1, D)
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        q = q.float()
    qp = Q_proj.reshape(BH, 1, D).to(q.dtype)
    q = q.contiguous()
    qp = qp.contiguous()

    kv = _lib.TQKVView()
    kv.idx = _contig_region(ts["k_idx_packed"], D // 4, Sk)
    kv.signs = _contig_region(ts["k_signs_packed"], D // 8, Sk)
    kv.norm = _contig_region(ts["k_norm"], 2, Sk)
    kv.rnorm = _contig_region(ts["k_r_norm"], 2, Sk)
    kv.centroids = cb.data_ptr()
    kv.bits, kv.qjl, kv.signs_permuted = 2, 1, 1
    kv.centroid_scale = _lib.centroid_scale(cb)
    vv = _lib.TQKVView()
    vv.idx = _contig_region(ts["v_idx_packed"], D // 4, Sk)
    vv.norm = _contig_region(ts["v_norm"], 2, Sk)
    vv.centroids = cb.data_ptr()
    vv.bits, vv.qjl, vv.signs_permuted = 2, 0, 0
    vv.centroid_scale = kv.centroid_scale

    seq_lens = torch.full((BH,), Sk, dtype=torch.int32, device=dev)
    out = torch.empty((BH, 1, D), dtype=torch.float16, device=dev)
    chunk = _chunk_for(BH, Sk, num_splits)
    nblk = math.ceil(Sk / BLOCK)
    run_decode(q, kv, vv, num_kv_heads=1, block_size=BLOCK, num_blocks=nblk, block_tables=None,
               max_blocks_per_seq=nblk, seq_lens=seq_lens, max_seq_len=Sk, sm_scale=1.0,
               corr_scale=float(corr_scale), q_proj=qp, sparse_threshold=0.0, tokens_per_chunk=chunk,
               out=out, workspace=None, skip_stats=None, keep_alive=(cb, ts))
    return out.reshape(BH, D)


def attention_unpacked_ref(Q, Q_proj, K_mse_rot, signs_float, k_r_norm, V_mse_rot, corr_scale):
    """Reference formulation on unpacked data (kernels/packed_attention.py:273-284).

    scores = Q.K_mse^T + Q_proj.(signs * rnorm * corr_scale)^T; softmax; . V_mse.  Plain torch
    ops, kept for API parity and as the formula the packed kernels are checked against.
    """
    score_mse = torch.bmm(Q.unsqueeze(1), K_mse_rot.transpose(1, 2).contiguous()).squeeze(1)
    K_qjl = signs_float * k_r_norm.unsqueeze(-1) * corr_scale
    score_qjl = torch.bmm(Q_proj.unsqueeze(1), K_qjl.transpose(1, 2).contiguous()).squeeze(1)
    attn = F.softmax(score_mse + score_qjl, dim=-1)
    return torch.bmm(attn.unsqueeze(1), V_mse_rot).squeeze(1)
