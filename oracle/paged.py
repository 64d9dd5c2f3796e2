"""Paged-cache oracle (test infrastructure only), numpy.

Per-token payload -> tile layout of the paged cache, written token by token:
  tile (block, head) = [bs x 16*bits idx][bs x 16 signs]? [bs x fp16 norm][bs x fp16 rnorm]?
(signs/rnorm for QJL keys only), token at slot s -> block s // bs, row s % bs
(integration/vllm_backend.py:223-230), negative or out-of-range slots dropped.
Reference array-of-slots layout [num_blocks, bs, Hkv, slot] (kernels/sparse_v.py:293-304):
per token idx bytes, [signs], fp16 norm, [fp16 rnorm], zero padding.
"""

from __future__ import annotations

import numpy as np


def tile_offsets(block_size: int, bits: int, qjl: bool):
    idx_row = 16 * bits
    off_signs = block_size * idx_row
    off_norm = block_size * (idx_row + (16 if qjl else 0))
    off_rnorm = off_norm + 2 * block_size
    tile = off_norm + 2 * block_size * (2 if qjl else 1)
    return idx_row, off_signs, off_norm, off_rnorm, tile


def scatter_tokens(payload: dict, slot_mapping: np.ndarray, num_blocks: int, num_heads: int,
                   block_size: int, bits: int, qjl: bool, cache: np.ndarray | None = None) -> np.ndarray:
    """payload[name]: per (token, head) arrays — idx [T,H,16b] u8, signs [T,H,16] u8,
    norm [T,H] u16 bits, rnorm [T,H] u16 bits.  Returns uint8 [num_blocks, H, tile]."""
    idx_row, off_signs, off_norm, off_rnorm, tile = tile_offsets(block_size, bits, qjl)
    if cache is None:
        cache = np.zeros((num_blocks, num_heads, tile), dtype=np.uint8)
    T = len(slot_mapping)
    for t in range(T):
        s = int(slot_mapping[t])
        if s < 0 or s >= num_blocks * block_size:
            continue
        blk, row = divmod(s, block_size)
        for h in range(num_heads):
            c = cache[blk, h]
            c[row * idx_row:(row + 1) * idx_row] = payload["idx"][t, h]
            c[off_norm + 2 * row: off_norm + 2 * row + 2] = np.array(
                [payload["norm"][t, h] & 0xFF, payload["norm"][t, h] >> 8], dtype=np.uint8)
            if qjl:
                c[off_signs + 16 * row: off_signs + 16 * row + 16] = payload["signs"][t, h]
                c[off_rnorm + 2 * row: off_rnorm + 2 * row + 2] = np.array(
                    [payload["rnorm"][t, h] & 0xFF, payload["rnorm"][t, h] >> 8], dtype=np.uint8)
    return cache


def gather_sequence(cache: np.ndarray, block_table: np.ndarray, seq_len: int, head: int,
                    block_size: int, bits: int, qjl: bool) -> dict:
    """Per-token payload of one (sequence, head) read back through the block table."""
    idx_row, off_signs, off_norm, off_rnorm, _ = tile_offsets(block_size, bits, qjl)
    out = {"idx": np.zeros((seq_len, idx_row), np.uint8), "norm": np.zeros(seq_len, np.uint16)}
    if qjl:
        out["signs"] = np.zeros((seq_len, 16), np.uint8)
        out["rnorm"] = np.zeros(seq_len, np.uint16)
    for t in range(seq_len):
        blk = int(block_table[t // block_size])
        row = t % block_size
        c = cache[blk, head]
        out["idx"][t] = c[row * idx_row:(row + 1) * idx_row]
        out["norm"][t] = int(c[off_norm + 2 * row]) | (int(c[off_norm + 2 * row + 1]) << 8)
        if qjl:
            out["signs"][t] = c[off_signs + 16 * row: off_signs + 16 * row + 16]
            out["rnorm"][t] = int(c[off_rnorm + 2 * row]) | (int(c[off_rnorm + 2 * row + 1]) << 8)
    return out


def to_slots(cache: np.ndarray, block_size: int, bits: int, qjl: bool, slot_bytes: int) -> np.ndarray:
    """Tile layout -> reference array-of-slots [num_blocks, bs, H, slot_bytes], per token."""
    nb, H, _ = cache.shape
    idx_row, off_signs, off_norm, off_rnorm, _ = tile_offsets(block_size, bits, qjl)
    out = np.zeros((nb, block_size, H, slot_bytes), dtype=np.uint8)
    for b in range(nb):
        for h in range(H):
            c = cache[b, h]
            for r in range(block_size):
                parts = [c[r * idx_row:(r + 1) * idx_row]]
                if qjl:
                    parts.append(c[off_signs + 16 * r: off_signs + 16 * r + 16])
                parts.append(c[off_norm + 2 * r: off_norm + 2 * r + 2])
                if qjl:
                    parts.append(c[off_rnorm + 2 * r: off_rnorm + 2 * r + 2])
                p = np.concatenate(parts)
                out[b, r, h, :len(p)] = p
    return out
