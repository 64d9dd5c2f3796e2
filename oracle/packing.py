"""Bit-format oracle (test infrastructure only), numpy.

Per-token formats of the reference (all little-endian bit streams over a row of bytes):
  pack_indices(bits=2): byte j = sum_c idx[4j+c] << 2c          (kernels/packed_compress.py:79-90)
  pack_indices(bits=3): idx[d] in bits 3d..3d+2                  (kernels/sparse_v.py:57-60,82-98)
  pack_indices(bits=4): byte j = idx[2j] | idx[2j+1] << 4        (docs/design/AITER_TURBO4_DESIGN.md:57-76)
  pack_signs:           byte j bit b = s[8j+b], s = 1 for a >= 0 projection (packed_compress.py:77,92-106)
  permute_signs:        out bit 32c+k = in bit 4k+c              (packed_compress.py:180-216)
Each is written field by field (no shared helper between formats) so that a test checking one
against brute force over all field values exercises the rule itself.
"""

from __future__ import annotations

import numpy as np


def pack_indices(idx: np.ndarray, bits: int) -> np.ndarray:
    idx = np.asarray(idx, dtype=np.int64)
    n, d = idx.shape
    out = np.zeros((n, d * bits // 8), dtype=np.uint8)
    if bits == 2:
        for j in range(d // 4):
            v = np.zeros(n, dtype=np.int64)
            for c in range(4):
                v |= (idx[:, 4 * j + c] & 3) << (2 * c)
            out[:, j] = v
    elif bits == 4:
        for j in range(d // 2):
            out[:, j] = (idx[:, 2 * j] & 15) | ((idx[:, 2 * j + 1] & 15) << 4)
    elif bits in (1, 3):
        acc = np.zeros((n, d * bits // 8 + 1), dtype=np.int64)
        for dd in range(d):
            for b in range(bits):
                pos = bits * dd + b
                acc[:, pos >> 3] |= ((idx[:, dd] >> b) & 1) << (pos & 7)
        out[:] = acc[:, : d * bits // 8]
    else:
        raise ValueError(bits)
    return out


def unpack_indices(packed: np.ndarray, bits: int, d: int = 128) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.int64)
    n = packed.shape[0]
    out = np.zeros((n, d), dtype=np.int64)
    for dd in range(d):
        v = np.zeros(n, dtype=np.int64)
        for b in range(bits):
            pos = bits * dd + b
            v |= ((packed[:, pos >> 3] >> (pos & 7)) & 1) << b
        out[:, dd] = v
    return out


def pack_signs(bits01: np.ndarray) -> np.ndarray:
    bits01 = np.asarray(bits01, dtype=np.int64)
    n, d = bits01.shape
    out = np.zeros((n, d // 8), dtype=np.uint8)
    for j in range(d // 8):
        v = np.zeros(n, dtype=np.int64)
        for b in range(8):
            v |= (bits01[:, 8 * j + b] & 1) << b
        out[:, j] = v
    return out


def unpack_signs(packed: np.ndarray, d: int = 128) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.int64)
    out = np.zeros((packed.shape[0], d), dtype=np.int64)
    for dd in range(d):
        out[:, dd] = (packed[:, dd >> 3] >> (dd & 7)) & 1
    return out


def permute_signs(rows: np.ndarray, d: int = 128) -> np.ndarray:
    bits = unpack_signs(rows, d)
    dq = d // 4
    perm = np.zeros_like(bits)
    for c in range(4):
        perm[:, c * dq:(c + 1) * dq] = bits[:, c::4]
    return pack_signs(perm)


def f16_bytes(values: np.ndarray) -> np.ndarray:
    """fp16 (round to nearest even) little-endian bytes [n, 2]."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint8).reshape(-1, 2)
