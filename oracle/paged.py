"""Paged-cache oracle (test infrastructure only), numpy.

Per-token payload -> tile of the paged cache, token at slot s -> block s // bs, row s % bs
(integration/vllm_backend.py:223-230), negative or out-of-range slots dropped.  A tile is
[payload: bs x (16*bits idx + 16 signs?) bytes][bs x fp16 norm][bs x fp16 rnorm]? (signs and
rnorm for QJL keys only).  The payload order is the layout:
  "rows"  : all idx rows (16*bits bytes each), then all sign rows (16 bytes each);
  "keys"  : per 16-row sub-tile, for row n = 0..15 and dim quarter g = 0..3, one chunk: the
            idx bytes of dims 32g..32g+31 of row n, then (QJL) their 4 sign bytes;
  "values": per 16-row sub-tile, for row group g = 0..3 and dim group n = 0..15, one chunk of
            4*bits bytes: a little-endian stream of 32 bits-wide fields, field 4j + r holding
            the index of dim 8n + j of row 4g + r (dimension-major: the four rows' fields of one
            dim are adjacent).
Here the sub-tiles are assembled chunk by chunk (build_subtile / split_subtile) rather than
through byte-position formulas.
Reference array-of-slots layout [num_blocks, bs, Hkv, slot] (kernels/sparse_v.py:293-304):
per token idx bytes, [signs], fp16 norm, [fp16 rnorm], zero padding.
"""

from __future__ import annotations

import numpy as np

from oracle import packing as _pack


def tile_offsets(block_size: int, bits: int, qjl: bool):
    """(idx row bytes, sign rows offset ("rows" layout), norm offset, rnorm offset, tile bytes)."""
    idx_row = 16 * bits
    off_signs = block_size * idx_row
    off_norm = block_size * (idx_row + (16 if qjl else 0))
    off_rnorm = off_norm + 2 * block_size
    tile = off_norm + 2 * block_size * (2 if qjl else 1)
    return idx_row, off_signs, off_norm, off_rnorm, tile


def build_subtile(idx: np.ndarray, signs: np.ndarray | None, bits: int, layout: str) -> bytes:
    """Payload bytes of 16 rows (idx [16, 16*bits], signs [16, 16] or None) in a lane-grouped
    layout, assembled chunk by chunk."""
    out = bytearray()
    if layout == "keys":
        for n in range(16):
            for g in range(4):
                out += bytes(idx[n, 4 * bits * g: 4 * bits * (g + 1)])
                if signs is not None:
                    out += bytes(signs[n, 4 * g: 4 * g + 4])
    elif layout == "values":
        assert signs is None
        f = _pack.unpack_indices(idx, bits)           # [16 rows, 128 dims]
        for g in range(4):
            for n in range(16):
                fields = [int(f[4 * g + r, 8 * n + j]) for j in range(8) for r in range(4)]
                out += bytes(_pack.pack_indices(np.array([fields]), bits)[0])
    else:
        raise ValueError(layout)
    return bytes(out)


def split_subtile(buf: bytes, bits: int, qjl: bool, layout: str):
    """Inverse of build_subtile: (idx [16, 16*bits], signs [16, 16] or None)."""
    idx = np.zeros((16, 16 * bits), np.uint8)
    signs = np.zeros((16, 16), np.uint8) if qjl else None
    it = iter(buf)
    take = lambda k: np.array([next(it) for _ in range(k)], np.uint8)  # noqa: E731
    if layout == "keys":
        for n in range(16):
            for g in range(4):
                idx[n, 4 * bits * g: 4 * bits * (g + 1)] = take(4 * bits)
                if qjl:
                    signs[n, 4 * g: 4 * g + 4] = take(4)
    else:
        f = np.zeros((16, 128), np.int64)
        for g in range(4):
            for n in range(16):
                fields = _pack.unpack_indices(take(4 * bits)[None], bits, 32)[0]
                for j in range(8):
                    for r in range(4):
                        f[4 * g + r, 8 * n + j] = fields[4 * j + r]
        idx[:] = _pack.pack_indices(f, bits)
    return idx, signs


def _tile_rows(tile: np.ndarray, block_size: int, bits: int, qjl: bool, layout: str):
    """(idx [bs, 16*bits], signs [bs, 16] or None) of one tile in any layout."""
    idx_row, off_signs, _, _, _ = tile_offsets(block_size, bits, qjl)
    if layout == "rows":
        idx = tile[:block_size * idx_row].reshape(block_size, idx_row).copy()
        signs = tile[off_signs:off_signs + 16 * block_size].reshape(block_size, 16).copy() if qjl else None
        return idx, signs
    P = idx_row + (16 if qjl else 0)
    if layout == "values":
        return values_subtiles_to_rows(tile[:block_size * P].reshape(block_size // 16, 16 * P), bits), None
    idx = np.zeros((block_size, idx_row), np.uint8)
    signs = np.zeros((block_size, 16), np.uint8) if qjl else None
    for j in range(block_size // 16):
        i_, s_ = split_subtile(tile[16 * P * j: 16 * P * (j + 1)].tobytes(), bits, qjl, layout)
        idx[16 * j:16 * j + 16] = i_
        if qjl:
            signs[16 * j:16 * j + 16] = s_
    return idx, signs


def _set_tile_rows(tile: np.ndarray, idx: np.ndarray, signs, block_size: int, bits: int, qjl: bool, layout: str):
    idx_row, off_signs, _, _, _ = tile_offsets(block_size, bits, qjl)
    if layout == "rows":
        tile[:block_size * idx_row] = idx.reshape(-1)
        if qjl:
            tile[off_signs:off_signs + 16 * block_size] = signs.reshape(-1)
        return
    P = idx_row + (16 if qjl else 0)
    if layout == "values":
        # vectorised form of build_subtile (the two are checked against each other)
        tile[:block_size * P] = rows_to_values_subtiles(idx, bits).reshape(-1)
        return
    for j in range(block_size // 16):
        b = build_subtile(idx[16 * j:16 * j + 16], signs[16 * j:16 * j + 16] if qjl else None, bits, layout)
        tile[16 * P * j: 16 * P * (j + 1)] = np.frombuffer(b, np.uint8)


def scatter_tokens(payload: dict, slot_mapping: np.ndarray, num_blocks: int, num_heads: int,
                   block_size: int, bits: int, qjl: bool, cache: np.ndarray | None = None,
                   layout: str = "rows") -> np.ndarray:
    """payload[name]: per (token, head) arrays - idx [T,H,16b] u8, signs [T,H,16] u8,
    norm [T,H] u16 bits, rnorm [T,H] u16 bits.  Returns uint8 [num_blocks, H, tile]."""
    idx_row, off_signs, off_norm, off_rnorm, tile = tile_offsets(block_size, bits, qjl)
    if cache is None:
        cache = np.zeros((num_blocks, num_heads, tile), dtype=np.uint8)
    touched = {}
    T = len(slot_mapping)
    for t in range(T):
        s = int(slot_mapping[t])
        if s < 0 or s >= num_blocks * block_size:
            continue
        blk, row = divmod(s, block_size)
        for h in range(num_heads):
            c = cache[blk, h]
            if (blk, h) not in touched:
                touched[(blk, h)] = _tile_rows(c, block_size, bits, qjl, layout)
            rows_idx, rows_sg = touched[(blk, h)]
            rows_idx[row] = payload["idx"][t, h]
            c[off_norm + 2 * row: off_norm + 2 * row + 2] = np.array(
                [payload["norm"][t, h] & 0xFF, payload["norm"][t, h] >> 8], dtype=np.uint8)
            if qjl:
                rows_sg[row] = payload["signs"][t, h]
                c[off_rnorm + 2 * row: off_rnorm + 2 * row + 2] = np.array(
                    [payload["rnorm"][t, h] & 0xFF, payload["rnorm"][t, h] >> 8], dtype=np.uint8)
    for (blk, h), (rows_idx, rows_sg) in touched.items():
        _set_tile_rows(cache[blk, h], rows_idx, rows_sg, block_size, bits, qjl, layout)
    return cache


def gather_sequence(cache: np.ndarray, block_table: np.ndarray, seq_len: int, head: int,
                    block_size: int, bits: int, qjl: bool, layout: str = "rows") -> dict:
    """Per-token payload of one (sequence, head) read back through the block table."""
    idx_row, off_signs, off_norm, off_rnorm, _ = tile_offsets(block_size, bits, qjl)
    out = {"idx": np.zeros((seq_len, idx_row), np.uint8), "norm": np.zeros(seq_len, np.uint16)}
    if qjl:
        out["signs"] = np.zeros((seq_len, 16), np.uint8)
        out["rnorm"] = np.zeros(seq_len, np.uint16)
    rows = {}
    for t in range(seq_len):
        blk = int(block_table[t // block_size])
        row = t % block_size
        c = cache[blk, head]
        if blk not in rows:
            rows[blk] = _tile_rows(c, block_size, bits, qjl, layout)
        out["idx"][t] = rows[blk][0][row]
        out["norm"][t] = int(c[off_norm + 2 * row]) | (int(c[off_norm + 2 * row + 1]) << 8)
        if qjl:
            out["signs"][t] = rows[blk][1][row]
            out["rnorm"][t] = int(c[off_rnorm + 2 * row]) | (int(c[off_rnorm + 2 * row + 1]) << 8)
    return out


def to_slots(cache: np.ndarray, block_size: int, bits: int, qjl: bool, slot_bytes: int,
             layout: str = "rows") -> np.ndarray:
    """Tile layout -> reference array-of-slots [num_blocks, bs, H, slot_bytes], per token."""
    nb, H, _ = cache.shape
    idx_row, off_signs, off_norm, off_rnorm, _ = tile_offsets(block_size, bits, qjl)
    out = np.zeros((nb, block_size, H, slot_bytes), dtype=np.uint8)
    for b in range(nb):
        for h in range(H):
            c = cache[b, h]
            ridx, rsg = _tile_rows(c, block_size, bits, qjl, layout)
            for r in range(block_size):
                parts = [ridx[r]]
                if qjl:
                    parts.append(rsg[r])
                parts.append(c[off_norm + 2 * r: off_norm + 2 * r + 2])
                if qjl:
                    parts.append(c[off_rnorm + 2 * r: off_rnorm + 2 * r + 2])
                p = np.concatenate(parts)
                out[b, r, h, :len(p)] = p
    return out


def subtile_row_positions(bits: int, qjl: bool, layout: str) -> np.ndarray:
    """pos[j] = byte of the row-major 16-row payload ([16 idx rows][16 sign rows]) that byte j
    of the "keys" sub-tile holds.  Derived by running build_subtile on byte ids (low and high
    byte planes separately: build_subtile only moves bytes in this layout), not by a second
    formula.  (The "values" layout moves bits-wide fields, not bytes: values_subtiles_to_rows.)"""
    if layout != "keys":
        raise ValueError("byte positions exist for the keys layout only")
    idx_row = 16 * bits
    ids_idx = np.arange(16 * idx_row, dtype=np.int64).reshape(16, idx_row)
    ids_sg = (16 * idx_row + np.arange(256, dtype=np.int64)).reshape(16, 16) if qjl else None
    planes = []
    for shift in (0, 8):
        i8 = ((ids_idx >> shift) & 0xFF).astype(np.uint8)
        s8 = ((ids_sg >> shift) & 0xFF).astype(np.uint8) if qjl else None
        planes.append(np.frombuffer(build_subtile(i8, s8, bits, layout), np.uint8).astype(np.int64))
    return planes[0] | (planes[1] << 8)


def values_subtiles_to_rows(sub: np.ndarray, bits: int) -> np.ndarray:
    """"values" sub-tile payloads [m, 256 * bits] -> packed index rows [16 m, 16 * bits],
    vectorised: every chunk's 32 fields are unpacked (little-endian bit order), indexed as
    (g, n, j, r) and transposed to (row 4g + r, dim 8n + j)."""
    m = sub.shape[0]
    b = np.unpackbits(np.ascontiguousarray(sub).reshape(m, 64, 4 * bits), axis=2, bitorder="little")
    f = (b.reshape(m, 64, 32, bits).astype(np.int64) << np.arange(bits)).sum(axis=3)
    f = f.reshape(m, 4, 16, 8, 4).transpose(0, 1, 4, 2, 3).reshape(16 * m, 128)
    return _pack.pack_indices(f, bits)


def rows_to_values_subtiles(idx: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of values_subtiles_to_rows: packed rows [16 m, 16 * bits] -> payloads [m, 256 * bits]."""
    m = idx.shape[0] // 16
    f = _pack.unpack_indices(idx, bits).reshape(m, 4, 4, 16, 8).transpose(0, 1, 3, 4, 2)  # (g, n, j, r)
    bitv = ((f.reshape(m, 64, 32, 1) >> np.arange(bits)) & 1).astype(np.uint8).reshape(m, 64, 32 * bits)
    return np.packbits(bitv, axis=2, bitorder="little").reshape(m, 256 * bits)


def tiles_to_tokens(tiles: np.ndarray, block_size: int, bits: int, qjl: bool, layout: str) -> dict:
    """Whole tiles [n, tile_bytes] (any layout) -> per-token payload of their n * block_size rows
    (idx [.., 16*bits] u8, signs [.., 16] u8, norm / rnorm [..] u16), vectorised."""
    tiles = np.ascontiguousarray(tiles)
    n = tiles.shape[0]
    idx_row, off_signs, off_norm, off_rnorm, _ = tile_offsets(block_size, bits, qjl)
    P = idx_row + (16 if qjl else 0)
    if layout == "rows":
        idx = tiles[:, :block_size * idx_row].reshape(n * block_size, idx_row)
        signs = tiles[:, off_signs:off_signs + 16 * block_size].reshape(n * block_size, 16) if qjl else None
    elif layout == "values":
        idx = values_subtiles_to_rows(tiles[:, :block_size * P].reshape(n * (block_size // 16), 16 * P), bits)
        signs = None
    else:
        pos = subtile_row_positions(bits, qjl, layout)
        sub = tiles[:, :block_size * P].reshape(n * (block_size // 16), 16 * P)
        rows = np.empty_like(sub)
        rows[:, pos] = sub
        idx = rows[:, :16 * idx_row].reshape(-1, idx_row)
        signs = rows[:, 16 * idx_row:].reshape(-1, 16) if qjl else None
    out = {"idx": idx,
           "norm": np.ascontiguousarray(tiles[:, off_norm:off_norm + 2 * block_size]).view(np.uint16).reshape(-1)}
    if qjl:
        out["signs"] = signs
        out["rnorm"] = np.ascontiguousarray(tiles[:, off_rnorm:off_rnorm + 2 * block_size]).view(np.uint16).reshape(-1)
    return out
