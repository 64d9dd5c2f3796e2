"""Paged packed-KV cache: format, fused compression, split-K decode attention.

Cache layout.  One tensor per K or V cache, uint8 [num_blocks, num_kv_heads, tile_bytes];
the tile of (physical block, KV head) stores its block_size tokens structure-of-arrays:

    [block_size x 16*bits index bytes][block_size x 16 sign bytes]  (signs: QJL keys only)
    [block_size x fp16 norm]          [block_size x fp16 residual norm] (QJL keys only)

Per token this is exactly the reference's payload (index bits as a little-endian bit stream,
sign bits, fp16 norms: kernels/packed_compress.py:79-106, kernels/sparse_v.py:57-98,
docs/design/AITER_TURBO4_DESIGN.md:57-76), regrouped so that the 16 tokens a wave reads
are contiguous (one 128-bit load per lane).  to_reference_slots / from_reference_slots convert
to and from the reference's array-of-slots layout [num_blocks, block_size, Hkv, slot_bytes]
(kernels/sparse_v.py:293-304, integration/vllm/compact_kv_allocator.py:36-75).

Slot addressing follows vLLM: token t goes to slot_mapping[t] = block * block_size + row
(integration/vllm_backend.py:223-230); negative slots are skipped.
"""

from __future__ import annotations

import ctypes
import functools
import math
from dataclasses import dataclass
from typing import Optional

import torch

from turboquant import _lib
from turboquant.core.rotation import wht_scale

MI355X_CUS = 256
# The dispatcher deals workgroups to the 8 XCDs in turn and, within an XCD, to its 4 shader
# engines in turn: workgroup b runs on shader engine (b % 8, (b // 8) % 4), i.e. b % 32.
MI355X_SE_SLOTS = 32


_LAYOUTS = {"rows": 0, "keys": 1, "values": 2}


@dataclass(frozen=True)
class PagedKVFormat:
    """Geometry of one paged cache (K or V).

    layout: how the payload (index bytes and QJL sign bytes) of a tile is ordered -
      "keys"   (default): per 16-token sub-tile, chunk (4n + g) holds the index bytes and then
               the sign bytes of row n, dims 32g..32g+31 - one load per decode lane for a key;
      "values": per 16-token sub-tile, chunk (16g + n) holds dims 8n..8n+7 of rows 4g..4g+3 -
               one load per decode lane for the value product (no QJL);
      "rows"   : all index rows, then all sign rows (row-major; read by the general kernel).
    A V cache uses layout="values"; decode_paged checks the roles.
    """

    bits: int = 4
    qjl: bool = False
    block_size: int = 16
    head_dim: int = 128
    layout: str = "keys"

    def __post_init__(self):
        if self.bits not in (2, 3, 4):
            raise ValueError(f"bits must be 2, 3 or 4, got {self.bits}")
        if self.block_size <= 0 or self.block_size % 16:
            raise ValueError(f"block_size must be a positive multiple of 16, got {self.block_size}")
        if self.head_dim != 128:
            raise ValueError("head_dim must be 128")
        if self.layout not in _LAYOUTS:
            raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}, got {self.layout!r}")
        if self.layout == "values" and self.qjl:
            raise ValueError("the values layout carries no QJL data")

    @classmethod
    def for_keys(cls, bits: int, qjl: bool = False, block_size: int = 16) -> "PagedKVFormat":
        return cls(bits=bits, qjl=qjl, block_size=block_size, layout="keys")

    @classmethod
    def for_values(cls, bits: int, block_size: int = 16) -> "PagedKVFormat":
        return cls(bits=bits, qjl=False, block_size=block_size, layout="values")

    @property
    def layout_code(self) -> int:
        return _LAYOUTS[self.layout]

    @property
    def payload_bytes(self) -> int:
        """Index + sign bytes per token (the payload region's row stride)."""
        return self.idx_bytes + (16 if self.qjl else 0)

    @property
    def idx_bytes(self) -> int:
        return self.head_dim * self.bits // 8

    @property
    def off_signs(self) -> int:
        """Sign rows of the "rows" layout (the lane-grouped layouts interleave them)."""
        return self.block_size * self.idx_bytes

    @property
    def off_norm(self) -> int:
        return self.block_size * (self.idx_bytes + (16 if self.qjl else 0))

    @property
    def off_rnorm(self) -> int:
        return self.off_norm + 2 * self.block_size

    @property
    def tile_bytes(self) -> int:
        return self.off_norm + 2 * self.block_size * (2 if self.qjl else 1)

    @property
    def token_bytes(self) -> int:
        """Payload bytes per (token, KV head)."""
        return self.tile_bytes // self.block_size

    @property
    def slot_bytes(self) -> int:
        """Size of the reference-layout slot (payload, no padding)."""
        return self.token_bytes


def allocate_cache(num_blocks: int, num_kv_heads: int, fmt: PagedKVFormat, device=None) -> torch.Tensor:
    """Zeroed uint8 cache [num_blocks, num_kv_heads, fmt.tile_bytes]."""
    return torch.zeros((num_blocks, num_kv_heads, fmt.tile_bytes), dtype=torch.uint8, device=device)


def _check_roles(k_fmt: PagedKVFormat, v_fmt: PagedKVFormat) -> None:
    if v_fmt.qjl:
        raise ValueError("the V cache carries no QJL data")
    if k_fmt.layout == "values":
        raise ValueError("the K cache format uses layout='values'; keys use 'keys' (or 'rows')")
    if v_fmt.layout == "keys":
        raise ValueError("the V cache format uses layout='keys'; values use 'values' (or 'rows')")


def _check_cache(cache: torch.Tensor, fmt: PagedKVFormat, what: str) -> None:
    if cache.dtype != torch.uint8 or cache.dim() != 3:
        raise ValueError(f"{what}: cache must be uint8 [num_blocks, num_kv_heads, tile_bytes]")
    if cache.shape[2] < fmt.tile_bytes or cache.stride(2) != 1:
        raise ValueError(f"{what}: cache tiles must hold {fmt.tile_bytes} contiguous bytes")


def compress_paged(
    x: torch.Tensor,
    slot_mapping: torch.Tensor,
    cache: torch.Tensor,
    fmt: PagedKVFormat,
    centroids: torch.Tensor,
    boundaries: torch.Tensor,
    rotate: bool = True,
) -> torch.Tensor:
    """Compress x [T, Hkv, 128] (f32/f16/bf16) into the paged cache at slot_mapping [T].

    With rotate=True the WHT is applied first (the reference's x @ make_wht_matrix(128));
    rotate=False takes already-rotated input (weights fused with the rotation).
    """
    dev = _lib.require_gpu("compress_paged", x, slot_mapping, cache, centroids, boundaries)
    if x.dim() != 3 or x.shape[2] != fmt.head_dim:
        raise ValueError(f"x must be [T, H, {fmt.head_dim}], got {tuple(x.shape)}")
    T, H, _ = x.shape
    _check_cache(cache, fmt, "compress_paged")
    if cache.shape[1] != H:
        raise ValueError(f"cache has {cache.shape[1]} heads, x has {H}")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != T:
        raise ValueError("slot_mapping must be [T]")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise TypeError("slot_mapping must be int32 or int64")
    if centroids.numel() != 2 ** fmt.bits:
        raise ValueError(f"need {2 ** fmt.bits} centroids for bits={fmt.bits}")
    if x.stride(2) != 1 or x.stride(0) % 8 or x.stride(1) % 8 or x.data_ptr() % 32:
        x = x.contiguous()
    slot_mapping = slot_mapping.contiguous()
    cent = centroids.to(device=dev, dtype=torch.float32).contiguous()
    bnd = boundaries.to(device=dev, dtype=torch.float32).contiguous()
    rc = _lib.lib().tq_compress_paged(
        x.data_ptr(), _lib.dtype_code(x), x.stride(0), x.stride(1), T, H, fmt.head_dim,
        slot_mapping.data_ptr(), _lib.dtype_code(slot_mapping),
        cache.data_ptr(), cache.stride(0), cache.stride(1), cache.shape[0], fmt.block_size,
        fmt.bits, int(fmt.qjl), fmt.layout_code, int(bool(rotate)), wht_scale(fmt.head_dim),
        cent.data_ptr(), bnd.data_ptr(), _lib.stream_handle(dev),
    )
    _lib.check(rc, "tq_compress_paged")
    return cache


def _f32_on(t: torch.Tensor, dev) -> torch.Tensor:
    if t.dtype == torch.float32 and t.is_cuda and t.get_device() == dev.index and t.is_contiguous():
        return t
    return t.to(device=dev, dtype=torch.float32).contiguous()


def _target(x: torch.Tensor, cache: torch.Tensor, fmt: PagedKVFormat, cb, dev, keep: list):
    cent = _f32_on(cb[0], dev)
    bnd = _f32_on(cb[1], dev)
    if cent.numel() != 2 ** fmt.bits or bnd.numel() != 2 ** fmt.bits - 1:
        raise ValueError(f"need {2 ** fmt.bits} centroids and {2 ** fmt.bits - 1} boundaries for bits={fmt.bits}")
    keep += [x, cent, bnd]
    return _lib.TQPagedTarget(x.data_ptr(), x.stride(0), x.stride(1), cache.data_ptr(), cache.stride(0), cache.stride(1),
                              fmt.bits, int(fmt.qjl), fmt.layout_code, cent.data_ptr(), bnd.data_ptr())


def compress_paged_kv(
    k: torch.Tensor,
    v: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_fmt: PagedKVFormat,
    v_fmt: PagedKVFormat,
    k_codebook,
    v_codebook,
    rotate: bool = True,
):
    """compress_paged of k into k_cache and of v into v_cache (same tokens and slots) in one
    launch: a layer's K + V cache update (the reference calls turbo4_fp8_compress_and_scatter
    once per tensor, integration/vllm_backend.py:179-230).  k_codebook / v_codebook are
    (centroids, boundaries)."""
    dev = _lib.require_gpu("compress_paged_kv", k, v, slot_mapping, k_cache, v_cache)
    _check_roles(k_fmt, v_fmt)
    if k.dim() != 3 or k.shape[2] != k_fmt.head_dim or v.shape != k.shape:
        raise ValueError(f"k and v must both be [T, H, {k_fmt.head_dim}], got {tuple(k.shape)} and {tuple(v.shape)}")
    if k.dtype != v.dtype:
        raise TypeError("k and v must share a dtype")
    if k_fmt.block_size != v_fmt.block_size:
        raise ValueError("k and v caches must share the block size")
    T, H, _ = k.shape
    _check_cache(k_cache, k_fmt, "compress_paged_kv (K)")
    _check_cache(v_cache, v_fmt, "compress_paged_kv (V)")
    if k_cache.shape[:2] != v_cache.shape[:2] or k_cache.shape[1] != H:
        raise ValueError("k_cache and v_cache must be [num_blocks, H, *] for the same blocks and heads")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != T:
        raise ValueError("slot_mapping must be [T]")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise TypeError("slot_mapping must be int32 or int64")

    def ok(x):
        return x if (x.stride(2) == 1 and x.stride(0) % 8 == 0 and x.stride(1) % 8 == 0 and x.data_ptr() % 32 == 0) \
            else x.contiguous()

    k, v = ok(k), ok(v)
    slot_mapping = slot_mapping.contiguous()
    keep: list = []
    tk = _target(k, k_cache, k_fmt, k_codebook, dev, keep)
    tv = _target(v, v_cache, v_fmt, v_codebook, dev, keep)
    rc = _lib.lib().tq_compress_paged_kv(
        ctypes.byref(tk), ctypes.byref(tv), _lib.dtype_code(k), T, H, k_fmt.head_dim,
        slot_mapping.data_ptr(), _lib.dtype_code(slot_mapping), k_cache.shape[0], k_fmt.block_size,
        int(bool(rotate)), wht_scale(k_fmt.head_dim), _lib.stream_handle(dev),
    )
    _lib.check(rc, "tq_compress_paged_kv")
    return k_cache, v_cache


_WORKSPACES: dict = {}


def decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """tq_decode workspace of at least nbytes for `device` and its current stream.

    One buffer per stream is reused (calls on one stream are ordered; calls that overlap in
    time must not share a workspace).
    """
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, _lib.stream_handle(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def choose_tokens_per_chunk(num_seqs: int, num_kv_heads: int, max_seq_len: int,
                            concurrent_units: int = MI355X_CUS * 4 * 3, seq_lens_host=None,
                            unit_overhead_tiles: float = 2.0, max_chunk: int = 65536) -> int:
    """Split-K chunk length (multiple of 16) for tq_decode.

    The grid has one work unit per (sequence, KV head, chunk of the sequence); concurrent_units
    of them run at once (tq_decode_concurrent_units).  With every sequence max_seq_len long the
    kernel takes ceil(units / concurrent_units) rounds of (chunk tiles + a fixed per-unit
    cost), and the chunk count per sequence minimising that is chosen (chunks balanced: the last
    is at most one tile shorter).  With the sequence lengths known on the host (seq_lens_host),
    the estimate is the balanced load (all work / concurrent_units) plus a quarter unit of tail
    (slots freed by short units are refilled, and waves left alone on a SIMD run faster), and
    never less than the longest unit.  Measured on MI355X with config-5-like lengths
    (log-uniform 2K..128K): chunks of ~170-260 tiles beat a single round of ~420-tile chunks by
    about 8 %.
    """
    slots = max(1, concurrent_units)
    ovh = unit_overhead_tiles
    tiles_max = max(1, -(-max(1, max_seq_len) // 16))
    lens = None
    if seq_lens_host is not None:
        lens = [max(0, -(-min(int(x), max(1, max_seq_len)) // 16)) for x in seq_lens_host]
        if not any(lens) or len(set(lens)) == 1:
            tiles_max = max(lens) if any(lens) else tiles_max
            lens = None  # uniform: the round model is exact
    base = max(1, num_seqs * num_kv_heads)
    max_nch = max(1, -(-tiles_max // 4))  # chunks of at least 4 tiles (64 tokens)
    best = None
    for nch in range(1, max_nch + 1):
        ct = -(-tiles_max // nch)
        if ct * 16 > max_chunk:
            continue
        if lens is None:
            cost = -(-(base * nch) // slots) * (ct + ovh)
        else:
            units = num_kv_heads * sum(-(-t // ct) for t in lens)
            work = num_kv_heads * sum(lens) + ovh * units
            cost = max(work / slots + 0.25 * (ct + ovh), ct + ovh)
        cost += 0.01 * nch  # partial results to merge
        if best is None or cost < best[0]:
            best = (cost, ct)
    if best is None:
        return max_chunk // 16 * 16
    return best[1] * 16


@functools.lru_cache(maxsize=256)
def _concurrent_units(device: int, k_bits: int, k_qjl: bool, v_bits: int, hq: int, hkv: int, norm_row: int,
                      share: bool) -> int:
    out = ctypes.c_int(0)
    with torch.cuda.device(device):
        _lib.check(_lib.lib().tq_decode_concurrent_units(k_bits, int(k_qjl), v_bits, hq, hkv, norm_row, int(share),
                                                         ctypes.byref(out)), "tq_decode_concurrent_units")
    return int(out.value)


def plan_tokens_per_chunk(device: torch.device, num_seqs: int, num_q_heads: int, num_kv_heads: int,
                          max_seq_len: int, k_fmt: "PagedKVFormat", v_fmt: "PagedKVFormat",
                          share_codebook: bool = False, seq_lens_host=None, norm_row_bytes: int = 2) -> int:
    """tokens_per_chunk for tq_decode on this device and configuration.

    With the sequence lengths known (seq_lens_host), fixed chunks from a round model whose
    per-unit cost beyond its tiles is about fourteen tiles of set-up (the workgroup's LDS
    tables, the query operands, the first loads; calibrated on MI355X with configs 3-5), plus
    writing and re-reading its partial results (group heads x 128 fp32, twice) expressed in
    tiles of K+V data, as long as its units fit in one round of resident waves: each wave then
    runs one unit inside one sequence.  When they would need more rounds, or the lengths are
    unknown, 0: the balanced schedule, every resident wave taking an equal share of all the
    tile pairs (balanced_partition).  Measured on MI355X: config 5 (log-uniform 2K..128K,
    several rounds) 387-390 us balanced vs 415-433 us in fixed chunks; config 3 (one round)
    49.3 vs 52.3 us and config 4 (equal lengths, one round) 405-408 vs 412 us the other way.
    """
    if seq_lens_host is None:
        return 0
    group = num_q_heads // max(1, num_kv_heads)
    tile_bytes = 16 * (k_fmt.token_bytes + v_fmt.token_bytes)
    overhead = 14.0 + group * 1024.0 / tile_bytes
    slots = concurrent_units(device, k_fmt.bits, k_fmt.qjl, v_fmt.bits, num_q_heads, num_kv_heads,
                             norm_row_bytes, share_codebook)
    msl = max(1, max_seq_len)
    tiles = [-(-min(max(int(x), 0), msl) // 16) for x in seq_lens_host]
    if len(set(tiles)) > 1:
        # Variable lengths: the shortest chunk (at least 4 tiles) whose busy workgroups leave a
        # slot free on every shader engine, so that all units run in one round (a unit's time is
        # its chunk plus its start-up), if that round is not much longer than the balanced
        # schedule's share per wave (which also pays its pieces' extra start-ups and a longer
        # merge).  Measured on MI355X, config 3 (8-wave workgroups, 16 slots per engine):
        # chunks of 384 tokens (15 busy on the fullest engine) 43.3 us, 400 (15) 45.4,
        # 336 / 352 / 368 (20 / 21 / 17, over) 52.9 / 53.6 / 53.6 us, balanced 47.9 us;
        # config 5 (one round only with 905-tile chunks against 369-tile shares) balanced.
        wgw = workgroup_waves(device, k_fmt.bits, k_fmt.qjl, v_fmt.bits, num_q_heads, num_kv_heads,
                              norm_row_bytes, share_codebook)
        cap = max(1, slots // max(1, wgw) // MI355X_SE_SLOTS)
        limit = cap - 1 if cap > 1 else cap
        tmax = max(1, -(-msl // 16))
        share = num_kv_heads * sum(tiles) / max(1, slots)
        for ct in range(min(4, tmax), tmax + 1):
            if ct + overhead > 1.3 * (share + overhead):
                break
            if chunk_engine_load(tiles, tmax, ct, num_kv_heads, wgw) <= limit:
                return ct * 16
        return 0
    chunk = choose_tokens_per_chunk(num_seqs, num_kv_heads, max_seq_len, slots, seq_lens_host, overhead)
    units = num_kv_heads * sum(-(-min(max(int(x), 0), msl) // chunk) for x in seq_lens_host)
    return chunk if units <= slots else 0


@functools.lru_cache(maxsize=256)
def _workgroup_waves(device: int, k_bits: int, k_qjl: bool, v_bits: int, hq: int, hkv: int, norm_row: int,
                     share: bool) -> int:
    out = ctypes.c_int(0)
    with torch.cuda.device(device):
        _lib.check(_lib.lib().tq_decode_workgroup_waves(k_bits, int(k_qjl), v_bits, hq, hkv, norm_row, int(share),
                                                        ctypes.byref(out)), "tq_decode_workgroup_waves")
    return int(out.value)


def workgroup_waves(device: torch.device, k_bits: int, k_qjl: bool, v_bits: int, num_q_heads: int,
                    num_kv_heads: int, norm_row_bytes: int = 2, share_codebook: bool = False) -> int:
    """Waves (work units) per workgroup of the decode kernel for this configuration."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _workgroup_waves(idx, k_bits, bool(k_qjl), v_bits, num_q_heads, num_kv_heads, norm_row_bytes,
                            bool(share_codebook))


def chunk_engine_load(tiles, tiles_max: int, ct: int, num_kv_heads: int, wg_waves: int,
                      engines: int = MI355X_SE_SLOTS) -> int:
    """Busy workgroups on the most loaded shader engine with chunks of ct tiles.

    Units in (sequence, chunk, KV head) order over ceil(tiles_max / ct) chunks per sequence,
    wg_waves units per workgroup, workgroup b on engine b % engines; a workgroup is busy when
    one of its units holds tokens (a sequence's busy units are one contiguous range)."""
    n = -(-tiles_max // ct)
    cnt = [0] * engines
    last = -1
    for s, t in enumerate(tiles):
        k = -(-t // ct)
        if k <= 0:
            continue
        b0 = max((s * n * num_kv_heads) // wg_waves, last + 1)
        b1 = ((s * n + k) * num_kv_heads - 1) // wg_waves
        if b1 < b0:
            continue
        full, rem = divmod(b1 - b0 + 1, engines)
        if full:
            cnt = [c + full for c in cnt]
        for j in range(rem):
            cnt[(b0 + j) % engines] += 1
        last = b1
    return max(cnt)


def concurrent_units(device: torch.device, k_bits: int, k_qjl: bool, v_bits: int, num_q_heads: int,
                     num_kv_heads: int, norm_row_bytes: int = 2, share_codebook: bool = False) -> int:
    """Decode work units resident at once on `device` for this configuration (occupancy query)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _concurrent_units(idx, k_bits, bool(k_qjl), v_bits, num_q_heads, num_kv_heads, norm_row_bytes,
                             bool(share_codebook))


def balanced_partition(seq_lens_host, num_kv_heads: int, workers: int, len_cap: int) -> dict:
    """The split-K pieces of tq_decode's balanced schedule (tokens_per_chunk = 0): for every
    (sequence, KV head) with tokens, the list of token ranges [t0, t1) that separate waves
    process (each with its own running max; the merge combines them).

    The work is the stream of 32-token tile pairs of the (sequence, KV head) segments, sequences
    in order and a sequence's KV heads after each other (ceil(min(len, len_cap) / 32) pairs per
    segment); with P pairs in all and R = min(P, workers) waves, wave w takes pairs
    [floor(w P / R), floor((w + 1) P / R)).  workers is concurrent_units(...) of the
    configuration and len_cap = min(max_seq_len, max_blocks_per_seq * block_size)."""
    lens = [max(0, min(int(x), int(len_cap))) for x in seq_lens_host]
    pairs = [(L + 31) // 32 for L in lens]
    P = num_kv_heads * sum(pairs)
    out = {}
    if P == 0:
        return out
    R = min(P, int(workers))
    pos = 0
    for s, (L, n) in enumerate(zip(lens, pairs)):
        for kh in range(num_kv_heads):
            if n == 0:
                continue
            a, b = pos, pos + n
            # worker boundaries strictly inside the segment
            w = (a * R) // P + 1                      # first boundary index past a (floor(wP/R) > a)
            while (w * P) // R <= a:
                w += 1
            cuts = [a]
            while w < R and (w * P) // R < b:
                cuts.append((w * P) // R)
                w += 1
            cuts.append(b)
            out[(s, kh)] = [(32 * (c0 - a), min(L, 32 * (c1 - a))) for c0, c1 in zip(cuts[:-1], cuts[1:])]
            pos = b
    return out


def _region(ptr: int, stride_block: int, stride_head: int, stride_row: int, stride_seq: int = 0) -> _lib.TQRegion:
    return _lib.TQRegion(ptr, stride_block, stride_head, stride_seq, stride_row)


def paged_view(cache: torch.Tensor, fmt: PagedKVFormat, centroids: torch.Tensor) -> _lib.TQKVView:
    """TQKVView over a cache tensor in this module's tile layouts."""
    base = cache.data_ptr()
    sb, sh = cache.stride(0), cache.stride(1)
    view = _lib.TQKVView()
    view.layout = fmt.layout_code
    if fmt.layout == "rows":
        view.idx = _region(base, sb, sh, fmt.idx_bytes)
        if fmt.qjl:
            view.signs = _region(base + fmt.off_signs, sb, sh, 16)
    else:
        view.idx = _region(base, sb, sh, fmt.payload_bytes)  # payload region; signs inside it
    if fmt.qjl:
        view.rnorm = _region(base + fmt.off_rnorm, sb, sh, 2)
    view.norm = _region(base + fmt.off_norm, sb, sh, 2)
    view.centroids = centroids.data_ptr()
    view.bits = fmt.bits
    view.qjl = int(fmt.qjl)
    view.signs_permuted = 0
    view.centroid_scale = _lib.centroid_scale(centroids)
    return view


def run_decode(
    q: torch.Tensor,
    k_view: _lib.TQKVView,
    v_view: _lib.TQKVView,
    *,
    num_kv_heads: int,
    block_size: int,
    num_blocks: int,
    block_tables: Optional[torch.Tensor],
    max_blocks_per_seq: int,
    seq_lens: Optional[torch.Tensor],
    max_seq_len: int,
    sm_scale: float,
    corr_scale: float,
    q_proj: Optional[torch.Tensor],
    sparse_threshold: float,
    tokens_per_chunk: int,
    out: torch.Tensor,
    workspace: Optional[torch.Tensor],
    skip_stats: Optional[torch.Tensor],
    keep_alive: tuple = (),
    rotate: bool = False,
) -> torch.Tensor:
    """Launch tq_decode for q [S, Hq, 128] given ready KV views (shared by all wrappers).

    rotate=True launches tq_decode_rotated: q in the original basis, out returned in it.
    seq_lens None: every sequence is max_seq_len tokens long (no length array is read)."""
    dev = q.device
    S, Hq, D = q.shape
    L = _lib.lib()
    need = L.tq_decode_workspace_bytes(S, Hq, max_seq_len, tokens_per_chunk)
    if workspace is None or workspace.numel() < need or workspace.data_ptr() % 256:
        workspace = decode_workspace(dev, need)
    if skip_stats is not None and (skip_stats.dtype != torch.int64 or skip_stats.numel() < 2 or not skip_stats.is_cuda):
        raise ValueError("skip_stats must be a device int64 tensor with 2 elements")
    bt_ptr = block_tables.data_ptr() if block_tables is not None else None
    bt_stride = block_tables.stride(0) if block_tables is not None else 0
    entry = L.tq_decode_rotated if rotate else L.tq_decode
    rc = entry(
        q.data_ptr(), _lib.dtype_code(q), q.stride(0), q.stride(1),
        _lib.ptr(q_proj), q_proj.stride(0) if q_proj is not None else 0, q_proj.stride(1) if q_proj is not None else 0,
        S, Hq, num_kv_heads, D,
        ctypes.byref(k_view), ctypes.byref(v_view),
        block_size, num_blocks,
        bt_ptr, bt_stride, max_blocks_per_seq,
        _lib.ptr(seq_lens), max_seq_len,
        float(sm_scale), float(corr_scale), float(sparse_threshold),
        tokens_per_chunk,
        workspace.data_ptr(), workspace.numel(),
        out.data_ptr(), _lib.dtype_code(out), out.stride(0), out.stride(1),
        _lib.ptr(skip_stats),
        _lib.stream_handle(dev),
    )
    _lib.check(rc, "tq_decode_rotated" if rotate else "tq_decode")
    del keep_alive
    return out


def decode_paged(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    k_fmt: PagedKVFormat,
    k_centroids: torch.Tensor,
    v_cache: torch.Tensor,
    v_fmt: PagedKVFormat,
    v_centroids: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    sm_scale: Optional[float] = None,
    corr_scale: Optional[float] = None,
    q_proj: Optional[torch.Tensor] = None,
    sparse_threshold: float = 0.0,
    max_seq_len: Optional[int] = None,
    tokens_per_chunk: Optional[int] = None,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    skip_stats: Optional[torch.Tensor] = None,
    seq_lens_host=None,
    rotate: bool = False,
) -> torch.Tensor:
    """Decode attention of q [S, Hq, 128] (rotated space) over paged packed K/V caches.

    rotate=True: q is in the original basis and so is the result - the kernels apply
    q @ make_wht_matrix(128) on load and rotate the output back on its write (the reference
    backend's rotate_query / rotate_output, integration/vllm_backend.py:158-177, fused).  An
    explicit q_proj is used as given; without one the QJL query is the rotated q.

    score = sm_scale * (q . k_mse + corr_scale * rnorm * (q_proj . signs)) with q_proj = q by
    default (QJL in the rotated basis, as polarquant_compress computes the signs);
    corr_scale defaults to sqrt(pi/2)/128 (reference/pytorch_reference.py:153-154).
    block_tables: int32 [S, max_blocks]; seq_lens: int32 [S]; max_seq_len: host-side upper
    bound of seq_lens (default: max_blocks * block_size).  sparse_threshold > 0 enables
    Sparse-V.  Output dtype = out.dtype or q.dtype.  seq_lens_host: the same lengths as a host
    sequence, if the caller has them; they only size the split-K chunks.  Passing one tensor as
    k_centroids and v_centroids (same codebook) lets the kernel keep one LDS table.
    """
    dev = _lib.require_gpu("decode_paged", q, k_cache, v_cache, block_tables, seq_lens, k_centroids, v_centroids)
    if q.dim() != 3 or q.shape[2] != 128:
        raise ValueError("q must be [S, Hq, 128]")
    if k_fmt.block_size != v_fmt.block_size:
        raise ValueError("K and V caches must share block_size")
    _check_roles(k_fmt, v_fmt)
    _check_cache(k_cache, k_fmt, "decode_paged(k)")
    _check_cache(v_cache, v_fmt, "decode_paged(v)")
    if k_cache.shape[0] != v_cache.shape[0] or k_cache.shape[1] != v_cache.shape[1]:
        raise ValueError("K and V caches must have the same [num_blocks, num_kv_heads]")
    S, Hq, _ = q.shape
    Hkv = k_cache.shape[1]
    if Hq % Hkv or Hq // Hkv > 16:
        raise ValueError(f"num_q_heads {Hq} must be a multiple of num_kv_heads {Hkv} with group <= 16")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("block_tables and seq_lens must be int32")
    if block_tables.dim() != 2 or block_tables.shape[0] != S or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be [S, max_blocks] with unit inner stride")
    seq_lens = seq_lens.contiguous()
    if q.stride(2) != 1:
        q = q.contiguous()
    if q_proj is not None:
        if q_proj.shape != q.shape:
            raise ValueError("q_proj must have q's shape")
        q_proj = q_proj.to(q.dtype)
        if q_proj.stride(2) != 1:
            q_proj = q_proj.contiguous()
    max_blocks = block_tables.shape[1]
    cap = max_blocks * k_fmt.block_size
    msl = cap if max_seq_len is None else min(int(max_seq_len), cap)
    if out is None:
        out = torch.empty_like(q)
    kc = k_centroids.to(device=dev, dtype=torch.float32).contiguous()
    vc = v_centroids.to(device=dev, dtype=torch.float32).contiguous()
    if kc.numel() != 2 ** k_fmt.bits or vc.numel() != 2 ** v_fmt.bits:
        raise ValueError("centroid counts must match the formats' bit widths")
    # One tensor for both codebooks lets the kernel keep a single LDS pair table.
    share = kc.data_ptr() == vc.data_ptr()
    chunk = (plan_tokens_per_chunk(dev, S, Hq, Hkv, msl, k_fmt, v_fmt, share, seq_lens_host)
             if tokens_per_chunk is None else int(tokens_per_chunk))
    kv = paged_view(k_cache, k_fmt, kc)
    vv = paged_view(v_cache, v_fmt, vc)
    return run_decode(
        q, kv, vv, num_kv_heads=Hkv, block_size=k_fmt.block_size, num_blocks=k_cache.shape[0],
        block_tables=block_tables, max_blocks_per_seq=max_blocks, seq_lens=seq_lens, max_seq_len=msl,
        sm_scale=(1.0 / math.sqrt(128)) if sm_scale is None else sm_scale,
        corr_scale=(math.sqrt(math.pi / 2) / 128) if corr_scale is None else corr_scale,
        q_proj=q_proj, sparse_threshold=sparse_threshold, tokens_per_chunk=chunk, out=out,
        workspace=workspace, skip_stats=skip_stats, keep_alive=(kc, vc), rotate=rotate,
    )


PREFILL_CAUSAL = 1
PREFILL_ROTATE = 2


def prefill_paged(
    q: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    k_cache: torch.Tensor,
    k_fmt: PagedKVFormat,
    k_centroids: torch.Tensor,
    v_cache: torch.Tensor,
    v_fmt: PagedKVFormat,
    v_centroids: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    sm_scale: Optional[float] = None,
    corr_scale: Optional[float] = None,
    q_proj: Optional[torch.Tensor] = None,
    causal: bool = True,
    rotate: bool = False,
    max_q_len: Optional[int] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Prefill / extend attention of q [T, Hq, 128] over paged packed K/V caches (tq_prefill).

    Sequence s owns query rows cu_seqlens_q[s] .. cu_seqlens_q[s+1] - 1 (int32 [S+1], device)
    and seq_lens[s] cache tokens, the new tokens included (written by compress_paged first).
    causal=True: query i of a sequence with n new tokens sits at position seq_lens - n + i and
    sees cache tokens up to it; causal=False: every query sees the whole sequence (the
    reference's Sq > 1 kernel, kernels/attention.py:146-196).  Scores and defaults as
    decode_paged; rotate=True takes q and returns the output in the model basis.  max_q_len:
    host-side bound of the per-sequence query counts (default: T).
    """
    dev = _lib.require_gpu("prefill_paged", q, cu_seqlens_q, k_cache, v_cache, block_tables, seq_lens,
                           k_centroids, v_centroids)
    if q.dim() != 3 or q.shape[2] != 128:
        raise ValueError("q must be [T, Hq, 128]")
    if k_fmt.block_size != v_fmt.block_size:
        raise ValueError("K and V caches must share block_size")
    _check_roles(k_fmt, v_fmt)
    _check_cache(k_cache, k_fmt, "prefill_paged(k)")
    _check_cache(v_cache, v_fmt, "prefill_paged(v)")
    if k_cache.shape[0] != v_cache.shape[0] or k_cache.shape[1] != v_cache.shape[1]:
        raise ValueError("K and V caches must have the same [num_blocks, num_kv_heads]")
    T, Hq, _ = q.shape
    Hkv = k_cache.shape[1]
    if Hq % Hkv:
        raise ValueError(f"num_q_heads {Hq} must be a multiple of num_kv_heads {Hkv}")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32 or cu_seqlens_q.dtype != torch.int32:
        raise TypeError("block_tables, seq_lens and cu_seqlens_q must be int32")
    S = seq_lens.shape[0]
    if cu_seqlens_q.dim() != 1 or cu_seqlens_q.shape[0] != S + 1:
        raise ValueError("cu_seqlens_q must be [num_seqs + 1]")
    if block_tables.dim() != 2 or block_tables.shape[0] != S or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be [S, max_blocks] with unit inner stride")
    seq_lens = seq_lens.contiguous()
    cu_seqlens_q = cu_seqlens_q.contiguous()
    if q.stride(2) != 1:
        q = q.contiguous()
    if q_proj is not None:
        if q_proj.shape != q.shape:
            raise ValueError("q_proj must have q's shape")
        q_proj = q_proj.to(q.dtype)
        if q_proj.stride(2) != 1:
            q_proj = q_proj.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.stride(2) != 1:
        raise ValueError("out must be [T, Hq, 128] with unit inner stride")
    kc = k_centroids.to(device=dev, dtype=torch.float32).contiguous()
    vc = v_centroids.to(device=dev, dtype=torch.float32).contiguous()
    if kc.numel() != 2 ** k_fmt.bits or vc.numel() != 2 ** v_fmt.bits:
        raise ValueError("centroid counts must match the formats' bit widths")
    kv = paged_view(k_cache, k_fmt, kc)
    vv = paged_view(v_cache, v_fmt, vc)
    flags = (PREFILL_CAUSAL if causal else 0) | (PREFILL_ROTATE if rotate else 0)
    mq = T if max_q_len is None else int(max_q_len)
    rc = _lib.lib().tq_prefill(
        q.data_ptr(), _lib.dtype_code(q), q.stride(0), q.stride(1),
        _lib.ptr(q_proj), q_proj.stride(0) if q_proj is not None else 0, q_proj.stride(1) if q_proj is not None else 0,
        cu_seqlens_q.data_ptr(), S, mq, Hq, Hkv, 128,
        ctypes.byref(kv), ctypes.byref(vv), k_fmt.block_size, k_cache.shape[0],
        block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1], seq_lens.data_ptr(),
        float((1.0 / math.sqrt(128)) if sm_scale is None else sm_scale),
        float((math.sqrt(math.pi / 2) / 128) if corr_scale is None else corr_scale), flags,
        out.data_ptr(), _lib.dtype_code(out), out.stride(0), out.stride(1), _lib.stream_handle(dev),
    )
    _lib.check(rc, "tq_prefill")
    return out


# ---- conversion to and from the reference's array-of-slots layout ------------------------

def _tile_fields(fmt: PagedKVFormat):
    """(name, offset in tile, bytes per token) of each per-token field, in slot order."""
    fields = [("idx", 0, fmt.idx_bytes)]
    if fmt.qjl:
        fields.append(("signs", fmt.off_signs, 16))
    fields.append(("norm", fmt.off_norm, 2))
    if fmt.qjl:
        fields.append(("rnorm", fmt.off_rnorm, 2))
    return fields


@functools.lru_cache(maxsize=None)
def _rows_positions(fmt: PagedKVFormat) -> Optional[torch.Tensor]:
    """pos[j] = byte of fmt's tile that holds byte j of the same tile in the "rows" layout
    (None for the rows layout itself, which needs no move, and for the values layout, whose
    chunks interleave bits-wide fields of four rows: see _values_to_rows).  Norm regions
    coincide."""
    if fmt.layout != "keys":
        return None
    bs, b, q = fmt.block_size, fmt.bits, fmt.qjl
    P = fmt.payload_bytes
    pos = torch.arange(fmt.tile_bytes, dtype=torch.int64)
    R = torch.arange(bs).view(bs, 1)
    sub, t16 = (R // 16) * 16 * P, R % 16
    k = torch.arange(16 * b).view(1, -1)                    # index byte of the token
    C = 4 * b + (4 if q else 0)
    pos[:bs * 16 * b] = (sub + (4 * t16 + k // (4 * b)) * C + k % (4 * b)).reshape(-1)
    if q:
        ks = torch.arange(16).view(1, -1)                   # sign byte of the token
        pos[fmt.off_signs:fmt.off_signs + bs * 16] = (sub + (4 * t16 + ks // 4) * C + 4 * b + ks % 4).reshape(-1)
    return pos


def _fields(b: torch.Tensor, bits: int, n: int) -> torch.Tensor:
    """uint8 [..., n * bits / 8] little-endian bit streams -> int64 fields [..., n]."""
    bitv = (b.to(torch.int64).unsqueeze(-1) >> torch.arange(8, device=b.device)) & 1
    return (bitv.reshape(*b.shape[:-1], n, bits) << torch.arange(bits, device=b.device)).sum(-1)


def _stream(f: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of _fields: int64 fields [..., n] -> uint8 [..., n * bits / 8]."""
    bitv = (f.unsqueeze(-1) >> torch.arange(bits, device=f.device)) & 1
    bitv = bitv.reshape(*f.shape[:-1], -1, 8)
    return (bitv << torch.arange(8, device=f.device)).sum(-1).to(torch.uint8)


_CONVERT_TILES = 2048  # tiles per batch of the field-level conversion (bounds the int64 temporaries)


def _values_to_rows(payload: torch.Tensor, bits: int) -> torch.Tensor:
    """values-layout payloads [m, bs * 16 * bits] -> row-major index rows, same shape.  Chunk
    16g + n of a 16-row sub-tile holds, at field 4j + r, dim 8n + j of row 4g + r."""
    m = payload.shape[0]
    f = _fields(payload.reshape(m, -1, 64, 4 * bits), bits, 32)          # [m, sub, chunk, field]
    f = f.reshape(m, -1, 4, 16, 8, 4).permute(0, 1, 2, 5, 3, 4)            # (g, r, n, j)
    return _stream(f.reshape(m, -1, 128), bits).reshape(m, -1)


def _rows_to_values(rows: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of _values_to_rows."""
    m = rows.shape[0]
    f = _fields(rows.reshape(m, -1, 16 * bits), bits, 128)                # [m, row, dim]
    f = f.reshape(m, -1, 4, 4, 16, 8).permute(0, 1, 2, 4, 5, 3)            # (g, n, j, r)
    return _stream(f.reshape(m, -1, 32), bits).reshape(m, -1)


def _convert_values(cache: torch.Tensor, fmt: PagedKVFormat, fn) -> torch.Tensor:
    out = cache[..., :fmt.tile_bytes].clone()
    nb, h, _ = out.shape
    flat = out.reshape(nb * h, -1)
    n_idx = fmt.block_size * fmt.idx_bytes
    for i in range(0, nb * h, _CONVERT_TILES):
        part = flat[i:i + _CONVERT_TILES, :n_idx]
        flat[i:i + _CONVERT_TILES, :n_idx] = fn(part, fmt.bits)
    return out


def to_rows_layout(cache: torch.Tensor, fmt: PagedKVFormat) -> torch.Tensor:
    """The same tiles in the "rows" layout (a copy)."""
    if fmt.layout == "values":
        return _convert_values(cache, fmt, _values_to_rows)
    pos = _rows_positions(fmt)
    if pos is None:
        return cache.clone()
    return cache[..., :fmt.tile_bytes].index_select(2, pos.to(cache.device))


def from_rows_layout(rows: torch.Tensor, fmt: PagedKVFormat) -> torch.Tensor:
    """Inverse of to_rows_layout."""
    if fmt.layout == "values":
        return _convert_values(rows, fmt, _rows_to_values)
    pos = _rows_positions(fmt)
    if pos is None:
        return rows.clone()
    out = torch.zeros(rows.shape[:2] + (fmt.tile_bytes,), dtype=torch.uint8, device=rows.device)
    out[..., pos.to(rows.device)] = rows[..., :fmt.tile_bytes]
    return out


def to_reference_slots(cache: torch.Tensor, fmt: PagedKVFormat, slot_bytes: Optional[int] = None) -> torch.Tensor:
    """Tile layout -> [num_blocks, block_size, Hkv, slot_bytes] slots holding, per token,
    index bytes, [sign bytes], fp16 norm, [fp16 residual norm], then zero padding."""
    cache = to_rows_layout(cache, fmt)
    nb, h, _ = cache.shape
    bs = fmt.block_size
    sb = slot_bytes or fmt.slot_bytes
    if sb < fmt.token_bytes:
        raise ValueError("slot too small")
    out = torch.zeros((nb, bs, h, sb), dtype=torch.uint8, device=cache.device)
    pos = 0
    for _, off, width in _tile_fields(fmt):
        part = cache[:, :, off: off + bs * width].reshape(nb, h, bs, width).permute(0, 2, 1, 3)
        out[..., pos: pos + width] = part
        pos += width
    return out


def compress_paged_slots(x: torch.Tensor, slot_mapping: torch.Tensor, slots: torch.Tensor, fmt: PagedKVFormat,
                         centroids: torch.Tensor, boundaries: torch.Tensor, rotate: bool = True) -> torch.Tensor:
    """compress_paged straight into an array-of-slots cache view slots [num_blocks, block_size,
    Hkv, slot_bytes] uint8 (the reference's per-token slot: index bytes, [sign bytes], fp16 norm,
    [fp16 residual norm], padding; kernels/sparse_v.py:293-304), token t at
    slots[slot_mapping[t] // block_size, slot_mapping[t] % block_size].  The view may be strided
    (e.g. tq_cache[:, 0] of a [num_blocks, 2, block_size, Hkv, slot] cache); fmt gives bits and
    QJL (its tile layout is not used).  One tq_compress_regions launch."""
    dev = _lib.require_gpu("compress_paged_slots", x, slot_mapping, slots, centroids, boundaries)
    if slots.dtype != torch.uint8 or slots.dim() != 4 or slots.stride(3) != 1:
        raise ValueError("slots must be uint8 [num_blocks, block_size, Hkv, slot_bytes] with contiguous slots")
    nb, bs, h, sb = slots.shape
    if sb < fmt.token_bytes:
        raise ValueError(f"slots of {sb} bytes cannot hold {fmt.token_bytes} bytes per token")
    if x.dim() != 3 or x.shape[2] != fmt.head_dim or x.shape[1] != h:
        raise ValueError(f"x must be [T, {h}, {fmt.head_dim}], got {tuple(x.shape)}")
    T = x.shape[0]
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != T:
        raise ValueError("slot_mapping must be [T]")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise TypeError("slot_mapping must be int32 or int64")
    cent = centroids.to(device=dev, dtype=torch.float32).contiguous()
    bnd = boundaries.to(device=dev, dtype=torch.float32).contiguous()
    if cent.numel() != 2 ** fmt.bits or bnd.numel() != 2 ** fmt.bits - 1:
        raise ValueError(f"need {2 ** fmt.bits} centroids and {2 ** fmt.bits - 1} boundaries for bits={fmt.bits}")
    if x.stride(2) != 1 or x.stride(0) % 8 or x.stride(1) % 8 or x.data_ptr() % 32:
        x = x.contiguous()
    slot_mapping = slot_mapping.contiguous()
    base = slots.data_ptr()
    s_blk, s_row, s_head = slots.stride(0), slots.stride(1), slots.stride(2)
    view = _lib.TQKVView()
    view.layout = _LAYOUTS["rows"]
    pos = 0
    for name, _, width in _tile_fields(fmt):
        setattr(view, name, _region(base + pos, s_blk, s_head, s_row))
        pos += width
    view.centroids = cent.data_ptr()
    view.bits, view.qjl, view.signs_permuted = fmt.bits, int(fmt.qjl), 0
    rc = _lib.lib().tq_compress_regions(
        x.data_ptr(), _lib.dtype_code(x), x.stride(0), x.stride(1), T, h, fmt.head_dim,
        slot_mapping.data_ptr(), _lib.dtype_code(slot_mapping), ctypes.byref(view), bnd.data_ptr(), nb, bs,
        int(bool(rotate)), wht_scale(fmt.head_dim), _lib.stream_handle(dev),
    )
    _lib.check(rc, "tq_compress_regions")
    return slots


def from_reference_slots(slots: torch.Tensor, fmt: PagedKVFormat) -> torch.Tensor:
    """Inverse of to_reference_slots: [num_blocks, block_size, Hkv, slot_bytes] -> tile layout."""
    nb, bs, h, _ = slots.shape
    if bs != fmt.block_size:
        raise ValueError("block_size mismatch")
    cache = torch.zeros((nb, h, fmt.tile_bytes), dtype=torch.uint8, device=slots.device)
    pos = 0
    for _, off, width in _tile_fields(fmt):
        part = slots[..., pos: pos + width].permute(0, 2, 1, 3).reshape(nb, h, bs * width)
        cache[:, :, off: off + bs * width] = part
        pos += width
    return from_rows_layout(cache, fmt)
