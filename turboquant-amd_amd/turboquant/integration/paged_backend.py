"""Serving-framework side of the packed paged hot path, without the framework itself.

vLLM is not part of this package (nor installed where it is built); what a backend needs from
the hot path is here, in the shapes the reference's backends use:

- TurboQuantPagedState: per-layer formats, codebooks and the two cache operations
  (compress-and-scatter, decode), plus rotate_query / rotate_output.  Follows
  TurboQuantFP8State (integration/vllm_backend.py:64-177): asymmetric K/V bit widths
  (`v_bits=None` means the K width), the WHT rotation (x @ make_wht_matrix(head_size)).  The
  reference compresses to FP8 through a dequantize step; this state writes the packed format
  itself and decodes it with the split-K kernels, with the query / output rotations fused into
  the decode call (rotate=True) unless the rotation is fused into the weights.
- TurboQuantPagedConfig / get_tq_paged_config: the boundary-layer policy of
  TurboQuantFP8Config / get_tq_fp8_config (integration/vllm_backend.py:237-337): the first and
  last `num_protected_layers` layers are not compressed (get_state returns None and the caller
  keeps its own attention for them, as the reference does), or, with `protected_bits`, get a
  4-bit (or other) packed format of their own.
- TurboQuantPagedImpl: an attention implementation in vLLM's shape
  (TurboQuantFP4Impl.do_kv_cache_update / forward and TurboQuantFP4Backend.get_kv_cache_shape,
  integration/tq_fp4_backend.py:389-735).  One uint8 tensor [num_blocks, num_kv_heads,
  k_tile + v_tile] holds both caches: each (block, KV head) has its K tile followed by its V
  tile.  forward runs the decode sequences (one new token each, first in the batch, as vLLM
  orders them) through the split-K decode kernels and the prefill / extend sequences through
  the tiled prefill kernel, both reading the packed cache (the reference FP4 backend falls back
  to dequantised attention for extends, tq_fp4_backend.py:558-601).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from turboquant.core import make_codebook, make_wht_matrix
from turboquant.kernels.paged import PagedKVFormat, compress_paged, compress_paged_kv, decode_paged, prefill_paged
from turboquant.kernels.rotation import wht_rows


class TurboQuantPagedState:
    """Per-layer state: K / V packed formats, codebooks, cache writes and decode.

    k_bits / v_bits: 2, 3 or 4 (v_bits None: same as k_bits); k_qjl: QJL residual signs on the
    keys; weights_fused: K, V and q arrive already rotated (the WHT folded into the
    projections, core/rotation.py:47-140) and the output is left in the rotated basis.
    """

    def __init__(self, head_size: int = 128, layer_idx: int = 0, device=None, k_bits: int = 4,
                 v_bits: Optional[int] = None, k_qjl: bool = False, block_size: int = 16,
                 weights_fused: bool = False):
        if head_size != 128:
            raise ValueError("the packed kernels take head_size 128")
        self.head_size = head_size
        self.layer_idx = layer_idx
        self.device = torch.device(device) if device is not None else None
        self.k_bits = k_bits
        self.v_bits = v_bits if v_bits is not None else k_bits
        self.k_qjl = bool(k_qjl)
        self.block_size = block_size
        self.weights_fused = bool(weights_fused)
        self.k_format = PagedKVFormat(bits=self.k_bits, qjl=self.k_qjl, block_size=block_size)
        self.v_format = PagedKVFormat(bits=self.v_bits, qjl=False, block_size=block_size, layout="values")
        self.wht = make_wht_matrix(head_size, self.device)
        self.k_centroids, self.k_boundaries = make_codebook(head_size, self.k_bits, device=self.device)
        if self.v_bits == self.k_bits:
            # one tensor for both: the decode kernel then keeps a single LDS table
            self.v_centroids, self.v_boundaries = self.k_centroids, self.k_boundaries
        else:
            self.v_centroids, self.v_boundaries = make_codebook(head_size, self.v_bits, device=self.device)

    # ---- rotations (stand-alone; decode() fuses them) ----
    def rotate_query(self, q: torch.Tensor) -> torch.Tensor:
        """q @ make_wht_matrix(128), in q's dtype."""
        return wht_rows(q)

    def rotate_output(self, out: torch.Tensor) -> torch.Tensor:
        """out @ make_wht_matrix(128) (the matrix is its own inverse), in out's dtype."""
        return wht_rows(out)

    # ---- cache geometry ----
    @property
    def tile_bytes(self) -> int:
        """Bytes per (block, KV head) of the combined cache: K tile then V tile."""
        return self.k_format.tile_bytes + self.v_format.tile_bytes

    def kv_cache_shape(self, num_blocks: int, num_kv_heads: int) -> tuple[int, int, int]:
        return (num_blocks, num_kv_heads, self.tile_bytes)

    def allocate_kv_cache(self, num_blocks: int, num_kv_heads: int, device=None) -> torch.Tensor:
        dev = device if device is not None else self.device
        return torch.zeros(self.kv_cache_shape(num_blocks, num_kv_heads), dtype=torch.uint8, device=dev)

    def split_kv_cache(self, kv_cache: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(K cache, V cache) views of a combined cache."""
        if kv_cache.dtype != torch.uint8 or kv_cache.dim() != 3 or kv_cache.shape[2] != self.tile_bytes:
            raise ValueError(f"kv_cache must be uint8 [num_blocks, num_kv_heads, {self.tile_bytes}]")
        kt = self.k_format.tile_bytes
        return kv_cache[:, :, :kt], kv_cache[:, :, kt:]

    # ---- cache operations ----
    def compress_and_scatter(self, x: torch.Tensor, cache: torch.Tensor, slot_mapping: torch.Tensor,
                             is_value: bool = False) -> None:
        """Compress x [T, Hkv, 128] into the K (or V) cache at slot_mapping (negative: skipped)."""
        if is_value:
            compress_paged(x, slot_mapping, cache, self.v_format, self.v_centroids, self.v_boundaries,
                           rotate=not self.weights_fused)
        else:
            compress_paged(x, slot_mapping, cache, self.k_format, self.k_centroids, self.k_boundaries,
                           rotate=not self.weights_fused)

    def compress_kv_and_scatter(self, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                                v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """The layer's K + V cache update in one launch: compress_and_scatter of k (K cache) and
        of v (V cache) at the same slots."""
        compress_paged_kv(k, v, slot_mapping, k_cache, v_cache, self.k_format, self.v_format,
                          (self.k_centroids, self.k_boundaries), (self.v_centroids, self.v_boundaries),
                          rotate=not self.weights_fused)

    def decode(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
               seq_lens: torch.Tensor, sm_scale: Optional[float] = None, sparse_threshold: float = 0.0,
               max_seq_len: Optional[int] = None, seq_lens_host: Optional[Sequence[int]] = None,
               out: Optional[torch.Tensor] = None, tokens_per_chunk: Optional[int] = None,
               workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode attention of q [S, Hq, 128] in the model's basis (rotations fused)."""
        return decode_paged(q, k_cache, self.k_format, self.k_centroids, v_cache, self.v_format, self.v_centroids,
                            block_tables, seq_lens, sm_scale=sm_scale, sparse_threshold=sparse_threshold,
                            max_seq_len=max_seq_len, seq_lens_host=seq_lens_host, out=out,
                            tokens_per_chunk=tokens_per_chunk, workspace=workspace,
                            rotate=not self.weights_fused)

    def prefill(self, q: torch.Tensor, cu_seqlens_q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                block_tables: torch.Tensor, seq_lens: torch.Tensor, sm_scale: Optional[float] = None,
                max_q_len: Optional[int] = None, out: Optional[torch.Tensor] = None,
                causal: bool = True) -> torch.Tensor:
        """Prefill / extend attention of q [T, Hq, 128] (new tokens of each sequence, already in
        the cache) in the model's basis."""
        return prefill_paged(q, cu_seqlens_q, k_cache, self.k_format, self.k_centroids, v_cache, self.v_format,
                             self.v_centroids, block_tables, seq_lens, sm_scale=sm_scale, causal=causal,
                             rotate=not self.weights_fused, max_q_len=max_q_len, out=out)


class TurboQuantPagedConfig:
    """Which layers are compressed, and with which formats.

    protect_boundary_layers / num_protected_layers: the first and last N layers are not
    compressed with the configured formats (integration/vllm_backend.py:266-278).  Their
    get_state is None (the caller's own attention, as in the reference) unless
    protected_bits is given: then they get k_bits = v_bits = protected_bits without QJL.
    """

    def __init__(self, head_size: int = 128, num_layers: int = 0, protect_boundary_layers: bool = True,
                 num_protected_layers: int = 2, k_bits: int = 4, v_bits: Optional[int] = None,
                 k_qjl: bool = False, block_size: int = 16, weights_fused: bool = False,
                 protected_bits: Optional[int] = None):
        self.head_size = head_size
        self.num_layers = num_layers
        self.protect_boundary_layers = protect_boundary_layers
        self.num_protected_layers = num_protected_layers
        self.k_bits = k_bits
        self.v_bits = v_bits
        self.k_qjl = k_qjl
        self.block_size = block_size
        self.weights_fused = weights_fused
        self.protected_bits = protected_bits
        self.layer_states: dict[int, TurboQuantPagedState] = {}

    def should_compress(self, layer_idx: int) -> bool:
        if not self.protect_boundary_layers or self.num_layers == 0:
            return True
        if layer_idx < self.num_protected_layers:
            return False
        if layer_idx >= self.num_layers - self.num_protected_layers:
            return False
        return True

    def get_state(self, layer_idx: int, device=None) -> Optional[TurboQuantPagedState]:
        protected = not self.should_compress(layer_idx)
        if protected and self.protected_bits is None:
            return None
        if layer_idx not in self.layer_states:
            if protected:
                kb, vb, kq = self.protected_bits, self.protected_bits, False
            else:
                kb, vb, kq = self.k_bits, self.v_bits, self.k_qjl
            self.layer_states[layer_idx] = TurboQuantPagedState(
                self.head_size, layer_idx, device, k_bits=kb, v_bits=vb, k_qjl=kq,
                block_size=self.block_size, weights_fused=self.weights_fused)
        return self.layer_states[layer_idx]


_tq_paged_config: Optional[TurboQuantPagedConfig] = None


def get_tq_paged_config(head_size: int = 128, num_layers: int = 0, protect_boundary_layers: bool = True,
                        num_protected_layers: int = 2, k_bits: int = 4, v_bits: Optional[int] = None,
                        k_qjl: bool = False, block_size: int = 16, weights_fused: bool = False,
                        protected_bits: Optional[int] = None) -> TurboQuantPagedConfig:
    """The process-wide config, created by the first call (later arguments are ignored, as in
    get_tq_fp8_config, integration/vllm_backend.py:295-337)."""
    global _tq_paged_config
    if _tq_paged_config is None:
        _tq_paged_config = TurboQuantPagedConfig(
            head_size=head_size, num_layers=num_layers, protect_boundary_layers=protect_boundary_layers,
            num_protected_layers=num_protected_layers, k_bits=k_bits, v_bits=v_bits, k_qjl=k_qjl,
            block_size=block_size, weights_fused=weights_fused, protected_bits=protected_bits)
    return _tq_paged_config


def reset_tq_paged_config() -> None:
    """Forget the process-wide config (tests, re-configuration)."""
    global _tq_paged_config
    _tq_paged_config = None


@dataclass
class PagedDecodeMetadata:
    """What forward needs of the framework's attention metadata.

    Without query_start_loc every sequence is a decode (one query token).  With it (int32
    [num_seqs + 1], vLLM's query_start_loc), the first num_decodes sequences are decodes and the
    rest prefill / extend sequences whose new tokens are the last ones of seq_lens.
    """

    block_tables: torch.Tensor                   # int32 [num_seqs, max_blocks]
    seq_lens: torch.Tensor                       # int32 [num_seqs], including the new tokens
    max_seq_len: int                             # host-side upper bound of seq_lens
    seq_lens_host: Optional[Sequence[int]] = None
    query_start_loc: Optional[torch.Tensor] = None
    num_decodes: Optional[int] = None            # default: all sequences when query_start_loc is None
    max_query_len: Optional[int] = None          # host-side bound of the prefill query counts


class TurboQuantPagedImpl:
    """Decode attention over the packed paged cache, in the shape of a vLLM AttentionImpl."""

    forward_includes_kv_cache_update = False  # do_kv_cache_update is called separately

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 state: TurboQuantPagedState, sparse_threshold: float = 0.0):
        if num_heads % num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        if head_size != state.head_size:
            raise ValueError("head_size differs from the layer state's")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.state = state
        self.sparse_threshold = float(sparse_threshold)

    @staticmethod
    def get_supported_kernel_block_sizes() -> list[int]:
        return [16, 32, 64]

    @staticmethod
    def get_supported_head_sizes() -> list[int]:
        return [128]

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           k_bits: int = 4, v_bits: Optional[int] = None, k_qjl: bool = False) -> tuple[int, ...]:
        """[num_blocks, num_kv_heads, k_tile + v_tile] uint8 (K tile, then V tile, per head)."""
        if block_size % 16:
            raise ValueError("Block size must be a multiple of 16.")
        if head_size != 128:
            raise ValueError("head_size must be 128")
        kf = PagedKVFormat(bits=k_bits, qjl=k_qjl, block_size=block_size)
        vf = PagedKVFormat(bits=v_bits if v_bits is not None else k_bits, qjl=False, block_size=block_size,
                           layout="values")
        return (num_blocks, num_kv_heads, kf.tile_bytes + vf.tile_bytes)

    def do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                           slot_mapping: torch.Tensor) -> None:
        """Compress key / value [num_tokens, num_kv_heads, head_size] into their slots (one
        launch for both: tq_compress_paged_kv)."""
        k_cache, v_cache = self.state.split_kv_cache(kv_cache)
        self.state.compress_kv_and_scatter(key, value, k_cache, v_cache, slot_mapping)

    def forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                attn_metadata: Optional[PagedDecodeMetadata], output: Optional[torch.Tensor] = None,
                output_scale: Optional[torch.Tensor] = None,
                output_block_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
        """query [num_tokens, num_heads * head_size] (or [num_tokens, num_heads, head_size]) ->
        output of the same shape: decode tokens first (one per sequence), then the new tokens of
        the prefill / extend sequences."""
        if output is None:
            raise ValueError("Output tensor must be provided.")
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("fused output quantization is not supported")
        if attn_metadata is None:
            return output.fill_(0)
        md = attn_metadata
        S = md.seq_lens.shape[0]
        nd = S if md.query_start_loc is None else (md.num_decodes if md.num_decodes is not None else 0)
        k_cache, v_cache = self.state.split_kv_cache(kv_cache)
        if nd:
            q = query[:nd].view(nd, self.num_heads, self.head_size)
            out = output[:nd].view(nd, self.num_heads, self.head_size)
            lens_host = md.seq_lens_host[:nd] if md.seq_lens_host is not None else None
            self.state.decode(q, k_cache, v_cache, md.block_tables[:nd], md.seq_lens[:nd],
                              sm_scale=self.scale, sparse_threshold=self.sparse_threshold,
                              max_seq_len=md.max_seq_len, seq_lens_host=lens_host, out=out)
        if nd < S:
            qsl = md.query_start_loc
            t0 = nd  # decode tokens come first, one per sequence
            cu = (qsl[nd:] - t0).to(torch.int32)
            tp = query.shape[0] - t0
            q = query[t0:].view(tp, self.num_heads, self.head_size)
            out = output[t0:].view(tp, self.num_heads, self.head_size)
            self.state.prefill(q, cu, k_cache, v_cache, md.block_tables[nd:], md.seq_lens[nd:], sm_scale=self.scale,
                               max_q_len=md.max_query_len, out=out)
        return output
