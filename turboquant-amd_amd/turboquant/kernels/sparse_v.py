"""Paged 3-bit decode over the reference's array-of-slots cache, dense (v11) and Sparse-V (v12).

The reference launches Triton kernels directly on a cache [num_blocks, 2 (K/V), block_size,
num_kv_heads, slot_bytes] uint8 whose slot holds 48 bytes of 3-bit indices (bits 3d..3d+2 =
dim d) and the fp16 norm at bytes 48-49 (kernels/sparse_v.py:25-159, 163-261, 293-304).
tq_v12_sparse_v / tq_v11 run tq_decode on that same memory through strided views, so a
cache written for the reference is read in place.  block_size is taken from the cache's
shape (docs/MI355X_BLOCKSIZE_FIX.md:18-21).

Sparse-V rule (kernels/sparse_v.py:108-149): with a running max m over the tokens processed
so far in the work unit, updated once per KV block (block_size tokens, as the reference's
KV_BLK_SZ = block_size loop does, for block sizes 16 and 32; every 32 tokens for larger
blocks), token t's V is skipped when max over the GQA group of exp(score - m) <= threshold;
skipped tokens still count in the softmax denominator.  The work unit here is a chunk of
tokens_per_chunk tokens (rounded up to a multiple of 32 for block sizes of 32 or more); with
tokens_per_chunk >= the sequence length it is the reference's single pass, one work unit per
(sequence, KV head) as the reference's grid (num_seqs, num_kv_heads) runs it
(kernels/sparse_v.py:316,341).  That is tq_v12_sparse_v's default, so the drop-in skips the
same tokens as the reference; a split-K chunk (faster for few long sequences, with the running
max restarting per chunk) is an opt-in through tokens_per_chunk.  tq_v11 (no skipping) keeps
the split-K planner by default: without the skip rule the chunking changes only the fp32
summation order, not the result.
"""

from __future__ import annotations

import torch

from turboquant import _lib
from turboquant.kernels.paged import (PagedKVFormat, choose_tokens_per_chunk, compress_paged_slots, concurrent_units,
                                     run_decode)

D = 128
DQ3 = D * 3 // 8  # 48 index bytes per slot
CD = 32
SPARSE_V_THRESHOLD = 1e-6


def _aos_view(cache: torch.Tensor, kv: int, centroids: torch.Tensor) -> _lib.TQKVView:
    nb, two, bs, hkv, slot = cache.shape
    base = cache.data_ptr() + kv * cache.stride(1)
    sb, sr, sh = cache.stride(0), cache.stride(2), cache.stride(3)
    view = _lib.TQKVView()
    view.idx = _lib.TQRegion(base, sb, sh, 0, sr)
    view.norm = _lib.TQRegion(base + DQ3, sb, sh, 0, sr)
    view.centroids = centroids.data_ptr()
    view.bits, view.qjl, view.signs_permuted = 3, 0, 0
    view.centroid_scale = _lib.centroid_scale(centroids)
    return view


def compress_to_tq_cache(x, slot_mapping, tq_cache, kv_idx: int, centroids, boundaries, rotate: bool = True):
    """Write x [T, Hkv, 128] into the 3-bit MSE-only slots of tq_cache [num_blocks, 2 (K/V),
    block_size, Hkv, slot_bytes] (48 index bytes + fp16 norm per slot, the layout the v11 / v12
    decode reads, kernels/sparse_v.py:293-304) at slot_mapping, K (kv_idx 0) or V (1), in place:
    one tq_compress_regions launch (negative slots skipped)."""
    if tq_cache.dtype != torch.uint8 or tq_cache.dim() != 5 or tq_cache.shape[1] != 2:
        raise ValueError("tq_cache must be uint8 [num_blocks, 2, block_size, num_kv_heads, slot_bytes]")
    if kv_idx not in (0, 1):
        raise ValueError("kv_idx must be 0 (K) or 1 (V)")
    fmt = PagedKVFormat(bits=3, qjl=False, block_size=tq_cache.shape[2])
    return compress_paged_slots(x, slot_mapping, tq_cache[:, kv_idx], fmt, centroids, boundaries, rotate=rotate)


def tq_paged_decode_3bit(out, q, tq_cache, centroids, block_tables, seq_lens, scale,
                         threshold: float = 0.0, max_seq_len=None, tokens_per_chunk=None, skip_stats=None):
    """out[S, Hq, 128] = attention of q over the 3-bit MSE-only K/V slots of tq_cache."""
    dev = _lib.require_gpu("tq_paged_decode_3bit", out, q, tq_cache, centroids, block_tables, seq_lens)
    if tq_cache.dtype != torch.uint8 or tq_cache.dim() != 5 or tq_cache.shape[1] != 2:
        raise ValueError("tq_cache must be uint8 [num_blocks, 2, block_size, num_kv_heads, slot_bytes]")
    nb, _, bs, hkv, slot = tq_cache.shape
    if slot < DQ3 + 2 or tq_cache.stride(4) != 1:
        raise ValueError("slots must hold 48 index bytes and an fp16 norm contiguously")
    S, Hq, d = q.shape
    if d != D or out.shape != q.shape:
        raise ValueError("q and out must be [S, Hq, 128]")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("block_tables and seq_lens must be int32")
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    cb = centroids.to(device=dev, dtype=torch.float32).contiguous()
    if cb.numel() != 8:
        raise ValueError("3-bit codebook needs 8 centroids")
    if q.stride(2) != 1:
        q = q.contiguous()
    max_blocks = block_tables.shape[1]
    cap = max_blocks * bs
    msl = cap if max_seq_len is None else min(int(max_seq_len), cap)
    if tokens_per_chunk is None and threshold > 0:
        # the reference's single pass: one unit per (sequence, KV head), whole sequence
        step = 32 if bs >= 32 else 16
        tokens_per_chunk = max(step, -(-msl // step) * step)
    chunk = tokens_per_chunk or choose_tokens_per_chunk(
        S, hkv, msl, concurrent_units(dev, 3, False, 3, Hq, hkv, tq_cache.stride(2), True))
    kv = _aos_view(tq_cache, 0, cb)
    vv = _aos_view(tq_cache, 1, cb)
    target = out if out.stride(2) == 1 else torch.empty_like(out)
    run_decode(q, kv, vv, num_kv_heads=hkv, block_size=bs, num_blocks=nb, block_tables=block_tables,
               max_blocks_per_seq=max_blocks, seq_lens=seq_lens.contiguous(), max_seq_len=msl, sm_scale=float(scale),
               corr_scale=0.0, q_proj=None, sparse_threshold=threshold, tokens_per_chunk=chunk, out=target,
               workspace=None, skip_stats=skip_stats, keep_alive=(cb,))
    if target is not out:
        out.copy_(target)
    return out


def tq_v12_sparse_v(out, q, tq_cache, centroids, block_tables, seq_lens, scale,
                    threshold: float = SPARSE_V_THRESHOLD, **kw):
    """Sparse-V decode (the role of _tq_v12_sparse_v_kernel, kernels/sparse_v.py:25-159).

    By default one pass over each (sequence, KV head), the reference's grid and skip
    semantics; tokens_per_chunk=N opts into split-K chunks of N tokens (the running max the
    skip test uses then restarts per chunk)."""
    return tq_paged_decode_3bit(out, q, tq_cache, centroids, block_tables, seq_lens, scale, threshold, **kw)


def tq_v11(out, q, tq_cache, centroids, block_tables, seq_lens, scale, **kw):
    """Dense decode without skipping (the role of _tq_v11_single_kernel, kernels/sparse_v.py:163-261)."""
    return tq_paged_decode_3bit(out, q, tq_cache, centroids, block_tables, seq_lens, scale, 0.0, **kw)


def benchmark(cases=((1, 1024), (1, 4096), (1, 16384), (1, 32768), (8, 4096), (32, 4096), (64, 4096), (192, 4096)),
              iters: int = 20, warmup: int = 3, seed: int = 42, verbose: bool = True) -> list:
    """tq_v11 (no skipping) against tq_v12_sparse_v on cuda:0 (the role of the reference
    module's benchmark(), kernels/sparse_v.py:264-380): 4 KV heads, GQA 6, block 32, 128-byte
    slots of random index bytes with fp16 norms of 0.5, the fixed 8-level codebook of that
    benchmark.  Per (batch, sequence length): mean device ms of v11, of v12 (the reference's
    single pass) and of v12 with split-K chunks, and the cosine between the v11 and v12 outputs.
    Returns the rows printed."""
    import math

    from turboquant.kernels._selfcheck import time_ms
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    hkv, gqa, bs, slot = 4, 6, 32, 128
    hq = hkv * gqa
    scale = 1.0 / math.sqrt(D)
    centroids = torch.tensor([-1.5, -0.8, -0.3, -0.05, 0.05, 0.3, 0.8, 1.5], dtype=torch.float32, device=dev)
    half = torch.tensor([0.5], dtype=torch.float16).view(torch.uint8)
    say = print if verbose else (lambda *a, **k: None)
    say(f"{'config':>16} | {'v11 ms':>9} | {'v12 ms':>9} | {'v12 split-K ms':>14} | {'speedup':>7} | {'cos':>7}")
    rows = []
    for ns, slen in cases:
        nblk = -(-slen // bs)
        total = ns * nblk + 16
        q = torch.randn(ns, hq, D, device=dev, generator=gen).half()
        cache = torch.randint(0, 256, (total, 2, bs, hkv, slot), dtype=torch.uint8, device=dev, generator=gen)
        cache[..., DQ3] = int(half[0])
        cache[..., DQ3 + 1] = int(half[1])
        bt = (torch.arange(nblk, dtype=torch.int32, device=dev).unsqueeze(0)
              + torch.arange(ns, dtype=torch.int32, device=dev).unsqueeze(1) * nblk).contiguous()
        lens = torch.full((ns,), slen, dtype=torch.int32, device=dev)
        o11, o12, o12s = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
        t11 = time_ms(lambda: tq_v11(o11, q, cache, centroids, bt, lens, scale), warmup, iters)
        t12 = time_ms(lambda: tq_v12_sparse_v(o12, q, cache, centroids, bt, lens, scale), warmup, iters)
        split = choose_tokens_per_chunk(ns, hkv, slen, concurrent_units(dev, 3, False, 3, hq, hkv, cache.stride(2), True))
        t12s = time_ms(lambda: tq_v12_sparse_v(o12s, q, cache, centroids, bt, lens, scale,
                                               tokens_per_chunk=split), warmup, iters)
        cos = torch.nn.functional.cosine_similarity(o11.flatten().float(), o12.flatten().float(), dim=0).item()
        rows.append({"batch": ns, "seq_len": slen, "v11_ms": t11, "v12_ms": t12, "v12_split_ms": t12s, "cos": cos})
        say(f"  B={ns:>3d},S={slen:>5d} | {t11:>9.3f} | {t12:>9.3f} | {t12s:>14.3f} | {t11 / t12:>6.2f}x | {cos:>7.4f}")
        del cache
    return rows


if __name__ == "__main__":
    benchmark()
