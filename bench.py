#!/usr/bin/env python3
"""Benchmark of the TurboQuant packed-KV hot path on one MI355X.

Prints ONE JSON line.  Headline (`value`): benchmark config 4 — Sparse-V split-K decode, turbo3
+ QJL keys / turbo3 values, batch 64 x context 32768, 48 query / 8 KV heads, block 16,
threshold 1e-4 — in us per layer (one tq_decode call = one layer's decode for the batch).
The same line carries configs 2 (turbo4 paged compress), 3 (turbo4 decode) and 5 (turbo2 + QJL
compress + decode step), the shapes the reference publishes numbers for, the roofline of the
headline kernel and a CPU baseline.

Inputs are synthetic (seeded) and resident in HBM before the timed region.  Each workload
first runs an untimed, reported settle phase (its own step, repeated for a fixed wall time:
the GPU's clocks ramp over the first tens of milliseconds of work), then W untimed warmup
steps, then exactly K timed steps bracketed by torch.cuda.synchronize().  HIP events on the
stream the kernels run on (torch's current stream) mark every step; `value` is the median
step, the mean is reported beside it.

The workload builders (WORKLOADS, build_decode_workload, compress workload) are shared with the
GPU parity tests, which check exactly the inputs timed here.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import random
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "turboquant-amd_amd"))

METRIC = "packed-KV decode attn μs/layer + HBM GB/s (% roofline); compress GB/s"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_TFLOPS = 2500.0
D = 128
SETTLE_S = 0.25
BRACKETS = 5


def outlier_kv(T, H, gen, device, dtype):
    """N(0,1) x per-channel log-normal(0, 0.5) scale, 2% of channels x8 (benchmark config 2)."""
    import torch
    scale = torch.exp(torch.randn(H, D, generator=gen, device=device) * 0.5)
    out = torch.rand(H, D, generator=gen, device=device) < 0.02
    scale = torch.where(out, scale * 8, scale)
    return (torch.randn(T, H, D, generator=gen, device=device) * scale).to(dtype)


def _lens3():
    rng = random.Random(3)  # one generator per workload: any subset gives the same lengths
    return [rng.randint(1024, 8192) for _ in range(32)]


def _lens5():
    rng = random.Random(5)
    return [int(round(math.exp(rng.uniform(math.log(2048), math.log(131072))))) for _ in range(64)]


# Benchmark configs 3-5; `lens` gives the per-sequence context lengths.
WORKLOADS = {
    "config3": dict(name="config3: turbo4 decode, B=32, Hq 32 / Hkv 8, ctx U[1K,8K], bs 16",
                    B=32, Hq=32, Hkv=8, lens=_lens3, kb=4, kq=False, vb=4, thresh=0.0, bs=16, seed=3),
    "config4": dict(name="config4: Sparse-V split-K decode, turbo3+QJL K / turbo3 V, B=64 x ctx 32768, "
                         "Hq 48 / Hkv 8, bs 16, T=1e-4",
                    B=64, Hq=48, Hkv=8, lens=lambda: [32768] * 64, kb=3, kq=True, vb=3, thresh=1e-4, bs=16, seed=4),
    "config5": dict(name="config5: turbo2+QJL compress 64 new tokens + decode, B=64, Hq 64 / Hkv 8, "
                         "ctx log-U[2K,128K], bs 16",
                    B=64, Hq=64, Hkv=8, lens=_lens5, kb=2, kq=True, vb=2, thresh=0.0, bs=16, seed=5, new_tokens=True),
}


def fill_paged(kv_cache_pair, fmts, centroids, boundaries, block_tables, seq_lens_host, Hkv, gen, dev,
               chunk_tokens=1 << 20):
    """Compress synthetic K and V for every sequence into the caches (untimed setup)."""
    import torch
    from turboquant.kernels.paged import compress_paged
    bs = fmts[0].block_size
    toks, slots = [], []
    pending = 0
    bt_host = block_tables.cpu()

    def flush():
        nonlocal toks, slots, pending
        if not toks:
            return
        slot = torch.cat(slots).to(dev)
        T = slot.numel()
        for which in (0, 1):
            x = outlier_kv(T, Hkv, gen, dev, torch.bfloat16)
            compress_paged(x, slot, kv_cache_pair[which], fmts[which], centroids[which], boundaries[which])
        toks, slots, pending = [], [], 0

    for s in range(len(seq_lens_host)):
        L = int(seq_lens_host[s])
        t = torch.arange(L)
        slots.append((bt_host[s, t // bs].long() * bs + t % bs).to(torch.int32))
        toks.append(L)
        pending += L
        if pending >= chunk_tokens:
            flush()
    flush()


def build_decode_workload(key, dev, lens=None):
    """Inputs of benchmark workload `key` on `dev`: caches filled by compress_paged from the
    outlier-channel distribution, random-permutation block tables, bf16 N(0,1) queries, the
    split-K chunk from the planner, the workspace; config 5 also its 64 new tokens and slots."""
    import torch
    from turboquant import _lib
    from turboquant.core import make_codebook
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, plan_tokens_per_chunk

    w = WORKLOADS[key]
    B, Hq, Hkv, bs, seed = w["B"], w["Hq"], w["Hkv"], w["bs"], w["seed"]
    lens_host = list(lens if lens is not None else w["lens"]())
    gen = torch.Generator(device=dev).manual_seed(seed)
    kf = PagedKVFormat(bits=w["kb"], qjl=w["kq"], block_size=bs)
    vf = PagedKVFormat(bits=w["vb"], qjl=False, block_size=bs, layout="values")
    blocks_per = [math.ceil(L / bs) for L in lens_host]
    maxb = max(blocks_per)
    nb = sum(blocks_per) + 64
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    bt = torch.full((B, maxb), -1, dtype=torch.int32)
    o = 0
    for s, n in enumerate(blocks_per):
        bt[s, :n] = perm[o:o + n].to(torch.int32)
        o += n
    bt = bt.to(dev)
    lens_t = torch.tensor(lens_host, dtype=torch.int32, device=dev)
    kc, kbnd = make_codebook(D, w["kb"], device=dev)
    # one codebook tensor per bit width, shared by K and V as a serving stack holds it
    vc, vbnd = (kc, kbnd) if w["vb"] == w["kb"] else make_codebook(D, w["vb"], device=dev)
    k_cache = allocate_cache(nb, Hkv, kf, device=dev)
    v_cache = allocate_cache(nb, Hkv, vf, device=dev)
    fill_paged((k_cache, v_cache), (kf, vf), (kc, vc), (kbnd, vbnd), bt, lens_host, Hkv, gen, dev)
    q = torch.randn((B, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    msl = max(lens_host)
    chunk = plan_tokens_per_chunk(dev, B, Hq, Hkv, msl, kf, vf, kc is vc, lens_host)
    ws = torch.empty(_lib.lib().tq_decode_workspace_bytes(B, Hq, msl, chunk), dtype=torch.uint8, device=dev)
    st = dict(key=key, name=w["name"], B=B, Hq=Hq, Hkv=Hkv, q=q, out=torch.empty_like(q), k_cache=k_cache,
              v_cache=v_cache, kf=kf, vf=vf, kc=kc, vc=vc, kbnd=kbnd, vbnd=vbnd, bt=bt, lens=lens_t,
              lens_host=lens_host, msl=msl, chunk=chunk, ws=ws, thresh=w["thresh"], new_tokens=None)
    if w.get("new_tokens"):
        # one new token per sequence, written into the last slot of its context
        last = torch.tensor([L - 1 for L in lens_host])
        slot_new = (bt.cpu()[torch.arange(B), last // bs].long() * bs + last % bs).to(torch.int32).to(dev)
        st["new_tokens"] = (outlier_kv(B, Hkv, gen, dev, torch.bfloat16), outlier_kv(B, Hkv, gen, dev, torch.bfloat16),
                            slot_new)
    return st


def decode_step(st, rotate=False, skip_stats=None):
    """One benchmark step of a decode workload: [compress the new tokens,] decode the batch."""
    from turboquant.kernels.paged import compress_paged_kv, decode_paged

    def step():
        if st["new_tokens"] is not None:
            newk, newv, slot_new = st["new_tokens"]
            compress_paged_kv(newk, newv, slot_new, st["k_cache"], st["v_cache"], st["kf"], st["vf"],
                              (st["kc"], st["kbnd"]), (st["vc"], st["vbnd"]))
        return decode_paged(st["q"], st["k_cache"], st["kf"], st["kc"], st["v_cache"], st["vf"], st["vc"], st["bt"],
                            st["lens"], sparse_threshold=st["thresh"], max_seq_len=st["msl"],
                            tokens_per_chunk=st["chunk"], out=st["out"], workspace=st["ws"], rotate=rotate,
                            skip_stats=skip_stats)
    return step


def settle(fn, seconds=SETTLE_S):
    """Untimed: run fn back to back for a fixed wall time; returns the milliseconds spent."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            break
    return round((time.perf_counter() - t0) * 1e3, 1), n


def timed(fn, steps, warmup, settle_s=SETTLE_S, brackets=BRACKETS):
    """Step time of fn: after a settle phase (untimed) and W warmup steps, K steps enqueued back
    to back between one pair of HIP events on the current stream, with a synchronize on both
    sides; `brackets` such runs, ms = the median of their total / K.

    A further run of K steps with an event recorded after every step gives the per-step
    distribution (event_median_ms, steps_ms).  Each of those events is a completion signal in
    the queue that the next launch waits behind (1.5-3 us per step measured on MI355X), so that figure
    carries the instrumentation and is reported beside the step time, not as it.
    Returns dict(ms, brackets_ms, event_median_ms, steps_ms, settle_ms, settle_steps)."""
    import torch
    settle_ms, settle_n = settle(fn, settle_s) if settle_s > 0 else (0.0, 0)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    brk = []
    for _ in range(brackets):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        brk.append(e0.elapsed_time(e1) / steps)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return {"ms": statistics.median(brk), "brackets_ms": brk, "event_median_ms": statistics.median(per),
            "steps_ms": per, "settle_ms": settle_ms, "settle_steps": settle_n}


def decode_case(key, dev, steps, warmup, time_rotated=False):
    import torch
    st = build_decode_workload(key, dev)
    t = timed(decode_step(st), steps, warmup)
    ms = t["ms"]
    res = {"workload": st["name"], "us_per_layer": ms * 1e3,
           "event_median_us": t["event_median_ms"] * 1e3, "settle_ms": t["settle_ms"]}
    if time_rotated:
        # the same decode with q and the output in the model basis (rotations fused)
        res["rotated_us_per_layer"] = timed(decode_step(st, rotate=True), steps, warmup, settle_s=0.05)["ms"] * 1e3
        # the same tiles in a K cache spanning more than 2 GiB (a serving pool), the blocks moved
        # past 2 GiB: the kernel's 64-bit per-tile addressing
        kc = st["k_cache"]
        shift = (3 << 30) // (kc.shape[1] * kc.shape[2]) + 1 - kc.shape[0] // 2
        big = torch.zeros((kc.shape[0] + shift,) + tuple(kc.shape[1:]), dtype=torch.uint8, device=dev)
        big[shift:] = kc
        bt_big = torch.where(st["bt"] >= 0, st["bt"] + shift, st["bt"])
        vbig = torch.zeros((big.shape[0],) + tuple(st["v_cache"].shape[1:]), dtype=torch.uint8, device=dev)
        vbig[shift:] = st["v_cache"]
        stb = dict(st, k_cache=big, v_cache=vbig, bt=bt_big, out=torch.empty_like(st["q"]))
        res["k_cache_beyond_2gib_us_per_layer"] = timed(decode_step(stb), steps, warmup, settle_s=0.05)["ms"] * 1e3
        del big, vbig, stb
    tokens = sum(st["lens_host"])
    kf, vf, Hkv = st["kf"], st["vf"], st["Hkv"]
    kv_bytes = tokens * Hkv * (kf.token_bytes + vf.token_bytes)
    io_bytes = 2 * st["B"] * st["Hq"] * D * 2 + st["bt"].numel() * 4 + st["B"] * 4
    alg = kv_bytes + io_bytes
    if st["new_tokens"] is not None:
        # the compress step: bf16 K and V in, the packed rows out
        alg += 2 * st["B"] * Hkv * D * 2 + st["B"] * Hkv * (kf.token_bytes + vf.token_bytes) + st["B"] * 4
    res.update(algorithmic_bytes=alg, kv_bytes=kv_bytes, hbm_gbs=alg / (ms * 1e-3) / 1e9,
               frac_of_8tbs=alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, tokens_per_chunk=st["chunk"],
               mean_ctx=tokens / st["B"])
    if st["thresh"] > 0:
        stats = torch.zeros(2, dtype=torch.int64, device=dev)
        decode_step(st, skip_stats=stats)()
        torch.cuda.synchronize()
        sk, tot = stats.tolist()
        frac = sk / max(tot, 1)
        res["sparse_v_skip_fraction"] = frac
        # V tiles are fetched whole (the skip test needs the scores of a pair, which arrive
        # after its loads were issued): skipped tokens save PV work, not bytes
        res["bytes_fetched"] = alg
        res["v_bytes_of_skipped_tokens"] = int(sk * vf.token_bytes)
    return res, st


def prefill_case(dev, steps, warmup, B=4, n=4096, Hq=48, Hkv=8, kb=3, kq=True, vb=3, bs=16, seed=7):
    """Full causal prefill over the packed cache: B sequences of n new tokens each (already
    compressed into the cache), one tq_prefill call per step."""
    import torch
    from turboquant.core import make_codebook
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, prefill_paged

    gen = torch.Generator(device=dev).manual_seed(seed)
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout="values")
    nbl = math.ceil(n / bs)
    nb = B * nbl + 8
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    bt = perm[:B * nbl].view(B, nbl).to(torch.int32).to(dev)
    lens_host = [n] * B
    lens = torch.tensor(lens_host, dtype=torch.int32, device=dev)
    kc, kbnd = make_codebook(D, kb, device=dev)
    vc, vbnd = (kc, kbnd) if vb == kb else make_codebook(D, vb, device=dev)
    k_cache = allocate_cache(nb, Hkv, kf, device=dev)
    v_cache = allocate_cache(nb, Hkv, vf, device=dev)
    fill_paged((k_cache, v_cache), (kf, vf), (kc, vc), (kbnd, vbnd), bt, lens_host, Hkv, gen, dev)
    q = torch.randn((B * n, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    cu = torch.arange(0, B * n + 1, n, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)

    def step():
        prefill_paged(q, cu, k_cache, kf, kc, v_cache, vf, vc, bt, lens, causal=True, max_q_len=n, out=out)

    ms = timed(step, steps, warmup, settle_s=0.1)["ms"]
    # (query row, visible key) pairs x 3 products (q.k, qp.signs, p.v) x 2 x 128 flops
    pairs = B * Hq * n * (n + 1) // 2
    flops = pairs * (3 if kq else 2) * 2 * D
    return {"workload": f"prefill: {B} x {n} new tokens (causal), Hq {Hq} / Hkv {Hkv}, "
                        f"turbo{kb}{'+QJL' if kq else ''} K / turbo{vb} V, bs {bs}",
            "us_per_layer": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12,
            "frac_of_fp16_mfma": flops / (ms * 1e-3) / 1e12 / FP16_MFMA_TFLOPS,
            "algorithmic_flops": flops}


COMPRESS_T, COMPRESS_H, COMPRESS_NB, COMPRESS_BS = 16384, 8, 8192, 16


def build_compress_workload(dev):
    """Benchmark config 2 inputs: K and V [16384, 8, 128] bf16 (outlier channels), slots of a
    seeded permutation of 8192 blocks of 16, turbo4 formats and codebook, zeroed caches."""
    import torch
    from turboquant.core import make_codebook
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache
    T, H, nb, bs = COMPRESS_T, COMPRESS_H, COMPRESS_NB, COMPRESS_BS
    gen = torch.Generator(device=dev).manual_seed(2)
    k = outlier_kv(T, H, gen, dev, torch.bfloat16)
    v = outlier_kv(T, H, gen, dev, torch.bfloat16)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(2))
    slots = (perm[torch.arange(T) // bs] * bs + torch.arange(T) % bs).to(torch.int32).to(dev)
    fmt = PagedKVFormat(bits=4, qjl=False, block_size=bs)
    vfmt = PagedKVFormat(bits=4, qjl=False, block_size=bs, layout="values")
    c, b = make_codebook(D, 4, device=dev)
    return dict(k=k, v=v, slots=slots, fmt=fmt, vfmt=vfmt, c=c, b=b,
                kc=allocate_cache(nb, H, fmt, device=dev), vc=allocate_cache(nb, H, vfmt, device=dev))


def compress_case(dev, steps, warmup):
    """Benchmark config 2: K and V [16384, 8, 128] bf16 -> turbo4 paged blocks of 16 in 8192 blocks."""
    from turboquant.kernels.paged import compress_paged_kv
    w = build_compress_workload(dev)

    def step():
        # the layer's K + V cache update: one launch (tq_compress_paged_kv)
        compress_paged_kv(w["k"], w["v"], w["slots"], w["kc"], w["vc"], w["fmt"], w["vfmt"], (w["c"], w["b"]),
                          (w["c"], w["b"]))

    t = timed(step, steps, warmup, settle_s=0.1)
    ms = t["ms"]
    T, H = COMPRESS_T, COMPRESS_H
    alg = 2 * (T * H * D * 2 + T * H * w["fmt"].token_bytes) + T * 4
    return {"workload": "config2: turbo4 paged compress K+V, 16384 tok x 8 heads bf16, bs 16",
            "us_per_layer": ms * 1e3, "event_median_us": t["event_median_ms"] * 1e3, "algorithmic_bytes": alg,
            "compress_gbs": alg / (ms * 1e-3) / 1e9, "frac_of_8tbs": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}, w


def config1_case(dev, steps, warmup):
    """Benchmark config 1 on the GPU: polarquant_compress of K [1024, 128] fp32 N(0,1) from seed 0,
    turbo3 + QJL, the 128 x 128 normalized WHT, d = 128 Lloyd-Max codebook (the reference's
    CPU-runnable case; int64 indices, fp32 norms, signs, k_mse as the reference returns them)."""
    import torch
    from turboquant.core import PolarQuantConfig, make_codebook, make_wht_matrix, polarquant_compress
    torch.manual_seed(0)
    K = torch.randn(1024, 128)
    cent, bnd = make_codebook(D, 3)
    H = make_wht_matrix(D)
    cfg = PolarQuantConfig(head_dim=D, bits=3, use_qjl=True)
    Kd, cd, bd, Hd = K.to(dev), cent.to(dev), bnd.to(dev), H.to(dev)
    t = timed(lambda: polarquant_compress(Kd, cd, bd, cfg, Hd), steps, warmup, settle_s=0.05)
    out = polarquant_compress(Kd, cd, bd, cfg, Hd)
    torch.cuda.synchronize()
    us = t["ms"] * 1e3
    return {"workload": "config1: polarquant_compress K [1024,128] fp32 N(0,1) seed 0, turbo3 + QJL, WHT",
            "us": us, "us_per_layer": us}, (K, cent, bnd, H, out)


def parity_leg(c1, w2):
    """Compress parity measured in this run, outside every timed region, with the CPU oracle as
    the checker: config 1's GPU output (polarquant_compress) and config 2's paged caches as the
    timed steps left them, every index against the oracle's fp32 restatement of the reference
    and its float64 shadow (oracle.compress.classify_strict: mismatches counted by their distance
    from the boundary between the two indices, in fp32 ulps; a mismatch beyond 1 ulp passes only
    where the GPU agrees with float64), sign bits likewise around the centroid."""
    import numpy as np
    import torch
    from oracle import compress as ocomp
    from oracle import packing as opack
    from oracle import paged as opaged
    from turboquant.core import make_wht_matrix
    res = {}
    K, cent, bnd, H, out = c1
    ref = ocomp.polarquant_compress(K, cent, bnd, 8, True, H)
    ref64 = ocomp.polarquant_compress_fp64(K, cent, bnd, True, True)
    st = ocomp.classify_strict(out["indices"].cpu().numpy(), ref["indices"].numpy(), ref["x_normalized"].numpy(),
                               bnd.numpy(), ref64["indices"].numpy())
    sg = (out["signs"].cpu() > 0).numpy()
    sr = (ref["signs"] > 0).numpy()
    s64 = (ref64["signs"] > 0).numpy()
    same = out["indices"].cpu().numpy() == ref["indices"].numpy()
    st["sign_mismatches"] = int((sg != sr).sum())
    st["sign_mismatches_fp64_differs"] = int(((sg != sr) & same & (sg != s64)).sum())
    st["norm_max_rel_err"] = float(((out["norms"].cpu() - ref["norms"]).abs() / ref["norms"].clamp_min(1e-30)).max())
    res["config1"] = st
    T, Hh, bs = COMPRESS_T, COMPRESS_H, COMPRESS_BS
    slots = w2["slots"].long().cpu().numpy()
    blk, row = slots // bs, slots % bs
    H128 = make_wht_matrix(D)
    c4, b4 = w2["c"].cpu(), w2["b"].cpu()
    for which, x, cache, fmt in (("K", w2["k"], w2["kc"], w2["fmt"]), ("V", w2["v"], w2["vc"], w2["vfmt"])):
        got = np.zeros((T, Hh, D), np.int64)
        for h in range(Hh):
            tok = opaged.tiles_to_tokens(cache[:, h].cpu().numpy(), bs, 4, False, fmt.layout)
            got[:, h] = opack.unpack_indices(tok["idx"][blk * bs + row], 4)
        xf = x.float().cpu().reshape(T * Hh, D)
        ref = ocomp.polarquant_compress(xf, c4, b4, 16, False, H128)
        ref64 = ocomp.polarquant_compress_fp64(xf, c4, b4, False, True)
        res[f"config2 {which}"] = ocomp.classify_strict(got.reshape(T * Hh, D), ref["indices"].numpy(),
                                                        ref["x_normalized"].numpy(), b4.numpy(), ref64["indices"].numpy())
    tot = {}
    for v in res.values():
        for k, n in v.items():
            if isinstance(n, int):
                tot[k] = tot.get(k, 0) + n
    res["all"] = tot
    res["source"] = "measured in this run (bench.py parity leg, oracle/ as the checker)"
    return res


def cpu_baseline_compress(c1, w2, seconds=6.0):
    """The reference's CPU polarquant_compress (oracle/compress.py, its torch fp32 formulation)
    timed on the host cores: config 1 whole (repeated), config 2 on a sample of 2048 tokens x 8
    heads of K and V, scaled by rows to the full 16384 tokens."""
    import torch
    from oracle import compress as ocomp
    from turboquant.core import make_wht_matrix
    K, cent, bnd, H, _ = c1
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        ocomp.polarquant_compress(K, cent, bnd, 8, True, H)
        n += 1
    c1_us = (time.perf_counter() - t0) / n * 1e6
    H128 = make_wht_matrix(D)
    c4, b4 = w2["c"].cpu(), w2["b"].cpu()
    rows = 2048 * COMPRESS_H
    xs = [w2[k][:2048].float().cpu().reshape(rows, D) for k in ("k", "v")]
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for x in xs:
            ocomp.polarquant_compress(x, c4, b4, 16, False, H128)
        n += 1
    c2_us = (time.perf_counter() - t0) / n * 1e6 * (COMPRESS_T / 2048)
    return {"config1": {"value": round(c1_us, 1), "unit": "us", "cores": torch.get_num_threads(), "kind": "port",
                        "sample": "the whole config-1 call, repeated"},
            "config2": {"value": round(c2_us, 1), "unit": "us/layer", "cores": torch.get_num_threads(), "kind": "port",
                        "sample": "K and V of 2048 of 16384 tokens x 8 heads, scaled by rows (the paged scatter "
                                  "is not included)"}}


def stream_reference(dev):
    """Untimed for the headline: this box's HBM streaming rates in the same process, so that a
    decode time can be read against the box it ran on (read: torch.amax over 2 GiB of int64;
    copy: 1 GiB read + 1 GiB written)."""
    import torch
    x = torch.ones(1 << 28, dtype=torch.int64, device=dev)
    y = torch.empty(1 << 27, dtype=torch.int64, device=dev)
    r = timed(lambda: torch.amax(x), 20, 3, settle_s=0.05)["ms"]
    c = timed(lambda: y.copy_(x[: 1 << 27]), 20, 3, settle_s=0.05)["ms"]
    del x, y
    torch.cuda.empty_cache()
    return {"read_2gib_gbs": round((2 << 30) / (r * 1e-3) / 1e9, 1), "copy_1gib_gbs": round((2 << 30) / (c * 1e-3) / 1e9, 1)}


def published_shapes(dev, steps, warmup):
    """The shapes the reference publishes MI355X numbers for (docs/BLOG_NOTES.md): the v7
    packed_attention API at BH 8/32/64 x Sk 32768 (turbo2 + QJL keys, turbo2 values), the
    end-to-end compress_k + compress_v + packed_attention pipeline at those shapes
    (:167-171: 1.41 / 5.33 / 10.84 ms) and compress_k at N = 2K..524K vectors (:66-71:
    0.050 / 0.059 / 0.098 / 0.271 ms)."""
    import torch
    from turboquant.kernels.packed_attention import packed_attention
    from turboquant.kernels.packed_compress import compress_k, compress_k_permuted, compress_v, solve_codebook
    out = {"attention": [], "pipeline": [], "compress_k": []}
    gen = torch.Generator(device=dev).manual_seed(11)
    cb = solve_codebook(D, 2).to(dev)
    bnd = (cb[:-1] + cb[1:]) / 2
    g64 = torch.Generator().manual_seed(12)
    Pi, _ = torch.linalg.qr(torch.randn(D, D, generator=g64, dtype=torch.float64))
    S = torch.randn(D, D, generator=g64, dtype=torch.float64)
    PiT = Pi.T.contiguous().float().to(dev)
    PiST = (Pi @ S.T).contiguous().float().to(dev)
    cs = math.sqrt(math.pi / 2) / D
    pub = {8: 1.41, 32: 5.33, 64: 10.84}
    for BH in (8, 32, 64):
        Sk = 32768
        K = torch.randn(BH * Sk, D, generator=gen, device=dev)
        V = torch.randn(BH * Sk, D, generator=gen, device=dev)
        Q = (torch.randn(BH, D, generator=gen, device=dev) * 0.1).half()
        Qp = (torch.randn(BH, D, generator=gen, device=dev) * 0.1).half()
        ki, ks, kr, kn = compress_k_permuted(K, PiT, PiST, cb, bnd)
        vi, vn = compress_v(V, PiT, cb, bnd)
        ki, ks, vi = ki.view(BH, Sk, -1), ks.view(BH, Sk, -1), vi.view(BH, Sk, -1)
        kr, kn, vn = kr.view(BH, Sk), kn.view(BH, Sk), vn.view(BH, Sk)

        def attend():
            return packed_attention(Q, Qp, ki, ks, kr, kn, vi, vn, cb, cs)

        ms = timed(attend, steps, warmup, settle_s=0.05)["ms"]
        nbytes = BH * Sk * (32 + 16 + 2 + 2 + 32 + 2) + 2 * BH * D * 2
        out["attention"].append({"BH": BH, "Sk": Sk, "us": ms * 1e3, "hbm_gbs": nbytes / (ms * 1e-3) / 1e9})

        def pipeline():
            a = compress_k_permuted(K, PiT, PiST, cb, bnd)
            b = compress_v(V, PiT, cb, bnd)
            return packed_attention(Q, Qp, a[0].view(BH, Sk, -1), a[1].view(BH, Sk, -1), a[2].view(BH, Sk),
                                    a[3].view(BH, Sk), b[0].view(BH, Sk, -1), b[1].view(BH, Sk), cb, cs)

        ms = timed(pipeline, max(3, steps // 4), 2, settle_s=0.05)["ms"]
        out["pipeline"].append({"BH": BH, "Sk": Sk, "us": ms * 1e3, "reference_published_us": pub[BH] * 1e3})
        del K, V, ki, ks, kr, kn, vi, vn
    pubk = {2048: 50, 32768: 59, 131072: 98, 524288: 271}
    for N in (2048, 32768, 131072, 524288):
        K = torch.randn(N, D, generator=gen, device=dev)
        ms = timed(lambda: compress_k(K, PiT, PiST, cb, bnd), steps, warmup, settle_s=0.05)["ms"]
        # two 128 x 128 fp32 products per row (rotation, sign projection)
        out["compress_k"].append({"N": N, "us": ms * 1e3, "reference_published_us": pubk[N],
                                  "fp32_tflops": N * 2 * 2 * D * D / (ms * 1e-3) / 1e12})
        del K
    return out


# batch and sequence length of each workload as the bench line's config states them (the
# longest context where the lengths vary)
WORKLOAD_SHAPE = {
    "config4": {"global_batch": 64, "seq_len": 32768},
    "config3": {"global_batch": 32, "seq_len": 8192},
    "config5": {"global_batch": 64, "seq_len": 131072},
    "config2": {"global_batch": 16384, "seq_len": 1},
    "prefill": {"global_batch": 4, "seq_len": 4096},
}


def profile_value(name, key):
    """A `key: value` line of a committed rocprof summary under profiles/ (None if absent)."""
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    m = re.search(rf"^{re.escape(key)}:\s*([-+0-9.eE]+)", path.read_text(), re.M)
    return None if m is None else float(m.group(1))


def profiled_traffic():
    """HBM bytes per launch of the headline decode kernel (two rocprofv3 --pmc runs of this script
    with --copy-calibration, FETCH_SIZE and WRITE_SIZE scaled by two kernels of known traffic)."""
    v = profile_value("decode_fast_kernel_config4_pmc.md", "traffic_bytes_per_launch")
    fs = profile_value("decode_fast_kernel_config4_pmc.md", "fetch_scale")
    ws = profile_value("decode_fast_kernel_config4_pmc.md", "write_scale")
    return (int(v), f"profiles/decode_fast_kernel_config4_pmc.md (FETCH_SIZE x{fs:g} + WRITE_SIZE x{ws:g}, calibrated on "
                    "a 256 MiB copy and multiply in the same profiled process)") \
        if v is not None and fs is not None and ws is not None else (None, None)


def cpu_info():
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    import torch
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "torch_num_threads": torch.get_num_threads()}


def cpu_baseline_decode(st, max_seconds=20.0):
    """The reference's PyTorch path in fp32 on the host cores (oracle/torch_ref.py: paged gather,
    dequantisation by table gather, bmm scores with the QJL term, softmax with the split-aware
    Sparse-V rule, bmm with V) on whole sequences of the headline workload, timed until
    max_seconds, scaled by tokens to the full batch."""
    import numpy as np
    import torch
    from oracle import paged as opaged
    from oracle import torch_ref
    kf, vf = st["kf"], st["vf"]
    bs, Hkv, G = kf.block_size, st["Hkv"], st["Hq"] // st["Hkv"]
    q = st["q"].float().cpu()
    kcb, vcb = st["kc"].float().cpu(), st["vc"].float().cpu()
    sm, cs = 1 / math.sqrt(D), math.sqrt(math.pi / 2) / D
    info = cpu_info()
    el = 0.0
    done_tokens = seqs = 0
    for s in range(st["B"]):
        L = st["lens_host"][s]
        nbl = math.ceil(L / bs)
        blocks = st["bt"][s, :nbl].long()
        # host copy of the sequence's tiles, in the row-major tile layout (untimed preparation)
        kt = st["k_cache"].index_select(0, blocks).cpu().numpy()
        vt = st["v_cache"].index_select(0, blocks).cpu().numpy()
        krows = torch.from_numpy(np.stack([_rows_tiles(kt[:, h], kf, opaged) for h in range(Hkv)], axis=1))
        vrows = torch.from_numpy(np.stack([_rows_tiles(vt[:, h], vf, opaged) for h in range(Hkv)], axis=1))
        local_bt = torch.arange(nbl, dtype=torch.int32)
        t0 = time.perf_counter()
        for kh in range(Hkv):
            kp = torch_ref.gather_rows(krows, local_bt, L, kh, bs, kf.idx_bytes, kf.qjl)
            vp = torch_ref.gather_rows(vrows, local_bt, L, kh, bs, vf.idx_bytes, False)
            k, sg, rn = torch_ref.dequant(kp, kcb, kf.bits, kf.qjl)
            v, _, _ = torch_ref.dequant(vp, vcb, vf.bits, False)
            qs = q[s, kh * G:(kh + 1) * G]
            torch_ref.decode(qs, qs, k, sg, rn, v, sm, cs, st["chunk"], st["thresh"])
        el += time.perf_counter() - t0
        done_tokens += L
        seqs += 1
        if el > max_seconds:
            break
    total = sum(st["lens_host"])
    return {"value": round(el / done_tokens * total * 1e6, 1), "unit": "us/layer", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{seqs} of {st['B']} sequences (all {Hkv} KV heads, {done_tokens} tokens), torch fp32 on the "
                      f"host (paged gather, dequant, bmm scores + QJL, split-aware Sparse-V softmax, bmm V), "
                      f"{el:.1f} s, scaled linearly by tokens",
            **info}


def _rows_tiles(tiles, fmt, opaged):
    """Tiles [n, tile_bytes] in fmt's layout -> the same tiles in the row-major layout."""
    import numpy as np
    tok = opaged.tiles_to_tokens(tiles, fmt.block_size, fmt.bits, fmt.qjl, fmt.layout)
    n, bs = tiles.shape[0], fmt.block_size
    parts = [tok["idx"].reshape(n, -1)]
    if fmt.qjl:
        parts.append(tok["signs"].reshape(n, -1))
    parts.append(tok["norm"].view(np.uint8).reshape(n, -1))
    if fmt.qjl:
        parts.append(tok["rnorm"].view(np.uint8).reshape(n, -1))
    return np.ascontiguousarray(np.concatenate(parts, axis=1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the host legs: CPU baselines and the oracle parity check")
    ap.add_argument("--no-published", action="store_true", help="skip the reference-published shapes")
    ap.add_argument("--only", choices=["config1", "config2", "config3", "config4", "config5", "prefill", "published"],
                    default=None)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 256 MiB device-to-device copy (reference for rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    steps, warmup = args.steps, args.warmup
    if args.copy_calibration:
        # Two kernels of known traffic: the runtime's device copy and an elementwise multiply,
        # each reading 256 MiB and writing 256 MiB.
        src = torch.ones(1 << 26, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        print("# copy calibration: copyBuffer and mul kernels, 268435456 bytes read and 268435456 bytes "
              "written each", file=sys.stderr, flush=True)
        del src, dst
    extra = {}

    def want(k):
        return args.only in (None, k)

    head = None
    cpu = None
    if want("config4"):
        head, state4 = decode_case("config4", dev, steps, warmup, time_rotated=True)
        print(f"# config4 {head['us_per_layer']:.1f} us/layer (per-step events {head['event_median_us']:.1f}), "
              f"{head['hbm_gbs']:.0f} GB/s",
              file=sys.stderr, flush=True)
        if args.only is None:
            extra["stream_reference"] = stream_reference(dev)
            print(f"# stream reference {extra['stream_reference']}", file=sys.stderr, flush=True)
        if not args.no_cpu_baseline:
            cpu = cpu_baseline_decode(state4)
            print(f"# cpu baseline {cpu['value']:.0f} us/layer ({cpu['cores']} threads)", file=sys.stderr, flush=True)
        del state4
        torch.cuda.empty_cache()
    for key in ("config3", "config5"):
        if want(key):
            r, _ = decode_case(key, dev, steps, warmup)
            extra[key] = r
            print(f"# {key} {r['us_per_layer']:.1f} us (per-step events {r['event_median_us']:.1f})", file=sys.stderr,
                  flush=True)
            torch.cuda.empty_cache()
    if want("prefill"):
        rp = prefill_case(dev, min(steps, 20), min(warmup, 5))
        extra["prefill"] = rp
        print(f"# prefill {rp['us_per_layer']:.1f} us/layer, {rp['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
    w2 = c1 = None
    if want("config2"):
        r2, w2 = compress_case(dev, steps, warmup)
        extra["config2"] = r2
        print(f"# config2 {r2['us_per_layer']:.1f} us (per-step events {r2['event_median_us']:.1f}), "
              f"{r2['compress_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    if want("config2") or args.only == "config1":
        r1, c1 = config1_case(dev, steps, warmup)
        extra["config1"] = r1
        print(f"# config1 {r1['us']:.1f} us", file=sys.stderr, flush=True)
    if c1 is not None and w2 is not None and not args.no_cpu_baseline:
        extra["parity"] = parity_leg(c1, w2)
        print(f"# parity leg: {extra['parity']['all']}", file=sys.stderr, flush=True)
        extra["cpu_baselines_compress"] = cpu_baseline_compress(c1, w2)
        print(f"# cpu baselines (compress): config1 {extra['cpu_baselines_compress']['config1']['value']:.0f} us, "
              f"config2 {extra['cpu_baselines_compress']['config2']['value']:.0f} us", file=sys.stderr, flush=True)
    if w2 is not None:
        del w2
        torch.cuda.empty_cache()
    if (args.only == "published") or (args.only is None and not args.no_published):
        extra["reference_published_shapes"] = published_shapes(dev, steps, warmup)
        print("# published shapes done", file=sys.stderr, flush=True)

    if head is None and args.only == "published":
        print(json.dumps({"reference_published_shapes": extra["reference_published_shapes"]}))
        return
    if head is None:
        key = next(iter(extra))
        head = extra.pop(key)
    us = head["us_per_layer"]
    traffic, traffic_src = profiled_traffic() if head["workload"].startswith("config4") else (None, None)
    mfma = profile_value("decode_fast_kernel_config4_pmc.md", "mfma_busy_fraction")
    details = {"headline": head, **extra,
               "timing": "after a settle phase (settle_ms, untimed) and W warmup steps: K steps back to back "
                         "between one pair of HIP events, synchronize on both sides, total / K; median of "
                         f"{BRACKETS} such brackets.  event_median_us: median of a further K steps with an "
                         "event recorded after each (the events' own queue signals included)",
               "reference_published_us_per_layer": {"turbo3_v12_sparse_v": 843, "turbo4": 797,
                                                    "note": "MI355X Triton, shape unstated (README.md:102-103)"}}
    if mfma is not None:
        details["mfma_busy_fraction_headline"] = mfma
    for name, prof in (("config3", "decode_fast_kernel_config3_pmc.md"), ("config5", "decode_fast_kernel_config5_pmc.md"),
                       ("prefill", "prefill_kernel_4x4096_pmc.md")):
        v = profile_value(prof, "mfma_busy_fraction")
        if v is not None:
            details.setdefault("mfma_busy_fraction_by_kernel", {})[name] = v
    details["operand_precision"] = {
        "qk": "q and dequantized K in fp16 (centroid tables scaled into [1, 2) x c), fp32 accumulation",
        "qjl": "fp4 +-1 signs x q_proj*corr as three fp6 e2m3 parts with per-32-element E8M0 scales "
               "(each element within 2^-14 of its block's largest magnitude; fp16 carries 2^-11 of each)",
        "pv": "dequantized V and p * norm in fp16, fp32 accumulation; softmax in fp32"}
    line = {
        "metric": METRIC,
        "value": round(us, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": head["workload"], **WORKLOAD_SHAPE.get(head["workload"].split(":")[0], {}),
                   "parallelism": "none"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(head.get("hbm_gbs", head.get("compress_gbs", 0.0)), 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head.get("frac_of_8tbs", 0.0), 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
        },
        "cpu_baseline": cpu,
        "details": details,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
