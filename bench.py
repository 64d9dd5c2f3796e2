#!/usr/bin/env python3
"""Benchmark of the TurboQuant packed-KV hot path on one MI355X.

Prints ONE JSON line.  Headline (`value`): benchmark config 4 — Sparse-V split-K decode, turbo3
+ QJL keys / turbo3 values, batch 64 x context 32768, 48 query / 8 KV heads, block 16,
threshold 1e-4 — in us per layer (one tq_decode call = one layer's decode for the batch).
The same line carries configs 2 (turbo4 paged compress), 3 (turbo4 decode) and 5 (turbo2 + QJL
compress + decode step), the roofline of the headline kernel and a CPU baseline.

Inputs are synthetic (seeded) and resident in HBM before the timed region; timing uses HIP
events on the stream the kernels run on (torch's current stream), W untimed warmup steps, then
exactly K timed steps bracketed by torch.cuda.synchronize().
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "turboquant-amd_amd"))

METRIC = "packed-KV decode attn μs/layer + HBM GB/s (% roofline); compress GB/s"
HBM_PEAK_GBS = 8000.0
D = 128


def outlier_kv(T, H, gen, device, dtype):
    """N(0,1) x per-channel log-normal(0, 0.5) scale, 2% of channels x8 (benchmark config 2)."""
    import torch
    scale = torch.exp(torch.randn(H, D, generator=gen, device=device) * 0.5)
    out = torch.rand(H, D, generator=gen, device=device) < 0.02
    scale = torch.where(out, scale * 8, scale)
    return (torch.randn(T, H, D, generator=gen, device=device) * scale).to(dtype)


def profiled_traffic(head):
    """HBM bytes per launch of the headline decode kernel from the committed rocprof summary.

    profiles/decode_fast_kernel_config4_pmc.md holds FETCH_SIZE and WRITE_SIZE of the kernel (two
    rocprofv3 --pmc runs of this script with --copy-calibration), scaled by what the same
    counters read for two kernels of known traffic.  Returned only for the config 4 headline.
    """
    import re
    path = ROOT / "profiles" / "decode_fast_kernel_config4_pmc.md"
    if not head.get("workload", "").startswith("config4") or not path.exists():
        return None, None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", path.read_text(), re.M)
    if not m:
        return None, None
    return int(m.group(1)), "profiles/decode_fast_kernel_config4_pmc.md (FETCH_SIZE x2.0 + WRITE_SIZE x1.0, copy-calibrated)"


def timed(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def read_stream_reference(dev, nbytes=1 << 31, steps=20, warmup=3):
    """A practical read ceiling of the GPU the bench runs on: torch's amax over a 2 GiB int64
    tensor (a library streaming reduction), timed like the workloads."""
    import torch
    x = torch.ones(nbytes // 8, dtype=torch.int64, device=dev)
    ms = timed(lambda: torch.amax(x), steps, warmup)
    del x
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"op": "torch.amax over a 2 GiB int64 tensor", "read_gbs": round(gbs, 1),
            "frac_of_8tbs": round(gbs / HBM_PEAK_GBS, 4)}


def fill_paged(kv_cache_pair, fmts, centroids, boundaries, block_tables, seq_lens_host, Hkv, gen, dev, chunk_tokens=1 << 20):
    """Compress synthetic K and V for every sequence into the caches (untimed setup)."""
    import torch
    from turboquant.kernels.paged import compress_paged
    bs = fmts[0].block_size
    S = len(seq_lens_host)
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

    for s in range(S):
        L = int(seq_lens_host[s])
        t = torch.arange(L)
        slots.append((bt_host[s, t // bs].long() * bs + t % bs).to(torch.int32))
        toks.append(L)
        pending += L
        if pending >= chunk_tokens:
            flush()
    flush()


def decode_case(name, B, Hq, Hkv, lens_host, kb, kq, vb, thresh, bs, seed, dev, steps, warmup, extra_compress=None,
                time_rotated=False):
    import torch
    from turboquant.core import make_codebook
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, decode_paged, plan_tokens_per_chunk

    gen = torch.Generator(device=dev).manual_seed(seed)
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout="values")
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
    lens = torch.tensor(lens_host, dtype=torch.int32, device=dev)
    kc, kbnd = make_codebook(D, kb, device=dev)
    # one codebook tensor per bit width, shared by K and V as a serving stack holds it
    vc, vbnd = (kc, kbnd) if vb == kb else make_codebook(D, vb, device=dev)
    k_cache = allocate_cache(nb, Hkv, kf, device=dev)
    v_cache = allocate_cache(nb, Hkv, vf, device=dev)
    fill_paged((k_cache, v_cache), (kf, vf), (kc, vc), (kbnd, vbnd), bt, lens_host, Hkv, gen, dev)
    q = torch.randn((B, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    msl = max(lens_host)
    chunk = plan_tokens_per_chunk(dev, B, Hq, Hkv, msl, kf, vf, kc is vc, lens_host)
    from turboquant import _lib
    ws = torch.empty(_lib.lib().tq_decode_workspace_bytes(B, Hq, msl, chunk), dtype=torch.uint8, device=dev)
    stats = torch.zeros(2, dtype=torch.int64, device=dev)

    def step():
        decode_paged(q, k_cache, kf, kc, v_cache, vf, vc, bt, lens, sparse_threshold=thresh,
                     max_seq_len=msl, tokens_per_chunk=chunk, out=out, workspace=ws)

    if extra_compress is not None:
        step_inner = step
        newk = outlier_kv(B, Hkv, gen, dev, torch.bfloat16)
        newv = outlier_kv(B, Hkv, gen, dev, torch.bfloat16)
        # one new token per sequence goes into the last slot of its context
        last = torch.tensor([L - 1 for L in lens_host])
        slot_new = (bt.cpu()[torch.arange(B), last // bs].long() * bs + last % bs).to(torch.int32).to(dev)
        from turboquant.kernels.paged import compress_paged

        def step():  # noqa: F811
            compress_paged(newk, slot_new, k_cache, kf, kc, kbnd)
            compress_paged(newv, slot_new, v_cache, vf, vc, vbnd)
            step_inner()

    ms = timed(step, steps, warmup)
    ms_rot = None
    if time_rotated:
        # the same decode with q and the output in the model basis (rotations fused)
        def step_rot():
            decode_paged(q, k_cache, kf, kc, v_cache, vf, vc, bt, lens, sparse_threshold=thresh,
                         max_seq_len=msl, tokens_per_chunk=chunk, out=out, workspace=ws, rotate=True)
        ms_rot = timed(step_rot, steps, warmup)
    skip_frac = None
    if thresh > 0:
        decode_paged(q, k_cache, kf, kc, v_cache, vf, vc, bt, lens, sparse_threshold=thresh,
                     max_seq_len=msl, tokens_per_chunk=chunk, out=out, workspace=ws, skip_stats=stats)
        torch.cuda.synchronize()
        sk, tot = stats.tolist()
        skip_frac = sk / max(tot, 1)
    tokens = sum(lens_host)
    kv_bytes = tokens * Hkv * (kf.token_bytes + vf.token_bytes)
    io_bytes = 2 * B * Hq * D * 2 + bt.numel() * 4 + B * 4
    alg_bytes = kv_bytes + io_bytes
    res = {
        "workload": name, "us_per_layer": ms * 1e3, "algorithmic_bytes": alg_bytes, "kv_bytes": kv_bytes,
        "hbm_gbs": alg_bytes / (ms * 1e-3) / 1e9, "frac_of_8tbs": alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_chunk": chunk, "mean_ctx": tokens / B,
    }
    if skip_frac is not None:
        res["sparse_v_skip_fraction"] = skip_frac
    if ms_rot is not None:
        res["rotated_us_per_layer"] = ms_rot * 1e3
    state = dict(q=q, k_cache=k_cache, v_cache=v_cache, kf=kf, vf=vf, kc=kc, vc=vc, bt=bt, lens=lens,
                 lens_host=lens_host, Hkv=Hkv, chunk=chunk)
    return res, state


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

    ms = timed(step, steps, warmup)
    # (query row, visible key) pairs x 3 products (q.k, qp.signs, p.v) x 2 x 128 flops
    pairs = B * Hq * n * (n + 1) // 2
    flops = pairs * (3 if kq else 2) * 2 * D
    return {"workload": f"prefill: {B} x {n} new tokens (causal), Hq {Hq} / Hkv {Hkv}, "
                        f"turbo{kb}{'+QJL' if kq else ''} K / turbo{vb} V, bs {bs}",
            "us_per_layer": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12,
            "frac_of_fp16_mfma": flops / (ms * 1e-3) / 1e12 / 2500.0,
            "algorithmic_flops": flops}


def compress_case(dev, steps, warmup):
    """Benchmark config 2: K and V [16384, 8, 128] bf16 -> turbo4 paged blocks of 16 in 8192 blocks."""
    import torch
    from turboquant.core import make_codebook
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, nb, bs = 16384, 8, 8192, 16
    gen = torch.Generator(device=dev).manual_seed(2)
    k = outlier_kv(T, H, gen, dev, torch.bfloat16)
    v = outlier_kv(T, H, gen, dev, torch.bfloat16)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(2))
    slots = (perm[torch.arange(T) // bs] * bs + torch.arange(T) % bs).to(torch.int32).to(dev)
    fmt = PagedKVFormat(bits=4, qjl=False, block_size=bs)
    vfmt = PagedKVFormat(bits=4, qjl=False, block_size=bs, layout="values")
    c, b = make_codebook(D, 4, device=dev)
    kc = allocate_cache(nb, H, fmt, device=dev)
    vc = allocate_cache(nb, H, vfmt, device=dev)

    def step():
        compress_paged(k, slots, kc, fmt, c, b)
        compress_paged(v, slots, vc, vfmt, c, b)

    ms = timed(step, steps, warmup)
    alg = 2 * (T * H * D * 2 + T * H * fmt.token_bytes) + T * 4
    return {"workload": "config2: turbo4 paged compress K+V, 16384 tok x 8 heads bf16, bs 16",
            "us_per_layer": ms * 1e3, "algorithmic_bytes": alg, "compress_gbs": alg / (ms * 1e-3) / 1e9,
            "frac_of_8tbs": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def _gather_tiles(cache_np, blocks, kh, fmt, L):
    """Vectorized read of one (sequence, KV head) through its block table -> per-token payload."""
    import numpy as np
    bs = fmt.block_size
    tiles = cache_np[blocks, kh]                                   # [nblk, tile]
    nblk = tiles.shape[0]
    out = {"idx": tiles[:, : bs * fmt.idx_bytes].reshape(nblk * bs, fmt.idx_bytes)[:L],
           "norm": tiles[:, fmt.off_norm: fmt.off_norm + 2 * bs].copy().view(np.uint16).reshape(-1)[:L]}
    if fmt.qjl:
        out["signs"] = tiles[:, fmt.off_signs: fmt.off_signs + 16 * bs].reshape(nblk * bs, 16)[:L]
        out["rnorm"] = tiles[:, fmt.off_rnorm: fmt.off_rnorm + 2 * bs].copy().view(np.uint16).reshape(-1)[:L]
    return out


def cpu_baseline_decode(state, max_seconds=20.0):
    """The oracle's float64 decode (a CPU restatement of the reference's PyTorch path:
    dequantize, scores, softmax, weighted sum, with the Sparse-V chunk walk) on whole sequences
    of the headline workload, scaled by tokens to the full batch."""
    import numpy as np
    from oracle import decode as odec
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    threads = min(os.cpu_count() or 1, 16)
    from turboquant.kernels.paged import to_rows_layout
    kf, vf = state["kf"], state["vf"]
    # the payload in row form (index rows, then sign rows): what _gather_tiles reads
    kc_np = to_rows_layout(state["k_cache"], kf).cpu().numpy()
    vc_np = to_rows_layout(state["v_cache"], vf).cpu().numpy()
    bt = state["bt"].cpu().numpy()
    q = state["q"].float().cpu().numpy().astype(np.float64)
    kcb = state["kc"].double().cpu().numpy()
    vcb = state["vc"].double().cpu().numpy()
    Hkv = state["Hkv"]
    G = q.shape[1] // Hkv
    limiter = threadpool_limits(limits=threads) if threadpool_limits is not None else None
    t0 = time.perf_counter()
    done_tokens = 0
    seqs = 0
    for s in range(len(state["lens_host"])):
        L = state["lens_host"][s]
        blocks = bt[s, : math.ceil(L / kf.block_size)]
        for kh in range(Hkv):
            kp = _gather_tiles(kc_np, blocks, kh, kf, L)
            vp = _gather_tiles(vc_np, blocks, kh, vf, L)
            k, sg, rn = odec.dequant_keys(kp, kcb, kf.bits, kf.qjl)
            v = odec.dequant_values(vp, vcb, vf.bits)
            hs = slice(kh * G, (kh + 1) * G)
            odec.decode_chunked(q[s, hs], q[s, hs], k, sg, rn, v, 1 / math.sqrt(D),
                                math.sqrt(math.pi / 2) / D, state["chunk"], 1e-4)
        done_tokens += L
        seqs += 1
        if time.perf_counter() - t0 > max_seconds:
            break
    el = time.perf_counter() - t0
    if limiter is not None:
        limiter.restore_original_limits()
    total = sum(state["lens_host"])
    us_full = el / done_tokens * total * 1e6
    return {"value": round(us_full, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "sample": f"{seqs} of {len(state['lens_host'])} sequences (all {Hkv} KV heads, {done_tokens} tokens), "
                      f"numpy float64 oracle incl. paged gather + dequant, {el:.1f} s, scaled linearly by tokens",
            "cpu_model": platform.processor() or platform.machine()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 100 + 100 by default: the first tens of milliseconds after the (host-side) set-up run
    # ~12 % slower on MI355X (measured: 530 us/layer for a 30-step window after 5 warm-up steps,
    # 463-471 us when re-timed right after), so the warm-up covers that ramp.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["config2", "config3", "config4", "config5", "prefill"], default=None)
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
    import random

    head = None
    state4 = None
    if args.only in (None, "config4"):
        head, state4 = decode_case(
            "config4: Sparse-V split-K decode, turbo3+QJL K / turbo3 V, B=64 x ctx 32768, Hq 48 / Hkv 8, bs 16, T=1e-4",
            64, 48, 8, [32768] * 64, 3, True, 3, 1e-4, 16, 4, dev, steps, warmup, time_rotated=True)
        print(f"# config4 {head['us_per_layer']:.1f} us/layer, {head['hbm_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    if args.only in (None, "config3"):
        rng = random.Random(3)  # one generator per workload: --only gives the same lengths
        lens3 = [rng.randint(1024, 8192) for _ in range(32)]
        r3, _ = decode_case("config3: turbo4 decode, B=32, Hq 32 / Hkv 8, ctx U[1K,8K], bs 16",
                            32, 32, 8, lens3, 4, False, 4, 0.0, 16, 3, dev, steps, warmup)
        extra["config3"] = r3
        print(f"# config3 {r3['us_per_layer']:.1f} us/layer", file=sys.stderr, flush=True)
    if args.only in (None, "config5"):
        rng = random.Random(5)
        lens5 = [int(round(math.exp(rng.uniform(math.log(2048), math.log(131072))))) for _ in range(64)]
        r5, _ = decode_case("config5: turbo2+QJL compress 64 new tokens + decode, B=64, Hq 64 / Hkv 8, "
                            "ctx log-U[2K,128K], bs 16", 64, 64, 8, lens5, 2, True, 2, 0.0, 16, 5, dev, steps, warmup,
                            extra_compress=True)
        extra["config5"] = r5
        print(f"# config5 {r5['us_per_layer']:.1f} us/step", file=sys.stderr, flush=True)
    if args.only in (None, "prefill"):
        rp = prefill_case(dev, min(steps, 20), min(warmup, 5))
        extra["prefill"] = rp
        print(f"# prefill {rp['us_per_layer']:.1f} us/layer, {rp['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
    if args.only in (None, "config2"):
        r2 = compress_case(dev, steps, warmup)
        extra["config2"] = r2
        print(f"# config2 {r2['us_per_layer']:.1f} us, {r2['compress_gbs']:.0f} GB/s", file=sys.stderr, flush=True)

    if head is None:
        key = next(iter(extra))
        head = extra.pop(key)
    stream_ref = read_stream_reference(dev)
    print(f"# read stream reference {stream_ref['read_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    cpu = None
    if state4 is not None and not args.no_cpu_baseline:
        cpu = cpu_baseline_decode(state4)
    us = head["us_per_layer"]
    traffic, traffic_src = profiled_traffic(head)
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
        "config": {"workload": head["workload"], "global_batch": 64, "seq_len": 32768, "parallelism": "none"},
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
        "details": {"headline": head, **extra, "read_stream_reference": stream_ref,
                    "reference_published_us_per_layer": {"turbo3_v12_sparse_v": 843, "turbo4": 797,
                                                          "note": "MI355X Triton, shape unstated (README.md:102-103)"}},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
