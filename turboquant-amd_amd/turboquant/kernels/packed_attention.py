"""Packed attention on contiguous per-head arrays (drop-in for the reference's v7 API).

packed_attention keeps the signature of kernels/packed_attention.py:290-344 and reads the
same arrays: 2-bit K/V indices [BH, Sk, 32], stride-4 permuted QJL sign rows [BH, Sk, 16],
fp16 norms / residual norms [BH, Sk].  It is one call of the C entry tq_packed_attention, whose
argument list is the reference function's: each of the BH query heads is a sequence with its
own KV (no GQA), 16-token tiles addressed by stride instead of a block table.  For Sk a
multiple of 16 the library runs its row-major kernel (decode_contig_kernel: the fast kernel's
pair loop with loads for these arrays); other Sk go through the general decode kernel.

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
from turboquant.kernels.paged import MI355X_CUS, decode_workspace

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


def packed_attention(Q, Q_proj, k_idx_packed, k_signs_packed, k_r_norm, k_norm,
                     v_idx_packed, v_norm, centroids, corr_scale,
                     num_splits=None, block_sk=None, num_warps=None, num_stages=None):
    """Split-K decode over packed 2-bit K (+ QJL) and 2-bit V; returns fp16 [BH, D].

    Q, Q_proj: [BH, D] (any float dtype; scores are not scaled, the caller pre-scales Q).
    k_signs_packed must be in the permuted order (permute_signs_for_chunked).
    num_splits selects the split count; block_sk / num_warps / num_stages are Triton tuning
    knobs of the reference and are accepted and ignored.  One call of the C entry
    tq_packed_attention, which takes the reference's argument list.
    """
    dev = _lib.require_gpu("packed_attention", Q, Q_proj, k_idx_packed, k_signs_packed, k_r_norm, k_norm,
                           v_idx_packed, v_norm, centroids)
    BH, D = Q.shape
    if D != 128:
        raise ValueError("head_dim must be 128")
    if tuple(Q_proj.shape) != (BH, D):
        raise ValueError(f"Q_proj must be {(BH, D)}, got {tuple(Q_proj.shape)}")
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
        ts[name] = t if t.is_contiguous() else t.contiguous()
    if centroids.numel() != 4:
        raise ValueError("packed_attention uses a 2-bit codebook (4 centroids)")
    cb = centroids
    if cb.dtype != torch.float32 or cb.device != dev or not cb.is_contiguous():
        cb = cb.to(device=dev, dtype=torch.float32).contiguous()
    q = Q if Q.dtype in (torch.float32, torch.float16, torch.bfloat16) else Q.float()
    qp = Q_proj if Q_proj.dtype == q.dtype else Q_proj.to(q.dtype)
    q = q if q.is_contiguous() else q.contiguous()
    qp = qp if qp.is_contiguous() else qp.contiguous()
    out = torch.empty((BH, D), dtype=torch.float16, device=dev)
    # num_splits given: that many chunks; otherwise the library's choice (for Sk a multiple of 16,
    # the row-major kernel with one round of the resident waves)
    chunk = _chunk_for(BH, Sk, num_splits) if num_splits else 0
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    ws = decode_workspace(dev, L.tq_packed_attention_workspace_bytes(BH, Sk, chunk))
    rc = L.tq_packed_attention(q.data_ptr(), qp.data_ptr(), _lib.dtype_code(q), ts["k_idx_packed"].data_ptr(),
                               ts["k_signs_packed"].data_ptr(), 1, ts["k_r_norm"].data_ptr(), ts["k_norm"].data_ptr(),
                               ts["v_idx_packed"].data_ptr(), ts["v_norm"].data_ptr(), cb.data_ptr(),
                               _lib.centroid_scale(cb), float(corr_scale), BH, Sk, chunk, ws.data_ptr(), ws.numel(),
                               out.data_ptr(), _lib.TQ_F16, stream)
    _lib.check(rc, "tq_packed_attention")
    return out


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


def _random_case(BH: int, Sk: int, D: int, dev, gen):
    u8 = lambda *s: torch.randint(0, 256, s, dtype=torch.uint8, device=dev, generator=gen)  # noqa: E731
    f16 = lambda *s: torch.rand(s, device=dev, generator=gen).half()  # noqa: E731
    return dict(k_idx_packed=u8(BH, Sk, D // 4), k_signs_packed=u8(BH, Sk, D // 8),
                k_r_norm=f16(BH, Sk) * 0.1, k_norm=f16(BH, Sk) + 0.5, v_idx_packed=u8(BH, Sk, D // 4),
                v_norm=f16(BH, Sk) + 0.5,
                Q=(torch.randn(BH, D, device=dev, generator=gen) * 0.1).half(),
                Q_proj=(torch.randn(BH, D, device=dev, generator=gen) * 0.1).half())


def _unpacked(case: dict, centroids, D: int):
    BH, Sk, _ = case["k_idx_packed"].shape
    k_idx = unpack_2bit(case["k_idx_packed"].reshape(-1, D // 4), D).reshape(BH, Sk, D).long()
    k_sg = unpack_1bit(case["k_signs_packed"].reshape(-1, D // 8), D).reshape(BH, Sk, D)
    v_idx = unpack_2bit(case["v_idx_packed"].reshape(-1, D // 4), D).reshape(BH, Sk, D).long()
    return (centroids[k_idx] * case["k_norm"].float().unsqueeze(-1), k_sg.float() * 2 - 1,
            case["k_r_norm"].float(), centroids[v_idx] * case["v_norm"].float().unsqueeze(-1))


def run(bh_list=(8, 32, 64), sk_check=(256, 4096, 16384, 32768), sk_bench=(256, 1024, 4096, 16384, 32768),
        warmup: int = 20, iters: int = 200, seed: int = 42, verbose: bool = True) -> dict:
    """Self-test and benchmark of packed_attention on cuda:0 (the role of the reference
    module's run(), kernels/packed_attention.py:347-460).

    Random packed K (2-bit + permuted QJL signs) and V with fp16 norms, the 2-bit kernel
    codebook, corr_scale = sqrt(pi/2)/sqrt(D).  Correctness: packed_attention against
    attention_unpacked_ref on the unpacked tensors (cosine and max abs difference).  Benchmark:
    mean device time of packed_attention and of attention_unpacked_ref per call.  Returns the
    figures printed."""
    from turboquant.kernels._selfcheck import time_ms
    from turboquant.kernels.packed_compress import permute_signs_for_chunked, solve_codebook
    dev = torch.device("cuda")
    D = 128
    centroids = solve_codebook(D, 2).to(dev)
    corr_scale = math.sqrt(math.pi / 2) / math.sqrt(D)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    say = print if verbose else (lambda *a, **k: None)
    say(f"Packed attention on {torch.cuda.get_device_name(0)}: D={D}, 2-bit K + QJL, 2-bit V")
    res = {"correctness": [], "benchmark": []}

    def call(c, perm):
        return packed_attention(c["Q"], c["Q_proj"], c["k_idx_packed"], perm, c["k_r_norm"], c["k_norm"],
                                c["v_idx_packed"], c["v_norm"], centroids, corr_scale)

    for BH in bh_list:
        for Sk in sk_check:
            c = _random_case(BH, Sk, D, dev, gen)
            kmse, sg, rn, vmse = _unpacked(c, centroids, D)
            ref = attention_unpacked_ref(c["Q"].float(), c["Q_proj"].float(), kmse, sg, rn, vmse, corr_scale)
            out = call(c, permute_signs_for_chunked(c["k_signs_packed"], D)).float()
            cos = F.cosine_similarity(ref.reshape(1, -1), out.reshape(1, -1)).item()
            err = (out - ref).abs().max().item()
            ok = cos > 0.99
            res["correctness"].append({"BH": BH, "Sk": Sk, "cos": cos, "max_abs_err": err, "pass": ok})
            say(f"  BH={BH:>3} Sk={Sk:>5}: cos={cos:.6f} max|diff|={err:.2e} {'PASS' if ok else 'FAIL'}")
            del c, kmse, sg, rn, vmse
    say(f"{'BH':>4} {'Sk':>6} {'packed ms':>10} {'torch ms':>10} {'speedup':>8}")
    for BH in bh_list:
        for Sk in sk_bench:
            c = _random_case(BH, Sk, D, dev, gen)
            perm = permute_signs_for_chunked(c["k_signs_packed"], D)
            p_ms = time_ms(lambda: call(c, perm), warmup, iters)
            kmse, sg, rn, vmse = _unpacked(c, centroids, D)
            q, qp = c["Q"].float(), c["Q_proj"].float()
            r_ms = time_ms(lambda: attention_unpacked_ref(q, qp, kmse, sg, rn, vmse, corr_scale), warmup, iters)
            res["benchmark"].append({"BH": BH, "Sk": Sk, "packed_ms": p_ms, "torch_ms": r_ms})
            say(f"{BH:>4} {Sk:>6} {p_ms:>10.4f} {r_ms:>10.4f} {r_ms / p_ms:>7.2f}x")
            del c, kmse, sg, rn, vmse
    return res


if __name__ == "__main__":
    run()
