"""Packed compression helpers (drop-in names of the reference's kernels/packed_compress.py).

Bit-level helpers run as HIP kernels: permute_signs_for_chunked (tq_permute_signs) and
unpack_2bit / unpack_1bit (tq_unpack_bits).  solve_codebook here is the kernel files' own
codebook recipe (kernels/packed_compress.py:21-41), which differs from
turboquant.core.make_codebook (fact documented by the reference: two codebooks exist).
"""

from __future__ import annotations

import math

import torch

from turboquant import _lib


def solve_codebook(d: int, bits: int) -> torch.Tensor:
    """Kernel-file Lloyd-Max variant: centroids start uniform on +-3.5 sigma (cell midpoints),
    cells extend to +-10.5 sigma, up to 200 rounds until the centroid change is < 1e-10.
    Returns fp32 centroids [2^bits] (kernels/packed_compress.py:21-41).  For d = 128, bits 1-4
    the values come from the committed table (turboquant/core/codebook_d128.json, written by the
    same recipe), so no scipy is needed."""
    from turboquant.core import codebook as _cb
    if int(d) == _cb.TABLE_D and int(bits) in _cb.TABLE_BITS:
        return torch.tensor(_cb.kernel_table()[int(bits)], dtype=torch.float32)
    return torch.tensor(_solve_kernel_recipe(int(d), int(bits)), dtype=torch.float32)


def _solve_kernel_recipe(d: int, bits: int) -> list:
    from scipy import integrate

    n_levels = 2 ** bits
    sigma = 1.0 / math.sqrt(d)

    def pdf(x):
        return (1.0 / math.sqrt(2 * math.pi * sigma**2)) * math.exp(-x * x / (2 * sigma**2))

    def first_moment(x):
        return x * pdf(x)

    lo, hi = -3.5 * sigma, 3.5 * sigma
    centroids = [lo + (hi - lo) * (i + 0.5) / n_levels for i in range(n_levels)]
    for _ in range(200):
        boundaries = [(centroids[i] + centroids[i + 1]) / 2.0 for i in range(n_levels - 1)]
        edges = [lo * 3] + boundaries + [hi * 3]
        new_c = []
        for i in range(n_levels):
            a, b = edges[i], edges[i + 1]
            num, _ = integrate.quad(first_moment, a, b)
            den, _ = integrate.quad(pdf, a, b)
            new_c.append(num / den if den > 1e-15 else centroids[i])
        if max(abs(new_c[i] - centroids[i]) for i in range(n_levels)) < 1e-10:
            break
        centroids = new_c
    return centroids


def _rows(packed: torch.Tensor, row_bytes: int, what: str) -> torch.Tensor:
    if packed.dtype == torch.int8:
        packed = packed.view(torch.uint8)
    if packed.dtype != torch.uint8 or packed.shape[-1] != row_bytes:
        raise ValueError(f"{what}: expected uint8 rows of {row_bytes} bytes, got {packed.dtype} {tuple(packed.shape)}")
    return packed.contiguous()


def unpack_bits(packed: torch.Tensor, bits: int, D: int = 128) -> torch.Tensor:
    """[..., D*bits/8] uint8 rows of little-endian b-bit fields -> int8 [N, D] (N = rows)."""
    _lib.require_gpu("unpack_bits", packed)
    if D != 128:
        raise ValueError("D must be 128")
    rows = _rows(packed, D * bits // 8, "unpack_bits")
    n = rows.numel() // (D * bits // 8)
    out = torch.empty((n, D), dtype=torch.int8, device=rows.device)
    rc = _lib.lib().tq_unpack_bits(rows.data_ptr(), out.data_ptr(), n, D, bits, _lib.stream_handle(rows.device))
    _lib.check(rc, "tq_unpack_bits")
    return out


def unpack_2bit(packed: torch.Tensor, D: int) -> torch.Tensor:
    """[N, D/4] -> int8 [N, D] with values 0..3 (kernels/packed_compress.py:145-148)."""
    return unpack_bits(packed, 2, D)


def unpack_1bit(packed: torch.Tensor, D: int) -> torch.Tensor:
    """[N, D/8] -> int8 [N, D] with values 0/1 (kernels/packed_compress.py:150-154)."""
    return unpack_bits(packed, 1, D)


def permute_signs_for_chunked(signs_packed: torch.Tensor, D: int = 128) -> torch.Tensor:
    """Reorder sign rows so chunk c (dims c, c+4, ..., c+124) fills bytes 4c..4c+3:
    output bit 32c+k = input bit 4k+c.  Same shape as the input (packed_compress.py:180-216)."""
    _lib.require_gpu("permute_signs_for_chunked", signs_packed)
    if D != 128:
        raise ValueError("D must be 128")
    shape = signs_packed.shape
    rows = _rows(signs_packed, D // 8, "permute_signs_for_chunked")
    n = rows.numel() // (D // 8)
    out = torch.empty_like(rows)
    rc = _lib.lib().tq_permute_signs(rows.data_ptr(), out.data_ptr(), n, D, _lib.stream_handle(rows.device))
    _lib.check(rc, "tq_permute_signs")
    return out.reshape(shape)


def _packed_compress(x: torch.Tensor, pit: torch.Tensor, pist, centroids: torch.Tensor,
                     boundaries: torch.Tensor, what: str):
    dev = _lib.require_gpu(what, x, pit, *( [pist] if pist is not None else []))
    if x.dim() != 2 or x.shape[1] != _lib.HEAD_DIM:
        raise ValueError(f"{what}: input must be [N, {_lib.HEAD_DIM}], got {tuple(x.shape)}")
    n, d = x.shape
    nc = centroids.numel()
    bits = nc.bit_length() - 1
    if nc != 2 ** bits or not 1 <= bits <= 4 or boundaries.numel() != nc - 1:
        raise ValueError(f"{what}: need 2^b centroids and 2^b - 1 boundaries (b = 1..4)")
    for name, m in (("PiT", pit), ("PiST", pist)):
        if m is not None and tuple(m.shape) != (d, d):
            raise ValueError(f"{what}: {name} must be [{d}, {d}]")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.float()
    if x.stride(1) != 1:
        x = x.contiguous()
    f32 = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()  # noqa: E731
    pit_f, cent, bnd = f32(pit), f32(centroids), f32(boundaries)
    pist_f = f32(pist) if pist is not None else None
    idx = torch.empty((n, d * bits // 8), dtype=torch.uint8, device=dev)
    norm = torch.empty((n,), dtype=torch.float16, device=dev)
    signs = torch.empty((n, d // 8), dtype=torch.uint8, device=dev) if pist is not None else None
    rnorm = torch.empty((n,), dtype=torch.float16, device=dev) if pist is not None else None
    rc = _lib.lib().tq_compress_packed(
        x.data_ptr(), _lib.dtype_code(x), x.stride(0), n, d, pit_f.data_ptr(), _lib.ptr(pist_f),
        cent.data_ptr(), bnd.data_ptr(), bits, idx.data_ptr(), _lib.ptr(signs), _lib.ptr(rnorm),
        norm.data_ptr(), _lib.stream_handle(dev))
    _lib.check(rc, "tq_compress_packed")
    return idx, signs, rnorm, norm


def compress_k(K: torch.Tensor, PiT: torch.Tensor, PiST: torch.Tensor, centroids: torch.Tensor,
               boundaries: torch.Tensor):
    """Packed K compression with explicit rotations (kernels/packed_compress.py:44-106,157-177).

    norm = |k|; k_n = k * (1 / (norm + 1e-8)); rot = k_n @ PiT; idx = #{boundaries <= rot};
    resid = (rot - centroids[idx]) * norm; rnorm = |resid|; sign bit = (resid @ PiST >= 0).
    Returns (k_idx uint8 [N, D*b/8], k_signs uint8 [N, D/8], k_rnorm fp16 [N], k_norm fp16 [N]);
    b = log2(#centroids) (the reference: 2, i.e. 4 indices per byte).  The products are fp32
    (the reference uses fp16 dot products, whose rounding is not reproduced)."""
    idx, signs, rnorm, norm = _packed_compress(K, PiT, PiST, centroids, boundaries, "compress_k")
    return idx, signs, rnorm, norm


def compress_k_permuted(K: torch.Tensor, PiT: torch.Tensor, PiST: torch.Tensor, centroids: torch.Tensor,
                        boundaries: torch.Tensor):
    """compress_k with the signs in the stride-4 order of permute_signs_for_chunked
    (kernels/packed_compress.py:219-223)."""
    idx, signs, rnorm, norm = compress_k(K, PiT, PiST, centroids, boundaries)
    return idx, permute_signs_for_chunked(signs), rnorm, norm


def compress_v(V: torch.Tensor, PiT: torch.Tensor, centroids: torch.Tensor, boundaries: torch.Tensor):
    """Packed V compression (kernels/packed_compress.py:109-142,226-240): as compress_k without
    the residual.  Returns (v_idx uint8 [N, D*b/8], v_norm fp16 [N])."""
    idx, _, _, norm = _packed_compress(V, PiT, None, centroids, boundaries, "compress_v")
    return idx, norm


def run(sizes=(2048, 32768, 131072, 524288), n_test: int = 131072, warmup: int = 25, iters: int = 300,
        seed: int = 42, verbose: bool = True) -> dict:
    """Self-test and benchmark of compress_k / compress_v on cuda:0 (the role of the reference
    module's run(), kernels/packed_compress.py:243-330).

    Correctness: n_test Gaussian rows through compress_k and compress_v with a seeded random
    rotation pair and the 2-bit kernel codebook; the unpacked indices are compared with the same
    formula in torch fp32 (norm, x / (norm + 1e-8) @ PiT, count of boundaries <= rot).  Then the
    packed footprint and the mean device time per call at each N in sizes.  Returns the
    figures printed."""
    from turboquant.kernels._selfcheck import random_rotations, time_ms
    dev = torch.device("cuda")
    D = _lib.HEAD_DIM
    PiT, PiST = random_rotations(D, seed, dev)
    centroids = solve_codebook(D, 2).to(dev)
    boundaries = ((centroids[:-1] + centroids[1:]) / 2.0).contiguous()
    say = print if verbose else (lambda *a, **k: None)
    say(f"Packed TurboQuant compress on {torch.cuda.get_device_name(0)}: D={D}, 2-bit indices + 1-bit QJL signs")
    res = {"correctness": {}, "benchmark": []}

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 1)
    K = torch.randn(n_test, D, device=dev, generator=gen)
    V = torch.randn(n_test, D, device=dev, generator=gen)
    k_idx, k_signs, k_rnorm, k_norm = compress_k(K, PiT, PiST, centroids, boundaries)
    v_idx, v_norm = compress_v(V, PiT, centroids, boundaries)
    for name, x, idx in (("K", K, k_idx), ("V", V, v_idx)):
        got = unpack_2bit(idx, D).long()
        norm = torch.linalg.vector_norm(x, dim=-1, keepdim=True)
        rot = (x / (norm + 1e-8)) @ PiT
        want = (rot.unsqueeze(-1) >= boundaries).sum(-1)
        match = (got == want).float().mean().item()
        recon_cos = torch.nn.functional.cosine_similarity(
            (centroids[got] * norm).reshape(1, -1), (centroids[want] * norm).reshape(1, -1)).item()
        ok = int(got.min()) >= 0 and int(got.max()) <= 3 and match > 0.99
        res["correctness"][name] = {"idx_match": match, "recon_cos": recon_cos, "pass": ok}
        say(f"  {name}: idx range [{int(got.min())}, {int(got.max())}], idx_match vs torch fp32 {match:.6f}, "
            f"recon cos {recon_cos:.8f} {'PASS' if ok else 'FAIL'}")
    sg = unpack_1bit(k_signs, D)
    say(f"  K signs range [{int(sg.min())}, {int(sg.max())}] (expected [0, 1])")

    fp16_bytes = D * 2 * 2
    packed = D // 4 + D // 8 + 2 + 2 + D // 4 + 2
    say(f"  memory per token-head: {fp16_bytes} B fp16 K+V -> {packed} B packed ({fp16_bytes / packed:.1f}x)")
    say(f"{'N':>8} {'K ms':>10} {'V ms':>10} {'K+V ms':>10}")
    for n in sizes:
        Kb = torch.randn(n, D, device=dev, generator=gen)
        Vb = torch.randn(n, D, device=dev, generator=gen)
        k_ms = time_ms(lambda: compress_k(Kb, PiT, PiST, centroids, boundaries), warmup, iters)
        v_ms = time_ms(lambda: compress_v(Vb, PiT, centroids, boundaries), warmup, iters)
        res["benchmark"].append({"N": n, "k_ms": k_ms, "v_ms": v_ms})
        say(f"{n:>8} {k_ms:>10.4f} {v_ms:>10.4f} {k_ms + v_ms:>10.4f}")
        del Kb, Vb
    return res


if __name__ == "__main__":
    run()
