"""Shared pieces of the modules' self-test / benchmark entry points (packed_compress.run,
packed_attention.run, sparse_v.benchmark): a seeded random rotation pair and a GPU timer.

The timer brackets the calls with HIP events on torch's current stream, the stream every
entry point of this package launches on, so it measures device time of the calls rather than
host dispatch."""

from __future__ import annotations

import torch


def random_rotations(D: int, seed: int, device):
    """(PiT, PiST) as the reference's self-tests build them: Pi from the QR of a seeded
    Gaussian matrix with R's diagonal signs folded in (kernels/packed_compress.py:243-254),
    S a second seeded Gaussian matrix, PiST = Pi @ S^T."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    G = torch.randn(D, D, device=device, generator=gen)
    Q, R = torch.linalg.qr(G)
    sign = torch.sign(torch.diag(R))
    sign[sign == 0] = 1.0
    Pi = Q * sign.unsqueeze(0)
    gen2 = torch.Generator(device=device)
    gen2.manual_seed(seed + 10000)
    S = torch.randn(D, D, device=device, generator=gen2)
    return Pi.T.contiguous(), (Pi @ S.T.contiguous()).contiguous()


def time_ms(fn, warmup: int, iters: int) -> float:
    """Mean device milliseconds per call of fn() over iters calls after warmup calls."""
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters
