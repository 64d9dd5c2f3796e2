"""tq_decode_noalloc (the split-K workspace in the library's fixed device array) against
tq_decode with a caller workspace: same kernels, same chunking, so the outputs and the Sparse-V
skip statistics must be identical.  Two calls in a row, the second smaller; a request beyond
the fixed array is refused before any launch."""

import ctypes
import math

import pytest
import torch

from turboquant import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = _lib.NOALLOC_SCRATCH_BYTES


def _fn():
    return _lib.lib().tq_decode_noalloc


def _case(dev, seed, lens, Hq=48, Hkv=8, kb=3, kq=True, vb=3, bs=16):
    from turboquant.core import make_codebook
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    g = torch.Generator(device=dev).manual_seed(seed)
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout="values")
    nbl = [math.ceil(L / bs) for L in lens]
    nb = sum(nbl) + 4
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    bt = torch.full((len(lens), max(nbl)), -1, dtype=torch.int32)
    o = 0
    for s, n in enumerate(nbl):
        bt[s, :n] = perm[o:o + n].to(torch.int32)
        o += n
    kc, kbnd = make_codebook(128, kb, device=dev)
    vc, vbnd = make_codebook(128, vb, device=dev)
    k_cache = allocate_cache(nb, Hkv, kf, device=dev)
    v_cache = allocate_cache(nb, Hkv, vf, device=dev)
    slots = torch.cat([(bt[s, torch.arange(L) // bs].long() * bs + torch.arange(L) % bs) for s, L in enumerate(lens)])
    T = slots.numel()
    compress_paged(torch.randn(T, Hkv, 128, generator=g, device=dev).bfloat16(), slots.to(torch.int32).to(dev), k_cache,
                   kf, kc, kbnd)
    compress_paged(torch.randn(T, Hkv, 128, generator=g, device=dev).bfloat16(), slots.to(torch.int32).to(dev), v_cache,
                   vf, vc, vbnd)
    q = (torch.randn(len(lens), Hq, 128, generator=g, device=dev) * 3).bfloat16()
    return dict(q=q, k_cache=k_cache, v_cache=v_cache, kf=kf, vf=vf, kc=kc, vc=vc, bt=bt.to(dev),
                lens=torch.tensor(lens, dtype=torch.int32, device=dev), Hkv=Hkv, bs=bs)


def _noalloc(c, chunk, thresh, out, stats):
    from turboquant.kernels.paged import paged_view
    kv = paged_view(c["k_cache"], c["kf"], c["kc"])
    vv = paged_view(c["v_cache"], c["vf"], c["vc"])
    S, Hq, _ = c["q"].shape
    msl = int(c["lens"].max())
    bt = c["bt"]
    return _fn()(c["q"].data_ptr(), _lib.dtype_code(c["q"]), c["q"].stride(0), c["q"].stride(1), None, 0, 0,
                 S, Hq, c["Hkv"], 128, ctypes.byref(kv), ctypes.byref(vv), c["bs"], c["k_cache"].shape[0],
                 bt.data_ptr(), bt.stride(0), bt.shape[1], c["lens"].data_ptr(), msl,
                 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128, thresh, chunk,
                 out.data_ptr(), _lib.dtype_code(out), out.stride(0), out.stride(1),
                 stats.data_ptr(), _lib.stream_handle(c["q"].device))


def _reference(c, chunk, thresh, stats):
    from turboquant.kernels.paged import decode_paged
    return decode_paged(c["q"], c["k_cache"], c["kf"], c["kc"], c["v_cache"], c["vf"], c["vc"], c["bt"], c["lens"],
                        sparse_threshold=thresh, max_seq_len=int(c["lens"].max()), tokens_per_chunk=chunk,
                        workspace=torch.empty(_lib.lib().tq_decode_workspace_bytes(
                            len(c["lens"]), c["q"].shape[1], int(c["lens"].max()), chunk),
                            dtype=torch.uint8, device=c["q"].device), skip_stats=stats)


@pytest.mark.parametrize("rounds", [[([3000, 17, 1200, 0, 2047, 512, 95, 4096], 256, 1e-4), ([700, 33, 160], 64, 0.0)],
                                    [([3000, 17, 1200, 0, 2047, 512, 95, 4096], 0, 1e-4), ([700, 33, 160], 0, 0.0)]])
def test_noalloc_matches_workspace_entry(dev, rounds):
    for i, (lens, chunk, thresh) in enumerate(rounds):
        c = _case(dev, 90 + i, lens)
        need = _lib.lib().tq_decode_workspace_bytes(len(lens), c["q"].shape[1], max(lens), chunk)
        assert 0 < need <= SCRATCH_BYTES
        st_ref = torch.zeros(2, dtype=torch.int64, device=dev)
        want = _reference(c, chunk, thresh, st_ref)
        out = torch.full_like(c["q"], float("nan"))
        st = torch.zeros(2, dtype=torch.int64, device=dev)
        rc = _noalloc(c, chunk, thresh, out, st)
        assert rc == 0, _lib.status_string(rc)
        torch.cuda.synchronize()
        print(f"call {i}: {len(lens)} sequences, chunk {chunk}, workspace {need} bytes", flush=True)
        assert torch.equal(out, want)
        if thresh > 0:
            assert torch.equal(st, st_ref)


def test_noalloc_refuses_requests_beyond_the_scratch(dev):
    c = _case(dev, 7, [100, 50])
    out = torch.empty_like(c["q"])
    st = torch.zeros(2, dtype=torch.int64, device=dev)
    # chunks of 16 tokens over a 1M-token bound: far more partial results than the array holds
    from turboquant.kernels.paged import paged_view
    kv = paged_view(c["k_cache"], c["kf"], c["kc"])
    vv = paged_view(c["v_cache"], c["vf"], c["vc"])
    q = c["q"]
    rc = _fn()(q.data_ptr(), _lib.dtype_code(q), q.stride(0), q.stride(1), None, 0, 0, 2, 48, 8, 128,
               ctypes.byref(kv), ctypes.byref(vv), 16, c["k_cache"].shape[0], c["bt"].data_ptr(), c["bt"].stride(0),
               c["bt"].shape[1], c["lens"].data_ptr(), 1 << 20, 0.1, 0.0, 0.0, 16,
               out.data_ptr(), _lib.dtype_code(out), out.stride(0), out.stride(1), None, _lib.stream_handle(dev))
    assert rc == -10 and "tokens_per_chunk" in _lib.status_string(rc)
