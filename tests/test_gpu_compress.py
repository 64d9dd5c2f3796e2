"""GPU parity: compression kernels vs the CPU oracle.

Bar: packed indices / sign bits / bytes bit-exact except elements whose
oracle value lies within a rounding band of a codebook boundary (counted and reported);
norms within rtol 1e-2 / atol 1e-3.  The band is BAND_ULPS fp32 ulps at the coordinate scale
1/sqrt(128) (2^-27): the WHT butterfly and the oracle's sgemm sum the same 128 terms in
different orders, which moves a rotated coordinate by ~1 such ulp.
"""

import math

import numpy as np
import pytest
import torch

from oracle import compress as ocomp
from oracle import packing as opack
from oracle import paged as opaged

pytestmark = pytest.mark.gpu

BAND_ULPS = 8.0
NORM_RTOL, NORM_ATOL = 1e-2, 1e-3


def _codebook(bits):
    from turboquant.core import make_codebook
    return make_codebook(128, bits)


def _report(name, stats):
    n, ok, bad, band = stats
    print(f"[{name}] index mismatches {n} (in band {ok}, out of band {bad}, max band {band:.2f} ulp)")


def check_against_oracle(res, ref, cent, bnd, bits, use_qjl, name):
    xn = ref["x_normalized"].reshape(-1, 128)
    idx_gpu = res["indices"].cpu().reshape(-1, 128)
    idx_ref = ref["indices"].reshape(-1, 128)
    stats = ocomp.classify_index_mismatch(idx_gpu, idx_ref, xn, bnd, BAND_ULPS)
    _report(name, stats)
    assert stats[2] == 0, f"{name}: {stats[2]} index mismatches outside the boundary band"
    assert stats[0] <= max(4, idx_ref.numel() // 20000), f"{name}: too many boundary mismatches {stats[0]}"
    torch.testing.assert_close(res["norms"].cpu(), ref["norms"], rtol=NORM_RTOL, atol=NORM_ATOL)
    # norms agree far tighter than the bar; keep a regression guard on it
    assert float(((res["norms"].cpu() - ref["norms"]).abs() / ref["norms"].clamp_min(1e-30)).max()) < 1e-5
    same = idx_gpu == idx_ref
    kg = res["k_mse_rot"].cpu().reshape(-1, 128)
    kr = ref["k_mse_rot"].reshape(-1, 128)
    torch.testing.assert_close(kg[same], kr[same], rtol=1e-5, atol=1e-7)
    if use_qjl:
        sg = res["signs"].cpu().reshape(-1, 128)
        sr = ref["signs"].reshape(-1, 128)
        diff = sg != sr
        cb = ocomp.centroid_band(xn, cent, idx_ref.reshape(-1, 128))
        explained = (~same) | (cb <= BAND_ULPS)
        assert not (diff & ~explained).any(), f"{name}: sign flips away from centroids/boundaries"
        rows_clean = same.all(dim=1)
        torch.testing.assert_close(res["rot_residual_norm"].cpu()[rows_clean], ref["rot_residual_norm"][rows_clean],
                                   rtol=1e-4, atol=1e-6)


def test_config1_polarquant_compress(dev):
    """K [1024,128] N(0,1) seed 0, bits=3, QJL, WHT."""
    from turboquant.core import PolarQuantConfig, make_wht_matrix, polarquant_compress
    torch.manual_seed(0)
    K = torch.randn(1024, 128)
    cent, bnd = _codebook(3)
    H = make_wht_matrix(128)
    cfg = PolarQuantConfig(head_dim=128, bits=3, use_qjl=True)
    res = polarquant_compress(K.to(dev), cent.to(dev), bnd.to(dev), cfg, H.to(dev))
    torch.cuda.synchronize()
    ref = ocomp.polarquant_compress(K, cent, bnd, 8, True, H)
    check_against_oracle(res, ref, cent, bnd, 3, True, "config1")
    assert res["indices"].dtype == torch.int64 and res["indices"].shape == (1024, 128)
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "config1_oracle.npz")
    gi = torch.from_numpy(opack.unpack_indices(golden["indices_packed"], 3))
    stats = ocomp.classify_index_mismatch(res["indices"].cpu(), gi, ref["x_normalized"], bnd, BAND_ULPS)
    assert stats[2] == 0


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("use_qjl", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rotate", [True, False])
def test_polarquant_variants(dev, bits, use_qjl, dtype, rotate):
    from turboquant.core import PolarQuantConfig, make_wht_matrix, polarquant_compress
    g = torch.Generator().manual_seed(1000 + bits * 10 + int(use_qjl))
    x = (torch.randn(777, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).to(dtype)
    cent, bnd = _codebook(bits)
    H = make_wht_matrix(128) if rotate else None
    cfg = PolarQuantConfig(head_dim=128, bits=bits, use_qjl=use_qjl)
    res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, None if H is None else H.to(dev))
    ref = ocomp.polarquant_compress(x.float(), cent, bnd, 2 ** bits, use_qjl, H)
    check_against_oracle(res, ref, cent, bnd, bits, use_qjl, f"b{bits} q{int(use_qjl)} {dtype} rot{int(rotate)}")


def test_polarquant_3d_and_edge_rows(dev):
    from turboquant.core import PolarQuantConfig, make_wht_matrix, polarquant_compress
    cent, bnd = _codebook(3)
    H = make_wht_matrix(128)
    cfg = PolarQuantConfig(head_dim=128, bits=3, use_qjl=True)
    torch.manual_seed(0)
    x = torch.randn(4, 8, 128)
    x[0, 0] = 0.0                      # zero vector: norm 0, x_n = 0
    x[0, 1] = 0.0
    x[0, 1, 5] = 3.0                   # basis vector: every rotated coordinate is +-h*3
    res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, H.to(dev))
    assert res["k_mse_rot"].shape == (4, 8, 128) and res["indices"].shape == (4, 8, 128)
    assert res["norms"].shape == (32,)
    ref = ocomp.polarquant_compress(x, cent, bnd, 8, True, H)
    check_against_oracle(res, ref, cent, bnd, 3, True, "3d")
    assert float(res["norms"][0]) == 0.0
    assert (res["signs"][0, 0] == 1.0).all()
    # single-row input
    res1 = polarquant_compress(x[1, 2:3].reshape(1, 128).to(dev), cent.to(dev), bnd.to(dev), cfg, H.to(dev))
    assert torch.equal(res1["indices"].cpu(), res["indices"][1, 2:3].cpu())


def _payload_from_oracle(ref, bits, qjl, T, H):
    idx = ref["indices"].reshape(T * H, 128).numpy()
    pl = {"idx": opack.pack_indices(idx, bits).reshape(T, H, -1),
          "norm": ref["norms"].numpy().astype(np.float16).view(np.uint16).reshape(T, H)}
    if qjl:
        s01 = (ref["signs"].reshape(T * H, 128).numpy() > 0).astype(np.int64)
        pl["signs"] = opack.pack_signs(s01).reshape(T, H, 16)
        pl["rnorm"] = ref["rot_residual_norm"].numpy().astype(np.float16).view(np.uint16).reshape(T, H)
    return pl


@pytest.mark.parametrize("bits,qjl", [(2, False), (2, True), (3, False), (3, True), (4, False), (4, True)])
@pytest.mark.parametrize("block_size", [16, 32])
def test_compress_paged_bytes(dev, bits, qjl, block_size):
    from turboquant.core import make_wht_matrix
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, nb = 203, 3, 20
    g = torch.Generator().manual_seed(7 + bits + 10 * int(qjl))
    x = torch.randn(T, H, 128, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb * block_size, generator=g)[:T].to(torch.int64)
    perm[5] = -1                       # padding token: skipped
    perm[6] = nb * block_size + 3      # out of range: skipped
    slots = perm.to(torch.int32)
    fmt = PagedKVFormat(bits=bits, qjl=qjl, block_size=block_size)
    cent, bnd = _codebook(bits)
    cache = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x.to(dev), slots.to(dev), cache, fmt, cent.to(dev), bnd.to(dev))
    got = cache.cpu().numpy()
    ref = ocomp.polarquant_compress(x.float().reshape(T * H, 128), cent, bnd, 2 ** bits, qjl, make_wht_matrix(128))
    pl = _payload_from_oracle(ref, bits, qjl, T, H)
    want = opaged.scatter_tokens(pl, perm.numpy(), nb, H, block_size, bits, qjl)
    if np.array_equal(got, want):
        return
    # Differences must come only from boundary-band indices / fp16 norm rounding of the same tokens.
    xn = ref["x_normalized"].reshape(T, H, 128)
    for t in range(T):
        s = int(perm[t])
        if s < 0 or s >= nb * block_size:
            continue
        for h in range(H):
            one = {k: v[t:t + 1, h:h + 1] for k, v in pl.items()}
            w = opaged.scatter_tokens(one, np.array([s]), nb, 1, block_size, bits, qjl)[s // block_size, 0]
            gt = got[s // block_size, h]
            if np.array_equal(gt[w != 0], w[w != 0]) and np.array_equal(np.nonzero(gt)[0], np.nonzero(w)[0]):
                continue
            iw = opack.unpack_indices(w[(s % block_size) * 16 * bits:(s % block_size + 1) * 16 * bits][None], bits)
            ig = opack.unpack_indices(gt[(s % block_size) * 16 * bits:(s % block_size + 1) * 16 * bits][None], bits)
            st = ocomp.classify_index_mismatch(torch.from_numpy(ig), torch.from_numpy(iw), xn[t, h][None], bnd, BAND_ULPS)
            assert st[2] == 0, f"token {t} head {h}: out-of-band index mismatch"
    # untouched blocks stay zero
    written = {int(p) // block_size for p in perm if 0 <= int(p) < nb * block_size}
    for b in range(nb):
        if b not in written:
            assert not got[b].any()


def test_config2_full_size_roundtrip(dev):
    """BASELINE config 2 at full size: 16384 tokens x 8 heads bf16 turbo4 into 8192 blocks."""
    from turboquant.core import make_wht_matrix
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged, to_reference_slots
    T, H, nb, bs = 16384, 8, 8192, 16
    g = torch.Generator().manual_seed(2)
    scale = torch.exp(torch.randn(H, 128, generator=g) * 0.5)
    out_ch = torch.rand(H, 128, generator=g) < 0.02
    scale[out_ch] *= 8
    x = (torch.randn(T, H, 128, generator=g) * scale).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g)
    slots = (perm[torch.arange(T) // bs] * bs + torch.arange(T) % bs).to(torch.int32)
    fmt = PagedKVFormat(bits=4, qjl=False, block_size=bs)
    cent, bnd = _codebook(4)
    cache = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x.to(dev), slots.to(dev), cache, fmt, cent.to(dev), bnd.to(dev))
    aos = to_reference_slots(cache, fmt).cpu().numpy()          # [nb, bs, H, 66]
    ref = ocomp.polarquant_compress(x.float().reshape(T * H, 128), cent, bnd, 16, False, make_wht_matrix(128))
    blk = (slots.long() // bs).numpy()
    row = (slots.long() % bs).numpy()
    tok_slots = aos[blk, row]                                   # [T, H, 66]
    got_idx = opack.unpack_indices(tok_slots[..., :64].reshape(T * H, 64), 4)
    stats = ocomp.classify_index_mismatch(torch.from_numpy(got_idx), ref["indices"], ref["x_normalized"], bnd, BAND_ULPS)
    _report("config2", stats)
    assert stats[2] == 0
    got_norm = tok_slots[..., 64:66].copy().view(np.float16).reshape(T * H).astype(np.float32)
    want_norm = ref["norms"].numpy().astype(np.float16).astype(np.float32)
    np.testing.assert_allclose(got_norm, want_norm, rtol=NORM_RTOL, atol=NORM_ATOL)
    assert np.mean(got_norm == want_norm) > 0.999
