"""GPU parity: compression kernels vs the CPU oracle.

Bar (the path's parity target): packed indices / sign bits / bytes bit-exact except elements whose
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


def check_against_oracle(res, ref, cent, bnd, bits, use_qjl, name, band_ulps=BAND_ULPS):
    xn = ref["x_normalized"].reshape(-1, 128)
    idx_gpu = res["indices"].cpu().reshape(-1, 128)
    idx_ref = ref["indices"].reshape(-1, 128)
    stats = ocomp.classify_index_mismatch(idx_gpu, idx_ref, xn, bnd, band_ulps)
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
        explained = (~same) | (cb <= band_ulps)
        assert not (diff & ~explained).any(), f"{name}: sign flips away from centroids/boundaries"
        rows_clean = same.all(dim=1)
        torch.testing.assert_close(res["rot_residual_norm"].cpu()[rows_clean], ref["rot_residual_norm"][rows_clean],
                                   rtol=1e-4, atol=1e-6)


def test_config1_polarquant_compress(dev):
    """Benchmark config 1: K [1024,128] N(0,1) seed 0, bits=3, QJL, WHT."""
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


def _random_rotation(seed):
    """Pi (orthogonal, from QR with the sign fix) and S (Gaussian) as the reference builds them
    (kernels/packed_compress.py:265-273): PiT = Pi^T, PiST = Pi S^T."""
    g = torch.Generator().manual_seed(seed)
    G = torch.randn(128, 128, generator=g, dtype=torch.float64)
    Q, R = torch.linalg.qr(G)
    ds = torch.sign(torch.diag(R))
    ds[ds == 0] = 1.0
    Pi = Q * ds.unsqueeze(0)
    S = torch.randn(128, 128, generator=torch.Generator().manual_seed(seed + 10000), dtype=torch.float64)
    return Pi.T.contiguous().float(), (Pi @ S.T).contiguous().float()


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_polarquant_general_rotation(dev, bits, dtype):
    """rotation_matrix that is not a WHT: fp32 product kernel vs the oracle's torch op sequence.
    The two sum x_d R_dj in different orders; the band allows 64 ulps at the coordinate scale."""
    from turboquant.core import PolarQuantConfig, polarquant_compress
    g = torch.Generator().manual_seed(2000 + bits)
    x = (torch.randn(515, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).to(dtype)
    R, _ = _random_rotation(40 + bits)
    cent, bnd = _codebook(bits)
    for use_qjl in (False, True):
        cfg = PolarQuantConfig(head_dim=128, bits=bits, use_qjl=use_qjl)
        res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, R.to(dev))
        ref = ocomp.polarquant_compress(x.float(), cent, bnd, 2 ** bits, use_qjl, R)
        check_against_oracle(res, ref, cent, bnd, bits, use_qjl, f"general b{bits} q{int(use_qjl)} {dtype}",
                             band_ulps=64.0)


# compress_k / compress_v: decisions compared with the float64 restatement.  A GPU decision may
# differ only where the oracle's margin is within fp32 rounding: |rot - boundary| <= ROT_BAND, or
# |proj| <= PROJ_REL * sum_d |resid_d PiST_dj|; rows with an index difference are exempt from the
# sign comparison (their residual differs).
ROT_BAND = 1e-6
PROJ_REL = 1e-5


def _kernel_codebook(bits):
    from oracle import codebook as ocb
    c = np.array(ocb.kernel_codebook(128, bits), dtype=np.float32)
    b = ((c[:-1] + c[1:]) / 2.0).astype(np.float32)
    return torch.from_numpy(c), torch.from_numpy(b)


@pytest.mark.parametrize("bits", [2, 1, 3, 4])
@pytest.mark.parametrize("n", [1, 1023, 4096])
def test_compress_k_v_against_oracle(dev, bits, n):
    from turboquant.kernels.packed_compress import compress_k, compress_k_permuted, compress_v
    g = torch.Generator().manual_seed(3000 + bits * 7 + n)
    K = torch.randn(n, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)
    PiT, PiST = _random_rotation(11 + bits)
    cent, bnd = _kernel_codebook(bits)
    t = lambda a: a.to(dev)  # noqa: E731
    k_idx, k_signs, k_rnorm, k_norm = compress_k(t(K), t(PiT), t(PiST), t(cent), t(bnd))
    torch.cuda.synchronize()
    assert k_idx.dtype == torch.uint8 and k_idx.shape == (n, 16 * bits)
    assert k_signs.shape == (n, 16) and k_rnorm.dtype == torch.float16 and k_norm.dtype == torch.float16
    ref = ocomp.compress_packed(K.double().numpy(), PiT.double().numpy(), PiST.double().numpy(),
                                cent.double().numpy(), bnd.double().numpy())
    idx_gpu = opack.unpack_indices(k_idx.cpu().numpy(), bits)
    diff = idx_gpu != ref["idx"]
    assert not (diff & (ref["rot_margin"] > ROT_BAND)).any(), "index differences outside the band"
    assert (np.abs(idx_gpu[diff].astype(int) - ref["idx"][diff]) == 1).all()
    print(f"[compress_k b{bits} n{n}] index differences in band: {int(diff.sum())}")
    # the kernel's bytes are exactly the oracle's packing of the oracle's decisions, where the
    # band-exempt elements take the GPU's value
    merged = np.where(diff, idx_gpu, ref["idx"])
    np.testing.assert_array_equal(k_idx.cpu().numpy(), opack.pack_indices(merged, bits))
    rows_ok = ~diff.any(axis=1)
    sg = opack.unpack_signs(k_signs.cpu().numpy())
    sdiff = (sg != ref["sign"]) & rows_ok[:, None]
    assert not (sdiff & (np.abs(ref["proj"]) > PROJ_REL * ref["proj_scale"])).any(), "sign flips outside the band"
    print(f"[compress_k b{bits} n{n}] sign differences in band: {int(sdiff.sum())}, rows exempt: {int((~rows_ok).sum())}")
    merged_s = np.where(sdiff | ~rows_ok[:, None], sg, ref["sign"])
    np.testing.assert_array_equal(k_signs.cpu().numpy(), opack.pack_signs(merged_s))
    np.testing.assert_allclose(k_norm.float().cpu().numpy(), ref["norm"], rtol=1e-3)
    np.testing.assert_allclose(k_rnorm.float().cpu().numpy()[rows_ok], ref["rnorm"][rows_ok], rtol=1e-3, atol=1e-6)
    # permuted variant = permutation of the natural signs
    _, k_sp, _, _ = compress_k_permuted(t(K), t(PiT), t(PiST), t(cent), t(bnd))
    np.testing.assert_array_equal(k_sp.cpu().numpy(), opack.permute_signs(k_signs.cpu().numpy()))
    # V: same rotation and quantizer, no residual
    v_idx, v_norm = compress_v(t(K), t(PiT), t(cent), t(bnd))
    np.testing.assert_array_equal(v_idx.cpu().numpy(), k_idx.cpu().numpy())
    np.testing.assert_array_equal(v_norm.cpu().numpy(), k_norm.cpu().numpy())


def test_compress_k_v_input_dtypes_and_rejections(dev):
    from turboquant.kernels.packed_compress import compress_k, compress_v
    PiT, PiST = _random_rotation(5)
    cent, bnd = _kernel_codebook(2)
    K = torch.randn(64, 128, generator=torch.Generator().manual_seed(9))
    t = lambda a: a.to(dev)  # noqa: E731
    base = compress_k(t(K), t(PiT), t(PiST), t(cent), t(bnd))
    for dt in (torch.bfloat16, torch.float16):
        Kd = K.to(dt)
        got = compress_k(t(Kd), t(PiT), t(PiST), t(cent), t(bnd))
        ref = ocomp.compress_packed(Kd.double().numpy(), PiT.double().numpy(), PiST.double().numpy(),
                                    cent.double().numpy(), bnd.double().numpy())
        idx = opack.unpack_indices(got[0].cpu().numpy(), 2)
        assert not ((idx != ref["idx"]) & (ref["rot_margin"] > ROT_BAND)).any()
    with pytest.raises(ValueError):
        compress_k(t(K[:, :64]), t(PiT), t(PiST), t(cent), t(bnd))
    with pytest.raises(ValueError):
        compress_v(t(K), t(PiT), t(cent[:3]), t(bnd))
    with pytest.raises(ValueError):
        compress_k(K, PiT, PiST, cent, bnd)  # CPU tensors: no CPU fallback
    assert base[0].shape == (64, 32)


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
@pytest.mark.parametrize("layout", ["keys", "values", "rows"])
def test_compress_paged_bytes(dev, bits, qjl, block_size, layout):
    if layout == "values" and qjl:
        pytest.skip("the values layout carries no QJL data")
    from turboquant.core import make_wht_matrix
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, nb = 203, 3, 20
    g = torch.Generator().manual_seed(7 + bits + 10 * int(qjl))
    x = torch.randn(T, H, 128, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb * block_size, generator=g)[:T].to(torch.int64)
    perm[5] = -1                       # padding token: skipped
    perm[6] = nb * block_size + 3      # out of range: skipped
    slots = perm.to(torch.int32)
    fmt = PagedKVFormat(bits=bits, qjl=qjl, block_size=block_size, layout=layout)
    cent, bnd = _codebook(bits)
    cache = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x.to(dev), slots.to(dev), cache, fmt, cent.to(dev), bnd.to(dev))
    got = cache.cpu().numpy()
    ref = ocomp.polarquant_compress(x.float().reshape(T * H, 128), cent, bnd, 2 ** bits, qjl, make_wht_matrix(128))
    pl = _payload_from_oracle(ref, bits, qjl, T, H)
    want = opaged.scatter_tokens(pl, perm.numpy(), nb, H, block_size, bits, qjl, layout=layout)
    if np.array_equal(got, want):
        return
    # Differences must come only from boundary-band indices / fp16 norm rounding of the same
    # tokens; compared per token in row form (the oracle reads any layout back into rows).
    xn = ref["x_normalized"].reshape(T, H, 128)
    _, _, off_norm, off_rnorm, _ = opaged.tile_offsets(block_size, bits, qjl)
    for t in range(T):
        s = int(perm[t])
        if s < 0 or s >= nb * block_size:
            continue
        blk, row = divmod(s, block_size)
        for h in range(H):
            gi, gs = opaged._tile_rows(got[blk, h], block_size, bits, qjl, layout)
            wi, ws = opaged._tile_rows(want[blk, h], block_size, bits, qjl, layout)
            same_norms = np.array_equal(got[blk, h, off_norm + 2 * row: off_norm + 2 * row + 2],
                                        want[blk, h, off_norm + 2 * row: off_norm + 2 * row + 2])
            if np.array_equal(gi[row], wi[row]) and (not qjl or np.array_equal(gs[row], ws[row])) and same_norms:
                continue
            ig = opack.unpack_indices(gi[row][None], bits)
            iw = opack.unpack_indices(wi[row][None], bits)
            st = ocomp.classify_index_mismatch(torch.from_numpy(ig), torch.from_numpy(iw), xn[t, h][None], bnd, BAND_ULPS)
            assert st[2] == 0, f"token {t} head {h}: out-of-band index mismatch"
    # untouched blocks stay zero
    written = {int(p) // block_size for p in perm if 0 <= int(p) < nb * block_size}
    for b in range(nb):
        if b not in written:
            assert not got[b].any()


def test_config2_full_size_roundtrip(dev):
    """Benchmark config 2 at full size: 16384 tokens x 8 heads bf16 turbo4 into 8192 blocks."""
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
    fmt = PagedKVFormat(bits=4, qjl=False, block_size=bs, layout="values")
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


def _quantizer_probe_rows(values):
    """Rows [t, c, 0, ...] with c = sqrt(1 - t^2) in fp32: the row norm is 1 (or within an ulp),
    so x / (norm + 1e-8) lands on t itself when the norm rounds to 1."""
    t = np.asarray(values, dtype=np.float32)
    c = np.sqrt(np.maximum(0.0, 1.0 - t.astype(np.float64) ** 2)).astype(np.float32)
    x = np.zeros((t.size, 128), dtype=np.float32)
    x[:, 0] = t
    x[:, 1] = c
    return x


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_searchsorted_at_boundaries_and_cell_edges(dev, bits):
    """Index of values exactly on every boundary, one fp32 ulp either side of it, on the edges of
    the kernel's 1/128-wide lookup cells and their neighbours, and at 0 and +-1, against
    np.searchsorted (left) of the same fp32 quotient."""
    from turboquant.core import PolarQuantConfig, polarquant_compress
    cent, bnd = _codebook(bits)
    b = bnd.numpy().astype(np.float32)
    edges = (-1.0 + np.arange(257, dtype=np.float64) / 128.0).astype(np.float32)
    vals = []
    for v in np.concatenate([b, edges, np.float32([0.0, 0.5, -0.5])]):
        vals += [v, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(-np.inf))]
    vals = np.asarray([v for v in vals if abs(v) <= 1.0], dtype=np.float32)
    x = torch.from_numpy(_quantizer_probe_rows(vals))
    cfg = PolarQuantConfig(head_dim=128, bits=bits, use_qjl=False)
    res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, None)
    norms = res["norms"].cpu().numpy().astype(np.float32)
    assert (norms == np.float32(1.0)).mean() > 0.5, "probe rows should mostly have norm exactly 1"
    xn = vals / (norms + np.float32(1e-8))                     # fp32, correctly rounded
    want = np.searchsorted(b, xn, side="left")
    got = res["indices"].cpu().numpy()[:, 0]
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"bits {bits}: x={xn[bad[:5]]} got {got[bad[:5]]} want {want[bad[:5]]}"


def test_searchsorted_close_boundaries_fallback(dev):
    """A codebook with two boundaries 1e-4 apart (inside one lookup cell) still quantizes exactly
    (the kernel counts linearly for such codebooks)."""
    from turboquant.core import PolarQuantConfig, polarquant_compress
    bnd = torch.tensor([-0.3, -0.05, 0.0, 1e-4, 0.02, 0.1, 0.4], dtype=torch.float32)
    cent = torch.tensor([-0.5, -0.2, -0.02, 5e-5, 0.01, 0.05, 0.2, 0.6], dtype=torch.float32)
    vals = []
    for v in np.concatenate([bnd.numpy(), np.float32([0.0, 5e-5, -1.0, 1.0, 0.99])]):
        vals += [v, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(-np.inf))]
    vals = np.asarray([v for v in vals if abs(v) <= 1.0], dtype=np.float32)
    x = torch.from_numpy(_quantizer_probe_rows(vals))
    cfg = PolarQuantConfig(head_dim=128, bits=3, use_qjl=False)
    res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, None)
    norms = res["norms"].cpu().numpy().astype(np.float32)
    xn = vals / (norms + np.float32(1e-8))
    want = np.searchsorted(bnd.numpy(), xn, side="left")
    got = res["indices"].cpu().numpy()[:, 0]
    np.testing.assert_array_equal(got, want)
