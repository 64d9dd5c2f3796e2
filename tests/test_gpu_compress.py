"""GPU parity: compression kernels vs the CPU oracle.

Bar (the path's parity target): packed indices / sign bits / bytes bit-exact except elements
within 1 ulp of a codebook boundary, which are counted and reported.  Every index mismatch
against the fp32 restatement of the reference is classified by the distance of the reference
value from the boundary between the two indices, in fp32 ulps (oracle.compress.classify_strict):
within 1 ulp it is accepted; further out it is accepted only when the GPU's index equals the
float64 shadow's (the reference's own fp32 rounding put its value on the wrong side), and
counted as such.  Sign bits follow the same rule around the centroid (where the residual's sign
flips).  Norms within rtol 1e-2 / atol 1e-3.  Counts go to the session's parity log
(written to $TQ_PARITY_OUT).
"""

import math

import numpy as np
import pytest
import torch

from oracle import compress as ocomp
from oracle import packing as opack
from oracle import paged as opaged

pytestmark = pytest.mark.gpu

NORM_RTOL, NORM_ATOL = 1e-2, 1e-3


def _codebook(bits):
    from turboquant.core import make_codebook
    return make_codebook(128, bits)


def _log(parity_log, name, stats):
    print(f"[{name}] {stats}")
    if parity_log is not None:
        parity_log[name] = stats


def check_against_oracle(res, ref, ref64, cent, bnd, use_qjl, name, parity_log=None):
    xn = ref["x_normalized"].reshape(-1, 128)
    idx_gpu = res["indices"].cpu().reshape(-1, 128)
    idx_ref = ref["indices"].reshape(-1, 128)
    stats = ocomp.classify_strict(idx_gpu.numpy(), idx_ref.numpy(), xn.numpy(), bnd.numpy(),
                                  ref64["indices"].reshape(-1, 128).numpy())
    _log(parity_log, name, stats)
    assert stats["failures"] == 0, f"{name}: index mismatches beyond 1 ulp not explained by the fp64 shadow: {stats}"
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
        s64 = ref64["signs"].reshape(-1, 128).to(sg.dtype)
        diff = (sg != sr).numpy()
        c = cent.double()[idx_ref.long()]
        cdist = (xn.double() - c).abs().numpy() / np.maximum(
            ocomp.ulp32(np.maximum(xn.double().abs().numpy(), c.abs().numpy())), 1e-300)
        ok = (~same).numpy() | (cdist <= 1.0) | (sg == s64).numpy()
        assert not (diff & ~ok).any(), f"{name}: sign flips away from centroids not explained by the fp64 shadow"
        if parity_log is not None:
            parity_log[name]["sign_mismatches"] = int(diff.sum())
        rows_clean = same.all(dim=1)
        torch.testing.assert_close(res["rot_residual_norm"].cpu()[rows_clean], ref["rot_residual_norm"][rows_clean],
                                   rtol=1e-4, atol=1e-6)


def test_config1_polarquant_compress(dev, parity_log):
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
    ref64 = ocomp.polarquant_compress_fp64(K, cent, bnd, True, True)
    check_against_oracle(res, ref, ref64, cent, bnd, True, "config1", parity_log)
    assert res["indices"].dtype == torch.int64 and res["indices"].shape == (1024, 128)
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "config1_oracle.npz")
    gi = opack.unpack_indices(golden["indices_packed"], 3)
    stats = ocomp.classify_strict(res["indices"].cpu().numpy(), gi, ref["x_normalized"].numpy(), bnd.numpy(),
                                  ref64["indices"].numpy())
    assert stats["failures"] == 0


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("use_qjl", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rotate", [True, False])
def test_polarquant_variants(dev, bits, use_qjl, dtype, rotate, parity_log):
    from turboquant.core import PolarQuantConfig, make_wht_matrix, polarquant_compress
    g = torch.Generator().manual_seed(1000 + bits * 10 + int(use_qjl))
    x = (torch.randn(777, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).to(dtype)
    cent, bnd = _codebook(bits)
    H = make_wht_matrix(128) if rotate else None
    cfg = PolarQuantConfig(head_dim=128, bits=bits, use_qjl=use_qjl)
    res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, None if H is None else H.to(dev))
    ref = ocomp.polarquant_compress(x.float(), cent, bnd, 2 ** bits, use_qjl, H)
    ref64 = ocomp.polarquant_compress_fp64(x.float(), cent, bnd, use_qjl, rotate)
    check_against_oracle(res, ref, ref64, cent, bnd, use_qjl, f"variant b{bits} q{int(use_qjl)} {dtype} rot{int(rotate)}",
                         parity_log)


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
def test_polarquant_general_rotation(dev, bits, dtype, parity_log):
    """rotation_matrix that is not a WHT: the product kernel vs the oracle's torch op sequence,
    under the same 1-ulp / fp64 rule."""
    from turboquant.core import PolarQuantConfig, polarquant_compress
    g = torch.Generator().manual_seed(2000 + bits)
    x = (torch.randn(515, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).to(dtype)
    R, _ = _random_rotation(40 + bits)
    cent, bnd = _codebook(bits)
    for use_qjl in (False, True):
        cfg = PolarQuantConfig(head_dim=128, bits=bits, use_qjl=use_qjl)
        res = polarquant_compress(x.to(dev), cent.to(dev), bnd.to(dev), cfg, R.to(dev))
        ref = ocomp.polarquant_compress(x.float(), cent, bnd, 2 ** bits, use_qjl, R)
        ref64 = ocomp.polarquant_compress_fp64(x.float(), cent, bnd, use_qjl, True, matrix=R)
        check_against_oracle(res, ref, ref64, cent, bnd, use_qjl, f"general b{bits} q{int(use_qjl)} {dtype}",
                             parity_log)


# compress_k / compress_v: decisions compared with the float64 restatement (the reference's
# fp16 tl.dot products are not a target).  An index may differ only within 1 fp32 ulp of the
# boundary (classify_strict_fp64).  A sign bit may differ from float64's only where |proj| is
# within the error bound of the kernel's arithmetic (derived in csrc/tq_packed.hip): rot's
# bound E = 2^-19 * max column norm of PiT + 2^-21 times the row norm and the column's 1-norm of
# PiST, plus 2^-19 of the summed terms sum_d |resid_d PiST_dj|, plus 2^-25 of the 1-norms of the
# PiST column and the residual (fp16 subnormals); float64 decides everywhere else.  Every such
# difference is counted in the parity log.  Rows with an index difference are exempt from the
# sign comparison (their residual differs).


def sign_band(ref, pit, pist):
    colmax = float(np.sqrt((np.asarray(pit, np.float64) ** 2).sum(axis=0)).max())
    e_rot = 2.0 ** -19 * colmax + 2.0 ** -21
    p1 = np.abs(np.asarray(pist, np.float64)).sum(axis=0)           # column 1-norms of PiST
    r1 = np.abs(ref["resid"]).sum(axis=1)                          # residual 1-norms
    return (e_rot * ref["norm"][:, None] * p1[None, :] + 2.0 ** -19 * ref["proj_scale"]
            + 2.0 ** -25 * (p1[None, :] + r1[:, None]))


def _kernel_codebook(bits):
    from oracle import codebook as ocb
    c = np.array(ocb.kernel_codebook(128, bits), dtype=np.float32)
    b = ((c[:-1] + c[1:]) / 2.0).astype(np.float32)
    return torch.from_numpy(c), torch.from_numpy(b)


@pytest.mark.parametrize("bits", [2, 1, 3, 4])
@pytest.mark.parametrize("n", [1, 1023, 4096, 131072])
def test_compress_k_v_against_oracle(dev, bits, n, parity_log):
    """compress_k / compress_v against the float64 restatement; 131,072 rows make every wave
    loop over several 32-row groups."""
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
    stats = ocomp.classify_strict_fp64(idx_gpu, ref["idx"], ref["rot"], bnd.double().numpy())
    _log(parity_log, f"compress_k b{bits} n{n}", stats)
    assert stats["failures"] == 0, f"index differences beyond 1 ulp of a boundary: {stats}"
    # the kernel's bytes are exactly the oracle's packing of the oracle's decisions, where the
    # band-exempt elements take the GPU's value
    merged = np.where(diff, idx_gpu, ref["idx"])
    np.testing.assert_array_equal(k_idx.cpu().numpy(), opack.pack_indices(merged, bits))
    rows_ok = ~diff.any(axis=1)
    sg = opack.unpack_signs(k_signs.cpu().numpy())
    sdiff = (sg != ref["sign"]) & rows_ok[:, None]
    band = sign_band(ref, PiT.double().numpy(), PiST.double().numpy())
    outside = sdiff & (np.abs(ref["proj"]) > band)
    assert not outside.any(), f"sign bits differ from float64 outside the arithmetic bound: {int(outside.sum())}"
    if parity_log is not None:
        parity_log[f"compress_k b{bits} n{n}"].update(
            sign_elements=int(rows_ok.sum()) * 128, sign_mismatches_in_bound=int(sdiff.sum()),
            sign_rows_exempt=int((~rows_ok).sum()), sign_band_max=float(band.max()))
    print(f"[compress_k b{bits} n{n}] sign differences within the bound: {int(sdiff.sum())}, "
          f"rows exempt: {int((~rows_ok).sum())}")
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
        assert ocomp.classify_strict_fp64(idx, ref["idx"], ref["rot"], bnd.double().numpy())["failures"] == 0
    with pytest.raises(ValueError):
        compress_k(t(K[:, :64]), t(PiT), t(PiST), t(cent), t(bnd))
    with pytest.raises(ValueError):
        compress_v(t(K), t(PiT), t(cent[:3]), t(bnd))
    with pytest.raises(ValueError):
        compress_k(K, PiT, PiST, cent, bnd)  # CPU tensors: no CPU fallback
    assert base[0].shape == (64, 32)


def test_polarquant_3d_and_edge_rows(dev, parity_log):
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
    ref64 = ocomp.polarquant_compress_fp64(x, cent, bnd, True, True)
    check_against_oracle(res, ref, ref64, cent, bnd, True, "3d", parity_log)
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


def compare_paged(cache, x, slots, fmt, cent, bnd, rotate=True, name=None, parity_log=None):
    """The paged cache written by compress_paged(x, slots) against the oracle, token by token
    (read back from any layout): indices under the 1-ulp / fp64 rule, sign bits under the same
    rule around the centroid, fp16 norms (NaN where the oracle's is NaN), residual norms of rows
    whose indices all match, and every block no slot points at still zero."""
    from turboquant.core import make_wht_matrix
    got = cache.cpu().numpy()
    nb, H = got.shape[0], got.shape[1]
    bs, bits, qjl = fmt.block_size, fmt.bits, fmt.qjl
    T = x.shape[0]
    slots = np.asarray(slots, np.int64)
    xf = x.float().cpu().reshape(T * H, 128)
    ref = ocomp.polarquant_compress(xf, cent, bnd, 2 ** bits, qjl, make_wht_matrix(128) if rotate else None)
    ref64 = ocomp.polarquant_compress_fp64(xf, cent, bnd, qjl, rotate)
    live = (slots >= 0) & (slots < nb * bs)
    # a slot written twice keeps one of its writers: only slots written once are compared
    uniq, counts = np.unique(slots[live], return_counts=True)
    once = np.isin(slots, uniq[counts == 1]) & live
    tok = np.nonzero(once)[0]
    sel = slots[tok]
    xn = ref["x_normalized"].reshape(T, H, 128).numpy()
    stats_all = None
    for h in range(H):
        pl = opaged.tiles_to_tokens(got[:, h], bs, bits, qjl, fmt.layout)
        gi = opack.unpack_indices(pl["idx"][sel], bits)
        ri = ref["indices"].reshape(T, H, 128)[tok, h].numpy()
        i64 = ref64["indices"].reshape(T, H, 128)[tok, h].numpy()
        st = ocomp.classify_strict(gi, ri, xn[tok, h], bnd.numpy(), i64)
        assert st["failures"] == 0, f"{name} head {h}: index mismatches beyond 1 ulp: {st}"
        stats_all = st if stats_all is None else {k: stats_all[k] + st[k] for k in st}
        gn = pl["norm"][sel].view(np.float16).astype(np.float32)
        rn = ref["norms"].reshape(T, H)[tok, h].numpy().astype(np.float16).astype(np.float32)
        np.testing.assert_array_equal(np.isnan(gn), np.isnan(rn))
        fin = ~np.isnan(rn)
        np.testing.assert_allclose(gn[fin], rn[fin], rtol=NORM_RTOL, atol=NORM_ATOL)
        if qjl:
            gs = opack.unpack_signs(pl["signs"][sel])
            rsg = (ref["signs"].reshape(T, H, 128)[tok, h].numpy() > 0).astype(gs.dtype)
            s64 = (ref64["signs"].reshape(T, H, 128)[tok, h].numpy() > 0).astype(gs.dtype)
            c = cent.double().numpy()[ri]
            xr = xn[tok, h].astype(np.float64)
            cdist = np.abs(xr - c) / np.maximum(ocomp.ulp32(np.maximum(np.abs(xr), np.abs(c))), 1e-300)
            ok = (gi != ri) | (cdist <= 1.0) | (gs == s64) | np.isnan(xr)
            assert not ((gs != rsg) & ~ok).any(), f"{name} head {h}: sign flips away from centroids"
            clean = (gi == ri).all(axis=1) & fin
            grn = pl["rnorm"][sel].view(np.float16).astype(np.float32)[clean]
            rrn = ref["rot_residual_norm"].reshape(T, H)[tok, h].numpy().astype(np.float16).astype(np.float32)[clean]
            np.testing.assert_allclose(grn, rrn, rtol=NORM_RTOL, atol=NORM_ATOL)
    if name is not None:
        _log(parity_log, name, stats_all)
    written = np.zeros(nb, bool)
    written[slots[live] // bs] = True
    assert not got[~written].any(), "blocks no slot points at were written"
    return stats_all


def block_order_slots(T, nb, bs, seed):
    """Token t -> slot perm[t // bs] * bs + t % bs for a seeded permutation of the blocks (how a
    prefill fills whole blocks)."""
    perm = np.random.default_rng(seed).permutation(nb)
    t = np.arange(T)
    return perm[t // bs] * bs + t % bs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rotate", [True, False])
@pytest.mark.parametrize("bits,qjl", [(4, False), (3, True), (2, True), (2, False)])
@pytest.mark.parametrize("layout", ["keys", "values", "rows"])
def test_compress_paged_16bit(dev, dtype, rotate, bits, qjl, layout, parity_log):
    """bf16 / fp16 rows (the matrix-core path): block-ordered slots (whole quads of rows land on
    consecutive slots), one padding slot inside a quad and an odd token count (a partial last
    group), with and without the rotation, every layout."""
    if layout == "values" and qjl:
        pytest.skip("the values layout carries no QJL data")
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, bs = 203, 3, 16
    nb = 20
    g = torch.Generator().manual_seed(11 + bits)
    x = (torch.randn(T, H, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)).to(dtype)
    slots = block_order_slots(T, nb, bs, 3)
    slots[37] = -1
    fmt = PagedKVFormat(bits=bits, qjl=qjl, block_size=bs, layout=layout)
    cent, bnd = _codebook(bits)
    cache = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x.to(dev), torch.from_numpy(slots).to(dev), cache, fmt, cent.to(dev), bnd.to(dev), rotate=rotate)
    torch.cuda.synchronize()
    compare_paged(cache, x, slots, fmt, cent, bnd, rotate, f"paged16 {dtype} rot{int(rotate)} b{bits} q{int(qjl)} {layout}",
                  parity_log)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["keys", "values"])
def test_compress_paged_16bit_subnormal_rows(dev, dtype, layout):
    """Rows of subnormal bf16 / fp16 values (all of them, or beside one normal element) and rows
    near the bottom of the normal range, through the matrix-core rotation: the products keep the
    subnormal inputs (a flush to zero would zero the row, and every positive element would then
    fall on the other side of the middle boundary), under the same parity rule."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, bs, nb = 64, 2, 16, 8
    g = torch.Generator().manual_seed(21)
    tiny = torch.finfo(dtype).tiny  # smallest normal
    x = torch.randn(T, H, 128, generator=g)
    x[0:16] *= tiny * 0.25          # every element subnormal
    x[16:32] *= tiny * 0.25
    x[16:32, :, 5] = 1.0            # one normal element beside subnormals
    x[32:48] *= tiny * 4.0          # just above the normal range
    x = x.to(dtype)
    qjl = layout == "keys"
    slots = block_order_slots(T, nb, bs, 9)
    fmt = PagedKVFormat(bits=4 if layout == "values" else 3, qjl=qjl, block_size=bs, layout=layout)
    cent, bnd = _codebook(fmt.bits)
    cache = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x.to(dev), torch.from_numpy(slots).to(dev), cache, fmt, cent.to(dev), bnd.to(dev), rotate=True)
    torch.cuda.synchronize()
    compare_paged(cache, x, slots, fmt, cent, bnd, True)


@pytest.mark.parametrize("rotate", [True, False])
@pytest.mark.parametrize("layout", ["keys", "values"])
def test_compress_paged_16bit_edge_rows(dev, rotate, layout):
    """A NaN row (every index past the last boundary, NaN norm), a zero row, a row whose sum of
    squares overflows (norm inf: x / inf = 0 for every element), a basis row, among ordinary
    rows; int64 slots."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, bs, nb = 48, 2, 16, 6
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, H, 128, generator=g)
    x[3, 0, 7] = float("nan")
    x[4, 1] = 0.0
    x[5, 0] = 3e19
    x[6, 1] = 0.0
    x[6, 1, 9] = 2.5
    x = x.to(torch.bfloat16)
    qjl = layout == "keys"
    slots = block_order_slots(T, nb, bs, 8)
    fmt = PagedKVFormat(bits=3, qjl=qjl, block_size=bs, layout=layout)
    cent, bnd = _codebook(3)
    cache = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x.to(dev), torch.from_numpy(slots).to(dev), cache, fmt, cent.to(dev), bnd.to(dev), rotate=rotate)
    torch.cuda.synchronize()
    compare_paged(cache, x, slots, fmt, cent, bnd, rotate)
    # the NaN row: every index 7, NaN norm; the overflowing row: inf norm, indices of 0
    pl = opaged.tiles_to_tokens(cache[:, 0].cpu().numpy(), bs, 3, qjl, layout)
    nan_idx = opack.unpack_indices(pl["idx"][slots[3]][None], 3)[0]
    assert (nan_idx == 7).all()
    assert np.isnan(pl["norm"][slots[3]].view(np.float16))
    big = opack.unpack_indices(pl["idx"][slots[5]][None], 3)[0]
    assert (big == int(np.searchsorted(bnd.numpy(), 0.0))).all()
    assert np.isinf(pl["norm"][slots[5]].view(np.float16))


def test_compress_paged_16bit_close_boundaries(dev):
    """A codebook with two boundaries 1e-4 apart (inside one lookup cell) runs the linear count
    of the matrix-core kernel; the probe rows put values on and next to every boundary."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    bnd = torch.tensor([-0.3, -0.05, 0.0, 1e-4, 0.02, 0.1, 0.4], dtype=torch.float32)
    cent = torch.tensor([-0.5, -0.2, -0.02, 5e-5, 0.01, 0.05, 0.2, 0.6], dtype=torch.float32)
    T, H, bs, nb = 64, 2, 16, 8
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(T, H, 128, generator=g) * 0.3).to(torch.bfloat16)
    slots = block_order_slots(T, nb, bs, 1)
    for layout, qjl in (("keys", True), ("values", False)):
        fmt = PagedKVFormat(bits=3, qjl=qjl, block_size=bs, layout=layout)
        cache = allocate_cache(nb, H, fmt, device=dev)
        compress_paged(x.to(dev), torch.from_numpy(slots).to(dev), cache, fmt, cent.to(dev), bnd.to(dev), rotate=False)
        torch.cuda.synchronize()
        compare_paged(cache, x, slots, fmt, cent, bnd, False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("kb,kq,vb,klayout,vlayout", [
    (4, False, 4, "keys", "values"),     # one launch, turbo4 K and V
    (3, True, 3, "keys", "values"),      # one launch, QJL signs in the K half only
    (2, True, 2, "rows", "rows"),        # one launch, row layout for both
    (4, True, 2, "keys", "values"),      # different bits: two launches behind the same call
])
def test_compress_paged_kv_matches_two_launches(dev, dtype, kb, kq, vb, klayout, vlayout):
    """compress_paged_kv writes byte-for-byte what compress_paged(K) then compress_paged(V) write,
    with padding and out-of-range slots, int64 slots and a second, shorter call into the same caches."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged, compress_paged_kv
    T, H, bs, nb = 203, 4, 16, 20
    g = torch.Generator().manual_seed(17 + kb + 5 * vb)
    k = (torch.randn(T, H, 128, generator=g) * 2.0).to(dtype).to(dev)
    v = torch.randn(T, H, 128, generator=g).to(dtype).to(dev)
    slots = torch.from_numpy(block_order_slots(T, nb, bs, 4)).to(torch.int64)
    slots[11] = -1
    slots[12] = nb * bs + 7
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs, layout=klayout)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout=vlayout)
    kcb = tuple(t.to(dev) for t in _codebook(kb))
    vcb = tuple(t.to(dev) for t in _codebook(vb))
    want_k = allocate_cache(nb, H, kf, device=dev)
    want_v = allocate_cache(nb, H, vf, device=dev)
    got_k = allocate_cache(nb, H, kf, device=dev)
    got_v = allocate_cache(nb, H, vf, device=dev)
    for n in (T, 61):
        s = slots[:n].to(dev)
        compress_paged(k[:n], s, want_k, kf, *kcb)
        compress_paged(v[:n], s, want_v, vf, *vcb)
        compress_paged_kv(k[:n], v[:n], s, got_k, got_v, kf, vf, kcb, vcb)
        torch.cuda.synchronize()
        assert torch.equal(got_k, want_k), f"K cache differs after a call over {n} tokens"
        assert torch.equal(got_v, want_v), f"V cache differs after a call over {n} tokens"
        k, v = k.flip(0).contiguous(), v.flip(0).contiguous()


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_compress_paged_values_appends(dev, bits):
    """Values tiles interleave the fields of four consecutive rows.  Writing a block's tokens one
    call at a time (decode appends: each call sets its own fields and keeps the neighbours'),
    in a scrambled order, over a block that held other data, gives the bytes of one call over
    all tokens; so does a call whose slots start mid-group (prefill after a partial block)."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged
    T, H, bs, nb = 40, 3, 16, 4
    g = torch.Generator().manual_seed(30 + bits)
    x = torch.randn(T, H, 128, generator=g).to(torch.bfloat16).to(dev)
    slots = torch.arange(5, 5 + T, dtype=torch.int64)     # starts at row 5 of block 0
    fmt = PagedKVFormat(bits=bits, qjl=False, block_size=bs, layout="values")
    cb = tuple(t.to(dev) for t in _codebook(bits))
    want = allocate_cache(nb, H, fmt, device=dev)
    compress_paged(x, slots.to(dev), want, fmt, *cb)
    got = allocate_cache(nb, H, fmt, device=dev)
    got.random_(0, 256, generator=torch.Generator(device=dev).manual_seed(1))
    pre = got.clone()
    order = torch.randperm(T, generator=g)
    for t in order.tolist():
        compress_paged(x[t:t + 1], slots[t:t + 1].to(dev), got, fmt, *cb)
    torch.cuda.synchronize()
    # rows 0-4 of block 0 were never written: their fields keep the old bits
    pl_got = opaged.tiles_to_tokens(got.reshape(nb * H, -1).cpu().numpy(), bs, bits, False, "values")
    pl_pre = opaged.tiles_to_tokens(pre.reshape(nb * H, -1).cpu().numpy(), bs, bits, False, "values")
    pl_want = opaged.tiles_to_tokens(want.reshape(nb * H, -1).cpu().numpy(), bs, bits, False, "values")
    rows = np.arange(nb * H * bs).reshape(nb, H, bs)
    written = np.zeros((nb, bs), bool)
    written.reshape(-1)[slots.numpy()] = True
    for b in range(nb):
        for h in range(H):
            for r in range(bs):
                i = rows[b, h, r]
                src = pl_want if written[b, r] else pl_pre
                assert np.array_equal(pl_got["idx"][i], src["idx"][i]), (b, h, r)
                if written[b, r]:
                    assert pl_got["norm"][i] == pl_want["norm"][i]
    # the same tokens again in one call over the appended cache: bytes of the whole-batch write
    # wherever a token was written
    compress_paged(x, slots.to(dev), got, fmt, *cb)
    pl_got2 = opaged.tiles_to_tokens(got.reshape(nb * H, -1).cpu().numpy(), bs, bits, False, "values")
    sel = rows[:, :, :][written[:, None, :].repeat(H, 1)]
    assert np.array_equal(pl_got2["idx"][sel], pl_want["idx"][sel])


def test_compress_paged_kv_rejections(dev):
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged_kv
    T, H, bs, nb = 8, 2, 16, 2
    k = torch.zeros(T, H, 128, dtype=torch.bfloat16, device=dev)
    slots = torch.arange(T, dtype=torch.int32, device=dev)
    kf = PagedKVFormat(bits=3, qjl=True, block_size=bs, layout="keys")
    vf = PagedKVFormat(bits=3, qjl=False, block_size=bs, layout="values")
    cb = tuple(t.to(dev) for t in _codebook(3))
    kc, vc = allocate_cache(nb, H, kf, device=dev), allocate_cache(nb, H, vf, device=dev)
    with pytest.raises(ValueError):   # V with QJL
        compress_paged_kv(k, k, slots, kc, vc, kf, PagedKVFormat(bits=3, qjl=True, block_size=bs, layout="rows"), cb, cb)
    with pytest.raises(ValueError):   # K in the values layout
        compress_paged_kv(k, k, slots, vc, vc, vf, vf, cb, cb)
    with pytest.raises(TypeError):    # dtypes differ
        compress_paged_kv(k, k.float(), slots, kc, vc, kf, vf, cb, cb)
    with pytest.raises(ValueError):   # shapes differ
        compress_paged_kv(k, k[:4], slots, kc, vc, kf, vf, cb, cb)
    with pytest.raises(ValueError):   # wrong codebook size
        compress_paged_kv(k, k, slots, kc, vc, kf, vf, cb, tuple(t.to(dev) for t in _codebook(2)))


@pytest.mark.parametrize("bits,qjl,slot_bytes", [
    (3, False, 50),    # the reference's 3-bit slot: 48 index bytes + fp16 norm (2-byte stores)
    (3, False, 64),    # padded slot: 4-byte aligned rows
    (3, True, 68),     # indices, signs, norm, residual norm
    (2, True, 54),     # signs at an offset that is only 2-byte aligned
    (4, False, 66),
])
@pytest.mark.parametrize("kv_view", [False, True])
def test_compress_paged_slots_matches_tiles(dev, bits, qjl, slot_bytes, kv_view):
    """compress_paged_slots writes into an array-of-slots cache [NB, BS, Hkv, slot] (or the K / V
    half of a [NB, 2, BS, Hkv, slot] cache) exactly the bytes to_reference_slots reads out of a
    compress_paged tile cache for every written token; padding bytes, unwritten slots and the
    other half of the cache keep what they held.  A second, shorter call follows."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged, compress_paged_slots, \
        to_reference_slots
    T, H, bs, nb = 203, 3, 16, 20
    g = torch.Generator().manual_seed(40 + bits + slot_bytes)
    x = torch.randn(T, H, 128, generator=g).to(torch.bfloat16).to(dev)
    perm = torch.randperm(nb * bs, generator=g)[:T].to(torch.int64)
    perm[5] = -1
    perm[6] = nb * bs + 3
    fmt = PagedKVFormat(bits=bits, qjl=qjl, block_size=bs, layout="keys" if qjl else "values")
    tb = fmt.token_bytes
    cb = tuple(t.to(dev) for t in _codebook(bits))
    tiles = allocate_cache(nb, H, fmt, device=dev)
    if kv_view:
        full = torch.randint(0, 256, (nb, 2, bs, H, slot_bytes), dtype=torch.uint8, generator=g).to(dev)
        slots = full[:, 1]
    else:
        full = torch.randint(0, 256, (nb, bs, H, slot_bytes), dtype=torch.uint8, generator=g).to(dev)
        slots = full
    pre = full.clone()
    for n in (T, 57):
        s = perm[:n].to(dev)
        compress_paged(x[:n], s, tiles, fmt, *cb)
        compress_paged_slots(x[:n], s, slots, fmt, *cb)
        torch.cuda.synchronize()
        want = to_reference_slots(tiles, fmt, slot_bytes).cpu()
        got = slots.cpu()
        written = torch.zeros(nb * bs, dtype=torch.bool)
        ok = perm[:T]
        written[ok[(ok >= 0) & (ok < nb * bs)]] = True
        written = written.reshape(nb, bs)
        assert torch.equal(got[written][..., :tb], want[written][..., :tb]), f"payload differs after {n} tokens"
        pre_s = (pre[:, 1] if kv_view else pre).cpu()
        assert torch.equal(got[..., tb:], pre_s[..., tb:]), "padding bytes changed"
        assert torch.equal(got[~written], pre_s[~written]), "unwritten slots changed"
        if kv_view:
            assert torch.equal(full[:, 0].cpu(), pre[:, 0].cpu()), "the other half of the cache changed"
        x = x.flip(0).contiguous()


def test_compress_to_tq_cache_then_decode(dev):
    """The reference's 3-bit [NB, 2, BS, Hkv, 128] slot cache filled by compress_to_tq_cache (K
    and V, one launch each) decodes with tq_v11 to what the tile-layout decode gives for the
    same tokens compressed into tiles (two kernels, two layouts, one answer)."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, compress_paged, decode_paged
    from turboquant.kernels.sparse_v import compress_to_tq_cache, tq_v11
    Hkv, G, bs, S, L = 4, 6, 32, 2, 300
    Hq = Hkv * G
    nblk = math.ceil(L / bs)
    nb = S * nblk + 3
    g = torch.Generator().manual_seed(5)
    k = torch.randn(S * L, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(S * L, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    bt = torch.randperm(nb, generator=g)[: S * nblk].reshape(S, nblk).to(torch.int32)
    tok = torch.arange(L)
    slot = torch.cat([bt[s, tok // bs].to(torch.int64) * bs + tok % bs for s in range(S)]).to(dev)
    cent, bnd = (t.to(dev) for t in _codebook(3))
    cache = torch.zeros((nb, 2, bs, Hkv, 128), dtype=torch.uint8, device=dev)
    compress_to_tq_cache(k, slot, cache, 0, cent, bnd)
    compress_to_tq_cache(v, slot, cache, 1, cent, bnd)
    kf = PagedKVFormat(bits=3, qjl=False, block_size=bs, layout="keys")
    vf = PagedKVFormat(bits=3, qjl=False, block_size=bs, layout="values")
    kc, vc = allocate_cache(nb, Hkv, kf, device=dev), allocate_cache(nb, Hkv, vf, device=dev)
    compress_paged(k, slot, kc, kf, cent, bnd)
    compress_paged(v, slot, vc, vf, cent, bnd)
    q = torch.randn(S, Hq, 128, generator=g).to(torch.float16).to(dev)
    lens = torch.full((S,), L, dtype=torch.int32, device=dev)
    sm = 1 / math.sqrt(128)
    out_aos = torch.empty_like(q)
    tq_v11(out_aos, q, cache, cent, bt.to(dev), lens, sm)
    out_tiles = decode_paged(q, kc, kf, cent, vc, vf, cent, bt.to(dev), lens, sm)
    torch.cuda.synchronize()
    torch.testing.assert_close(out_aos.float(), out_tiles.float(), rtol=1e-2, atol=1e-3)


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
    ref64 = ocomp.polarquant_compress_fp64(x.float().reshape(T * H, 128), cent, bnd, qjl, True)
    pl = _payload_from_oracle(ref, bits, qjl, T, H)
    want = opaged.scatter_tokens(pl, perm.numpy(), nb, H, block_size, bits, qjl, layout=layout)
    if np.array_equal(got, want):
        return
    # Differences must come only from boundary-band indices / fp16 norm rounding of the same
    # tokens; compared per token in row form (the oracle reads any layout back into rows).
    xn = ref["x_normalized"].reshape(T, H, 128).numpy()
    i64 = ref64["indices"].reshape(T, H, 128).numpy()
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
            st = ocomp.classify_strict(ig, iw, xn[t, h][None], bnd.numpy(), i64[t, h][None])
            assert st["failures"] == 0, f"token {t} head {h}: index mismatch beyond 1 ulp: {st}"
    # untouched blocks stay zero
    written = {int(p) // block_size for p in perm if 0 <= int(p) < nb * block_size}
    for b in range(nb):
        if b not in written:
            assert not got[b].any()


def test_config2_full_size_roundtrip(dev, parity_log):
    """Benchmark config 2 at full size, on the bench's own inputs (bench.build_compress_workload):
    K and V [16384, 8, 128] bf16 with outlier channels, turbo4, into 8192 permuted blocks of 16
    (K in the keys layout, V in the values layout).  Every stored index against the oracle
    (1-ulp / fp64 rule, counted), every fp16 norm, and the untouched blocks."""
    import bench
    from turboquant.core import make_wht_matrix
    from turboquant.kernels.paged import compress_paged
    w = bench.build_compress_workload(dev)
    T, H, bs = bench.COMPRESS_T, bench.COMPRESS_H, bench.COMPRESS_BS
    slots = w["slots"].long().cpu().numpy()
    cent, bnd = w["c"].cpu(), w["b"].cpu()
    H128 = make_wht_matrix(128)
    for which, x, cache, fmt in (("K", w["k"], w["kc"], w["fmt"]), ("V", w["v"], w["vc"], w["vfmt"])):
        compress_paged(x, w["slots"], cache, fmt, w["c"], w["b"])
        torch.cuda.synchronize()
        blk, row = slots // bs, slots % bs
        got_idx = np.zeros((T, H, 128), np.int64)
        got_norm = np.zeros((T, H), np.uint16)
        for h in range(H):
            tok = opaged.tiles_to_tokens(cache[:, h].cpu().numpy(), bs, 4, False, fmt.layout)
            sel = blk * bs + row
            got_idx[:, h] = opack.unpack_indices(tok["idx"][sel], 4)
            got_norm[:, h] = tok["norm"][sel]
        xf = x.float().cpu().reshape(T * H, 128)
        ref = ocomp.polarquant_compress(xf, cent, bnd, 16, False, H128)
        ref64 = ocomp.polarquant_compress_fp64(xf, cent, bnd, False, True)
        stats = ocomp.classify_strict(got_idx.reshape(T * H, 128), ref["indices"].numpy(), ref["x_normalized"].numpy(),
                                      bnd.numpy(), ref64["indices"].numpy())
        _log(parity_log, f"config2 {which}", stats)
        assert stats["failures"] == 0, stats
        gn = got_norm.reshape(-1).view(np.float16).astype(np.float32)
        want_norm = ref["norms"].numpy().astype(np.float16).astype(np.float32)
        np.testing.assert_allclose(gn, want_norm, rtol=NORM_RTOL, atol=NORM_ATOL)
        assert np.mean(gn == want_norm) > 0.999
        written = np.zeros(cache.shape[0], bool)
        written[blk] = True
        assert not cache[torch.from_numpy(~written).to(dev)].any()


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
