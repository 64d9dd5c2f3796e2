"""Pinning the CPU oracle (no GPU): closed forms, brute force, invariants, golden fixtures.

The reference's own tests hold no golden vectors for this path (only invariants:
tests/test_codebook.py, tests/test_compress.py, tests/test_rotation.py); every oracle function
is pinned here by something other than re-typing its formula.
"""

import hashlib
import itertools
import json
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import codebook as ocb
from oracle import compress as ocomp
from oracle import decode as odec
from oracle import packing as opack
from oracle import paged as opaged

GOLDEN = pathlib.Path(__file__).parent / "golden"


# ---------------------------------------------------------------- codebook
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_quad_equals_closed_form(bits):
    c, b = ocb.solve_codebook_quad(128, bits)
    cc, bb = ocb.solve_codebook_closed_form(128, bits)
    assert max(abs(x - y) for x, y in zip(c, cc)) < 1e-10
    assert max(abs(x - y) for x, y in zip(b, bb)) < 1e-10


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_invariants(bits):
    # tests/test_codebook.py:12-49 of the reference
    c, b = ocb.solve_codebook_quad(128, bits)
    assert len(c) == 2 ** bits and len(b) == 2 ** bits - 1
    assert all(c[i] < c[i + 1] for i in range(len(c) - 1))
    assert all(c[i] < b[i] < c[i + 1] for i in range(len(b)))
    assert all(abs(c[i] + c[-1 - i]) < 1e-6 for i in range(len(c)))
    # 100 rounds reach the Lloyd-Max fixed point for bits <= 3; for bits = 4 the reference's
    # codebook stops short of it (slow convergence), and 2000 rounds of the same map converge.
    res = ocb.lloyd_residual(c, b, 128)
    if bits <= 3:
        assert res < 1e-7
    else:
        assert 1e-5 < res < 1e-3
        c2, b2 = ocb.solve_codebook_closed_form(128, bits, iters=2000)
        assert ocb.lloyd_residual(c2, b2, 128) < res / 1000


def test_codebook_known_lloyd_max_values():
    # Max (1960) optimal Gaussian quantizers, in units of sigma = 1/sqrt(d)
    sigma = 1 / math.sqrt(128)
    known = {1: [0.7979], 2: [0.4528, 1.510], 3: [0.2451, 0.7560, 1.344, 2.152]}
    for bits, pos in known.items():
        c, _ = ocb.solve_codebook_quad(128, bits)
        half = [x / sigma for x in c[len(c) // 2:]]
        np.testing.assert_allclose(half, pos, rtol=2e-3)


def test_codebook_sigma_scaling():
    c64, _ = ocb.solve_codebook_quad(64, 2)
    c256, _ = ocb.solve_codebook_quad(256, 2)
    assert abs(c64[-1] / c256[-1] - 2.0) < 1e-9


def test_codebook_golden_fixture():
    g = json.loads((GOLDEN / "codebooks.json").read_text())
    for bits in (1, 2, 3, 4):
        c, b = ocb.solve_codebook_quad(128, bits)
        assert g["books"][str(bits)]["centroids"] == c
        assert g["books"][str(bits)]["boundaries"] == b


def test_kernel_codebook_variant_differs_but_is_lloyd_max():
    kc = ocb.kernel_codebook(128, 2)
    c, _ = ocb.solve_codebook_quad(128, 2)
    bnd = [(kc[i] + kc[i + 1]) / 2 for i in range(3)]
    assert ocb.lloyd_residual(kc, bnd, 128) < 1e-8
    assert max(abs(x - y) for x, y in zip(kc, c)) < 1e-6


# ---------------------------------------------------------------- WHT
@pytest.mark.parametrize("d", [2, 4, 8, 16, 32, 64, 128])
def test_wht_closed_form_and_involution(d):
    H = ocomp.wht_matrix(d)
    h = float(H[0, 0])
    np.testing.assert_array_equal(H.numpy(), ocomp.wht_closed_form(d, h).astype(np.float32))
    assert abs(h - 1 / math.sqrt(d)) < 1e-7
    assert (H @ H - torch.eye(d)).abs().max() < 1e-5


# ---------------------------------------------------------------- compress
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("use_qjl", [False, True])
def test_compress_oracle_vs_fp64_shadow(bits, use_qjl):
    g = torch.Generator().manual_seed(bits)
    x = torch.randn(2000, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 0.5)
    c, b = ocb.solve_codebook_quad(128, bits)
    cent, bnd = torch.tensor(c), torch.tensor(b)
    ref = ocomp.polarquant_compress(x, cent, bnd, 2 ** bits, use_qjl, ocomp.wht_matrix(128))
    sh = ocomp.polarquant_compress_fp64(x, cent, bnd, use_qjl, True)
    n, ok, bad, band = ocomp.classify_index_mismatch(ref["indices"], sh["indices"], sh["x_normalized"], bnd, 8)
    assert bad == 0 and n <= 3
    np.testing.assert_allclose(ref["norms"].numpy(), sh["norms"].numpy(), rtol=1e-6)
    if use_qjl:
        same = ref["indices"] == sh["indices"]
        cbd = ocomp.centroid_band(sh["x_normalized"], cent, sh["indices"])
        flips = (ref["signs"].double() != sh["signs"]) & same & (cbd > 8)
        assert not flips.any()
        np.testing.assert_allclose(ref["rot_residual_norm"].numpy(), sh["rot_residual_norm"].numpy(), rtol=1e-4)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_compress_packed_agrees_with_polarquant_shadow_for_wht(bits):
    """compress_packed (norm first, multiply by the reciprocal, >= rule, residual through PiST)
    and the polarquant fp64 shadow (rotate first, divide, > rule, residual signs) describe the
    same quantizer when PiT is the WHT and PiST = I: indices, signs and norms must agree except
    at exact ties.  A slip in either restatement (order, the 1e-8, the residual scaling, the
    sign convention) breaks this."""
    torch.manual_seed(7)
    x = torch.randn(400, 128) * torch.exp(torch.randn(128) * 0.5)
    c, b = ocb.solve_codebook_quad(128, bits)
    c, b = torch.tensor(c), torch.tensor(b)
    h = float(ocomp.wht_matrix(128)[0, 0])
    H = ocomp.wht_closed_form(128, h)
    pk = ocomp.compress_packed(x.double().numpy(), H, np.eye(128), c.numpy(), b.numpy())
    sh = ocomp.polarquant_compress_fp64(x, c, b, use_qjl=True, rotate=True)
    np.testing.assert_array_equal(pk["idx"], sh["indices"].numpy())
    # |x| vs |x H|: H's entries are the fp32-rounded h, so H is orthogonal to ~2e-8 only
    np.testing.assert_allclose(pk["norm"], sh["norms"].numpy(), rtol=5e-8)
    np.testing.assert_allclose(pk["rnorm"], sh["rot_residual_norm"].numpy(), rtol=5e-7)
    sign_sh = (sh["signs"].numpy() > 0).astype(np.uint8)
    np.testing.assert_array_equal(pk["sign"], sign_sh)


def test_compress_packed_tie_rule_on_basis_vectors():
    """Known answers with PiT = PiST = I: rows 3 e_d against c = (-1.5, -0.5, 0.5, 1.5)/s,
    b = (-1, 0, 1)/s.  Zero coordinates sit exactly on the middle boundary: the >= rule gives
    index 2 (searchsorted-left would give 1), residual (0 - c2) * 3 < 0 -> sign bit 0; the unit
    coordinate gives index 3, residual (1 - c3) * 3 > 0 -> sign bit 1."""
    s = math.sqrt(128)
    c = np.array([-1.5, -0.5, 0.5, 1.5]) / s
    b = np.array([-1.0, 0.0, 1.0]) / s
    x = 3.0 * np.eye(128)
    pk = ocomp.compress_packed(x, np.eye(128), np.eye(128), c, b)
    want_idx = np.full((128, 128), 2)
    np.fill_diagonal(want_idx, 3)
    np.testing.assert_array_equal(pk["idx"], want_idx)
    np.testing.assert_allclose(pk["norm"], 3.0)
    want_sign = np.eye(128, dtype=np.uint8)
    np.testing.assert_array_equal(pk["sign"], want_sign)
    # the unit coordinate is u = 3 * (1 / (3 + 1e-8)); rnorm^2 = 127 * (0.5/s * 3)^2 + ((u - 1.5/s) * 3)^2
    u = 3.0 * (1.0 / (3.0 + 1e-8))
    want_rn = math.sqrt(127 * (1.5 / s) ** 2 + (3 * (u - 1.5 / s)) ** 2)
    np.testing.assert_allclose(pk["rnorm"], want_rn, rtol=1e-12)


def test_compress_oracle_known_answers():
    c, b = ocb.solve_codebook_quad(128, 3)
    cent, bnd = torch.tensor(c), torch.tensor(b)
    x = torch.zeros(3, 128)
    x[1, 7] = 2.5                       # basis vector: rotated coords are +-h*2.5, x_n = +-1/sqrt(128)
    x[2] = 1.0                          # all-ones: rotated vector is sqrt(128) e_0
    r = ocomp.polarquant_compress(x, cent, bnd, 8, True, ocomp.wht_matrix(128))
    # zero vector: x_n = 0 -> idx = #{b < 0} = 3 (boundary 0 itself is not < 0); signs +1
    assert (r["indices"][0] == 3).all() and r["norms"][0] == 0 and (r["signs"][0] == 1).all()
    # basis vector: +-0.0884 -> idx 5 (0.0442 < x < 0.0928) or 2
    Hrow = ocomp.wht_matrix(128)[7]
    want = torch.where(Hrow > 0, 5, 2)
    assert torch.equal(r["indices"][1], want)
    # all-ones: x_n = e_0 -> coordinate 0 is 1.0 (top cell 7), the others exactly 0 -> 3
    assert r["indices"][2, 0] == 7 and (r["indices"][2, 1:] == 3).all()


def test_compress_oracle_reference_test_invariants():
    # tests/test_compress.py:23-72 of the reference (seed 42, 64 x 128, bits 3)
    torch.manual_seed(42)
    c, b = ocb.solve_codebook_quad(128, 3)
    cent, bnd = torch.tensor(c), torch.tensor(b)
    x = torch.randn(64, 128)
    H = ocomp.wht_matrix(128)
    r = ocomp.polarquant_compress(x, cent, bnd, 8, True, H)
    assert r["indices"].min() >= 0 and r["indices"].max() < 8
    assert (r["norms"] >= 0).all()
    assert ((r["signs"] == 1) | (r["signs"] == -1)).all()
    cos = torch.nn.functional.cosine_similarity(x @ H, r["k_mse_rot"], dim=-1)
    assert cos.mean() > 0.95


def test_config1_golden_fixture():
    g = np.load(GOLDEN / "config1_oracle.npz")
    torch.manual_seed(0)
    K = torch.randn(1024, 128)
    assert hashlib.sha256(K.numpy().tobytes()).digest() == g["input_sha256"].tobytes()
    c, b = ocb.solve_codebook_quad(128, 3)
    cent, bnd = torch.tensor(c), torch.tensor(b)
    r = ocomp.polarquant_compress(K, cent, bnd, 8, True, ocomp.wht_matrix(128))
    gi = torch.from_numpy(opack.unpack_indices(g["indices_packed"], 3))
    n, ok, bad, _ = ocomp.classify_index_mismatch(r["indices"], gi, r["x_normalized"], bnd, 8)
    assert bad == 0 and n <= 2
    np.testing.assert_allclose(r["norms"].numpy(), g["norms"], rtol=1e-6)


# ---------------------------------------------------------------- packing
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_brute_force_single_fields(bits):
    # every (dim, value) alone in a row lands in exactly the bits [bits*d, bits*d + bits)
    for d in range(128):
        for v in range(1, 2 ** bits):
            idx = np.zeros((1, 128), np.int64)
            idx[0, d] = v
            row = opack.pack_indices(idx, bits)[0]
            stream = int.from_bytes(row.tobytes(), "little")
            assert stream == v << (bits * d)
            assert np.array_equal(opack.unpack_indices(row[None], bits), idx)


def test_pack_known_answers():
    idx = np.arange(128)[None] % 4
    assert opack.pack_indices(idx, 2)[0, 0] == 0 | (1 << 2) | (2 << 4) | (3 << 6)   # packed_compress.py:79-90
    idx4 = (np.arange(128)[None] % 16)
    assert opack.pack_indices(idx4, 4)[0, 0] == 0x10 and opack.pack_indices(idx4, 4)[0, 1] == 0x32
    idx3 = np.full((1, 128), 2)
    assert list(opack.pack_indices(idx3, 3)[0, :3]) == [0x92, 0x24, 0x49]


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_roundtrip_random_bytes(bits):
    rng = np.random.default_rng(bits)
    rows = rng.integers(0, 256, (50, 16 * bits), dtype=np.uint8)
    assert np.array_equal(opack.pack_indices(opack.unpack_indices(rows, bits), bits), rows)


def test_permute_signs_brute_force():
    for src in range(128):
        bits01 = np.zeros((1, 128), np.int64)
        bits01[0, src] = 1
        out = opack.permute_signs(opack.pack_signs(bits01))[0]
        pos = int.from_bytes(out.tobytes(), "little").bit_length() - 1
        c, k = src % 4, src // 4
        assert pos == 32 * c + k
    rng = np.random.default_rng(0)
    for v in range(256):      # all byte values at every byte position
        rows = rng.integers(0, 256, (1, 16), dtype=np.uint8)
        rows[0, v % 16] = v
        p = opack.permute_signs(rows)
        bits = opack.unpack_signs(rows)
        pb = opack.unpack_signs(p)
        for c in range(4):
            assert np.array_equal(pb[0, 32 * c:32 * (c + 1)], bits[0, c::4])


# ---------------------------------------------------------------- paged
@pytest.mark.parametrize("layout", ["rows", "keys", "values"])
def test_paged_scatter_gather_roundtrip(layout):
    rng = np.random.default_rng(1)
    cases = [(4, False, 16), (3, True, 32), (2, True, 16), (3, False, 32)]
    for bits, qjl, bs in cases:
        if layout == "values" and qjl:
            continue
        T, H, nb = 70, 3, 9
        pl = {"idx": rng.integers(0, 256, (T, H, 16 * bits), dtype=np.uint8),
              "norm": rng.integers(0, 65536, (T, H)).astype(np.uint16)}
        if qjl:
            pl["signs"] = rng.integers(0, 256, (T, H, 16), dtype=np.uint8)
            pl["rnorm"] = rng.integers(0, 65536, (T, H)).astype(np.uint16)
        perm = rng.permutation(nb * bs)[:T]
        cache = opaged.scatter_tokens(pl, perm, nb, H, bs, bits, qjl, layout=layout)
        # a block table listing, for a sequence made of the tokens in slot order
        order = np.argsort(perm)
        slots_sorted = perm[order]
        for h in range(H):
            for t_i, t in enumerate(order):
                blk, row = divmod(int(perm[t]), bs)
                got = opaged.gather_sequence(cache, np.array([blk]), row + 1, h, bs, bits, qjl, layout=layout)
                assert np.array_equal(got["idx"][row], pl["idx"][t, h])
                assert got["norm"][row] == pl["norm"][t, h]
                if qjl:
                    assert np.array_equal(got["signs"][row], pl["signs"][t, h])
                    assert got["rnorm"][row] == pl["rnorm"][t, h]
        assert len(slots_sorted) == T
        slots = opaged.to_slots(cache, bs, bits, qjl, 16 * bits + (20 if qjl else 2), layout=layout)
        blk, row = divmod(int(perm[0]), bs)
        assert np.array_equal(slots[blk, row, 0, :16 * bits], pl["idx"][0, 0])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_values_layout_field_provenance(bits):
    """The values layout on field provenance: in a 16-row sub-tile, decode lane (n, g) reads
    chunk 16g + n (4*bits bytes), and its field 4j + r is dim 8n + j of row 4g + r, so one table
    lookup of 4 adjacent fields gives the four rows of one dim (the PV operand).  Every field is
    tagged with its (row, dim) id, bits of the id at a time, through build_subtile."""
    ids = np.arange(16 * 128).reshape(16, 128)
    got = np.zeros(64 * 32, np.int64)
    for c in range((11 + bits - 1) // bits):
        f = (ids >> (bits * c)) & ((1 << bits) - 1)
        buf = np.frombuffer(opaged.build_subtile(opack.pack_indices(f, bits), None, bits, "values"), np.uint8)
        assert buf.size == 16 * 16 * bits
        got |= opack.unpack_indices(buf.reshape(64, 4 * bits), bits, 32).reshape(-1) << (bits * c)
    got = got.reshape(4, 16, 8, 4)   # chunk (g, n), field (j, r)
    for g in range(4):
        for n in range(16):
            for j in range(8):
                for r in range(4):
                    assert got[g, n, j, r] == (4 * g + r) * 128 + 8 * n + j
    # the vectorised converters are this permutation and its inverse
    rng = np.random.default_rng(bits)
    rows = rng.integers(0, 256, (48, 16 * bits), dtype=np.uint8)
    sub = opaged.rows_to_values_subtiles(rows, bits)
    assert np.array_equal(sub[1], np.frombuffer(opaged.build_subtile(rows[16:32], None, bits, "values"), np.uint8))
    assert np.array_equal(opaged.values_subtiles_to_rows(sub, bits), rows)
    back, _ = opaged.split_subtile(sub[2].tobytes(), bits, False, "values")
    assert np.array_equal(back, rows[32:48])


@pytest.mark.parametrize("bits,qjl", [(2, False), (2, True), (3, False), (3, True), (4, False), (4, True)])
def test_lane_grouped_layouts_one_chunk_per_lane(bits, qjl):
    """The property the keys layout exists for, checked on byte provenance: in a 16-row
    sub-tile, decode lane (n, g) needs the index bytes of row n, dims 32g..32g+31, and their sign
    bytes; each such set must be one contiguous run of bytes, the runs tiling the payload in
    lane order."""
    bs = 32
    # tag every payload byte with (kind, row, byte index): kind 0 index, 1 sign
    idx = np.arange(bs * 16 * bits).reshape(bs, 16 * bits)
    sg = 100000 + np.arange(bs * 16).reshape(bs, 16)
    for layout in ("keys",):
        P = 16 * bits + (16 if qjl else 0)
        # payload built through the oracle with 16-bit tags split over two byte planes
        planes = []
        for shift in (0, 8, 16):
            tile = np.zeros(bs * P + 64 * bs, np.uint8)
            opaged._set_tile_rows(tile, ((idx >> shift) & 0xFF).astype(np.uint8),
                                  ((sg >> shift) & 0xFF).astype(np.uint8) if qjl else None, bs, bits, qjl, layout)
            planes.append(tile[:bs * P].astype(np.int64) << shift)
        tag = planes[0] | planes[1] | planes[2]
        for j in range(bs // 16):
            sub = tag[16 * P * j:16 * P * (j + 1)]
            pos = 0
            for n in range(16):
                for g in range(4):
                    want = list(idx[16 * j + n, 4 * bits * g:4 * bits * (g + 1)])
                    if qjl:
                        want += list(sg[16 * j + n, 4 * g:4 * g + 4])
                    assert list(sub[pos:pos + len(want)]) == want, (layout, j, n, g)
                    pos += len(want)
            assert pos == 16 * P


def test_paged_layout_matches_product_format():
    import sys
    sys.path.insert(0, str(pathlib.Path(__file__).parents[1] / "turboquant-amd_amd"))
    from turboquant.kernels.paged import PagedKVFormat
    for bits, qjl, bs in itertools.product((2, 3, 4), (False, True), (16, 32, 64)):
        f = PagedKVFormat(bits=bits, qjl=qjl, block_size=bs)
        idx_row, off_s, off_n, off_r, tile = opaged.tile_offsets(bs, bits, qjl)
        assert (f.idx_bytes, f.off_norm, f.tile_bytes) == (idx_row, off_n, tile)
        if qjl:
            assert (f.off_signs, f.off_rnorm) == (off_s, off_r)


def test_reference_slot_converters_roundtrip():
    import sys
    sys.path.insert(0, str(pathlib.Path(__file__).parents[1] / "turboquant-amd_amd"))
    from turboquant.kernels.paged import PagedKVFormat, from_reference_slots, to_reference_slots
    rng = np.random.default_rng(5)
    for bits, qjl, layout, bs in [(4, False, "rows", 16), (3, True, "rows", 16), (3, True, "keys", 32),
                                  (2, False, "keys", 16), (4, True, "keys", 16), (3, False, "values", 32),
                                  (2, False, "values", 16), (4, False, "values", 16)]:
        f = PagedKVFormat(bits=bits, qjl=qjl, block_size=bs, layout=layout)
        cache = torch.from_numpy(rng.integers(0, 256, (4, 2, f.tile_bytes), dtype=np.uint8))
        slots = to_reference_slots(cache, f, slot_bytes=f.slot_bytes + 6)
        assert np.array_equal(slots.numpy(), opaged.to_slots(cache.numpy(), bs, bits, qjl, f.slot_bytes + 6, layout=layout))
        assert torch.equal(from_reference_slots(slots, f), cache)


# ---------------------------------------------------------------- decode
def _tiny_case(rng, L, G, kb, qjl, vb):
    kp = {"idx": rng.integers(0, 256, (L, 16 * kb), dtype=np.uint8),
          "norm": rng.uniform(1, 3, L).astype(np.float16).view(np.uint16)}
    if qjl:
        kp["signs"] = rng.integers(0, 256, (L, 16), dtype=np.uint8)
        kp["rnorm"] = rng.uniform(0, 1, L).astype(np.float16).view(np.uint16)
    vp = {"idx": rng.integers(0, 256, (L, 16 * vb), dtype=np.uint8),
          "norm": rng.uniform(1, 3, L).astype(np.float16).view(np.uint16)}
    q = rng.standard_normal((G, 128))
    qp = rng.standard_normal((G, 128))
    return kp, vp, q, qp


def test_decode_oracle_vs_python_loops():
    rng = np.random.default_rng(2)
    kc = np.array(ocb.solve_codebook_quad(128, 3)[0])
    vc = np.array(ocb.solve_codebook_quad(128, 2)[0])
    L, G = 9, 3
    kp, vp, q, qp = _tiny_case(rng, L, G, 3, True, 2)
    k, sg, rn = odec.dequant_keys(kp, kc, 3, True)
    v = odec.dequant_values(vp, vc, 2)
    out = odec.decode_dense(q, qp, k, sg, rn, v, 0.3, 0.05)
    for h in range(G):
        sc = []
        for t in range(L):
            row = int.from_bytes(kp["idx"][t].tobytes(), "little")
            srow = int.from_bytes(kp["signs"][t].tobytes(), "little")
            n = float(np.float16(kp["norm"].view(np.float16)[t]))
            r = float(kp["rnorm"].view(np.float16)[t])
            s = 0.0
            for d in range(128):
                s += q[h, d] * kc[(row >> (3 * d)) & 7] * n
                s += 0.05 * r * qp[h, d] * (1.0 if (srow >> d) & 1 else -1.0)
            sc.append(0.3 * s)
        w = [math.exp(x - max(sc)) for x in sc]
        for d in range(0, 128, 17):
            num = 0.0
            for t in range(L):
                vrow = int.from_bytes(vp["idx"][t].tobytes(), "little")
                num += w[t] * vc[(vrow >> (2 * d)) & 3] * float(vp["norm"].view(np.float16)[t])
            assert abs(out[h, d] - num / sum(w)) < 1e-12


def test_prefill_oracle_vs_masked_score_matrix():
    """prefill_dense (rows of decode_dense over a growing prefix) against one masked score
    tensor [n, G, L] with the causal limit L - n + i written as a comparison of positions."""
    rng = np.random.default_rng(12)
    kc = np.array(ocb.solve_codebook_quad(128, 3)[0])
    vc = np.array(ocb.solve_codebook_quad(128, 4)[0])
    L, G, n = 23, 3, 7
    kp, vp, _, _ = _tiny_case(rng, L, G, 3, True, 4)
    k, sg, rn = odec.dequant_keys(kp, kc, 3, True)
    v = odec.dequant_values(vp, vc, 4)
    q = rng.standard_normal((n, G, 128))
    qp = rng.standard_normal((n, G, 128))
    sm, cs = 0.2, 0.03
    s = sm * (np.einsum("igd,td->igt", q, k) + cs * np.einsum("igd,td->igt", qp, sg) * rn[None, None, :])
    pos_q = (L - n + np.arange(n))[:, None, None]
    s = np.where(np.arange(L)[None, None, :] <= pos_q, s, -np.inf)
    w = np.exp(s - s.max(axis=2, keepdims=True))
    want = np.einsum("igt,td->igd", w / w.sum(axis=2, keepdims=True), v)
    got = odec.prefill_dense(q, qp, k, sg, rn, v, sm, cs, causal=True)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # the last new token sees the whole sequence: a decode step
    np.testing.assert_allclose(got[-1], odec.decode_dense(q[-1], qp[-1], k, sg, rn, v, sm, cs), rtol=1e-12)
    # without the mask every row is a full decode
    nc = odec.prefill_dense(q, qp, k, sg, rn, v, sm, cs, causal=False)
    for i in range(n):
        np.testing.assert_allclose(nc[i], odec.decode_dense(q[i], qp[i], k, sg, rn, v, sm, cs), rtol=1e-12)
    # more new tokens than cache tokens: the rows before the sequence start see nothing
    few = odec.prefill_dense(q, qp, k[:4], sg[:4], rn[:4], v[:4], sm, cs)
    assert np.all(few[:3] == 0.0) and np.all(np.isfinite(few))
    np.testing.assert_allclose(few[3], odec.decode_dense(q[3], qp[3], k[:1], sg[:1], rn[:1], v[:1], sm, cs))


def test_decode_chunked_equals_dense_without_threshold():
    rng = np.random.default_rng(3)
    kc = np.array(ocb.solve_codebook_quad(128, 4)[0])
    kp, vp, q, qp = _tiny_case(rng, 300, 4, 4, False, 4)
    k, _, _ = odec.dequant_keys(kp, kc, 4, False)
    v = odec.dequant_values(vp, kc, 4)
    dense = odec.decode_dense(q, None, k, None, None, v, 0.2, 0.0)
    for chunk in (16, 48, 112, 1024):
        o, sk, tot = odec.decode_chunked(q, None, k, None, None, v, 0.2, 0.0, chunk)
        np.testing.assert_allclose(o, dense, rtol=1e-12, atol=1e-14)
        assert sk == 0 and tot == 300


def test_decode_sparse_rule_brute_force():
    """Skip decisions of decode_chunked vs a token-by-token restatement of sparse_v.py:108-149."""
    rng = np.random.default_rng(4)
    kc = np.array(ocb.solve_codebook_quad(128, 3)[0])
    kp, vp, q, qp = _tiny_case(rng, 80, 2, 3, False, 3)
    q *= 6
    k, _, _ = odec.dequant_keys(kp, kc, 3, False)
    v = odec.dequant_values(vp, kc, 3)
    thr = 1e-3
    o, sk, tot = odec.decode_chunked(q, None, k, None, None, v, 1.0, 0.0, 32, thr)
    s = q @ k.T
    skipped = 0
    outs = []
    for c0 in range(0, 80, 32):
        m = np.full(2, -np.inf)
        l = np.zeros(2)
        acc = np.zeros((2, 128))
        for t0 in range(c0, min(c0 + 32, 80), 16):
            m_new = np.maximum(m, s[:, t0:t0 + 16].max(axis=1))
            l *= np.exp(m - m_new)
            acc *= np.exp(m - m_new)[:, None]
            for t in range(t0, t0 + 16):
                p = np.exp(s[:, t] - m_new)
                l += p
                if p.max() > thr:
                    acc += p[:, None] * v[t][None, :]
                else:
                    skipped += 1
            m = m_new
        outs.append((m, l, acc))
    M = np.max([x[0] for x in outs], axis=0)
    num = sum(np.exp(x[0] - M)[:, None] * x[2] for x in outs)
    den = sum(np.exp(x[0] - M) * x[1] for x in outs)
    np.testing.assert_allclose(o, num / den[:, None], rtol=1e-12)
    assert sk == skipped and sk > 0 and tot == 80


def test_decode_constant_values_closed_form():
    rng = np.random.default_rng(6)
    kc = np.array(ocb.solve_codebook_quad(128, 2)[0])
    kp, vp, q, _ = _tiny_case(rng, 50, 2, 2, False, 2)
    vp["idx"][:] = 0xFF                      # every 2-bit field = 3
    vp["norm"][:] = np.float16(1.5).view(np.uint16)
    k, _, _ = odec.dequant_keys(kp, kc, 2, False)
    v = odec.dequant_values(vp, kc, 2)
    o = odec.decode_dense(q, None, k, None, None, v, 1.0, 0.0)
    np.testing.assert_allclose(o, np.full((2, 128), kc[3] * 1.5), rtol=1e-12)


def test_permuted_sign_dequant_matches_natural():
    rng = np.random.default_rng(7)
    kc = np.array(ocb.solve_codebook_quad(128, 2)[0])
    kp, _, _, _ = _tiny_case(rng, 20, 1, 2, True, 2)
    _, s_nat, _ = odec.dequant_keys(kp, kc, 2, True)
    kp2 = dict(kp, signs=opack.permute_signs(kp["signs"]))
    _, s_perm, _ = odec.dequant_keys(kp2, kc, 2, True, signs_permuted=True)
    assert np.array_equal(s_nat, s_perm)


@pytest.mark.parametrize("bits,qjl,layout", [(3, True, "keys"), (2, True, "keys"), (4, False, "keys"),
                                             (3, False, "values"), (2, False, "values"), (4, False, "values"),
                                             (3, True, "rows")])
@pytest.mark.parametrize("bs", [16, 32])
def test_tiles_to_tokens_matches_per_token_gather(bits, qjl, layout, bs):
    """The vectorised tile reader (a permutation derived from build_subtile) equals the per-token,
    chunk-by-chunk gather_sequence on random caches."""
    rng = np.random.default_rng(bits * 10 + bs + int(qjl))
    tb = opaged.tile_offsets(bs, bits, qjl)[4]
    cache = rng.integers(0, 256, (6, 2, tb), dtype=np.uint8)
    bt = np.array([3, 1, 4, 0, 2])
    L = bs * 5 - 3
    for h in range(2):
        slow = opaged.gather_sequence(cache, bt, L, h, bs, bits, qjl, layout)
        fast = opaged.tiles_to_tokens(cache[bt, h], bs, bits, qjl, layout)
        for k in slow:
            np.testing.assert_array_equal(slow[k], fast[k][:L])


def test_sparse_v_margins_decide_like_decode_chunked():
    """A token is dropped by decode_chunked exactly when its margin is <= log(threshold)."""
    rng = np.random.default_rng(5)
    G, L = 6, 300
    q = rng.standard_normal((G, 128)) * 8
    k = rng.standard_normal((L, 128))
    v = rng.standard_normal((L, 128))
    for thr in (1e-4, 1e-2):
        _, sk, _ = odec.decode_chunked(q, None, k, None, None, v, 0.1, 0.0, 96, thr)
        m = odec.sparse_v_margins(q, None, k, None, None, 0.1, 0.0, 96)
        assert sk == int((m <= math.log(thr)).sum()) and sk > 0


@pytest.mark.parametrize("kb,kq,vb", [(3, True, 3), (2, True, 2), (4, False, 4)])
def test_torch_reference_path_matches_oracle(kb, kq, vb):
    """oracle/torch_ref.py (the fp32 torch formulation bench.py times as the CPU baseline) against
    the float64 numpy oracle: dequantisation exact, outputs and Sparse-V skip counts equal (run in
    float64), and within 1e-5 in float32."""
    from oracle import torch_ref
    rng = np.random.default_rng(kb * 3 + vb)
    L, G, bs = 700, 6, 16
    kp = {"idx": rng.integers(0, 256, (L, 16 * kb), dtype=np.uint8),
          "norm": (rng.uniform(5, 15, L)).astype(np.float16).view(np.uint16)}
    if kq:
        kp["signs"] = rng.integers(0, 256, (L, 16), dtype=np.uint8)
        kp["rnorm"] = (rng.uniform(0, 3, L)).astype(np.float16).view(np.uint16)
    vp = {"idx": rng.integers(0, 256, (L, 16 * vb), dtype=np.uint8),
          "norm": (rng.uniform(5, 15, L)).astype(np.float16).view(np.uint16)}
    kc = (np.sort(rng.standard_normal(2 ** kb)) * 0.1).astype(np.float32).astype(np.float64)
    vc = (np.sort(rng.standard_normal(2 ** vb)) * 0.1).astype(np.float32).astype(np.float64)
    k, sg, rn = odec.dequant_keys(kp, kc, kb, kq)
    v = odec.dequant_values(vp, vc, vb)
    tp = lambda pl: {n: torch.from_numpy(a.copy().view(np.uint8).reshape(L, -1)) for n, a in pl.items()}  # noqa: E731
    tk, tsg, trn = torch_ref.dequant(tp(kp), torch.from_numpy(kc), kb, kq)
    tv, _, _ = torch_ref.dequant(tp(vp), torch.from_numpy(vc), vb, False)
    np.testing.assert_array_equal(tk.double().numpy(), k.astype(np.float32).astype(np.float64))
    np.testing.assert_array_equal(tv.double().numpy(), v.astype(np.float32).astype(np.float64))
    if kq:
        np.testing.assert_array_equal(tsg.numpy(), sg)
    q = rng.standard_normal((G, 128)) * 4
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    for chunk, thr in ((None, 0.0), (256, 1e-4), (96, 1e-2)):
        want, sk, _ = odec.decode_chunked(q, q, k, sg, rn, v, sm, cs, chunk or L, thr)
        t64 = lambda a: None if a is None else torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
        got, tsk = torch_ref.decode(t64(q), t64(q), t64(k), t64(sg), t64(rn), t64(v), sm, cs, chunk, thr)
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)
        assert tsk == sk
        got32, _ = torch_ref.decode(torch.from_numpy(q).float(), torch.from_numpy(q).float(), tk,
                                    tsg, trn, tv, sm, cs, chunk, thr)
        np.testing.assert_allclose(got32.double().numpy(), want, rtol=1e-4, atol=1e-5)
