"""GPU parity: decode attention kernels vs the float64 CPU oracle.

Bar (the path's parity target): attention outputs within rtol 1e-2 / atol 1e-3 of the reference
path (attention_unpacked_ref semantics with the correct split combine).  The kernel computes
Q and the dequantized K/V in fp16 with fp32 accumulation.
"""

import math

import numpy as np
import pytest
import torch

from oracle import decode as odec
from oracle import packing as opack
from oracle import paged as opaged

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _cb(bits):
    from turboquant.core import make_codebook
    return make_codebook(128, bits)[0]


def random_payload(rng, n, bits, qjl, norm_scale=10.0):
    pl = {"idx": rng.integers(0, 256, size=(n, 16 * bits), dtype=np.uint8),
          "norm": (rng.uniform(0.5, 1.5, size=n) * norm_scale).astype(np.float16).view(np.uint16)}
    if qjl:
        pl["signs"] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
        pl["rnorm"] = (rng.uniform(0.0, 0.3, size=n) * norm_scale).astype(np.float16).view(np.uint16)
    return pl


def build_case(seed, S, Hq, Hkv, seq_lens, kb, kq, vb, bs, extra_blocks=3, layouts=("keys", "values")):
    rng = np.random.default_rng(seed)
    maxb = max(1, max(math.ceil(L / bs) for L in seq_lens))
    nb = S * maxb + extra_blocks
    perm = rng.permutation(nb)
    bt = np.full((S, maxb), -1, dtype=np.int32)
    k_cache = np.zeros((nb, Hkv, opaged.tile_offsets(bs, kb, kq)[4]), np.uint8)
    v_cache = np.zeros((nb, Hkv, opaged.tile_offsets(bs, vb, False)[4]), np.uint8)
    k_tok, v_tok = {}, {}
    nxt = 0
    for s, L in enumerate(seq_lens):
        nbl = math.ceil(L / bs)
        bt[s, :nbl] = perm[nxt:nxt + nbl]
        nxt += nbl
        slots = np.array([bt[s, t // bs] * bs + t % bs for t in range(L)], dtype=np.int64)
        kp = random_payload(rng, L * Hkv, kb, kq)
        vp = random_payload(rng, L * Hkv, vb, False)
        kp3 = {k: v.reshape(L, Hkv, *v.shape[1:]) for k, v in kp.items()}
        vp3 = {k: v.reshape(L, Hkv, *v.shape[1:]) for k, v in vp.items()}
        opaged.scatter_tokens(kp3, slots, nb, Hkv, bs, kb, kq, k_cache, layout=layouts[0])
        opaged.scatter_tokens(vp3, slots, nb, Hkv, bs, vb, False, v_cache, layout=layouts[1])
        k_tok[s], v_tok[s] = kp3, vp3
    q = rng.standard_normal((S, Hq, 128)).astype(np.float32)
    return dict(q=q, bt=bt, nb=nb, k_cache=k_cache, v_cache=v_cache, k_tok=k_tok, v_tok=v_tok,
                seq_lens=np.array(seq_lens, np.int32), layouts=layouts)


def oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, qp=None, chunk=None, thresh=0.0, q_round=None, tile=16,
               margins=None):
    """Oracle outputs (and Sparse-V skip totals) of a case; margins: a list that receives, per
    (sequence, KV head), the tokens' keep margins (oracle.decode.sparse_v_margins)."""
    G = Hq // Hkv
    kc, vc = _cb(kb).double().numpy(), _cb(vb).double().numpy()
    S = len(case["seq_lens"])
    out = np.zeros((S, Hq, 128))
    skipped = total = 0
    q = case["q"].astype(np.float64) if q_round is None else q_round
    qpv = q if qp is None else qp
    for s in range(S):
        L = int(case["seq_lens"][s])
        for kh in range(Hkv):
            kp = {k: v[:, kh] for k, v in case["k_tok"][s].items()} if L else None
            vp = {k: v[:, kh] for k, v in case["v_tok"][s].items()} if L else None
            hs = slice(kh * G, (kh + 1) * G)
            if L == 0:
                continue
            k, sg, rn = odec.dequant_keys(kp, kc, kb, kq)
            v = odec.dequant_values(vp, vc, vb)
            if chunk is None:
                out[s, hs] = odec.decode_dense(q[s, hs], qpv[s, hs], k, sg, rn, v, sm, cs)
            else:
                ch = chunk[(s, kh)] if isinstance(chunk, dict) else chunk   # dict: per-segment pieces
                o, sk, tt = odec.decode_chunked(q[s, hs], qpv[s, hs], k, sg, rn, v, sm, cs, ch, thresh, tile=tile)
                if margins is not None:
                    margins.append(odec.sparse_v_margins(q[s, hs], qpv[s, hs], k, sg, rn, sm, cs, ch, tile=tile))
                out[s, hs] = o
                skipped += sk
                total += tt
    return out, skipped, total


def run_gpu(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, dtype=torch.bfloat16, chunk=None, thresh=0.0, stats=False,
            share_codebook=False):
    from turboquant.kernels.paged import PagedKVFormat, decode_paged
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs, layout=case["layouts"][0])
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout=case["layouts"][1])
    q = torch.from_numpy(case["q"]).to(dtype).to(dev)
    st = torch.zeros(2, dtype=torch.int64, device=dev) if stats else None
    kc = _cb(kb).to(dev)
    vc = kc if share_codebook else _cb(vb).to(dev)
    out = decode_paged(q, torch.from_numpy(case["k_cache"]).to(dev), kf, kc,
                       torch.from_numpy(case["v_cache"]).to(dev), vf, vc,
                       torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                       sm_scale=sm, corr_scale=cs, sparse_threshold=thresh, tokens_per_chunk=chunk, skip_stats=st)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), (st.cpu().numpy() if stats else None), q.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("kb,kq,vb", [(4, False, 4), (3, True, 3), (2, True, 2), (3, False, 3),
                                      (4, True, 2), (2, False, 4), (3, True, 4), (4, False, 3),
                                      (2, True, 3), (3, False, 2), (2, False, 2)])
def test_decode_bit_widths(dev, kb, kq, vb):
    S, Hq, Hkv, bs = 3, 8, 2, 16
    lens = [37, 1, 300]
    case = build_case(11 + kb * 7 + vb, S, Hq, Hkv, lens, kb, kq, vb, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    got, _, qr = run_gpu(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, chunk=64)
    want, _, _ = oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, q_round=qr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,kq", [(2, True), (2, False), (3, True), (4, False)])
def test_decode_shared_codebook(dev, kb, kq):
    """One centroid tensor for K and V (as a serving stack holds it): the kernel builds one
    shared table, or, for 2-bit values, its own V table at the fixed address."""
    S, Hq, Hkv, bs = 3, 12, 2, 16
    lens = [200, 17, 64]
    case = build_case(5 + kb, S, Hq, Hkv, lens, kb, kq, kb, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    got, _, qr = run_gpu(dev, case, Hq, Hkv, kb, kq, kb, bs, sm, cs, chunk=96, share_codebook=True)
    want, _, _ = oracle_out(case, Hq, Hkv, kb, kq, kb, sm, cs, q_round=qr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,kq,vb", [(4, False, 4), (3, True, 3), (2, True, 2), (3, False, 2)])
@pytest.mark.parametrize("layouts", [("rows", "rows"), ("keys", "rows"), ("rows", "values")])
def test_decode_row_major_paged_tiles(dev, kb, kq, vb, layouts):
    """Paged caches with row-major tiles (or one row-major and one lane-grouped) run the general
    kernel; the results match the oracle like the lane-grouped fast path's."""
    S, Hq, Hkv, bs = 3, 8, 2, 16
    lens = [37, 1, 300]
    case = build_case(71 + kb * 5 + vb, S, Hq, Hkv, lens, kb, kq, vb, bs, layouts=layouts)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    got, _, qr = run_gpu(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, chunk=64)
    want, _, _ = oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, q_round=qr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("G", [1, 4, 6, 8, 16])
@pytest.mark.parametrize("bs", [16, 32])
def test_decode_gqa_and_block_size(dev, G, bs):
    Hkv = 2
    Hq = G * Hkv
    lens = [15, 16, 17, 129, 513]
    case = build_case(100 + G * 3 + bs, len(lens), Hq, Hkv, lens, 3, True, 3, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / math.sqrt(128)
    for chunk in (16, 48, None):
        got, _, qr = run_gpu(dev, case, Hq, Hkv, 3, True, 3, bs, sm, cs, chunk=chunk)
        want, _, _ = oracle_out(case, Hq, Hkv, 3, True, 3, sm, cs, q_round=qr)
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_decode_empty_and_fp32_out(dev):
    from turboquant.kernels.paged import PagedKVFormat, decode_paged
    lens = [0, 5]
    case = build_case(5, 2, 4, 1, lens, 4, False, 4, 16)
    case["bt"][0, :] = -1
    got, _, qr = run_gpu(dev, case, 4, 1, 4, False, 4, 16, 0.1, 0.0, dtype=torch.float32)
    assert np.all(got[0] == 0.0)
    want, _, _ = oracle_out(case, 4, 1, 4, False, 4, 0.1, 0.0, q_round=qr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_decode_sparse_v_matches_chunked_oracle(dev):
    S, Hq, Hkv, bs = 2, 12, 2, 16
    lens = [700, 1500]
    case = build_case(77, S, Hq, Hkv, lens, 3, True, 3, bs)
    case["q"] *= 4.0                            # sharper softmax -> many skips
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    vmax = float(_cb(3).abs().max()) * 15.0          # |centroid| * largest payload norm
    for thresh in (1e-4, 1e-2):
        got, st, qr = run_gpu(dev, case, Hq, Hkv, 3, True, 3, bs, sm, cs, chunk=256, thresh=thresh, stats=True)
        want, sk, tot = oracle_out(case, Hq, Hkv, 3, True, 3, sm, cs, chunk=256, thresh=thresh, q_round=qr)
        # A token whose p lies within rounding of the threshold may be skipped on one side only;
        # each such flip moves an output by at most thresh * max|v| (the denominator is >= 1).
        flip_tol = 0.0 if thresh < 1e-3 else 2 * thresh * vmax
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL + flip_tol)
        assert int(st[1]) == tot
        print(f"thresh {thresh}: skipped gpu {int(st[0])} oracle {sk} of {tot}")
        assert abs(int(st[0]) - sk) <= max(3, tot // 200)
        assert sk > 0
    dense, _, qr = run_gpu(dev, case, Hq, Hkv, 3, True, 3, bs, sm, cs, chunk=256, thresh=0.0)
    want_dense, _, _ = oracle_out(case, Hq, Hkv, 3, True, 3, sm, cs, q_round=qr)
    np.testing.assert_allclose(dense, want_dense, rtol=RTOL, atol=ATOL)


def _balanced_pieces(dev, lens, Hq, Hkv, kb, kq, vb, max_blocks, bs, share=False):
    """The pieces tq_decode's balanced schedule cuts, from the device's resident waves."""
    from turboquant.kernels.paged import balanced_partition, concurrent_units
    R = max(4, concurrent_units(dev, kb, kq, vb, Hq, Hkv, 2, share))
    return balanced_partition(lens, Hkv, R, max_blocks * bs)


@pytest.mark.parametrize("scale", ["short", "long"])
@pytest.mark.parametrize("kb,kq,vb,G,bs", [(3, True, 3, 6, 16), (2, True, 2, 8, 16), (4, False, 4, 4, 32),
                                           (3, False, 2, 1, 64), (2, False, 4, 3, 16)])
def test_decode_balanced_many_sequences(dev, kb, kq, vb, G, bs, scale):
    """tokens_per_chunk = 0 (the balanced schedule) over 150 ragged sequences: empty ones, single
    tokens, lengths off the 32-token pairs.  Every wave's scan of seq_lens crosses three
    64-sequence blocks; "short" has fewer pairs than resident waves (one pair per wave, segments
    merged from up to ~50 pieces), "long" more (pieces cross sequences and KV heads)."""
    Hkv = 2
    Hq = G * Hkv
    rng = np.random.default_rng(kb * 10 + vb + G)
    pool = [0, 1, 31, 32, 33, 95, 200, 640, 1500] if scale == "short" else [0, 1, 33, 700, 1999, 4100]
    lens = [int(x) for x in rng.choice(pool, size=150)]
    case = build_case(300 + kb + 7 * vb + G, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    pieces = _balanced_pieces(dev, lens, Hq, Hkv, kb, kq, vb, case["bt"].shape[1], bs)
    print(f"{sum(len(v) for v in pieces.values())} pieces over {len(pieces)} segments", flush=True)
    got, _, qr = run_gpu(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, chunk=0)
    want, _, _ = oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, q_round=qr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    assert np.all(got[np.array(lens) == 0] == 0.0)


def test_decode_balanced_all_empty(dev):
    """No tokens at all: no wave has work, the plan still says so, every output is zero."""
    lens = [0, 0, 0]
    case = build_case(9, 3, 8, 2, [1, 1, 1], 3, True, 3, 16)
    case["seq_lens"] = np.array(lens, np.int32)
    got, _, _ = run_gpu(dev, case, 8, 2, 3, True, 3, 16, 0.1, 0.0, chunk=0)
    assert np.all(got == 0.0)


@pytest.mark.parametrize("bs", [16, 32])
def test_decode_balanced_sparse_v_pieces(dev, bs):
    """Sparse-V under the balanced schedule: the kernel's pieces (balanced_partition with the
    device's resident waves) are the chunks the oracle walks; outputs agree and skip counts agree
    up to the tokens within rounding of the threshold."""
    S, Hq, Hkv = 5, 12, 2
    lens = [4000, 9000, 3, 2500, 6000]
    case = build_case(61 + bs, S, Hq, Hkv, lens, 3, True, 3, bs)
    case["q"] *= 4.0
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    pieces = _balanced_pieces(dev, lens, Hq, Hkv, 3, True, 3, case["bt"].shape[1], bs)
    thresh = 1e-4
    got, st, qr = run_gpu(dev, case, Hq, Hkv, 3, True, 3, bs, sm, cs, chunk=0, thresh=thresh, stats=True)
    margins = []
    want, sk, tot = oracle_out(case, Hq, Hkv, 3, True, 3, sm, cs, chunk=pieces, thresh=thresh, q_round=qr,
                               tile=32 if bs >= 32 else 16, margins=margins)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    allow = _skip_allowance(margins, thresh)
    print(f"balanced Sparse-V: skipped gpu {int(st[0])} oracle {sk} of {tot} (within rounding {allow})")
    assert int(st[1]) == tot and sk > 0
    assert abs(int(st[0]) - sk) <= allow


def test_decode_workspace_reuse(dev):
    """One workspace across repeated and differently shaped calls (split into several chunks,
    one chunk, and empty sequences) keeps matching the oracle."""
    from turboquant import _lib
    from turboquant.kernels.paged import PagedKVFormat, decode_paged

    ws = torch.full((1 << 22,), 0x7f, dtype=torch.uint8, device=dev)  # stale contents do not matter
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    for rep, (lens, chunk) in enumerate([([300, 17, 64], 32), ([300, 17, 64], 32), ([1000, 0, 5, 77], 48)]):
        S, Hq, Hkv = len(lens), 8, 2
        case = build_case(40 + rep, S, Hq, Hkv, lens, 3, True, 3, 16)
        kf, vf = PagedKVFormat(bits=3, qjl=True), PagedKVFormat(bits=3, layout="values")
        cb = _cb(3).to(dev)
        q = torch.from_numpy(case["q"]).to(torch.bfloat16).to(dev)
        msl = max(lens)
        out = decode_paged(q, torch.from_numpy(case["k_cache"]).to(dev), kf, cb,
                           torch.from_numpy(case["v_cache"]).to(dev), vf, cb,
                           torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                           sm_scale=sm, corr_scale=cs, max_seq_len=msl, tokens_per_chunk=chunk, workspace=ws)
        torch.cuda.synchronize()
        qr = q.float().cpu().numpy().astype(np.float64)
        want, _, _ = oracle_out(case, Hq, Hkv, 3, True, 3, sm, cs, q_round=qr)
        np.testing.assert_allclose(out.float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)
        assert _lib.lib().tq_decode_workspace_bytes(S, Hq, msl, chunk) <= ws.numel()


def test_decode_bad_block_entries_are_skipped(dev):
    """Block-table entries outside [0, num_blocks) are ignored instead of read."""
    lens = [40]
    case = build_case(9, 1, 2, 1, lens, 4, False, 4, 16)
    bt = case["bt"].copy()
    bt[0, 1] = case["nb"] + 100            # second block (tokens 16..31) unreadable
    case2 = dict(case, bt=bt)
    got, _, qr = run_gpu(dev, case2, 2, 1, 4, False, 4, 16, 0.1, 0.0, chunk=16)
    keep = {k: np.concatenate([v[:16], v[32:40]]) for k, v in case["k_tok"][0].items()}
    keepv = {k: np.concatenate([v[:16], v[32:40]]) for k, v in case["v_tok"][0].items()}
    k, _, _ = odec.dequant_keys({k: v[:, 0] for k, v in keep.items()}, _cb(4).double().numpy(), 4, False)
    v = odec.dequant_values({k: v[:, 0] for k, v in keepv.items()}, _cb(4).double().numpy(), 4)
    want = odec.decode_dense(qr[0], None, k, None, None, v, 0.1, 0.0)
    np.testing.assert_allclose(got[0], want, rtol=RTOL, atol=ATOL)


def test_packed_attention_v7_api(dev):
    """packed_attention against the fp64 oracle and against the product's attention_unpacked_ref
    (kernels/packed_attention.py:273-284 of the reference) on the same unpacked data."""
    from turboquant.kernels.packed_attention import attention_unpacked_ref, packed_attention
    from turboquant.kernels.packed_compress import permute_signs_for_chunked
    rng = np.random.default_rng(3)
    cb = _cb(2)
    cs = math.sqrt(math.pi / 2) / math.sqrt(128)
    # num_splits 100 and 256 give 94 and 256 chunks per head: the merge's 8- and 16-wave forms
    for BH, Sk, splits in [(8, 1, None), (4, 100, None), (3, 4097, None), (2, 4096, None), (5, 2048, 7),
                           (3, 3000, 100), (2, 4096, 256)]:
        ki = rng.integers(0, 256, (BH, Sk, 32), dtype=np.uint8)
        ks = rng.integers(0, 256, (BH, Sk, 16), dtype=np.uint8)
        vi = rng.integers(0, 256, (BH, Sk, 32), dtype=np.uint8)
        kr = (rng.random((BH, Sk)) * 0.1).astype(np.float16)
        kn = (rng.random((BH, Sk)) + 0.5).astype(np.float16)
        vn = (rng.random((BH, Sk)) + 0.5).astype(np.float16)
        Q = (rng.standard_normal((BH, 128)) * 0.1).astype(np.float16)
        Qp = (rng.standard_normal((BH, 128)) * 0.1).astype(np.float16)
        t = lambda a: torch.from_numpy(a).to(dev)
        ks_perm = permute_signs_for_chunked(t(ks), 128)
        out = packed_attention(t(Q), t(Qp), t(ki), ks_perm, t(kr), t(kn), t(vi), t(vn), cb.to(dev), cs,
                               num_splits=splits)
        assert out.dtype == torch.float16 and out.shape == (BH, 128)
        got = out.float().cpu().numpy()
        for h in range(BH):
            k, sg, rn = odec.dequant_keys({"idx": ki[h], "norm": kn[h].view(np.uint16), "signs": ks[h],
                                           "rnorm": kr[h].view(np.uint16)}, cb.double().numpy(), 2, True)
            v = odec.dequant_values({"idx": vi[h], "norm": vn[h].view(np.uint16)}, cb.double().numpy(), 2)
            want = odec.decode_dense(Q[h:h + 1].astype(np.float64), Qp[h:h + 1].astype(np.float64), k, sg, rn, v, 1.0, cs)
            np.testing.assert_allclose(got[h], want[0], rtol=RTOL, atol=ATOL)
            # the product's unpacked formulation on the GPU (fp32 torch ops) on the same data
            f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).float().to(dev)[None]  # noqa: E731
            ref = attention_unpacked_ref(f(Q[h]), f(Qp[h]), f(k), f(sg), f(rn), f(v), cs)
            np.testing.assert_allclose(ref[0].cpu().numpy(), want[0], rtol=1e-4, atol=1e-5)
            np.testing.assert_allclose(got[h], ref[0].cpu().numpy(), rtol=RTOL, atol=ATOL)


def test_packed_attention_c_entry_dtypes(dev):
    """tq_packed_attention called through the C-ABI with bf16 / fp32 queries and fp32 / bf16
    output, natural or permuted sign rows, fixed and library-chosen chunks, against the fp64
    oracle (the Python packed_attention always passes fp16 in and out)."""
    from turboquant import _lib
    from turboquant.kernels.paged import decode_workspace
    rng = np.random.default_rng(17)
    cb = _cb(2).to(dev)
    cs = math.sqrt(math.pi / 2) / math.sqrt(128)
    L = _lib.lib()
    for BH, Sk, qdt, odt, perm, chunk in [(6, 1000, torch.bfloat16, torch.float32, True, 0),
                                          (3, 2048, torch.float32, torch.bfloat16, False, 256),
                                          (5, 37, torch.float16, torch.float32, True, 16)]:
        ki = rng.integers(0, 256, (BH, Sk, 32), dtype=np.uint8)
        ks = rng.integers(0, 256, (BH, Sk, 16), dtype=np.uint8)
        vi = rng.integers(0, 256, (BH, Sk, 32), dtype=np.uint8)
        kr = (rng.random((BH, Sk)) * 0.1).astype(np.float16)
        kn = (rng.random((BH, Sk)) + 0.5).astype(np.float16)
        vn = (rng.random((BH, Sk)) + 0.5).astype(np.float16)
        Q = (rng.standard_normal((BH, 128)) * 0.1).astype(np.float32)
        Qp = (rng.standard_normal((BH, 128)) * 0.1).astype(np.float32)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        ks_dev = opack.permute_signs(ks.reshape(-1, 16)).reshape(ks.shape) if perm else ks
        q, qp = t(Q).to(qdt), t(Qp).to(qdt)
        arrs = [t(ki), t(ks_dev), t(kr), t(kn), t(vi), t(vn)]
        out = torch.full((BH, 128), float("nan"), dtype=odt, device=dev)
        ws = decode_workspace(dev, L.tq_packed_attention_workspace_bytes(BH, Sk, chunk))
        rc = L.tq_packed_attention(q.data_ptr(), qp.data_ptr(), _lib.dtype_code(q), arrs[0].data_ptr(), arrs[1].data_ptr(),
                                   1 if perm else 0, arrs[2].data_ptr(), arrs[3].data_ptr(), arrs[4].data_ptr(),
                                   arrs[5].data_ptr(), cb.data_ptr(), _lib.centroid_scale(cb), cs, BH, Sk, chunk,
                                   ws.data_ptr(), ws.numel(), out.data_ptr(), _lib.dtype_code(out), _lib.stream_handle(dev))
        assert rc == 0, _lib.status_string(rc)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        qr = q.float().cpu().numpy().astype(np.float64)
        qpr = qp.float().cpu().numpy().astype(np.float64)
        # bf16 output: the contract tolerance plus the output's own rounding (2^-9 relative)
        tol = dict(rtol=RTOL, atol=ATOL) if odt == torch.float32 else dict(rtol=RTOL + 2.0 ** -8, atol=ATOL)
        for h in range(BH):
            k, sg, rn = odec.dequant_keys({"idx": ki[h], "norm": kn[h].view(np.uint16), "signs": ks[h],
                                           "rnorm": kr[h].view(np.uint16)}, cb.double().cpu().numpy(), 2, True)
            v = odec.dequant_values({"idx": vi[h], "norm": vn[h].view(np.uint16)}, cb.double().cpu().numpy(), 2)
            want = odec.decode_dense(qr[h:h + 1], qpr[h:h + 1], k, sg, rn, v, 1.0, cs)
            np.testing.assert_allclose(got[h], want[0], err_msg=f"BH {BH} Sk {Sk} head {h}", **tol)


@pytest.mark.parametrize("perm", [True, False])
@pytest.mark.parametrize("S,Sk,hkv,G,chunk", [(8, 256, 1, 1, 0), (3, 4096, 2, 6, 0), (2, 16, 1, 1, 0),
                                              (5, 1024, 1, 3, 512), (4, 2048, 2, 8, 96), (3, 1024, 1, 2, 16)])
def test_decode_row_major_arrays(dev, perm, S, Sk, hkv, G, chunk):
    """The row-major per-sequence arrays of the v7 layout (2-bit keys with QJL, 2-bit values, no
    block tables; Sk a multiple of 16) through tq_decode's contiguous kernel, against the fp64
    oracle: sign rows in natural or stride-4 permuted order, GQA groups 1-8, several KV heads,
    sequence lengths ending inside a tile, a sequence of length 0, fixed and library-chosen
    chunks (up to 64 per sequence: the merge's four-wave form)."""
    from turboquant import _lib
    from turboquant.kernels.paged import run_decode
    rng = np.random.default_rng(1000 + Sk + 7 * G + perm)
    cb = _cb(2)
    cs = math.sqrt(math.pi / 2) / math.sqrt(128)
    Hq = hkv * G
    ki = rng.integers(0, 256, (S, hkv, Sk, 32), dtype=np.uint8)
    ks = rng.integers(0, 256, (S, hkv, Sk, 16), dtype=np.uint8)
    vi = rng.integers(0, 256, (S, hkv, Sk, 32), dtype=np.uint8)
    kr = (rng.random((S, hkv, Sk)) * 0.1).astype(np.float16)
    kn = (rng.random((S, hkv, Sk)) + 0.5).astype(np.float16)
    vn = (rng.random((S, hkv, Sk)) + 0.5).astype(np.float16)
    q = (rng.standard_normal((S, Hq, 128)) * 0.3).astype(np.float16)
    qp = (rng.standard_normal((S, Hq, 128)) * 0.3).astype(np.float16)
    lens = np.array([Sk, max(Sk - 5, 1), 0, 17, Sk - 16, 3, Sk, Sk // 2 + 1][:S], dtype=np.int32)
    ks_dev = opack.permute_signs(ks.reshape(-1, 16)).reshape(ks.shape) if perm else ks
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    arrs = {"ki": t(ki), "ks": t(ks_dev), "kr": t(kr), "kn": t(kn), "vi": t(vi), "vn": t(vn)}

    def region(x, row):
        return _lib.TQRegion(x.data_ptr(), 16 * row, Sk * row, hkv * Sk * row, row)

    kv = _lib.TQKVView()
    kv.idx, kv.signs, kv.norm, kv.rnorm = region(arrs["ki"], 32), region(arrs["ks"], 16), region(arrs["kn"], 2), \
        region(arrs["kr"], 2)
    cbd = cb.to(dev)
    kv.centroids = cbd.data_ptr()
    kv.bits, kv.qjl, kv.signs_permuted = 2, 1, 1 if perm else 0
    kv.centroid_scale = _lib.centroid_scale(cbd)
    vv = _lib.TQKVView()
    vv.idx, vv.norm = region(arrs["vi"], 32), region(arrs["vn"], 2)
    vv.centroids = cbd.data_ptr()
    vv.bits, vv.qjl, vv.signs_permuted = 2, 0, 0
    vv.centroid_scale = kv.centroid_scale
    out = torch.full((S, Hq, 128), float("nan"), dtype=torch.float16, device=dev)
    sm = 1 / math.sqrt(128)
    run_decode(t(q), kv, vv, num_kv_heads=hkv, block_size=16, num_blocks=Sk // 16, block_tables=None,
               max_blocks_per_seq=Sk // 16, seq_lens=t(lens), max_seq_len=Sk, sm_scale=sm, corr_scale=cs,
               q_proj=t(qp), sparse_threshold=0.0, tokens_per_chunk=chunk, out=out, workspace=None,
               skip_stats=None, keep_alive=(cbd, arrs))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for s in range(S):
        L = int(lens[s])
        for kh in range(hkv):
            hs = slice(kh * G, (kh + 1) * G)
            if L == 0:
                assert np.all(got[s, hs] == 0), "an empty sequence decodes to zeros"
                continue
            k, sg, rn = odec.dequant_keys({"idx": ki[s, kh, :L], "norm": kn[s, kh, :L].view(np.uint16),
                                           "signs": ks[s, kh, :L], "rnorm": kr[s, kh, :L].view(np.uint16)},
                                          cb.double().numpy(), 2, True)
            v = odec.dequant_values({"idx": vi[s, kh, :L], "norm": vn[s, kh, :L].view(np.uint16)},
                                    cb.double().numpy(), 2)
            want = odec.decode_dense(q[s, hs].astype(np.float64), qp[s, hs].astype(np.float64), k, sg, rn, v, sm, cs)
            np.testing.assert_allclose(got[s, hs], want, rtol=RTOL, atol=ATOL, err_msg=f"seq {s} head {kh}")


@pytest.mark.parametrize("layouts,kb,kq,vb,chunk", [(("keys", "values"), 3, True, 3, 64),
                                                    (("keys", "values"), 2, True, 2, 0),
                                                    (("rows", "rows"), 4, False, 4, 48)])
def test_decode_null_seq_lens(dev, layouts, kb, kq, vb, chunk):
    """seq_lens NULL means every sequence is max_seq_len tokens long: the same bits as a length
    array of max_seq_len for every sequence, in the lane-grouped fast kernel, the general kernel
    (row-major tiles) and the split-K merge; and the oracle's answer."""
    from turboquant.kernels.paged import PagedKVFormat, paged_view, run_decode
    S, Hq, Hkv, bs, L = 3, 8, 2, 16, 300
    case = build_case(90 + kb, S, Hq, Hkv, [L] * S, kb, kq, vb, bs, layouts=layouts)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs, layout=layouts[0])
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout=layouts[1])
    kc, vc = _cb(kb).to(dev), _cb(vb).to(dev)
    kcache, vcache = torch.from_numpy(case["k_cache"]).to(dev), torch.from_numpy(case["v_cache"]).to(dev)
    bt = torch.from_numpy(case["bt"]).to(dev)
    q = torch.from_numpy(case["q"]).to(torch.bfloat16).to(dev)
    outs = []
    for lens in (torch.from_numpy(case["seq_lens"]).to(dev), None):
        out = torch.full((S, Hq, 128), float("nan"), dtype=torch.bfloat16, device=dev)
        run_decode(q, paged_view(kcache, kf, kc), paged_view(vcache, vf, vc), num_kv_heads=Hkv, block_size=bs,
                   num_blocks=kcache.shape[0], block_tables=bt, max_blocks_per_seq=bt.shape[1], seq_lens=lens,
                   max_seq_len=L, sm_scale=sm, corr_scale=cs, q_proj=None, sparse_threshold=0.0,
                   tokens_per_chunk=chunk, out=out, workspace=None, skip_stats=None, keep_alive=(kc, vc))
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    want, _, _ = oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, q_round=q.float().cpu().numpy().astype(np.float64))
    np.testing.assert_allclose(outs[1], want, rtol=RTOL, atol=ATOL)


def _skip_allowance(margins, thresh, delta=2e-3):
    """Tokens whose keep margin lies within delta (natural-log units, well above the kernels'
    score rounding) of log(threshold): either decision is within rounding."""
    return int(sum((np.abs(m - math.log(thresh)) < delta).sum() for m in margins))


def test_sparse_v_reference_slot_layout(dev):
    """tq_v11 / tq_v12_sparse_v read the reference's [NB, 2, BS, Hkv, 128] slot cache in place
    (block 32, GQA 6, the reference's own benchmark shape, kernels/sparse_v.py:270-274).  Dense
    against the oracle; Sparse-V (T = 1e-6, the reference's threshold) against the oracle's
    chunk walk with the running max updated once per 32-token KV block, outputs at the contract
    tolerance and skip counts equal up to the tokens within rounding of the threshold."""
    from turboquant.kernels.sparse_v import tq_v11, tq_v12_sparse_v
    rng = np.random.default_rng(8)
    Hkv, G, bs, S = 4, 6, 32, 3
    Hq = Hkv * G
    lens = [100, 1024, 33]
    maxb = max(math.ceil(L / bs) for L in lens)
    nb = S * maxb + 2
    cache = rng.integers(0, 256, (nb, 2, bs, Hkv, 128), dtype=np.uint8)
    norms = (rng.uniform(5, 15, (nb, 2, bs, Hkv))).astype(np.float16)
    cache[..., 48:50] = norms.view(np.uint8).reshape(nb, 2, bs, Hkv, 2)
    bt = rng.permutation(nb)[: S * maxb].reshape(S, maxb).astype(np.int32)
    q = (rng.standard_normal((S, Hq, 128)) * 6).astype(np.float16)
    cent = _cb(3)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    sm = 1 / math.sqrt(128)
    chunk, thresh = 256, 1e-6
    out11 = torch.empty((S, Hq, 128), dtype=torch.float16, device=dev)
    out12 = torch.empty_like(out11)
    st = torch.zeros(2, dtype=torch.int64, device=dev)
    tq_v11(out11, t(q), t(cache), cent.to(dev), t(bt), t(np.array(lens, np.int32)), sm, tokens_per_chunk=chunk)
    tq_v12_sparse_v(out12, t(q), t(cache), cent.to(dev), t(bt), t(np.array(lens, np.int32)), sm, thresh,
                    tokens_per_chunk=chunk, skip_stats=st)
    torch.cuda.synchronize()
    skipped = total = 0
    margins = []
    for s, L in enumerate(lens):
        for kh in range(Hkv):
            blks = bt[s, np.arange(L) // bs]
            rows = np.arange(L) % bs
            ksl = cache[blks, 0, rows, kh]
            vsl = cache[blks, 1, rows, kh]
            kp = {"idx": ksl[:, :48], "norm": ksl[:, 48:50].copy().view(np.uint16).reshape(-1)}
            vp = {"idx": vsl[:, :48], "norm": vsl[:, 48:50].copy().view(np.uint16).reshape(-1)}
            k, _, _ = odec.dequant_keys(kp, cent.double().numpy(), 3, False)
            v = odec.dequant_values(vp, cent.double().numpy(), 3)
            hs = slice(kh * G, (kh + 1) * G)
            qs = q[s, hs].astype(np.float64)
            want = odec.decode_dense(qs, None, k, None, None, v, sm, 0.0)
            np.testing.assert_allclose(out11[s, hs].float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)
            want12, sk, tot = odec.decode_chunked(qs, None, k, None, None, v, sm, 0.0, chunk, thresh, tile=32)
            margins.append(odec.sparse_v_margins(qs, None, k, None, None, sm, 0.0, chunk, tile=32))
            np.testing.assert_allclose(out12[s, hs].float().cpu().numpy(), want12, rtol=RTOL, atol=ATOL)
            skipped += sk
            total += tot
    gsk, gtot = st.tolist()
    allow = _skip_allowance(margins, thresh)
    print(f"tq_v12_sparse_v: skipped gpu {gsk} oracle {skipped} of {total} (within rounding {allow})")
    assert gtot == total and skipped > 0
    assert abs(gsk - skipped) <= allow


@pytest.mark.parametrize("bs", [16, 32])
def test_sparse_v_default_is_the_reference_single_pass(dev, bs):
    """tq_v12_sparse_v without tokens_per_chunk walks each (sequence, KV head) in one pass, as
    the reference's grid does: against decode_chunked(chunk = whole sequence, tile = the KV
    block), outputs at the contract tolerance and skip counts equal up to the tokens within
    rounding of the threshold; and it differs from a split-K chunking of the same data in which
    tokens it skips."""
    from turboquant.kernels.sparse_v import tq_v12_sparse_v
    rng = np.random.default_rng(80 + bs)
    Hkv, G, S = 2, 6, 3
    Hq = Hkv * G
    lens = [1500, 700, 2100]
    maxb = max(math.ceil(L / bs) for L in lens)
    nb = S * maxb + 2
    cache = rng.integers(0, 256, (nb, 2, bs, Hkv, 128), dtype=np.uint8)
    norms = (rng.uniform(5, 15, (nb, 2, bs, Hkv))).astype(np.float16)
    cache[..., 48:50] = norms.view(np.uint8).reshape(nb, 2, bs, Hkv, 2)
    bt = rng.permutation(nb)[: S * maxb].reshape(S, maxb).astype(np.int32)
    q = (rng.standard_normal((S, Hq, 128)) * 6).astype(np.float16)
    cent = _cb(3)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    sm, thresh = 1 / math.sqrt(128), 1e-4
    out = torch.empty((S, Hq, 128), dtype=torch.float16, device=dev)
    st = torch.zeros(2, dtype=torch.int64, device=dev)
    tq_v12_sparse_v(out, t(q), t(cache), cent.to(dev), t(bt), t(np.array(lens, np.int32)), sm, thresh, skip_stats=st)
    out_split = torch.empty_like(out)
    st_split = torch.zeros(2, dtype=torch.int64, device=dev)
    tq_v12_sparse_v(out_split, t(q), t(cache), cent.to(dev), t(bt), t(np.array(lens, np.int32)), sm, thresh,
                    tokens_per_chunk=256, skip_stats=st_split)
    torch.cuda.synchronize()
    skipped = total = 0
    margins = []
    for s, L in enumerate(lens):
        for kh in range(Hkv):
            blks = bt[s, np.arange(L) // bs]
            rows = np.arange(L) % bs
            ksl = cache[blks, 0, rows, kh]
            vsl = cache[blks, 1, rows, kh]
            kp = {"idx": ksl[:, :48], "norm": ksl[:, 48:50].copy().view(np.uint16).reshape(-1)}
            vp = {"idx": vsl[:, :48], "norm": vsl[:, 48:50].copy().view(np.uint16).reshape(-1)}
            k, _, _ = odec.dequant_keys(kp, cent.double().numpy(), 3, False)
            v = odec.dequant_values(vp, cent.double().numpy(), 3)
            hs = slice(kh * G, (kh + 1) * G)
            qs = q[s, hs].astype(np.float64)
            want, sk, tot = odec.decode_chunked(qs, None, k, None, None, v, sm, 0.0, L, thresh, tile=bs)
            margins.append(odec.sparse_v_margins(qs, None, k, None, None, sm, 0.0, L, tile=bs))
            np.testing.assert_allclose(out[s, hs].float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)
            skipped += sk
            total += tot
    gsk, gtot = st.tolist()
    allow = _skip_allowance(margins, thresh)
    print(f"single pass: skipped gpu {gsk} oracle {skipped} of {total} (within rounding {allow}); "
          f"split-K 256 skipped {st_split.tolist()[0]}")
    assert gtot == total and skipped > 0
    assert abs(gsk - skipped) <= allow
    assert st_split.tolist()[0] != gsk


@pytest.mark.parametrize("layouts", [("keys", "values"), ("rows", "rows")])
@pytest.mark.parametrize("chunk", [256, 240])
def test_decode_sparse_v_block32(dev, layouts, chunk):
    """Block size 32 with Sparse-V on the fast (lane-grouped) and general (row-major) kernels:
    the running max the skip test uses is updated once per 32-token KV block; a chunk that is
    not a multiple of 32 is rounded up to one.  Against decode_chunked(tile=32) with skip
    counts."""
    S, Hq, Hkv, bs = 2, 12, 2, 32
    lens = [700, 1500]
    case = build_case(79, S, Hq, Hkv, lens, 3, True, 3, bs, layouts=layouts)
    case["q"] *= 4.0
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    eff = chunk + 16 if chunk % 32 else chunk
    for thresh in (1e-4, 1e-2):
        got, st, qr = run_gpu(dev, case, Hq, Hkv, 3, True, 3, bs, sm, cs, chunk=chunk, thresh=thresh, stats=True)
        margins = []
        want, sk, tot = oracle_out(case, Hq, Hkv, 3, True, 3, sm, cs, chunk=eff, thresh=thresh, q_round=qr, tile=32,
                                   margins=margins)
        vmax = float(_cb(3).abs().max()) * 15.0
        flip_tol = 0.0 if thresh < 1e-3 else 2 * thresh * vmax
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL + flip_tol)
        allow = _skip_allowance(margins, thresh)
        print(f"block 32, chunk {chunk}, thresh {thresh}: skipped gpu {int(st[0])} oracle {sk} of {tot} ({allow})")
        assert int(st[1]) == tot and sk > 0
        assert abs(int(st[0]) - sk) <= allow


def test_decode_constant_values_full_size(dev):
    """Benchmark config 4 shape (B=64, ctx 32768, Hq 48 / Hkv 8): with every V token equal,
    the output equals that vector whatever the scores (size-independent property), dense and
    Sparse-V; plus one sequence checked against the oracle in full."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, decode_paged
    B, Hq, Hkv, ctx, bs = 64, 48, 8, 32768, 16
    kf = PagedKVFormat(bits=3, qjl=True, block_size=bs)
    vf = PagedKVFormat(bits=3, qjl=False, block_size=bs, layout="values")
    nb = B * ctx // bs
    g = torch.Generator(device=dev).manual_seed(4)
    k_cache = torch.randint(0, 256, (nb, Hkv, kf.tile_bytes), dtype=torch.uint8, device=dev, generator=g)
    nrm = (torch.rand((nb, Hkv, bs), device=dev, generator=g) * 10 + 5).half()
    k_cache[:, :, kf.off_norm:kf.off_norm + 2 * bs] = nrm.view(torch.uint8).reshape(nb, Hkv, 2 * bs)
    k_cache[:, :, kf.off_rnorm:kf.off_rnorm + 2 * bs] = (nrm * 0.1).view(torch.uint8).reshape(nb, Hkv, 2 * bs)
    v_cache = allocate_cache(nb, Hkv, vf, device=dev)
    # 3-bit fields all equal to 2 (bits 010): the little-endian stream repeats every 3 bytes
    pattern = torch.tensor([0x92, 0x24, 0x49], dtype=torch.uint8, device=dev)
    v_cache[:, :, : bs * 48] = pattern.repeat(bs * 16)
    v_cache[:, :, vf.off_norm:] = torch.tensor([2.0], dtype=torch.float16).view(torch.uint8).to(dev).repeat(bs)
    bt = torch.randperm(nb, device=dev, generator=g).to(torch.int32).reshape(B, ctx // bs)
    lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    q = torch.randn((B, Hq, 128), device=dev, generator=g).to(torch.bfloat16)
    cb = _cb(3)
    want_val = float(cb[2]) * 2.0
    for thr in (0.0, 1e-4):
        out = decode_paged(q, k_cache, kf, cb.to(dev), v_cache, vf, cb.to(dev), bt, lens,
                           sparse_threshold=thr)
        torch.cuda.synchronize()
        err = (out.float() - want_val).abs().max().item()
        assert err <= ATOL + RTOL * abs(want_val), err
    # sequence 0 in full against the oracle, with random V
    v_cache[:, :, : bs * 48] = torch.randint(0, 256, (nb, Hkv, bs * 48), dtype=torch.uint8, device=dev, generator=g)
    out = decode_paged(q, k_cache, kf, cb.to(dev), v_cache, vf, cb.to(dev), bt, lens)
    torch.cuda.synchronize()
    kc_np, vc_np = k_cache.cpu().numpy(), v_cache.cpu().numpy()
    bt0 = bt[0].cpu().numpy()
    qr = q[0].float().cpu().numpy().astype(np.float64)
    G = Hq // Hkv
    for kh in range(Hkv):
        kp = opaged.gather_sequence(kc_np, bt0, ctx, kh, bs, 3, True, layout="keys")
        vp = opaged.gather_sequence(vc_np, bt0, ctx, kh, bs, 3, False, layout="values")
        k, sg, rn = odec.dequant_keys(kp, cb.double().numpy(), 3, True)
        v = odec.dequant_values(vp, cb.double().numpy(), 3)
        hs = slice(kh * G, (kh + 1) * G)
        want = odec.decode_dense(qr[hs], qr[hs], k, sg, rn, v, 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128)
        np.testing.assert_allclose(out[0, hs].float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,vb", [(3, 3), (2, 2), (4, 4)])
@pytest.mark.parametrize("layouts", [("keys", "values"), ("rows", "rows")])
def test_decode_per_head_query_scales(dev, kb, vb, layouts):
    """Query magnitudes spanning 1e-2 .. 1e2 across the heads of one GQA group (q_proj = q, so
    the QJL operand spans the same range): every head against the fp64 oracle at the contract
    tolerance.  Fast kernel (lane-grouped tiles) and general kernel (row-major tiles)."""
    S, Hkv, G, bs = 2, 2, 8, 16
    Hq = Hkv * G
    case = build_case(620 + kb, S, Hq, Hkv, [300, 77], kb, True, vb, bs, layouts=layouts)
    scales = 10.0 ** np.linspace(-2.0, 2.0, G)
    case["q"] = (case["q"] * scales[np.arange(Hq) % G][None, :, None]).astype(np.float32)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    got, _, qr = run_gpu(dev, case, Hq, Hkv, kb, True, vb, bs, sm, cs, chunk=64)
    want, _, _ = oracle_out(case, Hq, Hkv, kb, True, vb, sm, cs, q_round=qr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,vb", [(3, 3), (2, 2), (4, 4)])
@pytest.mark.parametrize("layouts", [("keys", "values"), ("rows", "rows")])
def test_decode_qjl_small_heads_beside_large(dev, kb, vb, layouts):
    """Explicit q_proj with magnitudes 1e-2 .. 1e2 across one GQA group, the key norms zero so
    the score is the QJL term alone, residual norms ~1e4 so the smallest head (1e-2) gets a
    softmax spread of ~1 log unit: precision its QJL operand would lose to a block scale shared
    with the head 1e4 larger (its elements would fall to the bottom of fp8's range) shows in its
    output.  That head is checked against the fp64 oracle at the contract tolerance; the larger
    ones only share the group: their logits span 4 to 1e4 log units, where the last bits of any
    operand and the oracle's own ties decide the one-hot softmax (every head at realistic logits:
    test_decode_qjl_operand_every_head)."""
    from turboquant.kernels.paged import PagedKVFormat, decode_paged
    S, Hkv, G, bs = 2, 2, 8, 16
    Hq = Hkv * G
    lens = [300, 77]
    case = build_case(600 + kb, S, Hq, Hkv, lens, kb, True, vb, bs, layouts=layouts)
    rng = np.random.default_rng(601 + kb)
    nb = case["nb"]
    _, _, off_norm, off_rnorm, _ = opaged.tile_offsets(bs, kb, True)
    case["k_cache"][:, :, off_norm:off_norm + 2 * bs] = 0
    rn = (rng.uniform(0.5, 1.5, (nb, Hkv, bs)) * 1e4).astype(np.float16)
    case["k_cache"][:, :, off_rnorm:off_rnorm + 2 * bs] = rn.view(np.uint8).reshape(nb, Hkv, 2 * bs)
    for s, L in enumerate(lens):
        t = np.arange(L)
        blk, row = case["bt"][s, t // bs], t % bs
        case["k_tok"][s]["norm"][:] = 0
        case["k_tok"][s]["rnorm"][:] = rn[blk, :, row].view(np.uint16)
    scales = 10.0 ** np.linspace(-2.0, 2.0, G)
    qp = (rng.standard_normal((S, Hq, 128)) * scales[np.arange(Hq) % G][None, :, None]).astype(np.float32)
    kf = PagedKVFormat(bits=kb, qjl=True, block_size=bs, layout=layouts[0])
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout=layouts[1])
    q_t = torch.from_numpy(case["q"]).to(torch.bfloat16).to(dev)
    qp_t = torch.from_numpy(qp).to(torch.bfloat16).to(dev)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    out = decode_paged(q_t, torch.from_numpy(case["k_cache"]).to(dev), kf, _cb(kb).to(dev),
                       torch.from_numpy(case["v_cache"]).to(dev), vf, _cb(vb).to(dev),
                       torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                       sm_scale=sm, corr_scale=cs, q_proj=qp_t, tokens_per_chunk=64)
    torch.cuda.synchronize()
    want, _, _ = oracle_out(case, Hq, Hkv, kb, True, vb, sm, cs,
                            qp=qp_t.float().cpu().numpy().astype(np.float64),
                            q_round=q_t.float().cpu().numpy().astype(np.float64))
    small = np.nonzero(scales[np.arange(Hq) % G] <= 0.011)[0]
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got[:, small], want[:, small], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,vb", [(3, 3), (2, 2), (4, 4)])
@pytest.mark.parametrize("layouts", [("keys", "values"), ("rows", "rows")])
def test_decode_qjl_operand_every_head(dev, kb, vb, layouts):
    """Explicit q_proj whose magnitudes span 1e-2 .. 1e2 across the heads of one GQA group and
    1 .. 64 across the four 32-dim blocks of each head (the blocks of the fast kernel's per-lane
    fp6 scales), the cache's own key and residual norms, N(0,1) queries: logits stay in a
    realistic range, and every head is checked against the fp64 oracle at the contract
    tolerance (the QJL term of the larger heads moves their logits by several log units)."""
    from turboquant.kernels.paged import PagedKVFormat, decode_paged
    S, Hkv, G, bs = 3, 2, 8, 16
    Hq = Hkv * G
    lens = [300, 77, 1000]
    case = build_case(640 + kb, S, Hq, Hkv, lens, kb, True, vb, bs, layouts=layouts)
    rng = np.random.default_rng(641 + kb)
    head_scale = 10.0 ** np.linspace(-2.0, 2.0, G)[np.arange(Hq) % G]
    block_scale = np.repeat(4.0 ** rng.permutation(4), 32) / 8.0  # dims 32b..32b+31 share one scale
    qp = (rng.standard_normal((S, Hq, 128)) * head_scale[None, :, None] * block_scale[None, None, :]).astype(np.float32)
    kf = PagedKVFormat(bits=kb, qjl=True, block_size=bs, layout=layouts[0])
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout=layouts[1])
    q_t = torch.from_numpy(case["q"]).to(torch.bfloat16).to(dev)
    qp_t = torch.from_numpy(qp).to(torch.bfloat16).to(dev)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    for chunk in (64, 0):
        out = decode_paged(q_t, torch.from_numpy(case["k_cache"]).to(dev), kf, _cb(kb).to(dev),
                           torch.from_numpy(case["v_cache"]).to(dev), vf, _cb(vb).to(dev),
                           torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                           sm_scale=sm, corr_scale=cs, q_proj=qp_t, tokens_per_chunk=chunk)
        torch.cuda.synchronize()
        want, _, _ = oracle_out(case, Hq, Hkv, kb, True, vb, sm, cs,
                                qp=qp_t.float().cpu().numpy().astype(np.float64),
                                q_round=q_t.float().cpu().numpy().astype(np.float64))
        got = out.float().cpu().numpy()
        assert np.isfinite(got).all()
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,kq,vb", [(3, True, 3), (4, False, 4), (2, True, 2)])
def test_decode_cache_beyond_2gib(dev, kb, kq, vb):
    """Caches spanning more than 2 GiB (the 64-bit per-tile addressing of the fast kernel): the
    sequences' blocks sit at both ends of a ~3 GiB K cache.  The output equals the same tiles'
    decode from a compact cache bit for bit, and the oracle at the contract tolerance."""
    from turboquant.kernels.paged import PagedKVFormat, allocate_cache, decode_paged
    S, Hkv, G, bs = 3, 2, 6, 16
    Hq = Hkv * G
    lens = [300, 1000, 45]
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout="values")
    nb_big = (3 << 30) // (Hkv * kf.tile_bytes) + 1
    small = build_case(700 + kb, S, Hq, Hkv, lens, kb, kq, vb, bs)
    nbs = small["nb"]
    # compact block b -> big block: the first half near the start, the rest past 2 GiB
    remap = np.where(np.arange(nbs) < nbs // 2, np.arange(nbs), nb_big - nbs + np.arange(nbs))
    assert int(remap.max()) * Hkv * kf.tile_bytes > (2 << 30)
    k_big = allocate_cache(nb_big, Hkv, kf, device=dev)
    v_big = allocate_cache(nb_big, Hkv, vf, device=dev)
    rm = torch.from_numpy(remap).to(dev)
    k_big[rm] = torch.from_numpy(small["k_cache"]).to(dev)
    v_big[rm] = torch.from_numpy(small["v_cache"]).to(dev)
    bt_small = small["bt"]
    bt_big = np.where(bt_small >= 0, remap[np.maximum(bt_small, 0)], -1).astype(np.int32)
    q = torch.from_numpy(small["q"]).to(torch.bfloat16).to(dev)
    lens_t = torch.from_numpy(small["seq_lens"]).to(dev)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    outs = []
    for kc, vc, bt in ((k_big, v_big, bt_big), (torch.from_numpy(small["k_cache"]).to(dev),
                                                   torch.from_numpy(small["v_cache"]).to(dev), bt_small)):
        outs.append(decode_paged(q, kc, kf, _cb(kb).to(dev), vc, vf, _cb(vb).to(dev), torch.from_numpy(bt).to(dev),
                                 lens_t, sm_scale=sm, corr_scale=cs, tokens_per_chunk=128, sparse_threshold=1e-4))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    want, _, _ = oracle_out(small, Hq, Hkv, kb, kq, vb, sm, cs, chunk=128, thresh=1e-4,
                            q_round=q.float().cpu().numpy().astype(np.float64))
    np.testing.assert_allclose(outs[0].float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)
    del k_big, v_big
    torch.cuda.empty_cache()
