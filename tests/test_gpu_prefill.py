"""GPU parity: prefill / extend attention over the packed paged cache (tq_prefill) vs the float64
oracle (oracle.decode.prefill_dense: each query row is a decode over the tokens it sees; pinned
against a masked score tensor in test_oracle.py).  Bar: rtol 1e-2 / atol 1e-3, as decode.
"""

import math

import numpy as np
import pytest
import torch

from oracle import compress as ocomp
from oracle import decode as odec
from test_gpu_decode import ATOL, RTOL, _cb, build_case

pytestmark = pytest.mark.gpu

H64 = ocomp.wht_closed_form(128, 1.0 / math.sqrt(128.0))


def make_queries(rng, n_new, Hq):
    cu = np.zeros(len(n_new) + 1, np.int32)
    cu[1:] = np.cumsum(n_new)
    q = rng.standard_normal((int(cu[-1]), Hq, 128)).astype(np.float32)
    return q, cu


def oracle_prefill(case, q, cu, Hq, Hkv, kb, kq, vb, sm, cs, causal=True, qp=None):
    G = Hq // Hkv
    kc, vc = _cb(kb).double().numpy(), _cb(vb).double().numpy()
    out = np.zeros(q.shape)
    qpv = q if qp is None else qp
    for s in range(len(case["seq_lens"])):
        L = int(case["seq_lens"][s])
        rows = slice(int(cu[s]), int(cu[s + 1]))
        if L == 0 or cu[s + 1] == cu[s]:
            continue
        for kh in range(Hkv):
            kp = {k: v[:, kh] for k, v in case["k_tok"][s].items()}
            vp = {k: v[:, kh] for k, v in case["v_tok"][s].items()}
            k, sg, rn = odec.dequant_keys(kp, kc, kb, kq)
            v = odec.dequant_values(vp, vc, vb)
            hs = slice(kh * G, (kh + 1) * G)
            out[rows, hs] = odec.prefill_dense(q[rows, hs], qpv[rows, hs], k, sg, rn, v, sm, cs, causal=causal)
    return out


def run_prefill(dev, case, q, cu, kb, kq, vb, bs, sm, cs, causal=True, rotate=False, qp=None,
                dtype=torch.bfloat16, out_dtype=None, max_q_len=None):
    from turboquant.kernels.paged import PagedKVFormat, prefill_paged
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs, layout=case["layouts"][0])
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout=case["layouts"][1])
    qt = torch.from_numpy(q).to(dtype).to(dev)
    qpt = torch.from_numpy(qp).to(dtype).to(dev) if qp is not None else None
    out = None
    if out_dtype is not None:
        out = torch.empty(qt.shape, dtype=out_dtype, device=dev)
    out = prefill_paged(qt, torch.from_numpy(cu).to(dev), torch.from_numpy(case["k_cache"]).to(dev), kf,
                        _cb(kb).to(dev), torch.from_numpy(case["v_cache"]).to(dev), vf, _cb(vb).to(dev),
                        torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                        sm_scale=sm, corr_scale=cs, q_proj=qpt, causal=causal, rotate=rotate, out=out,
                        max_q_len=max_q_len)
    torch.cuda.synchronize()
    qr = qt.float().cpu().numpy().astype(np.float64)
    qpr = qpt.float().cpu().numpy().astype(np.float64) if qpt is not None else None
    return out.float().cpu().numpy(), qr, qpr


SM, CS = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128


@pytest.mark.parametrize("kb,kq,vb,G", [(3, True, 3, 6), (4, False, 4, 4), (2, True, 2, 8), (3, True, 4, 1),
                                        (2, False, 3, 3), (4, True, 2, 12)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_bit_widths_and_groups(dev, kb, kq, vb, G, causal):
    Hkv, bs = 2, 16
    Hq = G * Hkv
    lens = [37, 1, 300, 70]
    n_new = [5, 1, 64, 0]
    case = build_case(900 + 5 * kb + vb + G, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    rng = np.random.default_rng(G + kb)
    q, cu = make_queries(rng, n_new, Hq)
    got, qr, _ = run_prefill(dev, case, q, cu, kb, kq, vb, bs, SM, CS, causal=causal)
    want = oracle_prefill(case, qr, cu, Hq, Hkv, kb, kq, vb, SM, CS, causal=causal)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("kb,kq,vb", [(3, True, 3), (2, False, 4)])
def test_prefill_row_major_paged_tiles(dev, kb, kq, vb):
    """Row-major tiles are read as well as the lane-grouped ones."""
    Hq, Hkv, bs = 8, 2, 32
    lens = [100, 37]
    n_new = [20, 37]
    case = build_case(31 + kb, len(lens), Hq, Hkv, lens, kb, kq, vb, bs, layouts=("rows", "rows"))
    rng = np.random.default_rng(kb)
    q, cu = make_queries(rng, n_new, Hq)
    got, qr, _ = run_prefill(dev, case, q, cu, kb, kq, vb, bs, SM, CS)
    want = oracle_prefill(case, qr, cu, Hq, Hkv, kb, kq, vb, SM, CS)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("bs", [32, 64])
def test_prefill_block_sizes_row_blocks_and_short_sequences(dev, bs):
    """Block sizes above 16, sequences whose rows span several 64-row blocks (130 x 6), more new
    tokens than cache tokens (the first rows see nothing: zero), f16 queries, f32 output."""
    kb, kq, vb, Hq, Hkv = 3, True, 3, 12, 2
    lens = [400, 3, 129]
    n_new = [130, 5, 129]
    case = build_case(1234 + bs, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    rng = np.random.default_rng(bs)
    q, cu = make_queries(rng, n_new, Hq)
    got, qr, _ = run_prefill(dev, case, q, cu, kb, kq, vb, bs, SM, CS, dtype=torch.float16,
                             out_dtype=torch.float32, max_q_len=max(n_new))
    want = oracle_prefill(case, qr, cu, Hq, Hkv, kb, kq, vb, SM, CS)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    assert np.all(got[int(cu[1]):int(cu[1]) + 2] == 0.0)


def test_prefill_rotated_and_explicit_q_proj(dev):
    kb, kq, vb, Hq, Hkv, bs = 3, True, 3, 8, 2, 16
    lens = [200, 45]
    n_new = [17, 45]
    case = build_case(77, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    rng = np.random.default_rng(8)
    q, cu = make_queries(rng, n_new, Hq)
    got, qr, _ = run_prefill(dev, case, q, cu, kb, kq, vb, bs, SM, CS, rotate=True)
    want = oracle_prefill(case, qr @ H64, cu, Hq, Hkv, kb, kq, vb, SM, CS) @ H64
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    qp = rng.standard_normal(q.shape).astype(np.float32)
    got, qr, qpr = run_prefill(dev, case, q, cu, kb, kq, vb, bs, SM, CS, qp=qp)
    want = oracle_prefill(case, qr, cu, Hq, Hkv, kb, kq, vb, SM, CS, qp=qpr)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_prefill_bad_block_entries_are_masked(dev):
    """A block-table entry outside [0, num_blocks) removes its tokens from every row."""
    kb, kq, vb, Hq, Hkv, bs = 4, False, 4, 4, 1, 16
    lens = [48]
    case = build_case(19, 1, Hq, Hkv, lens, kb, kq, vb, bs)
    case["bt"][0, 1] = case["nb"] + 5        # tokens 16..31 unreadable
    rng = np.random.default_rng(1)
    q, cu = make_queries(rng, [6], Hq)
    got, qr, _ = run_prefill(dev, case, q, cu, kb, kq, vb, bs, 0.1, 0.0)
    keep = np.r_[0:16, 32:48]
    kc, vc = _cb(kb).double().numpy(), _cb(vb).double().numpy()
    kp = {k: v[keep, 0] for k, v in case["k_tok"][0].items()}
    vp = {k: v[keep, 0] for k, v in case["v_tok"][0].items()}
    k, _, _ = odec.dequant_keys(kp, kc, kb, False)
    v = odec.dequant_values(vp, vc, vb)
    pos_keep = keep
    for i in range(6):
        lim = int(np.searchsorted(pos_keep, 48 - 6 + i, side="right"))
        want = odec.decode_dense(qr[i], None, k[:lim], None, None, v[:lim], 0.1, 0.0)
        np.testing.assert_allclose(got[i], want, rtol=RTOL, atol=ATOL)


def test_prefill_last_row_is_a_decode_step(dev):
    """Full causal prefill of 1000 tokens (G = 6): its last row equals decode_paged of that token on
    the same cache, and sampled rows match the oracle."""
    from turboquant.kernels.paged import PagedKVFormat, decode_paged
    kb, kq, vb, Hq, Hkv, bs = 3, True, 3, 12, 2, 16
    lens = [1000]
    case = build_case(5, 1, Hq, Hkv, lens, kb, kq, vb, bs)
    rng = np.random.default_rng(9)
    q, cu = make_queries(rng, [1000], Hq)
    got, qr, _ = run_prefill(dev, case, q, cu, kb, kq, vb, bs, SM, CS)
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout="values")
    qlast = torch.from_numpy(qr[-1:]).to(torch.bfloat16).to(dev)
    dec = decode_paged(qlast, torch.from_numpy(case["k_cache"]).to(dev), kf, _cb(kb).to(dev),
                       torch.from_numpy(case["v_cache"]).to(dev), vf, _cb(vb).to(dev),
                       torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                       sm_scale=SM, corr_scale=CS, tokens_per_chunk=256)
    np.testing.assert_allclose(got[-1], dec.float().cpu().numpy()[0], rtol=RTOL, atol=ATOL)
    kc, vc = _cb(kb).double().numpy(), _cb(vb).double().numpy()
    G = Hq // Hkv
    for kh in range(Hkv):
        kp = {k: v[:, kh] for k, v in case["k_tok"][0].items()}
        vp = {k: v[:, kh] for k, v in case["v_tok"][0].items()}
        k, sg, rn = odec.dequant_keys(kp, kc, kb, kq)
        v = odec.dequant_values(vp, vc, vb)
        for i in (0, 1, 15, 16, 17, 511, 998, 999):
            hs = slice(kh * G, (kh + 1) * G)
            want = odec.decode_dense(qr[i, hs], qr[i, hs], k[:i + 1], sg[:i + 1], rn[:i + 1], v[:i + 1], SM, CS)
            np.testing.assert_allclose(got[i, hs], want, rtol=RTOL, atol=ATOL)
