"""GPU parity: the Walsh-Hadamard rotations of queries and outputs, alone (tq_wht_rows) and fused
into decode (tq_decode_rotated), and the paged backend built on them.

The rotation is pinned by the closed form of make_wht_matrix (entries (-1)^popcount(i&j) / sqrt(128),
oracle.compress.wht_closed_form, itself checked against the restated matrix in test_oracle.py):
rotate_query(q) = q @ H, rotate_output(o) = o @ H (integration/vllm_backend.py:158-177; H is
symmetric and H @ H = I).  Decode bar: rtol 1e-2 / atol 1e-3 against the float64 oracle.
"""

import math

import numpy as np
import pytest
import torch

from oracle import compress as ocomp
from oracle import decode as odec
from oracle import paged as opaged
from test_gpu_decode import ATOL, RTOL, _cb, build_case, oracle_out

pytestmark = pytest.mark.gpu

H64 = ocomp.wht_closed_form(128, 1.0 / math.sqrt(128.0))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_wht_rows_matches_closed_form(dev, dtype):
    from turboquant.kernels.rotation import wht_rows
    g = torch.Generator().manual_seed(5)
    x = torch.randn(5, 7, 128, generator=g).to(dtype)
    got = wht_rows(x.to(dev)).cpu()
    assert got.dtype == dtype
    want = x.double().numpy() @ H64
    # fp32 butterflies (7 additions deep) then one rounding to the output dtype
    rtol = {torch.float32: 1e-6, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]
    np.testing.assert_allclose(got.double().numpy(), want, rtol=rtol, atol=4e-6 + rtol * 2)


def test_wht_rows_layouts_and_involution(dev):
    from turboquant.kernels.rotation import wht_rows
    g = torch.Generator().manual_seed(6)
    base = torch.randn(6, 9, 128, generator=g)
    want = base.double().numpy() @ H64
    xd = base.to(dev)
    # strided rows (every other head), 2-D input, 4-D input, in place, mixed output dtype
    np.testing.assert_allclose(wht_rows(xd[:, ::2]).cpu().double().numpy(), want[:, ::2], rtol=1e-6, atol=4e-6)
    np.testing.assert_allclose(wht_rows(xd[1]).cpu().double().numpy(), want[1], rtol=1e-6, atol=4e-6)
    np.testing.assert_allclose(wht_rows(xd.view(2, 3, 9, 128)).cpu().double().numpy(), want.reshape(2, 3, 9, 128),
                               rtol=1e-6, atol=4e-6)
    y = xd.clone()
    assert wht_rows(y, out=y) is y
    np.testing.assert_allclose(y.cpu().double().numpy(), want, rtol=1e-6, atol=4e-6)
    o16 = torch.empty(6, 9, 128, dtype=torch.bfloat16, device=dev)
    wht_rows(xd, out=o16)
    np.testing.assert_allclose(o16.cpu().double().numpy(), want, rtol=2.0 ** -8, atol=1e-5)
    # H @ H = I: twice is the identity up to fp32 rounding
    np.testing.assert_allclose(wht_rows(wht_rows(xd)).cpu().numpy(), base.numpy(), rtol=1e-5, atol=1e-5)
    assert wht_rows(torch.empty(0, 4, 128, device=dev)).shape == (0, 4, 128)
    with pytest.raises(ValueError):
        wht_rows(torch.empty(3, 64, device=dev))


def _decode(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, chunk, rotate, q=None, q_proj=None):
    from turboquant.kernels.paged import PagedKVFormat, decode_paged
    kf = PagedKVFormat(bits=kb, qjl=kq, block_size=bs)
    vf = PagedKVFormat(bits=vb, qjl=False, block_size=bs, layout="values")
    if q is None:
        q = torch.from_numpy(case["q"]).to(torch.bfloat16).to(dev)
    out = decode_paged(q, torch.from_numpy(case["k_cache"]).to(dev), kf, _cb(kb).to(dev),
                       torch.from_numpy(case["v_cache"]).to(dev), vf, _cb(vb).to(dev),
                       torch.from_numpy(case["bt"]).to(dev), torch.from_numpy(case["seq_lens"]).to(dev),
                       sm_scale=sm, corr_scale=cs, tokens_per_chunk=chunk, q_proj=q_proj, rotate=rotate)
    torch.cuda.synchronize()
    return out, q


@pytest.mark.parametrize("kb,kq,vb,G", [(3, True, 3, 6), (4, False, 4, 4), (2, True, 2, 8), (3, True, 4, 12)])
def test_decode_rotated_matches_oracle(dev, kb, kq, vb, G):
    """q in the model basis: out = decode(q H) H.  G = 12 runs the general kernel, the others
    the paged fast path; chunk 64 splits the 300-token sequence, the others take one chunk
    (the rotated output is then written by the split-K merge), the empty one is zero."""
    Hkv, bs = 2, 16
    Hq = G * Hkv
    lens = [37, 1, 300, 0]
    case = build_case(500 + 7 * kb + vb + G, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    for chunk in (64, 512, 0):      # 0: the balanced schedule
        out, q = _decode(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, chunk, rotate=True)
        q64 = q.float().cpu().numpy().astype(np.float64)
        want_rot, _, _ = oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, q_round=q64 @ H64)
        want = want_rot @ H64
        got = out.float().cpu().numpy()
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
        assert np.all(got[3] == 0.0)


def test_decode_rotated_explicit_q_proj_is_not_rotated(dev):
    """A q_proj given by the caller enters the QJL term as it is; q is rotated."""
    kb, kq, vb, Hq, Hkv, bs = 3, True, 3, 8, 2, 16
    lens = [200, 45]
    case = build_case(612, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    rng = np.random.default_rng(3)
    qp = torch.from_numpy(rng.standard_normal((len(lens), Hq, 128)).astype(np.float32)).to(torch.bfloat16).to(dev)
    for chunk in (32, 256):
        out, q = _decode(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, chunk, rotate=True, q_proj=qp)
        q64 = q.float().cpu().numpy().astype(np.float64)
        qp64 = qp.float().cpu().numpy().astype(np.float64)
        want_rot, _, _ = oracle_out(case, Hq, Hkv, kb, kq, vb, sm, cs, qp=qp64, q_round=q64 @ H64)
        np.testing.assert_allclose(out.float().cpu().numpy(), want_rot @ H64, rtol=RTOL, atol=ATOL)


def test_decode_rotated_equals_rotations_around_decode(dev):
    """tq_decode_rotated = rotate_output(tq_decode(rotate_query(q))) up to fp32/fp16 rounding of q
    (the stand-alone path rounds q H to bf16 first)."""
    from turboquant.kernels.rotation import wht_rows
    kb, kq, vb, Hq, Hkv, bs = 3, True, 3, 12, 2, 16
    lens = [513, 64, 7]
    case = build_case(700, len(lens), Hq, Hkv, lens, kb, kq, vb, bs)
    sm, cs = 1 / math.sqrt(128), math.sqrt(math.pi / 2) / 128
    q = torch.from_numpy(case["q"]).to(torch.float32).to(dev)
    fused, _ = _decode(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, 64, rotate=True, q=q)
    plain, _ = _decode(dev, case, Hq, Hkv, kb, kq, vb, bs, sm, cs, 64, rotate=False, q=wht_rows(q))
    composed = wht_rows(plain)
    np.testing.assert_allclose(fused.cpu().numpy(), composed.cpu().numpy(), rtol=2e-3, atol=2e-4)


def test_paged_backend_decode_step(dev):
    """TurboQuantPagedImpl: do_kv_cache_update writes what compress_paged writes into each half
    of the combined cache; forward equals decode_paged(rotate=True) and, on the written bytes,
    the oracle's decode of q H rotated back."""
    from turboquant.integration.paged_backend import (PagedDecodeMetadata, TurboQuantPagedImpl,
                                                      TurboQuantPagedState)
    from turboquant.kernels.paged import compress_paged, decode_paged

    Hq, Hkv, bs, kb, vb = 12, 2, 16, 3, 2
    state = TurboQuantPagedState(128, layer_idx=3, device=dev, k_bits=kb, v_bits=vb, k_qjl=True, block_size=bs)
    impl = TurboQuantPagedImpl(Hq, 128, 1 / math.sqrt(128), Hkv, state)
    assert impl.get_kv_cache_shape(40, bs, Hkv, 128, k_bits=kb, v_bits=vb, k_qjl=True) == (40, Hkv, state.tile_bytes)
    lens = [70, 33]
    S = len(lens)
    g = torch.Generator().manual_seed(21)
    perm = torch.randperm(40, generator=g)
    bt = torch.full((S, 8), -1, dtype=torch.int32)
    bt[0, :5] = perm[:5].int()
    bt[1, :3] = perm[5:8].int()
    slots = torch.cat([torch.tensor([int(bt[s, t // bs]) * bs + t % bs for t in range(L)]) for s, L in enumerate(lens)])
    T = int(slots.numel())
    key = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    kv = state.allocate_kv_cache(40, Hkv)
    impl.do_kv_cache_update(None, key, value, kv, slots.to(dev))
    k_cache, v_cache = state.split_kv_cache(kv)
    k_ref = torch.zeros(40, Hkv, state.k_format.tile_bytes, dtype=torch.uint8, device=dev)
    v_ref = torch.zeros(40, Hkv, state.v_format.tile_bytes, dtype=torch.uint8, device=dev)
    compress_paged(key, slots.to(dev), k_ref, state.k_format, state.k_centroids, state.k_boundaries)
    compress_paged(value, slots.to(dev), v_ref, state.v_format, state.v_centroids, state.v_boundaries)
    assert torch.equal(k_cache, k_ref) and torch.equal(v_cache, v_ref)

    q = torch.randn(S, Hq, 128, generator=g).to(torch.bfloat16).to(dev)
    meta = PagedDecodeMetadata(block_tables=bt.to(dev), seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev),
                               max_seq_len=max(lens), seq_lens_host=lens)
    output = torch.empty(S, Hq * 128, dtype=torch.bfloat16, device=dev)
    assert impl.forward(None, q.view(S, Hq * 128), None, None, kv, meta, output=output) is output
    direct = decode_paged(q, k_ref, state.k_format, state.k_centroids, v_ref, state.v_format, state.v_centroids,
                          meta.block_tables, meta.seq_lens, sm_scale=impl.scale, max_seq_len=max(lens),
                          seq_lens_host=lens, rotate=True)
    torch.cuda.synchronize()
    assert torch.equal(output.view(S, Hq, 128), direct)

    kc64, vc64 = state.k_centroids.double().cpu().numpy(), state.v_centroids.double().cpu().numpy()
    kn, vn = k_ref.cpu().numpy(), v_ref.cpu().numpy()
    q64 = q.float().cpu().numpy().astype(np.float64) @ H64
    G = Hq // Hkv
    cs = math.sqrt(math.pi / 2) / 128
    want = np.zeros((S, Hq, 128))
    for s, L in enumerate(lens):
        for h in range(Hkv):
            kp = opaged.gather_sequence(kn, bt[s].numpy(), L, h, bs, kb, True, layout="keys")
            vp = opaged.gather_sequence(vn, bt[s].numpy(), L, h, bs, vb, False, layout="values")
            k, sg, rn = odec.dequant_keys(kp, kc64, kb, True)
            v = odec.dequant_values(vp, vc64, vb)
            hs = slice(h * G, (h + 1) * G)
            want[s, hs] = odec.decode_dense(q64[s, hs], q64[s, hs], k, sg, rn, v, impl.scale, cs) @ H64
    np.testing.assert_allclose(output.view(S, Hq, 128).float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)


def test_paged_backend_mixed_batch(dev):
    """A batch of two decode sequences followed by two extend sequences (vLLM order): the
    decode rows equal decode_paged(rotate=True), the extend rows prefill_paged(rotate=True) -
    bit for bit - and the extend rows match the oracle's causal prefill of q H rotated back."""
    from turboquant.integration.paged_backend import (PagedDecodeMetadata, TurboQuantPagedImpl,
                                                      TurboQuantPagedState)
    from turboquant.kernels.paged import decode_paged, prefill_paged

    Hq, Hkv, bs = 8, 2, 16
    state = TurboQuantPagedState(128, device=dev, k_bits=3, v_bits=3, k_qjl=True, block_size=bs)
    impl = TurboQuantPagedImpl(Hq, 128, 1 / math.sqrt(128), Hkv, state)
    lens = [90, 17, 40, 129]
    n_new = [1, 1, 40, 33]             # the third is a full prefill, the fourth an extend
    S = len(lens)
    g = torch.Generator().manual_seed(4)
    nb = 40
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((S, 9), -1, dtype=torch.int32)
    o = 0
    for s, L in enumerate(lens):
        nbl = (L + bs - 1) // bs
        bt[s, :nbl] = perm[o:o + nbl].int()
        o += nbl
    slots = torch.cat([torch.tensor([int(bt[s, t // bs]) * bs + t % bs for t in range(L)]) for s, L in enumerate(lens)])
    key = torch.randn(slots.numel(), Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(slots.numel(), Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    kv = state.allocate_kv_cache(nb, Hkv)
    impl.do_kv_cache_update(None, key, value, kv, slots.to(dev))
    k_cache, v_cache = state.split_kv_cache(kv)

    T = sum(n_new)
    qsl = torch.tensor([0] + list(np.cumsum(n_new)), dtype=torch.int32, device=dev)
    q = torch.randn(T + 3, Hq * 128, generator=g).to(torch.bfloat16).to(dev)  # 3 padding rows
    output = torch.full((T + 3, Hq * 128), 7.0, dtype=torch.bfloat16, device=dev)
    btd, lensd = bt.to(dev), torch.tensor(lens, dtype=torch.int32, device=dev)
    md = PagedDecodeMetadata(btd, lensd, max(lens), seq_lens_host=lens, query_start_loc=qsl, num_decodes=2,
                             max_query_len=40)
    impl.forward(None, q, None, None, kv, md, output=output)
    torch.cuda.synchronize()
    dec = decode_paged(q[:2].view(2, Hq, 128), k_cache, state.k_format, state.k_centroids, v_cache, state.v_format,
                       state.v_centroids, btd[:2], lensd[:2], sm_scale=impl.scale, max_seq_len=max(lens),
                       seq_lens_host=lens[:2], rotate=True)
    pre = prefill_paged(q[2:T].view(T - 2, Hq, 128), qsl[2:] - 2, k_cache, state.k_format, state.k_centroids,
                        v_cache, state.v_format, state.v_centroids, btd[2:], lensd[2:], sm_scale=impl.scale,
                        rotate=True)
    torch.cuda.synchronize()
    assert torch.equal(output[:2].view(2, Hq, 128), dec)
    assert torch.equal(output[2:T].view(T - 2, Hq, 128), pre)
    assert torch.all(output[T:] == 7.0)            # padding rows untouched

    kc64 = state.k_centroids.double().cpu().numpy()
    kn, vn = k_cache.cpu().numpy(), v_cache.cpu().numpy()
    G = Hq // Hkv
    cs = math.sqrt(math.pi / 2) / 128
    qn = q[:T].view(T, Hq, 128).float().cpu().numpy().astype(np.float64) @ H64
    got = output[:T].view(T, Hq, 128).float().cpu().numpy()
    for s in (2, 3):
        L, n = lens[s], n_new[s]
        r0 = int(sum(n_new[:s]))
        for h in range(Hkv):
            kp = opaged.gather_sequence(kn, bt[s].numpy(), L, h, bs, 3, True, layout="keys")
            vp = opaged.gather_sequence(vn, bt[s].numpy(), L, h, bs, 3, False, layout="values")
            k, sg, rn = odec.dequant_keys(kp, kc64, 3, True)
            v = odec.dequant_values(vp, kc64, 3)
            hs = slice(h * G, (h + 1) * G)
            want = odec.prefill_dense(qn[r0:r0 + n, hs], qn[r0:r0 + n, hs], k, sg, rn, v, impl.scale, cs) @ H64
            np.testing.assert_allclose(got[r0:r0 + n, hs], want, rtol=RTOL, atol=ATOL)
