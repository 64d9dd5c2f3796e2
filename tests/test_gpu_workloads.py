"""GPU parity at the benchmark workloads themselves (configs 3, 4 and 5 of BASELINE.json).

Each test builds exactly the inputs bench.py times (bench.build_decode_workload: caches filled
by compress_paged from the outlier-channel distribution, random-permutation block tables, bf16
queries, the planner's tokens_per_chunk), runs the timed step once, and checks the output:
  - against the float64 oracle (attention_unpacked_ref semantics, kernels/packed_attention.py:
    273-284) read back from the cache bytes, at rtol 1e-2 / atol 1e-3;
  - through the constant-V closed form over every sequence (every V token equal: the output is
    that vector whatever the scores);
  - config 4: Sparse-V skip counts at the planner's chunk against the oracle's chunk walk, up
    to the tokens whose keep/skip margin lies within the kernel's score rounding.
"""

import math

import numpy as np
import pytest
import torch

import bench
from oracle import compress as ocomp
from oracle import decode as odec
from oracle import packing as opack
from oracle import paged as opaged

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3
SM = 1 / math.sqrt(128)
CS = math.sqrt(math.pi / 2) / 128


def seq_tokens(st, s):
    """Per-(KV head) token payloads of sequence s, read back from the caches' bytes."""
    bs = st["kf"].block_size
    L = st["lens_host"][s]
    nbl = math.ceil(L / bs)
    blocks = st["bt"][s, :nbl].long()
    kt = st["k_cache"].index_select(0, blocks).cpu().numpy()
    vt = st["v_cache"].index_select(0, blocks).cpu().numpy()
    out = []
    for kh in range(st["Hkv"]):
        kp = opaged.tiles_to_tokens(kt[:, kh], bs, st["kf"].bits, st["kf"].qjl, st["kf"].layout)
        vp = opaged.tiles_to_tokens(vt[:, kh], bs, st["vf"].bits, False, st["vf"].layout)
        out.append(({k: v[:L] for k, v in kp.items()}, {k: v[:L] for k, v in vp.items()}))
    return out


def check_sequence(st, out, s, chunk=None, thresh=0.0):
    """Output rows of sequence s (all query heads) against the oracle; returns (skipped, total)."""
    kb, vb, kq = st["kf"].bits, st["vf"].bits, st["kf"].qjl
    kc, vc = st["kc"].double().cpu().numpy(), st["vc"].double().cpu().numpy()
    G = st["Hq"] // st["Hkv"]
    q = st["q"][s].float().cpu().numpy().astype(np.float64)
    got = out[s].float().cpu().numpy()
    skipped = total = 0
    for kh, (kp, vp) in enumerate(seq_tokens(st, s)):
        k, sg, rn = odec.dequant_keys(kp, kc, kb, kq)
        v = odec.dequant_values(vp, vc, vb)
        hs = slice(kh * G, (kh + 1) * G)
        if chunk is None:
            want = odec.decode_dense(q[hs], q[hs], k, sg, rn, v, SM, CS)
        else:
            want, sk, tot = odec.decode_chunked(q[hs], q[hs], k, sg, rn, v, SM, CS, chunk, thresh)
            skipped += sk
            total += tot
        np.testing.assert_allclose(got[hs], want, rtol=RTOL, atol=ATOL, err_msg=f"sequence {s} KV head {kh}")
    return skipped, total


def constant_values(st, code_byte, norm=2.0):
    """Overwrite every V payload byte with code_byte and every V norm with `norm`; returns the
    value every output element must then take."""
    vf = st["vf"]
    v = st["v_cache"]
    v[:, :, :vf.off_norm] = code_byte
    v[:, :, vf.off_norm:vf.tile_bytes] = torch.tensor([norm], dtype=torch.float16).view(torch.uint8).to(v.device).repeat(
        vf.block_size)
    idx = opack.unpack_indices(np.full((1, 16 * vf.bits), code_byte, np.uint8), vf.bits)[0]
    assert (idx == idx[0]).all()
    return float(st["vc"][int(idx[0])]) * norm


def check_constant_v(st, out_fn):
    # every V field = the same index in every layout: bytes 0x33 (4 bits), 0xAA (2 bits) or the
    # repeating 3-byte pattern of 3-bit fields equal to 2 (written here byte-wise per position)
    vb = st["vf"].bits
    if vb == 3:
        pat = torch.tensor([0x92, 0x24, 0x49], dtype=torch.uint8, device=st["v_cache"].device)
        st["v_cache"][:, :, :st["vf"].off_norm] = pat.repeat(st["vf"].off_norm // 3)
        st["v_cache"][:, :, st["vf"].off_norm:st["vf"].tile_bytes] = torch.tensor(
            [2.0], dtype=torch.float16).view(torch.uint8).to(st["v_cache"].device).repeat(st["vf"].block_size)
        want = float(st["vc"][2]) * 2.0
    else:
        want = constant_values(st, 0x33 if vb == 4 else 0xAA)
    out = out_fn()
    torch.cuda.synchronize()
    live = torch.tensor([L > 0 for L in st["lens_host"]], device=out.device)
    err = (out[live].float() - want).abs().max().item()
    assert err <= ATOL + RTOL * abs(want), f"constant-V closed form: max error {err} (value {want})"


def test_config3_full_workload(dev):
    """Config 3 (turbo4, B 32, Hq 32 / Hkv 8, ctx U[1K, 8K]): every sequence and KV head against
    the oracle, then the constant-V closed form."""
    st = bench.build_decode_workload("config3", dev)
    print(f"config3: chunk {st['chunk']}, lengths {min(st['lens_host'])}..{max(st['lens_host'])}", flush=True)
    out = bench.decode_step(st)().clone()
    torch.cuda.synchronize()
    for s in range(st["B"]):
        check_sequence(st, out, s)
    check_constant_v(st, bench.decode_step(st))


def test_config5_full_workload(dev, parity_log):
    """Config 5 (turbo2 + QJL, B 64, Hq 64 / Hkv 8, ctx log-U[2K, 128K]): the timed step
    (compress 64 new tokens into the last slot of each sequence, then decode).  The new tokens'
    stored indices against the compress oracle (1-ulp / fp64 rule); the shortest, the longest
    and every eighth sequence against the decode oracle; the constant-V closed form."""
    st = bench.build_decode_workload("config5", dev)
    lens = st["lens_host"]
    print(f"config5: chunk {st['chunk']}, lengths {min(lens)}..{max(lens)}", flush=True)
    out = bench.decode_step(st)().clone()
    torch.cuda.synchronize()
    # the new tokens (position L - 1 of each sequence) as stored
    newk, newv, _ = st["new_tokens"]
    from turboquant.core import make_wht_matrix
    H128 = make_wht_matrix(128)
    for which, x, fmt, cb, bnd in (("K", newk, st["kf"], st["kc"], st["kbnd"]), ("V", newv, st["vf"], st["vc"], st["vbnd"])):
        cache = st["k_cache"] if which == "K" else st["v_cache"]
        got = np.zeros((st["B"], st["Hkv"], 128), np.int64)
        bs = fmt.block_size
        for s in range(st["B"]):
            t = lens[s] - 1
            tile = cache[int(st["bt"][s, t // bs])].cpu().numpy()      # [Hkv, tile_bytes]
            for kh in range(st["Hkv"]):
                pl = opaged.tiles_to_tokens(tile[kh][None], bs, fmt.bits, fmt.qjl, fmt.layout)
                got[s, kh] = opack.unpack_indices(pl["idx"][t % bs][None], fmt.bits)[0]
        xf = x.float().cpu().reshape(-1, 128)
        ref = ocomp.polarquant_compress(xf, cb.cpu(), bnd.cpu(), 2 ** fmt.bits, fmt.qjl, H128)
        ref64 = ocomp.polarquant_compress_fp64(xf, cb.cpu(), bnd.cpu(), fmt.qjl, True)
        stats = ocomp.classify_strict(got.reshape(-1, 128), ref["indices"].numpy(), ref["x_normalized"].numpy(),
                                      bnd.cpu().numpy(), ref64["indices"].numpy())
        parity_log[f"config5 new tokens {which}"] = stats
        assert stats["failures"] == 0, stats
    order = sorted(range(st["B"]), key=lambda s: lens[s])
    for s in sorted({order[0], order[-1], *range(0, st["B"], 8)}):
        check_sequence(st, out, s)
    # decode alone from here (the step's compress would overwrite the constant V rows)
    check_constant_v(st, bench.decode_step(dict(st, new_tokens=None)))


def _single(st, s):
    """The workload reduced to sequence s (same caches, same chunk): skip statistics per sequence."""
    return dict(st, B=1, q=st["q"][s:s + 1], out=torch.empty_like(st["q"][s:s + 1]), bt=st["bt"][s:s + 1],
                lens=st["lens"][s:s + 1], lens_host=[st["lens_host"][s]], new_tokens=None)


def test_config4_sparse_v_skip_counts(dev):
    """Config 4 (turbo3 + QJL K / turbo3 V, B 64 x 32768, GQA 6, T = 1e-4) at the planner's
    chunk: two sequences decoded on their own with skip statistics against the oracle's chunk
    walk (decode_chunked).  A token whose keep margin (log of max_h p relative to the running
    max, minus log T) is within DELTA may fall either way under the kernel's rounding of the
    scores; the skip counts must agree up to the number of such tokens."""
    DELTA = 2e-3  # natural-log units: the kernel's score error is ~1e-4 here (fp8 QJL operand)
    st = bench.build_decode_workload("config4", dev)
    chunk = st["chunk"]
    print(f"config4: chunk {chunk}", flush=True)
    full = bench.decode_step(st)().clone()
    torch.cuda.synchronize()
    G = st["Hq"] // st["Hkv"]
    kc = st["kc"].double().cpu().numpy()
    skipped_total = 0
    for s in (0, 21, 37):
        one = _single(st, s)
        stats = torch.zeros(2, dtype=torch.int64, device=dev)
        out = bench.decode_step(one, skip_stats=stats)()
        torch.cuda.synchronize()
        # the batch run and the single-sequence run make the same decisions
        torch.testing.assert_close(out[0], full[s], rtol=0, atol=0)
        gsk, gtot = stats.tolist()
        sk, tot = check_sequence(one, out, 0, chunk=chunk, thresh=st["thresh"])
        q = one["q"][0].float().cpu().numpy().astype(np.float64)
        ambiguous = 0
        for kh, (kp, _) in enumerate(seq_tokens(one, 0)):
            k, sg, rn = odec.dequant_keys(kp, kc, 3, True)
            hs = slice(kh * G, (kh + 1) * G)
            marg = odec.sparse_v_margins(q[hs], q[hs], k, sg, rn, SM, CS, chunk)
            ambiguous += int((np.abs(marg - math.log(st["thresh"])) < DELTA).sum())
        print(f"sequence {s}: skipped gpu {gsk} oracle {sk} of {tot} (ambiguous {ambiguous})", flush=True)
        assert gtot == tot
        assert abs(gsk - sk) <= ambiguous, (gsk, sk, ambiguous)
        skipped_total += sk
    assert skipped_total > 0
