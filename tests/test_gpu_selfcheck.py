"""The reference modules' self-test / benchmark entry points, run small: packed_compress.run(),
packed_attention.run() and sparse_v.benchmark() exist under the drop-in package, run on the
GPU, and report passing correctness figures (the full-size parity of the same kernels is in
the other GPU tests)."""

import pytest

pytestmark = pytest.mark.gpu


def test_packed_compress_run(dev):
    from turboquant.kernels import packed_compress
    res = packed_compress.run(sizes=(2048,), n_test=8192, warmup=1, iters=2, verbose=False)
    for name in ("K", "V"):
        c = res["correctness"][name]
        assert c["pass"] and c["idx_match"] > 0.999 and c["recon_cos"] > 0.9999, (name, c)
    assert res["benchmark"][0]["k_ms"] > 0 and res["benchmark"][0]["v_ms"] > 0


def test_packed_attention_run(dev):
    from turboquant.kernels import packed_attention
    res = packed_attention.run(bh_list=(8,), sk_check=(256, 4096), sk_bench=(256,), warmup=1, iters=2,
                               verbose=False)
    for c in res["correctness"]:
        assert c["pass"] and c["cos"] > 0.999 and c["max_abs_err"] < 1e-3, c
    assert res["benchmark"][0]["packed_ms"] > 0


def test_sparse_v_benchmark(dev):
    from turboquant.kernels import sparse_v
    rows = sparse_v.benchmark(cases=((1, 1024), (8, 4096)), iters=2, warmup=1, verbose=False)
    assert len(rows) == 2
    for r in rows:
        assert r["cos"] > 0.99 and r["v11_ms"] > 0 and r["v12_ms"] > 0 and r["v12_split_ms"] > 0, r
