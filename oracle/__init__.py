"""CPU oracle for the TurboQuant packed-KV hot path — TEST INFRASTRUCTURE ONLY.

A restatement of the reference's algorithms (andyluo7/turboquant-amd) on the CPU, used to
check the HIP kernels.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import this package; the product (turboquant-amd_amd/turboquant) never does.

Modules and what pins each function (beyond restating the reference's formula):
  codebook  solve_codebook_quad (core/codebook.py:17-54) is pinned by an independent
            closed-form Gaussian-moment iteration (same 100 steps) to ~1e-12, by the reference
            tests' invariants (tests/test_codebook.py) and by Lloyd-Max optimality at the fixed
            point; kernel_codebook (kernels/packed_compress.py:21-41) by the same closed form.
  wht       wht_matrix (core/rotation.py:28-44) pinned by the closed form
            H[i][j] = (-1)^popcount(i&j) h and H @ H = I.
  compress  polarquant_compress (core/quantizer.py:111-183) pinned by an fp64 shadow
            computation (indices equal except within a rounding band of a boundary), basis
            and zero vectors with known answers, and the reference tests' invariants.
            compress_packed (kernels/packed_compress.py:64-142) pinned by agreement with the
            polarquant shadow for PiT = WHT, PiST = I (the two orders of operations differ only
            inside the band), and by basis vectors with PiT = I that pin the >= tie rule.
  packing   bit formats (Appendix-A rules: packed_compress.py:79-106,145-154,180-216;
            sparse_v.py:57-98; AITER_TURBO4_DESIGN.md:57-76) pinned by brute force over every
            field value / bit position and pack-unpack round trips.
  paged     tile layout / slot scatter pinned by a per-token brute-force scatter-gather round trip.
  decode    attention (kernels/packed_attention.py:273-284 with the correct combine of
            kernels/attention.py:121-140; Sparse-V of kernels/sparse_v.py:108-149) pinned by
            pure-Python loops on tiny inputs, chunking invariance of the dense result, and the
            closed form for constant values.
"""
