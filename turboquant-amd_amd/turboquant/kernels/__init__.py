"""HIP (gfx950) kernels of the TurboQuant packed-KV hot path.

Modules keep the reference's names (turboquant/kernels/__init__.py):
  packed_compress   bit-level helpers (sign permutation, unpacking) and the kernel-file codebook
  packed_attention  packed_attention: split-K decode over contiguous per-head packed arrays
  sparse_v          paged 3-bit decode over the reference's slot layout, dense and Sparse-V
  paged             paged packed cache: fused compression and GQA split-K decode
  rotation          stand-alone Walsh-Hadamard rotation of query / output rows
"""
