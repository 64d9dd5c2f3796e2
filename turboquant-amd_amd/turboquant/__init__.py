"""TurboQuant packed-KV hot path for AMD Instinct MI355X (gfx950).

Drop-in for the reference's `turboquant.core` and `turboquant.kernels` APIs
(andyluo7/turboquant-amd): host-side setup (codebooks, rotation, configuration) in Python,
every per-token computation in hand-written HIP kernels behind a C ABI
(include/turboquant_hip.h, loaded by turboquant._lib).
"""

__version__ = "0.1.0"
