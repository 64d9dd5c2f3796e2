"""Write the committed fixtures of tests/golden/ from the CPU oracle.

  codebooks.json      make_codebook values (d = 128, bits 1..4) from the restated QUADPACK
                      iteration, cross-checked against the closed-form iteration before writing.
  config1_oracle.npz  benchmark config 1 (torch.manual_seed(0); randn(1024, 128); bits 3; QJL;
                      WHT): packed indices / signs, norms, residual norms, and a checksum of the
                      input so a change of RNG or torch build is detected.

Run from the repository root: python tests/golden/make_golden.py
"""

import hashlib
import json
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import codebook as ocb  # noqa: E402
from oracle import compress as ocomp  # noqa: E402
from oracle import packing as opack  # noqa: E402


def main():
    books = {}
    for bits in (1, 2, 3, 4):
        c, b = ocb.solve_codebook_quad(128, bits)
        cc, bb = ocb.solve_codebook_closed_form(128, bits)
        assert max(abs(x - y) for x, y in zip(c, cc)) < 1e-9
        books[str(bits)] = {"centroids": c, "boundaries": b}
    (HERE / "codebooks.json").write_text(json.dumps({"d": 128, "books": books}, indent=1))

    torch.manual_seed(0)
    K = torch.randn(1024, 128)
    cent = torch.tensor(books["3"]["centroids"], dtype=torch.float32)
    bnd = torch.tensor(books["3"]["boundaries"], dtype=torch.float32)
    H = ocomp.wht_matrix(128)
    ref = ocomp.polarquant_compress(K, cent, bnd, 8, True, H)
    np.savez_compressed(
        HERE / "config1_oracle.npz",
        input_sha256=np.frombuffer(hashlib.sha256(K.numpy().tobytes()).digest(), dtype=np.uint8),
        indices_packed=opack.pack_indices(ref["indices"].numpy(), 3),
        signs_packed=opack.pack_signs((ref["signs"].numpy() > 0).astype(np.int64)),
        norms=ref["norms"].numpy(),
        rot_residual_norm=ref["rot_residual_norm"].numpy(),
    )
    print("wrote", HERE / "codebooks.json", HERE / "config1_oracle.npz")


if __name__ == "__main__":
    main()
