"""Regenerates codebook_d128.json: the Lloyd-Max codebooks for d = 128, bits 1-4, as computed by
codebook._solve with scipy's QUADPACK, and the centroids of the kernel files' own recipe
(packed_compress._solve_kernel_recipe).  codebook.solve_codebook serves these values for d = 128
so that hosts without scipy get the same floats.

    python turboquant-amd_amd/turboquant/core/make_codebook_table.py
"""

import json
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", ".."))

from turboquant.core.codebook import TABLE_BITS, TABLE_D, TABLE_PATH, _solve  # noqa: E402
from turboquant.kernels.packed_compress import _solve_kernel_recipe  # noqa: E402


def main() -> None:
    table = {"d": TABLE_D, "solver": "Lloyd-Max on N(0, 1/d), 100 rounds, scipy.integrate.quad", "bits": {}}
    for b in TABLE_BITS:
        c, bd = _solve(TABLE_D, b)
        table["bits"][str(b)] = {"centroids": list(c), "boundaries": list(bd)}
    table["kernel_recipe_centroids"] = {str(b): list(_solve_kernel_recipe(TABLE_D, b)) for b in TABLE_BITS}
    with open(TABLE_PATH, "w") as f:
        json.dump(table, f, indent=1)
        f.write("\n")
    print("wrote", TABLE_PATH)


if __name__ == "__main__":
    main()
