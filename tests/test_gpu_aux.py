"""GPU parity: bit-level helper kernels vs the oracle (bit-exact)."""

import numpy as np
import pytest
import torch

from oracle import packing as opack

pytestmark = pytest.mark.gpu


def test_permute_signs_kernel(dev):
    from turboquant.kernels.packed_compress import permute_signs_for_chunked
    rng = np.random.default_rng(0)
    rows = rng.integers(0, 256, (3, 1000, 16), dtype=np.uint8)
    got = permute_signs_for_chunked(torch.from_numpy(rows).to(dev), 128).cpu().numpy()
    assert got.shape == rows.shape
    assert np.array_equal(got.reshape(-1, 16), opack.permute_signs(rows.reshape(-1, 16)))


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_unpack_kernel(dev, bits):
    from turboquant.kernels.packed_compress import unpack_bits, unpack_1bit, unpack_2bit
    rng = np.random.default_rng(bits)
    rows = rng.integers(0, 256, (517, 16 * bits), dtype=np.uint8)
    got = unpack_bits(torch.from_numpy(rows).to(dev), bits).cpu().numpy()
    assert got.dtype == np.int8
    assert np.array_equal(got, opack.unpack_indices(rows, bits))
    if bits == 2:
        assert np.array_equal(unpack_2bit(torch.from_numpy(rows).to(dev), 128).cpu().numpy(), got)
    if bits == 1:
        assert np.array_equal(unpack_1bit(torch.from_numpy(rows).to(dev), 128).cpu().numpy(), got)
