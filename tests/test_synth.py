"""The synthetic-input generator's torch path (used by the bench to draw
configuration 4 on the GPU) against its numpy path: the same SplitMix64
draws and Irwin-Hall normals, bit for bit, on the CPU."""
import importlib

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def syn(olamd):
    return importlib.import_module("onnx_light_amd.synth")


@pytest.mark.parametrize("seed,start,n", [(0, 0, 1000), (4000, 12345, 4096), (3002, 0, 77), (2**63 + 5, 7, 300)])
def test_draws_match(syn, seed, start, n):
    a = syn.splitmix64_draws(seed, n, start)
    b = syn.splitmix64_draws_torch(seed, n, start).numpy().view(np.uint64)
    assert np.array_equal(a, b)


def test_splitmix64_published_values(syn):
    """First outputs of SplitMix64 seeded with 0 (the published algorithm)."""
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert [int(v) for v in syn.splitmix64_draws(0, 3)] == want
    assert [int(v) for v in syn.splitmix64_draws_torch(0, 3).numpy().view(np.uint64)] == want


def test_randn_matches_across_chunks(syn):
    x = syn.randn(4000, 200003)
    y = syn.randn_torch(4000, 200003, chunk=1 << 15).numpy()
    assert np.array_equal(x.view(np.uint64), y.view(np.uint64))

