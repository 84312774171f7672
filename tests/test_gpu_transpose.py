"""onnxl_amd_transpose_2d (Transpose, perm [1, 0]; tensor/kernel_transpose.cc
:98-111) on the GPU: bit for bit against numpy's transpose for 1-, 2-, 4- and
8-byte elements at tile-aligned, ragged and single-row / single-column
shapes, from device and host inputs; the preallocated-output errors."""
import numpy as np
import pytest
import torch

from test_gpu_float import T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


@pytest.mark.parametrize("dtype", [np.uint8, np.float16, np.float32, np.float64])
@pytest.mark.parametrize("shape", [(64, 64), (1, 1), (1, 300), (300, 1), (130, 67), (4096, 1000), (17, 4097)])
def test_bit_exact(olamd, dev, dtype, shape):
    rng = np.random.default_rng(shape[0] * 7 + shape[1])
    x = rng.integers(0, 1 << 8 * np.dtype(dtype).itemsize, shape, dtype=np.uint64)
    x = x.astype({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[np.dtype(dtype).itemsize]).view(dtype)
    y = olamd.transpose_2d(T(x, dev))
    assert np.array_equal(y.cpu().numpy().view(x.dtype).view(np.uint8), np.ascontiguousarray(x.T).view(np.uint8))
    yh = olamd.transpose_2d(np.ascontiguousarray(x))
    assert np.array_equal(yh.cpu().numpy().view(np.uint8), np.ascontiguousarray(x.T).view(np.uint8))


def test_errors(olamd, dev):
    x = T(np.zeros((3, 5), np.float32), dev)
    with pytest.raises(olamd.InvalidArgument, match="preallocated output shape mismatch"):
        olamd.transpose_2d(x, torch.zeros((3, 5), dtype=torch.float32, device=dev))
    with pytest.raises(olamd.InvalidArgument, match="preallocated output dtype must match"):
        olamd.transpose_2d(x, torch.zeros((5, 3), dtype=torch.float16, device=dev))
    with pytest.raises(olamd.Unsupported):
        olamd.transpose_2d(T(np.zeros((2, 3, 4), np.float32), dev))
