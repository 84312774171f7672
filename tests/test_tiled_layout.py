"""CPU checks of the tiled-layout restatement and of the prepared-weight
entry points' validation (no GPU work)."""
import ctypes

import numpy as np
import pytest

from tiled_layout import tile_int4


def test_tile_restatement_known_answer():
    """Hand-built 8-row column: rows 0..7 hold 1..8 (UINT4) -> one dword."""
    K, N = 8, 2
    vals = np.zeros((K, N), dtype=np.uint8)
    vals[:, 0] = np.arange(1, 9)
    flat = vals.reshape(-1)
    packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)
    words = tile_int4(packed, K, N, False)
    # rows (0,1) -> bits 0 / 16, (2,3) -> 4 / 20, (4,5) -> 8 / 24, (6,7) -> 12 / 28
    assert words[0] == (1 | 2 << 16 | 3 << 4 | 4 << 20 | 5 << 8 | 6 << 24 | 7 << 12 | 8 << 28)
    assert words[1] == 0  # chunk 1 of lane 0: rows 32.. (padding)


def test_tile_restatement_is_a_permutation():
    """Every input nibble lands in exactly one place: tiling distinct values
    and reading them back by the layout formula returns the matrix."""
    K, N = 260, 37
    rng = np.random.default_rng(3)
    vals = rng.integers(0, 16, K * N).astype(np.uint8)
    packed = (vals[0::2] | (np.append(vals[1::2], 0)[: (vals.size + 1) // 2] << 4)).astype(np.uint8) \
        if vals.size % 2 else (vals[0::2] | (vals[1::2] << 4)).astype(np.uint8)
    words = tile_int4(packed, K, N, False)
    ng = (K + 127) // 128
    for k, n in [(0, 0), (7, 0), (8, 1), (31, 15), (32, 16), (127, 36), (128, 5), (259, 36), (200, 20)]:
        t, i, q, c, g, j = n // 16, n % 16, k // 128, (k // 32) % 4, (k // 8) % 4, k % 8
        w = int(words[((t * ng + q) * 64 + g * 16 + i) * 4 + c])
        sh = 16 + 4 * (j // 2) if j % 2 else 4 * (j // 2)
        assert (w >> sh) & 15 == vals[k * N + n], (k, n)


def _desc(olamd, dtype, shape, layout=0):
    d = olamd.Tensor()
    d.data_type = dtype
    d.rank = len(shape)
    for i, s in enumerate(shape):
        d.dims[i] = s
    d.location = olamd.DEVICE
    d.layout = layout
    return d


def test_prepare_weight_size(olamd):
    for K, N, want in [(4096, 11008, 688 * 32 * 1024), (200, 40, 3 * 2 * 1024), (1, 1, 1024), (0, 16, 0)]:
        n = ctypes.c_int64(-1)
        d = _desc(olamd, olamd.INT4, (K, N))
        d.size_bytes = (K * N + 1) // 2
        d.data = 1  # never read: no device work for a size query
        olamd._check(olamd.lib().onnxl_amd_prepare_weight_size(ctypes.byref(d), ctypes.byref(n)))
        assert n.value == want, (K, N)


def test_prepare_weight_validation(olamd):
    n = ctypes.c_int64(0)
    d = _desc(olamd, olamd.INT8, (16, 16))
    d.size_bytes, d.data = 256, 1
    with pytest.raises(olamd.InvalidArgument, match="INT4 / UINT4"):
        olamd._check(olamd.lib().onnxl_amd_prepare_weight_size(ctypes.byref(d), ctypes.byref(n)))
    d = _desc(olamd, olamd.UINT4, (2, 16, 16))
    d.size_bytes, d.data = 256, 1
    with pytest.raises(olamd.InvalidArgument, match="2-D"):
        olamd._check(olamd.lib().onnxl_amd_prepare_weight_size(ctypes.byref(d), ctypes.byref(n)))


def test_tiled_layout_rejected_outside_dq_matmul(olamd):
    """Only the x input of the fused DequantizeLinear -> MatMul takes a
    prepared weight; elsewhere the layout is an argument error."""
    a = _desc(olamd, olamd.INT8, (4, 8), layout=olamd.LAYOUT_TILED_INT4)
    a.size_bytes, a.data = 32, 1
    b = _desc(olamd, olamd.INT8, (8, 4))
    b.size_bytes, b.data = 32, 1
    y = _desc(olamd, olamd.INT32, (4, 4))
    y.size_bytes, y.data = 64, 1
    rc = olamd.lib().onnxl_amd_matmul_integer(ctypes.byref(a), ctypes.byref(b), None, None, ctypes.byref(y), None)
    assert rc == olamd.INVALID_ARGUMENT
    assert "layout" in olamd.lib().onnxl_amd_last_error().decode()
