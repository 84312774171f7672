"""The ORT MatMulNBits decode of the oracle (oracle.ort_nbits_decode) and the
test packer (tests/nbits_cases.py), pinned by the reference's golden test
OrtMatMulNBitsGoldenInputsAndColumnPadding (test_quantization.cc:2382-2453:
K = 35, N = 2, block 16, code (row + column) & mask, zero point
(column + group + 1) & mask, scale 0.5 (group + 1); its byte values) and by
OrtMatMulNBitsImplicitAndFloatingZeroPoints (:2498-2513, fractional zero
points)."""
import numpy as np
import pytest

from nbits_cases import ort_pack


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_golden_inputs_and_column_padding(oracle, bits):
    K, N, block, groups = 35, 2, 16, 3
    mask = (1 << bits) - 1
    codes = np.array([[(r + c) & mask for c in range(N)] for r in range(K)])
    zp = np.array([[(c + g + 1) & mask for c in range(N)] for g in range(groups)])
    scale_ng = np.array([[0.5 * (g + 1) for g in range(groups)] for _ in range(N)])
    B, zpk = ort_pack(codes, zp, bits, block)
    assert B.shape == (N, groups, block * bits // 8)
    assert B.reshape(-1)[0] == {2: 0xE4, 4: 0x10, 8: 0}[bits]
    if bits == 2:
        assert zpk.reshape(-1).tolist() == [0x39, 0x0E]
    elif bits == 4:
        assert zpk.reshape(-1).tolist() == [0x21, 0x03, 0x32, 0x04]
    got = oracle.ort_nbits_decode(B, scale_ng, zpk, K, N, bits, block)
    want = np.array([[float(((r + c) & mask) - ((c + r // block + 1) & mask)) * 0.5 * (r // block + 1)
                      for c in range(N)] for r in range(K)])
    assert np.array_equal(got, want)


def test_fractional_zero_points(oracle):
    """zero points 3.25 / 4.5, scales -0.5 / 0.5 (one block per column)."""
    codes = np.array([[0, 0], [3, 5], [7, 10]])
    B, _ = ort_pack(codes, None, 4, 16)
    got = oracle.ort_nbits_decode(B, np.array([[-0.5], [0.5]]), np.array([[3.25], [4.5]], np.float32), 3, 2, 4, 16)
    assert np.array_equal(got, np.array([[1.625, -2.25], [0.125, 0.25], [-1.875, 2.75]]))


def test_implicit_zero_point_is_half_range(oracle):
    rng = np.random.default_rng(3)
    for bits in (2, 4, 8):
        K, N, block = 64, 5, 32
        codes = rng.integers(0, 1 << bits, (K, N))
        sc = rng.uniform(0.01, 0.1, (N, K // block))
        B, _ = ort_pack(codes, None, bits, block)
        got = oracle.ort_nbits_decode(B, sc, None, K, N, bits, block)
        want = (codes - (1 << (bits - 1))) * sc.T[np.arange(K) // block, :]
        assert np.array_equal(got, want)
