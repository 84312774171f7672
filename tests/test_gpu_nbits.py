"""ORT MatMulNBits weights (2, 4 and 8 bits) on the GPU: prepared by
onnxl_amd_prepare_matmul_nbits into the fused DequantizeLinear -> MatMul
operands (2-bit codes as 4-bit ones in the same tiled layout), then MatMul(A, W) with
W = oracle.ort_nbits_decode rounded to FLOAT16 (the reference's decode,
pinned by its golden test in test_oracle_nbits.py).  One-hot activations
read single rows of W back bit for bit (one exact product per output);
random activations match the oracle chain (decode, fp16 MatMul) within the
float path's tolerance |got - ref| <= 1e-2 |ref| + 2^-11 sum_k |a w|."""
import numpy as np
import pytest
import torch

from nbits_cases import ort_pack
from test_gpu_float import T, assert_close, tensor_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _weight(oracle, rng, K, N, bits, block, with_zp):
    groups = K // block
    codes = rng.integers(0, 1 << bits, (K, N))
    zp = rng.integers(0, 1 << bits, (groups, N)) if with_zp else None
    scale_bits = oracle.f32_to_f16_bits(rng.uniform(0.002, 0.05, (N, groups)).astype(np.float32))
    B, zpk = ort_pack(codes, zp, bits, block)
    w = oracle.ort_nbits_decode(B, oracle.f16_bits_to_f32(scale_bits), zpk, K, N, bits, block)
    w_bits = oracle.f32_to_f16_bits(w.astype(np.float32))  # exact in fp32: one fp16 rounding
    return B, scale_bits, zpk, w_bits


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("with_zp", [False, True])
@pytest.mark.parametrize("K,N,block", [(256, 96, 32), (512, 40, 128), (128, 34, 16)])
def test_one_hot_rows_bit_exact(olamd, oracle, dev, bits, with_zp, K, N, block):
    rng = np.random.default_rng(K + N + block + bits + with_zp)
    B, sb, zpk, w_bits = _weight(oracle, rng, K, N, bits, block, with_zp)
    prep = olamd.prepare_matmul_nbits(T(B, dev), T(sb.view(np.int16), dev).view(torch.float16),
                                      None if zpk is None else T(zpk, dev), K, N, bits, block)
    rows = [0, 1, 2, 31, block, K // 2 + 3, K - 2, K - 1]
    a = np.zeros((8, K), np.uint16)
    a[np.arange(8), rows] = 0x3C00  # 1.0
    y = olamd.matmul_nbits(T(a.view(np.int16), dev).view(torch.float16), prep)
    assert np.array_equal(tensor_bits(y), w_bits[rows]), "rows of W"


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("with_zp", [False, True])
@pytest.mark.parametrize("M", [1, 8, 24])
def test_random_vs_oracle_chain(olamd, oracle, dev, bits, with_zp, M):
    K, N, block = 1024, 352, 64
    rng = np.random.default_rng(M * 13 + bits + with_zp)
    B, sb, zpk, w_bits = _weight(oracle, rng, K, N, bits, block, with_zp)
    a = oracle.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    prep = olamd.prepare_matmul_nbits(B, sb, zpk, K, N, bits, block)  # host payloads
    y = olamd.matmul_nbits(T(a.view(np.int16), dev).view(torch.float16), prep)
    ref = oracle.matmul_half(a, w_bits, oracle.FLOAT16)
    mag = np.abs(oracle.f16_bits_to_f32(a).astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64))
    assert_close(tensor_bits(y), ref, mag, "f16", oracle, f"nbits {bits} zp={with_zp} M={M}")


def test_llama_mlp_shape_int4_with_zero_points(olamd, oracle, dev):
    """The decode GEMV shape of configuration 3 (fp16 [8, 4096] x [4096, 11008],
    block 32) in the ORT 4-bit format with zero points."""
    K, N, block = 4096, 11008, 32
    rng = np.random.default_rng(2024)
    B, sb, zpk, w_bits = _weight(oracle, rng, K, N, 4, block, True)
    a = oracle.f32_to_f16_bits(rng.standard_normal((8, K)).astype(np.float32))
    prep = olamd.prepare_matmul_nbits(T(B, dev), T(sb.view(np.int16), dev).view(torch.float16), T(zpk, dev), K, N, 4,
                                      block)
    y = olamd.matmul_nbits(T(a.view(np.int16), dev).view(torch.float16), prep)
    ref = oracle.matmul_half(a, w_bits, oracle.FLOAT16, nthreads=8)
    mag = np.abs(oracle.f16_bits_to_f32(a).astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64))
    assert_close(tensor_bits(y), ref, mag, "f16", oracle, "nbits llama shape")


def test_unsupported_and_invalid(olamd, oracle, dev):
    rng = np.random.default_rng(1)
    B, sb, zpk, _ = _weight(oracle, rng, 64, 8, 4, 16, True)
    with pytest.raises(olamd.Unsupported, match="multiple of block_size"):  # the reference's K = 35 golden shape
        olamd.prepare_matmul_nbits(np.zeros((2, 3, 8), np.uint8), np.zeros((2, 3), np.uint16), None, 35, 2, 4, 16)
    with pytest.raises(olamd.InvalidArgument, match="power of two"):
        olamd.prepare_matmul_nbits(B, sb, zpk, 64, 8, 4, 8)
    bad = sb.copy()
    bad[0, 0] = 0x7C00  # +inf
    with pytest.raises(olamd.InvalidArgument, match="Nonfinite ORT MatMulNBits scale"):
        olamd.prepare_matmul_nbits(B, bad, zpk, 64, 8, 4, 16)
    # 4 groups, 2 per byte: no padding; 3 groups (K = 48) pad the high nibble
    B3, sb3, zp3, _ = _weight(oracle, rng, 48, 8, 4, 16, True)
    zbad = zp3.copy()
    zbad[0, -1] |= 0x10
    with pytest.raises(olamd.InvalidArgument, match="zero-point padding"):
        olamd.prepare_matmul_nbits(B3, sb3, zbad, 48, 8, 4, 16)
