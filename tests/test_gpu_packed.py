"""GPU parity of DequantizePacked for all 27 GGUF profiles (the codebook
profiles iq2_xxs, iq2_xs, iq2_s, iq3_xxs, iq3_s, iq1_s and iq1_m included)
against the oracle: bit-exact in all four output dtypes (FLOAT, FLOAT16,
BFLOAT16, DOUBLE).  The reference test's corpus is checked against its GGML-C hashes
through the GPU too; random blocks include NaN, infinite, subnormal and
maximal fp16 scales; outputs at unaligned addresses take the per-element
stores."""
import numpy as np
import pytest
import torch

from test_oracle_packed import ALL_FORMATS, FORMATS, block_values, corpus, d_offset, fnv1a64

pytestmark = pytest.mark.gpu
OUT = {"float": (1, torch.float32), "float16": (10, torch.float16), "bfloat16": (16, torch.bfloat16),
       "double": (11, torch.float64)}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _bits(t, out):
    c = t.cpu()
    if out in ("float16", "bfloat16"):
        return c.view(torch.int16).numpy().view(np.uint16)
    return c.numpy()


@pytest.mark.parametrize("fmt", ALL_FORMATS)
def test_corpus_hashes_on_gpu(olamd, oracle, golden, dev, fmt):
    g = golden["dequantize_packed_gguf"]
    x = corpus(oracle, fmt, g["corpus_scales"])
    y = olamd.dequantize_packed(torch.from_numpy(x).to(dev), fmt, (2, 32 * block_values(fmt)))
    assert fnv1a64(y.cpu().numpy()) == g["fnv1a64"][fmt]


@pytest.mark.parametrize("out", list(OUT))
@pytest.mark.parametrize("fmt", ALL_FORMATS)
def test_random_blocks_vs_oracle(olamd, oracle, dev, fmt, out):
    rng = np.random.default_rng(len(fmt) * 7 + len(out) + ALL_FORMATS.index(fmt) * 101)
    size = oracle.packed_block_bytes(fmt)
    bv = block_values(fmt)
    shapes = [(bv,), (3, 5, 2 * bv), (7, 4096), (1, 3 * bv)]
    at = d_offset(fmt)  # the fp16 d (None: q8_k's fp32 d, the fp4 scale bytes)
    for shape in shapes:
        nb = int(np.prod(shape)) // bv
        x = rng.integers(0, 256, (nb, size)).astype(np.uint8)
        if at is not None:
            # scales: random fp16 bit patterns, with NaN, inf, subnormal and 65504 among them
            special = np.array([0x7E00, 0xFC00, 0x0001, 0x7BFF, 0x8000, 0x3C00], np.uint16)
            d = rng.integers(0, 65536, nb).astype(np.uint16)
            d[: min(nb, len(special))] = special[: min(nb, len(special))]
            x[:, at], x[:, at + 1] = d & 255, d >> 8
        elif fmt == "gguf:q8_k":
            # fp32 d: NaN, -inf, the smallest subnormal, the largest finite, -0, 1
            special = np.array([0x7FC00000, 0xFF800000, 0x00000001, 0x7F7FFFFF, 0x80000000, 0x3F800000], np.uint32)
            d = rng.integers(0, 2 ** 32, nb, dtype=np.uint64).astype(np.uint32)
            d[: min(nb, len(special))] = special[: min(nb, len(special))]
            for b in range(4):
                x[:, b] = (d >> (8 * b)) & 255
        elif fmt == "gguf:mxfp4":
            x[: min(nb, 4), 0] = [0, 1, 2, 255][: min(nb, 4)]  # the two subnormal scales, the largest
        x = x.reshape(-1)
        want = oracle.dequantize_packed(x, fmt, shape, OUT[out][0])
        for offset in (0, 1):
            if offset:
                raw = torch.empty(int(np.prod(shape)) + 1, dtype=OUT[out][1], device=dev)
                y = raw[1:].view(shape)
            else:
                y = None
            got = olamd.dequantize_packed(torch.from_numpy(x).to(dev), fmt, shape, OUT[out][0], out=y)
            g = _bits(got, out)
            if out in ("float", "double"):
                same = np.array_equal(g.view(np.uint32 if out == "float" else np.uint64),
                                      want.view(np.uint32 if out == "float" else np.uint64))
            else:
                same = np.array_equal(g, want)
            assert same, (fmt, out, shape, offset)


def test_empty_shape(olamd, dev):
    y = olamd.dequantize_packed(torch.zeros(0, dtype=torch.uint8, device=dev), "gguf:q4_0", (0, 32))
    assert tuple(y.shape) == (0, 32)


# ---- fused q4_0 / q8_0 GEMV: y = a @ DequantizePacked(W)^T -------------------

def _block_weight(rng, N, K, block_bytes):
    blocks = rng.integers(0, 256, (N * K // 32, block_bytes)).astype(np.uint8)
    d = np.float16(rng.uniform(0.001, 0.05, N * K // 32)).view(np.uint16)
    blocks[:, 0], blocks[:, 1] = d & 255, d >> 8
    return blocks.reshape(-1)


def _q4_0_weight(rng, N, K):
    return _block_weight(rng, N, K, 18)


def _k_weight(rng, N, K, fmt):
    """Random q4_k / q6_k blocks with small finite fp16 d (and dmin)."""
    size = 144 if fmt == "gguf:q4_k" else 210
    blocks = rng.integers(0, 256, (N * K // 256, size)).astype(np.uint8)
    d = np.float16(rng.uniform(0.0005, 0.004, N * K // 256)).view(np.uint16)
    at = 208 if fmt == "gguf:q6_k" else 0
    blocks[:, at], blocks[:, at + 1] = d & 255, d >> 8
    if fmt == "gguf:q4_k":
        m = np.float16(rng.uniform(0.0005, 0.004, N * K // 256)).view(np.uint16)
        blocks[:, 2], blocks[:, 3] = m & 255, m >> 8
    return blocks.reshape(-1)


_K_SHAPES = [(1, 96, 256), (3, 200, 512), (8, 64, 4096), (2, 1000, 1024), (1, 4096, 11008 // 256 * 256), (5, 37, 2304)]


@pytest.mark.parametrize("fmt", ["gguf:q2_k", "gguf:q3_k", "gguf:q4_k", "gguf:q5_k", "gguf:q6_k", "gguf:iq4_xs"])
@pytest.mark.parametrize("M,N,K", _K_SHAPES)
def test_k_quant_gemv_vs_chain(olamd, oracle, dev, fmt, M, N, K):
    """The fused 256-value GEMVs against the chain DequantizePacked(FLOAT16)
    -> MatMul(a, W^T): same weight rounding, fp32 sums in another order."""
    from test_gpu_float import assert_close
    rng = np.random.default_rng(M * 7919 + N * 31 + K + len(fmt))
    x = (_k_weight(rng, N, K, fmt) if fmt in ("gguf:q4_k", "gguf:q6_k")
         else _finite_blocks(oracle, rng, fmt, N * K // 256))
    a = np.float16(rng.standard_normal((M, K)))
    w_bits = oracle.dequantize_packed(x, fmt, (N, K), 10)
    ref = oracle.matmul_half(a.view(np.uint16), np.ascontiguousarray(w_bits.T), 10)
    got = olamd.dequantize_packed_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(x).to(dev), fmt, (N, K))
    got_bits = got.cpu().view(torch.int16).numpy().view(np.uint16)
    mag = np.abs(a.astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64)).T
    assert_close(got_bits, ref, mag, "f16", oracle, f"{fmt} gemv {M}x{N}x{K}")


_GEMV_SHAPES = [(1, 96, 64), (3, 200, 256), (8, 64, 4096), (2, 1000, 1024), (1, 14336, 4096), (5, 37, 2112),
                (4, 129, 6144), (1, 37, 256), (2, 129, 6144), (1, 1024, 14336), (2, 6, 8448)]


@pytest.mark.parametrize("fmt,block_bytes", [("gguf:q4_0", 18), ("gguf:q8_0", 34)])
@pytest.mark.parametrize("M,N,K", _GEMV_SHAPES)
def test_packed_gemv_vs_chain(olamd, oracle, dev, fmt, block_bytes, M, N, K):
    """The chain: DequantizePacked(fmt, [N, K], FLOAT16), then the fp16
    MatMul of a with its transpose (fp32 accumulation).  The fused kernel
    rounds the weights exactly as the chain does; only the summation order
    differs, so the float path's tolerance applies:
        |got - ref| <= 1e-2 * |ref| + 2^-11 * sum_k |a_mk * w_nk|."""
    from test_gpu_float import assert_close
    rng = np.random.default_rng(M * 7919 + N * 31 + K + block_bytes)
    x = _block_weight(rng, N, K, block_bytes)
    a = np.float16(rng.standard_normal((M, K)))
    w_bits = oracle.dequantize_packed(x, fmt, (N, K), 10)
    ref = oracle.matmul_half(a.view(np.uint16), np.ascontiguousarray(w_bits.T), 10)
    got = olamd.dequantize_packed_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(x).to(dev), fmt, (N, K))
    got_bits = got.cpu().view(torch.int16).numpy().view(np.uint16)
    mag = np.abs(a.astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64)).T
    assert_close(got_bits, ref, mag, "f16", oracle, f"{fmt} gemv {M}x{N}x{K}")


def _finite_blocks(oracle, rng, fmt, nblocks):
    """Random blocks of `fmt` with small finite scales (whatever the format
    keeps them in): the codes random, the outputs finite."""
    size = oracle.packed_block_bytes(fmt)
    x = rng.integers(0, 256, (nblocks, size)).astype(np.uint8)
    at = d_offset(fmt)
    if at is not None:
        d = oracle.f32_to_f16_bits(rng.uniform(0.001, 0.01, nblocks).astype(np.float32))
        x[:, at], x[:, at + 1] = d & 255, d >> 8
        if fmt in ("gguf:q4_1", "gguf:q5_1", "gguf:q2_k", "gguf:q4_k", "gguf:q5_k"):
            m = oracle.f32_to_f16_bits(rng.uniform(-0.01, 0.01, nblocks).astype(np.float32))
            x[:, at + 2], x[:, at + 3] = m & 255, m >> 8
    elif fmt == "gguf:q8_k":
        d = rng.uniform(0.001, 0.01, nblocks).astype(np.float32).view(np.uint32)
        for b in range(4):
            x[:, b] = (d >> (8 * b)) & 255
    elif fmt == "gguf:mxfp4":
        x[:, 0] = rng.integers(118, 124, nblocks)  # 2^-9 .. 2^-4
    elif fmt == "gguf:nvfp4":
        x[:, 0:4] = rng.integers(0x18, 0x28, (nblocks, 4))  # ue4m3 2^-5 .. 2^-3 range
    elif fmt == "gguf:iq1_m":
        d = oracle.f32_to_f16_bits(rng.uniform(0.001, 0.01, nblocks).astype(np.float32)).astype(np.int64)
        for j in range(4):
            w = (x[:, 48 + 2 * j].astype(np.int64) | (x[:, 49 + 2 * j].astype(np.int64) << 8)) & 0x0FFF
            w |= ((d >> (4 * j)) & 15) << 12
            x[:, 48 + 2 * j], x[:, 49 + 2 * j] = w & 255, w >> 8
    return x.reshape(-1)


def _chain_vs_gpu(olamd, oracle, dev, fmt, M, N, K, seed):
    from test_gpu_float import assert_close
    rng = np.random.default_rng(seed)
    x = _finite_blocks(oracle, rng, fmt, N * K // block_values(fmt))
    a = np.float16(rng.standard_normal((M, K)))
    w_bits = oracle.dequantize_packed(x, fmt, (N, K), 10)
    ref = oracle.matmul_half(a.view(np.uint16), np.ascontiguousarray(w_bits.T), 10, nthreads=8)
    got = olamd.dequantize_packed_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(x).to(dev), fmt, (N, K))
    got_bits = got.cpu().view(torch.int16).numpy().view(np.uint16)
    mag = np.abs(a.astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64)).T
    assert_close(got_bits, ref, mag, "f16", oracle, f"{fmt} {M}x{N}x{K}")


@pytest.mark.parametrize("fmt", ALL_FORMATS)
def test_packed_matmul_prefill_every_format(olamd, oracle, dev, fmt):
    """M = 40 (past the decode GEMVs): the weight decoded to FLOAT16 [N, K] on
    the device, then the MFMA GEMM reading its rows as B; the oracle chain
    DequantizePacked(FLOAT16) -> Transpose -> MatMul within the float
    tolerance (same weight rounding, another fp32 summation order)."""
    _chain_vs_gpu(olamd, oracle, dev, fmt, 40, 96, 512, ALL_FORMATS.index(fmt))


@pytest.mark.parametrize("fmt,M,N,K", [("gguf:q4_0", 300, 160, 1024), ("gguf:q4_k", 257, 48, 2048),
                                       ("gguf:iq2_xs", 9, 64, 256), ("gguf:q5_0", 1, 32, 64),
                                       ("gguf:q8_0", 3, 40, 32), ("gguf:q6_k", 24, 37, 512),
                                       ("gguf:mxfp4", 5, 21, 96)])
def test_packed_matmul_general_shapes(olamd, oracle, dev, fmt, M, N, K):
    """Ragged M tiles, a decode shape of a format without a fused GEMV, K %
    64 != 0 for q8_0, and N % 16 != 0 (the one-thread-per-output kernel)."""
    _chain_vs_gpu(olamd, oracle, dev, fmt, M, N, K, M * N + K)


@pytest.mark.parametrize("fmt,bpb", [("gguf:q4_0", 18), ("gguf:q8_0", 34)])
def test_packed_gemv_empty(olamd, dev, fmt, bpb):
    """MatMul semantics: a [0, K] activation gives an empty [0, N] result, and
    N = 0 an empty [M, 0] one (no launch)."""
    y = olamd.dequantize_packed_matmul(torch.zeros((0, 64), dtype=torch.float16, device=dev),
                                       torch.zeros(4 * 2 * bpb, dtype=torch.uint8, device=dev), fmt, (4, 64))
    assert tuple(y.shape) == (0, 4)
    y = olamd.dequantize_packed_matmul(torch.zeros((3, 64), dtype=torch.float16, device=dev),
                                       torch.zeros(0, dtype=torch.uint8, device=dev), fmt, (0, 64))
    torch.cuda.synchronize()
    assert tuple(y.shape) == (3, 0)
