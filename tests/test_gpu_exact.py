"""Bit-exact GPU checks of every k-term of the float GEMM / GEMV paths.

The tolerance tests (test_gpu_float.py and others) bound the fp32 summation
order, and at K = 4096 a BFLOAT16 bound is loose enough to miss a few
dropped or repeated k-terms.  These tests leave no room: on dyadic inputs
(tests/dyadic.py: small-integer activations, weights that are small integers
times powers of two, power-of-two scales) every fp32 partial sum is exact in
any order, so the GPU result must equal, bit for bit,

- the exact sum rounded once to the output type (every element), and
- the oracle chain (the reference's weight rounding, then its k-sequential
  fp32 MatMul, km/kernel_matmul.cc:136-141) on the rows it is run on.

tests/test_exact_inputs.py shows on the CPU, at these depths, that the
premise holds and that one k-term removed per row changes >= 99% of the
outputs it touches.  One-hot activations (one nonzero per row, over every k
of K) read each row of the dequantised weight back exactly, with the
reference data's own scales.
"""
import os

import numpy as np
import pytest
import torch

import dyadic as dy
from test_gpu_float import T, _synth, bits_tensor, tensor_bits

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _exact_on_gpu(oracle, a, w, out, dev):
    """The exact a @ w on the device in float64 (exact under the premise,
    checked here), rounded once to `out` by the oracle's encoder."""
    a64, w64 = torch.from_numpy(a).to(dev, torch.float64), torch.from_numpy(w).to(dev, torch.float64)
    e = dy.lsb_exponent(a) + dy.lsb_exponent(w)
    assert float((a64.abs() @ w64.abs()).max()) < 2.0 ** (24 + e), "dyadic premise"
    y = a64 @ w64
    y32 = y.to(torch.float32)
    assert torch.equal(y32.to(torch.float64), y)
    y32 = y32.cpu().numpy()
    return oracle.f32_to_bf16_bits(y32) if out == "bf16" else oracle.f32_to_f16_bits(y32)


def _chain_rows(oracle, case, rows):
    dt = case["out"]
    w_bits = dy.enc(oracle, case["w"], dt)
    code = oracle.BFLOAT16 if dt == "bf16" else oracle.FLOAT16
    return oracle.matmul_half(case["a_bits"][rows], w_bits, code, nthreads=NT)


def _plus0(x):
    """A one-hot row's exact output as the chain's MatMul forms it: the sum
    starts at +0.0, so a -0 weight (an fp8 or k-quant -0) gives +0."""
    return (np.asarray(x, np.float32) + np.float32(0.0)).astype(np.float32)


def _assert_exact(got, want, what):
    bad = got != want
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outputs differ (first at {np.argwhere(bad)[0]})"


# ---- configuration 4: bf16 x DequantizeLinear(fp8) -> Cast -> MatMul --------

def test_config4_shape_dyadic_bit_exact(olamd, oracle, dev):
    """The full [4096, 4096] x [4096, 14336] fp8 GEMM (the 256 x 256 tiles of
    the first 12288 columns and the 256 x 128 tiles of the rest): every output
    against the exact sum, four rows against the oracle chain."""
    M, K, N = 4096, 4096, 14336
    case = dy.fp8_case(oracle, np.random.default_rng(404), M, K, N)
    y = olamd.dequantize_linear_matmul(bits_tensor(case["a_bits"], "bf16", dev), T(case["x"], dev),
                                       T(case["scale"], dev), None, axis=1, cast_to=olamd.BFLOAT16,
                                       x_dtype=olamd.FLOAT8E4M3FN, x_shape=(K, N))
    got = tensor_bits(y)
    _assert_exact(got, _exact_on_gpu(oracle, case["a"], case["w"], "bf16", dev), "config 4 shape")
    rows = np.array([0, 1, 2049, 4095])
    _assert_exact(got[rows], _chain_rows(oracle, case, rows), "config 4 shape, oracle chain rows")


def test_config4_one_hot_rows_all_k(olamd, oracle, dev):
    """Configuration 4's own weights and scales (N(0,1) fp8 codes, scales
    U(0.005, 0.05)); row m of A is a_m * e_m with a_m in {1, -1, 2, -2}, so
    row m of Y is a_m * W[m] for every k = m of K and every column: W =
    bf16(fp32(decode(q)) * s), the chain's weight (the fused kernel scales the
    single product instead, the same value)."""
    K, N = 4096, 14336
    c4 = _synth().config4_torch(dev, scale=1.0)
    coef = np.array([1.0, -1.0, 2.0, -2.0], np.float32)[np.arange(K) % 4]
    a = np.zeros((K, K), np.float32)
    a[np.arange(K), np.arange(K)] = coef
    y = olamd.dequantize_linear_matmul(bits_tensor(dy.enc(oracle, a, "bf16"), "bf16", dev), c4["w"], c4["scale"],
                                       None, axis=1, cast_to=olamd.BFLOAT16, x_dtype=olamd.FLOAT8E4M3FN,
                                       x_shape=(K, N))
    got = tensor_bits(y)
    w = oracle.dequantize_linear(c4["w"].cpu().numpy(), oracle.FLOAT8E4M3FN, (K, N), c4["scale"].cpu().numpy(),
                                 oracle.FLOAT, None, 1)
    wb = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(w))
    _assert_exact(got, oracle.f32_to_bf16_bits(_plus0(wb * coef[:, None])), "config 4 one-hot rows")


# ---- FLOAT16 / BFLOAT16 MatMul ---------------------------------------------

@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M,K,N", [(1024, 4096, 2048), (300, 4096, 144), (37, 448, 40)])
def test_matmul_half_dyadic_bit_exact(olamd, oracle, dev, dt, M, K, N):
    case = dy.half_case(oracle, np.random.default_rng(M + K + N + len(dt)), M, K, N, dt)
    y = olamd.matmul(bits_tensor(case["a_bits"], dt, dev), bits_tensor(case["b_bits"], dt, dev))
    got = tensor_bits(y)
    _assert_exact(got, dy.exact_out_bits(oracle, case["a"], case["w"], dt), f"MatMul {dt} {M}x{K}x{N}")
    rows = np.array([0, M // 2, M - 1])
    _assert_exact(got[rows], _chain_rows(oracle, case, rows), f"MatMul {dt} oracle rows")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_matmul_half_one_hot_rows_all_k(olamd, oracle, dev, dt):
    M = K = 2048
    N = 512
    rng = np.random.default_rng(17 + len(dt))
    b32 = rng.standard_normal((K, N)).astype(np.float32)
    b = oracle.f32_to_bf16_bits(b32) if dt == "bf16" else oracle.f32_to_f16_bits(b32)
    coef = np.array([1.0, -2.0, 0.5, -1.0], np.float32)[np.arange(K) % 4]
    a = np.zeros((M, K), np.float32)
    a[np.arange(M), np.arange(M) % K] = coef
    y = olamd.matmul(bits_tensor(dy.enc(oracle, a, dt), dt, dev), bits_tensor(b, dt, dev))
    dec = oracle.bf16_bits_to_f32 if dt == "bf16" else oracle.f16_bits_to_f32
    want = _plus0(dec(b) * coef[:, None])
    want = oracle.f32_to_bf16_bits(want) if dt == "bf16" else oracle.f32_to_f16_bits(want)
    _assert_exact(tensor_bits(y), want, f"MatMul {dt} one-hot rows")


# ---- int4 DequantizeLinear -> MatMul: configuration 3's GEMVs and the rest --

@pytest.mark.parametrize("layout", ["onnx", "prepared"])
@pytest.mark.parametrize("signed,zp", [(True, False), (False, True)])
def test_config3_shape_dyadic_bit_exact(olamd, oracle, dev, layout, signed, zp):
    """[8, 4096] x [4096, 11008], block 32 on K, fp16 scales: both GEMVs."""
    M, K, N = 8, 4096, 11008
    case = dy.int4_case(oracle, np.random.default_rng(33 + signed + 2 * zp), M, K, N, 32, signed, zp, "f16")
    code = olamd.INT4 if signed else olamd.UINT4
    x = T(case["x"], dev)
    if layout == "prepared":
        x = olamd.prepare_weight(x, code, (K, N))
    y = olamd.dequantize_linear_matmul(bits_tensor(case["a_bits"], "f16", dev), x, T(case["scale"], dev),
                                       None if case["zp"] is None else T(case["zp"], dev), axis=0, x_dtype=code,
                                       x_shape=(K, N))
    got = tensor_bits(y)
    _assert_exact(got, dy.exact_out_bits(oracle, case["a"], case["w"], "f16"), f"config 3 {layout}")
    _assert_exact(got, _chain_rows(oracle, case, np.arange(M)), f"config 3 {layout}, oracle chain")


@pytest.mark.parametrize("M", [1, 9, 64, 300])
def test_int4_bf16_dyadic_bit_exact(olamd, oracle, dev, M):
    """BFLOAT16 activations: DequantizeLinear(INT4, FLOAT scales) -> Cast ->
    MatMul through the general fused path (dequantised weight, MFMA GEMM)."""
    K, N = 2048, 512
    case = dy.int4_case(oracle, np.random.default_rng(M), M, K, N, 64, True, M % 2 == 1, "bf16")
    y = olamd.dequantize_linear_matmul(bits_tensor(case["a_bits"], "bf16", dev), T(case["x"], dev),
                                       T(case["scale"], dev), None if case["zp"] is None else T(case["zp"], dev),
                                       axis=0, cast_to=olamd.BFLOAT16, x_dtype=olamd.INT4, x_shape=(K, N))
    got = tensor_bits(y)
    _assert_exact(got, dy.exact_out_bits(oracle, case["a"], case["w"], "bf16"), f"int4 bf16 M={M}")


@pytest.mark.parametrize("layout", ["onnx", "prepared"])
def test_int4_gemv_one_hot_rows_all_k(olamd, oracle, dev, layout):
    """Every k of K = 4096 read back by one-hot rows, 16 per GEMV call (the
    decode shape), random fp16 scales (block 32) and zero points."""
    K, N = 4096, 1024
    rng = np.random.default_rng(99)
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(0, 16, (K // 32, N))
    sc = rng.uniform(0.002, 0.02, (K // 32, N)).astype(np.float16)
    x = T(oracle.pack_int4(q.reshape(-1)), dev)
    if layout == "prepared":
        x = olamd.prepare_weight(x, olamd.UINT4, (K, N))
    w = oracle.dequantize_linear(oracle.pack_int4(q.reshape(-1)), oracle.UINT4, (K, N), sc.view(np.uint16),
                                 oracle.FLOAT16, oracle.pack_int4(z.reshape(-1)), 0)
    wf = oracle.f16_bits_to_f32(w)
    zt, st = T(oracle.pack_int4(z.reshape(-1)), dev), T(sc, dev)
    for k0 in range(0, K, 16):
        a = np.zeros((16, K), np.float32)
        coef = np.where(np.arange(16) % 2 == 0, 1.0, -2.0).astype(np.float32)
        a[np.arange(16), k0 + np.arange(16)] = coef
        y = olamd.dequantize_linear_matmul(bits_tensor(dy.enc(oracle, a, "f16"), "f16", dev), x, st, zt, axis=0,
                                           x_dtype=olamd.UINT4, x_shape=(K, N))
        want = oracle.f32_to_f16_bits(_plus0(wf[k0:k0 + 16] * coef[:, None]))
        _assert_exact(tensor_bits(y), want, f"int4 GEMV one-hot rows {k0}..{k0 + 15} ({layout})")


# ---- packed GGUF GEMVs ------------------------------------------------------

@pytest.mark.parametrize("fmt", ["gguf:q4_0", "gguf:q8_0", "gguf:q2_k", "gguf:q3_k", "gguf:q4_k", "gguf:q5_k",
                                 "gguf:q6_k", "gguf:iq4_xs"])
@pytest.mark.parametrize("M,N", [(1, 14336), (8, 2048), (40, 512)])
def test_packed_gemv_dyadic_bit_exact(olamd, oracle, dev, fmt, M, N):
    """The fused GEMVs (M <= 8) and the general path (M = 40: the weight
    decoded to FLOAT16 [N, K], the MFMA GEMM reading its rows)."""
    K = 4096
    case = dy.gguf_case(oracle, np.random.default_rng(M * N + len(fmt)), M, K, N, fmt)
    y = olamd.dequantize_packed_matmul(bits_tensor(case["a_bits"], "f16", dev), T(case["x"], dev), fmt, (N, K))
    got = tensor_bits(y)
    _assert_exact(got, dy.exact_out_bits(oracle, case["a"], case["w"], "f16"), f"{fmt} GEMV {M}x{N}")
    _assert_exact(got, _chain_rows(oracle, case, np.arange(M)), f"{fmt} GEMV, oracle chain")


@pytest.mark.parametrize("fmt", ["gguf:q4_0", "gguf:q8_0"])
@pytest.mark.parametrize("M,N,K", [(1, 37, 256), (2, 129, 6144), (1, 1024, 14336), (2, 6, 8448), (2, 4096, 4096)])
def test_streamed_q0_gemv_dyadic_bit_exact(olamd, oracle, dev, fmt, M, N, K):
    """The streamed q4_0 / q8_0 GEMV (M <= 2, K % 256 == 0): one partial
    chunk, several chunks with a partial last one, N not a multiple of the 4
    outputs of a workgroup."""
    case = dy.gguf_case(oracle, np.random.default_rng(M * N + K + len(fmt)), M, K, N, fmt)
    y = olamd.dequantize_packed_matmul(bits_tensor(case["a_bits"], "f16", dev), T(case["x"], dev), fmt, (N, K))
    got = tensor_bits(y)
    _assert_exact(got, dy.exact_out_bits(oracle, case["a"], case["w"], "f16"), f"{fmt} GEMV {M}x{N}x{K}")


@pytest.mark.parametrize("fmt,block_bytes", [("gguf:q4_0", 18), ("gguf:q8_0", 34), ("gguf:q2_k", 84),
                                             ("gguf:q3_k", 110), ("gguf:q4_k", 144), ("gguf:q5_k", 176),
                                             ("gguf:q6_k", 210), ("gguf:iq4_xs", 136)])
def test_packed_gemv_one_hot_rows_all_k(olamd, oracle, dev, fmt, block_bytes):
    """Random blocks (random finite fp16 scales), every k of K read back by
    one-hot rows, 8 per call."""
    N, K = 512, 2048
    rng = np.random.default_rng(block_bytes)
    bv = oracle.packed_block_values(fmt)
    x = rng.integers(0, 256, (N * K // bv, block_bytes)).astype(np.uint8)
    at = {"gguf:q6_k": 208, "gguf:q2_k": 80, "gguf:q3_k": 108}.get(fmt, 0)
    d = np.float16(rng.uniform(0.0005, 0.004, x.shape[0])).view(np.uint16)
    x[:, at], x[:, at + 1] = d & 255, d >> 8
    if fmt in ("gguf:q2_k", "gguf:q4_k", "gguf:q5_k"):  # dmin follows d
        m = np.float16(rng.uniform(0.0005, 0.004, x.shape[0])).view(np.uint16)
        x[:, at + 2], x[:, at + 3] = m & 255, m >> 8
    x = x.reshape(-1)
    w = oracle.f16_bits_to_f32(oracle.dequantize_packed(x, fmt, (N, K), oracle.FLOAT16))  # [N, K]
    xt = T(x, dev)
    for k0 in range(0, K, 8):
        a = np.zeros((8, K), np.float32)
        coef = np.where(np.arange(8) % 2 == 0, 1.0, -2.0).astype(np.float32)
        a[np.arange(8), k0 + np.arange(8)] = coef
        y = olamd.dequantize_packed_matmul(bits_tensor(dy.enc(oracle, a, "f16"), "f16", dev), xt, fmt, (N, K))
        want = oracle.f32_to_f16_bits(_plus0(w[:, k0:k0 + 8].T * coef[:, None]))
        _assert_exact(tensor_bits(y), want, f"{fmt} one-hot rows {k0}..{k0 + 7}")


# ---- AWQ / GPTQ / MatMulNBits prepared weights -------------------------------

def _prepare(olamd, case, kind, K, N, group, dt, dev):
    ck = case["ckpt"]
    if kind == "awq":
        s = torch.from_numpy(ck["scales"]).to(dev, torch.bfloat16 if dt == "bf16" else torch.float16)
        return olamd.prepare_awq("gemm", T(ck["qweight"], dev), T(ck["qzeros"], dev), s, K, N, group)
    if kind.startswith("gptq"):
        s = torch.from_numpy(ck["scales"]).to(dev, torch.bfloat16 if dt == "bf16" else torch.float16)
        return olamd.prepare_gptq("gptq_v2", T(ck["qweight"], dev), T(ck["qzeros"], dev), s, T(ck["g_idx"], dev),
                                  K, N, 8 if kind.endswith("8") else 4, group)
    return olamd.prepare_matmul_nbits(T(ck["B"], dev), T(ck["scale_bits"].view(np.int16), dev).view(torch.float16),
                                      T(ck["zp"], dev), K, N, ck["bits"], group)


CKPT = [("awq", "f16"), ("awq", "bf16"), ("gptq4", "bf16"), ("gptq8", "f16"), ("gptq8", "bf16"), ("nbits2", "f16"),
        ("nbits4", "f16"), ("nbits8", "f16")]


@pytest.mark.parametrize("kind,dt", CKPT)
@pytest.mark.parametrize("M", [8, 40])
def test_checkpoint_dyadic_bit_exact(olamd, oracle, dev, kind, dt, M):
    """The decode GEMV (M = 8) and the prefill path (M = 40) of prepared AWQ,
    GPTQ and MatMulNBits weights, [M, 4096] x [4096, 1024], group 128."""
    K, N, group = 4096, 1024, 128
    case = dy.ckpt_case(oracle, np.random.default_rng(M + len(kind) * 7 + len(dt)), kind, M, K, N, group, dt)
    prep = _prepare(olamd, case, kind, K, N, group, dt, dev)
    act = torch.bfloat16 if dt == "bf16" else torch.float16
    y = olamd.matmul_nbits(T(case["a_bits"].view(np.int16), dev).view(act), prep)
    got = tensor_bits(y)
    _assert_exact(got, dy.exact_out_bits(oracle, case["a"], case["w"], dt), f"{kind} {dt} M={M}")
    rows = np.array([0, M - 1])
    _assert_exact(got[rows], _chain_rows(oracle, case, rows), f"{kind} {dt}, oracle chain rows")


@pytest.mark.parametrize("kind,dt", [("awq", "bf16"), ("gptq8", "f16"), ("nbits4", "f16")])
def test_checkpoint_one_hot_rows_all_k(olamd, oracle, dev, kind, dt):
    """Every k of K = 1024 read back by one-hot rows, 16 per call (the GEMV)
    and all 1024 rows in one call (the prefill path)."""
    K, N, group = 1024, 256, 64
    case = dy.ckpt_case(oracle, np.random.default_rng(5 + len(kind)), kind, 1, K, N, group, dt)
    prep = _prepare(olamd, case, kind, K, N, group, dt, dev)
    act = torch.bfloat16 if dt == "bf16" else torch.float16
    coef = np.where(np.arange(K) % 2 == 0, 1.0, -2.0).astype(np.float32)
    a = np.zeros((K, K), np.float32)
    a[np.arange(K), np.arange(K)] = coef
    want = dy.enc(oracle, _plus0(case["w"] * coef[:, None]), dt)
    a_bits = dy.enc(oracle, a, dt)
    for r0 in range(0, K, 16):
        y = olamd.matmul_nbits(T(a_bits[r0:r0 + 16].view(np.int16), dev).view(act), prep)
        _assert_exact(tensor_bits(y), want[r0:r0 + 16], f"{kind} {dt} one-hot rows {r0}..")
    y = olamd.matmul_nbits(T(a_bits.view(np.int16), dev).view(act), prep)
    _assert_exact(tensor_bits(y), want, f"{kind} {dt} one-hot rows, one call")
