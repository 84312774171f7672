"""Quantized MoE experts on the GPU: onnxl_amd_dequantize_linear_grouped_matmul,
the fused DequantizeLinear -> [Cast] -> GroupedMatMul chain.

- fp8 experts on the matrix cores (FLOAT scales constant along K within an
  expert, Cast to BFLOAT16): on dyadic inputs (tests/dyadic.py: small-integer
  activations, fp8 codes times power-of-two scales) every fp32 partial sum is
  exact and the skipped bf16 rounding of q * s is exact too, so the result
  must equal the oracle chain (oracle.dequantize_linear, the Cast,
  oracle.grouped_matmul: the reference's k-sequential sums,
  math/kernel_grouped_matmul.cc:30-44) bit for bit, in every scale layout,
  with and without a bias; random data against the float64 closed form of the
  chain within the fp8 path's bound (the one configuration 4 uses).
- every other operand set (4- and 8-bit integer experts, zero points, blocked
  scales, FLOAT16 scales, transB): the experts dequantized with the chain's
  roundings, then the library's GroupedMatMul kernels, so the result must
  equal onnxl_amd_grouped_matmul on the oracle-dequantised experts bit for
  bit (that kernel is pinned against the oracle in test_gpu_grouped.py).
"""
import zlib

import numpy as np
import pytest
import torch

import dyadic as dy
from test_gpu_float import T, bits_tensor, tensor_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _routing(rng, M, S, G):
    """Every expert used, one (the last) left empty when G > 2: the routing
    of a top-S MoE step with an idle expert."""
    idx = rng.integers(0, max(G - 1, 1), (M, S)).astype(np.int32)
    idx[0, 0] = 0
    return idx


def _chain(oracle, a_bits, codes, xdt, shape, scale, sdt, zp, axis, cast, idx, bias_bits, tb, out):
    """The oracle chain: DequantizeLinear (scale dtype), optional Cast, then
    GroupedMatMul in the output dtype."""
    w = oracle.dequantize_linear(codes, xdt, shape, scale, sdt, zp, axis)
    if cast == oracle.BFLOAT16:
        w = oracle.f32_to_bf16_bits(w)
    elif cast == oracle.FLOAT16:
        w = oracle.f32_to_f16_bits(w)
    return oracle.grouped_matmul(a_bits, w, idx, bias_bits, tb, out), w


# scale layouts the fp8 core takes: (name, axis, scale shape for [G, K, N])
FP8_LAYOUTS = [("tensor", 1, lambda G, K, N: ()), ("expert", 0, lambda G, K, N: (G,)),
               ("column", 2, lambda G, K, N: (N,)), ("expert_column", 1, lambda G, K, N: (G, 1, N))]


@pytest.mark.parametrize("layout", FP8_LAYOUTS, ids=[f[0] for f in FP8_LAYOUTS])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("K,N", [(1024, 384), (96, 48)], ids=["wide_tiles", "half_k_step"])
def test_fp8_experts_dyadic_bit_exact(olamd, oracle, dev, layout, with_bias, K, N):
    """256 x 256 tiles when K takes whole 64-deep K steps (K = 1024, with a
    partly filled last column tile), 256 x 128 tiles otherwise (K = 96)."""
    name, axis, sshape = layout
    G, M, S = 8, 300, 2
    rng = np.random.default_rng(zlib.crc32(f"{name}{with_bias}{K}".encode()))
    a = dy.sparse_act(rng, (M, K), dy.DENSITY["fp8"])
    codes, q = dy.fp8_codes(oracle, rng, (G, K, N))
    scale = dy.pow2(rng, sshape(G, K, N), 3, 6)
    if name == "expert":
        w = q * scale[:, None, None]
    else:  # a scalar, [N] or [G, 1, N]: NumPy broadcasting over [G, K, N]
        w = q * scale
    for g in range(G):
        dy.check_premise(a.astype(np.float64), w[g].astype(np.float64))
    idx = _routing(rng, M, S, G)
    bias = (rng.integers(-4, 5, (G, N)) * 0.25).astype(np.float32) if with_bias else None
    a_bits = dy.enc(oracle, a, "bf16")
    b_bits = None if bias is None else dy.enc(oracle, bias, "bf16")
    want, _ = _chain(oracle, a_bits, codes, oracle.FLOAT8E4M3FN, (G, K, N), scale, oracle.FLOAT, None, axis,
                     oracle.BFLOAT16, idx, b_bits, 0, oracle.BFLOAT16)
    y = olamd.dequantize_linear_grouped_matmul(
        bits_tensor(a_bits, "bf16", dev), T(codes, dev), T(scale, dev), T(idx, dev), None, axis=axis,
        cast_to=olamd.BFLOAT16, bias=None if b_bits is None else bits_tensor(b_bits, "bf16", dev),
        x_dtype=olamd.FLOAT8E4M3FN, x_shape=(G, K, N))
    got = tensor_bits(y)
    bad = got != want
    assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.size} differ (first at {np.argwhere(bad)[0]})"
    assert np.count_nonzero(got) > 0.3 * got.size  # the outputs are not mostly zero


def test_fp8_experts_random_closed_form(olamd, oracle, dev):
    """Mixtral-like proportions at a small size: N(0,1) bf16 activations, fp8
    codes of N(0,1), per (expert, column) scales U(0.005, 0.05); every
    output against the float64 closed form of the chain (W = bf16(q * s),
    sum in float64) within the bound of the fp8 path: the skipped weight
    rounding (u = 2^-8 relative), fp32 sums in another order (2 K 2^-24 of
    sum |a W|) and one output rounding."""
    G, K, N, M, S = 8, 2048, 1024, 512, 2
    rng = np.random.default_rng(77)
    a_bits = oracle.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    codes = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(G * K * N).astype(np.float32)).reshape(G, K, N)
    scale = rng.uniform(0.005, 0.05, (G, 1, N)).astype(np.float32)
    idx = _routing(rng, M, S, G)
    y = olamd.dequantize_linear_grouped_matmul(
        bits_tensor(a_bits, "bf16", dev), T(codes, dev), T(scale, dev), T(idx, dev), None, axis=1,
        cast_to=olamd.BFLOAT16, x_dtype=olamd.FLOAT8E4M3FN, x_shape=(G, K, N))
    w = T(codes, dev).view(torch.float8_e4m3fn).to(torch.float32) * T(scale, dev)
    w64 = w.to(torch.bfloat16).to(torch.float64)
    a64 = bits_tensor(a_bits, "bf16", dev).to(torch.float64)
    yi = y.to(torch.float64)
    c = 2.0 ** -8 * (1 + 2.0 ** -7)
    for g in range(G):
        pairs = np.argwhere(idx == g)
        if pairs.size == 0:
            continue
        rows = torch.from_numpy(pairs[:, 0]).to(dev)
        ref = a64[rows] @ w64[g]
        mag = a64[rows].abs() @ w64[g].abs()
        err = (yi[rows, torch.from_numpy(pairs[:, 1]).to(dev)] - ref).abs()
        bad = ~(err <= c * ref.abs() + (c + 2.0 * K * 2.0 ** -24) * mag)
        assert int(bad.sum()) == 0, f"expert {g}: {int(bad.sum())} outside the bound (max err {float(err.max()):.3g})"
    assert bool(torch.isfinite(y.float()).all())
    # the chain itself on a few pairs, to pin the weight decode and scale layout
    pick = np.array([0, 1, M - 1])
    want, _ = _chain(oracle, a_bits[pick], codes, oracle.FLOAT8E4M3FN, (G, K, N), scale, oracle.FLOAT, None, 1,
                     oracle.BFLOAT16, idx[pick], None, 0, oracle.BFLOAT16)
    got = oracle.bf16_bits_to_f32(tensor_bits(y)[pick]).astype(np.float64)
    ref = oracle.bf16_bits_to_f32(want).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2.0 ** -6 * np.abs(ref) + 1e-2)


# (x dtype, scale kind, axis, zero point, scale dtype, cast, activation dtype, transB)
GENERAL = [
    ("int4", "block32", 1, True, "f32", "bf16", "bf16", 0),
    ("uint4", "block64", 1, True, "f16", None, "f16", 0),
    ("int8", "tensor", 1, True, "f32", "f16", "f16", 0),
    ("uint8", "column", 2, True, "f32", "bf16", "bf16", 0),
    ("uint8", "expert", 0, False, "f16", None, "f16", 1),
    ("int4", "column_t", 1, False, "f32", "bf16", "bf16", 1),
    ("fp8", "column", 2, False, "f16", None, "f16", 0),
    ("fp8", "block32_t", 2, False, "f32", "bf16", "bf16", 1),
    ("fp8", "column", 2, True, "f32", "bf16", "bf16", 0),
]


@pytest.mark.parametrize("case", GENERAL, ids=["-".join(str(v) for v in c) for c in GENERAL])
def test_general_experts_match_grouped_matmul(olamd, oracle, dev, case):
    xname, kind, axis, with_zp, sdt, cast, adt, tb = case
    G, K, N, M, S = 6, 256, 96, 130, 2
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    shape = (G, N, K) if tb else (G, K, N)
    xdt = {"int4": oracle.INT4, "uint4": oracle.UINT4, "int8": oracle.INT8, "uint8": oracle.UINT8,
           "fp8": oracle.FLOAT8E4M3FN}[xname]
    if xname in ("int4", "uint4"):
        vals = dy.int4_codes(rng, shape, xname == "int4")
        codes = oracle.pack_int4(vals.reshape(-1))
    elif xname == "fp8":
        codes = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(int(np.prod(shape))).astype(np.float32))
    else:
        info = np.iinfo(np.int8 if xname == "int8" else np.uint8)
        codes = rng.integers(info.min, info.max + 1, shape).astype(np.int8 if xname == "int8" else np.uint8)
        codes = codes.view(np.uint8).reshape(-1)
    ax_len = shape[axis]
    sshape = {"tensor": (), "column": (ax_len,), "expert": (ax_len,), "column_t": (ax_len,),
              "block32": tuple(d // 32 if i == axis else d for i, d in enumerate(shape)),
              "block64": tuple(d // 64 if i == axis else d for i, d in enumerate(shape)),
              "block32_t": tuple(d // 32 if i == axis else d for i, d in enumerate(shape))}[kind]
    scale = rng.uniform(0.002, 0.02, sshape).astype(np.float32)
    if sdt == "f16":
        scale_arg = oracle.f32_to_f16_bits(scale).reshape(sshape)
        scale_code = oracle.FLOAT16
        scale_t = T(scale_arg.view(np.int16), dev).view(torch.float16)
    else:
        scale_arg, scale_code, scale_t = scale, oracle.FLOAT, T(scale, dev)
    zp = zp_t = None
    if with_zp:
        n = int(np.prod(sshape)) if sshape else 1
        if xname in ("int4", "uint4"):
            zv = dy.int4_codes(rng, (n,), xname == "int4")
            zp = oracle.pack_int4(zv)
        elif xname == "fp8":
            zp = np.zeros(n, np.uint8)  # an all-zero fp8 zero point (not the fused path)
        else:
            info = np.iinfo(np.int8 if xname == "int8" else np.uint8)
            zp = rng.integers(info.min, info.max + 1, n).astype(np.int8 if xname == "int8" else np.uint8)
            zp = zp.view(np.uint8)
        zp = zp.reshape(sshape) if zp.size == n and xname not in ("int4", "uint4") else zp
        zp_t = T(zp, dev)
    a = rng.standard_normal((M, K)).astype(np.float32)
    a_bits = oracle.f32_to_bf16_bits(a) if adt == "bf16" else oracle.f32_to_f16_bits(a)
    out = oracle.BFLOAT16 if adt == "bf16" else oracle.FLOAT16
    cast_code = {None: 0, "bf16": oracle.BFLOAT16, "f16": oracle.FLOAT16}[cast]
    idx = _routing(rng, M, S, G)
    w = oracle.dequantize_linear(codes, xdt, shape, scale_arg, scale_code, zp, axis)
    if cast_code == oracle.BFLOAT16:
        w = oracle.f32_to_bf16_bits(w)
    elif cast_code == oracle.FLOAT16:
        w = oracle.f32_to_f16_bits(w)
    w = np.asarray(w, np.uint16).reshape(shape)
    y = olamd.dequantize_linear_grouped_matmul(
        bits_tensor(a_bits, adt, dev), T(codes, dev), scale_t, T(idx, dev), zp_t, axis=axis, cast_to=cast_code,
        transB=tb, x_dtype=xdt, x_shape=shape)
    ref = olamd.grouped_matmul(bits_tensor(a_bits, adt, dev), bits_tensor(w, adt, dev), T(idx, dev), None, tb)
    got, want = tensor_bits(y), tensor_bits(ref)
    bad = got != want
    assert not bad.any(), f"{case}: {int(bad.sum())} of {bad.size} differ"
    # and one pair against the oracle's own GroupedMatMul, within the float tolerance
    chain = oracle.grouped_matmul(a_bits[:1], w, idx[:1], None, tb, out)
    dec = oracle.bf16_bits_to_f32 if adt == "bf16" else oracle.f16_bits_to_f32
    assert np.allclose(dec(got[:1]), dec(chain), rtol=2e-2, atol=2e-2)


def test_validation_order(olamd, dev):
    """The chain's node checks, in its order: DequantizeLinear's, the Cast's,
    then GroupedMatMul's."""
    a = torch.zeros((4, 64), dtype=torch.bfloat16, device=dev)
    x = torch.zeros((2, 64, 32), dtype=torch.uint8, device=dev)
    idx = torch.zeros((4, 1), dtype=torch.int32, device=dev)
    sc = torch.ones((32,), device=dev)
    with pytest.raises(olamd.InvalidArgument, match="axis out of range"):
        olamd.dequantize_linear_grouped_matmul(a, x, sc, idx, axis=3, cast_to=olamd.BFLOAT16,
                                               x_dtype=olamd.FLOAT8E4M3FN)
    with pytest.raises(olamd.InvalidArgument, match="element count must equal axis dimension"):
        olamd.dequantize_linear_grouped_matmul(a, x, sc, idx, axis=1, cast_to=olamd.BFLOAT16,
                                               x_dtype=olamd.FLOAT8E4M3FN)
    with pytest.raises(olamd.InvalidArgument, match="weights must match the input dtype"):
        olamd.dequantize_linear_grouped_matmul(a, x, sc, idx, axis=2, cast_to=olamd.FLOAT16,
                                               x_dtype=olamd.FLOAT8E4M3FN)
    with pytest.raises(olamd.InvalidArgument, match="incompatible input dimensions"):
        olamd.dequantize_linear_grouped_matmul(torch.zeros((4, 32), dtype=torch.bfloat16, device=dev), x, sc, idx,
                                               axis=2, cast_to=olamd.BFLOAT16, x_dtype=olamd.FLOAT8E4M3FN)
    y = olamd.dequantize_linear_grouped_matmul(a, x, sc, idx, axis=2, cast_to=olamd.BFLOAT16,
                                               x_dtype=olamd.FLOAT8E4M3FN)
    assert tuple(y.shape) == (4, 1, 32) and not bool(y.float().abs().sum())
