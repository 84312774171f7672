"""AWQ and GPTQ checkpoint weights on the GPU, against the oracle's decodes
(oracle.awq_decode / oracle.gptq_decode, pinned by the reference tests'
fixtures in test_oracle_awq_gptq.py).

- onnxl_amd_dequantize_awq / _gptq: every value bit for bit, in FLOAT,
  FLOAT16, BFLOAT16 and DOUBLE (the oracle's FLOAT values rounded to nearest
  even), on the reference tests' own fixtures and on larger packed weights
  (act-order group maps and partial groups included).
- onnxl_amd_prepare_awq / _gptq, then the fused DequantizeLinear -> MatMul:
  one-hot activations read rows of W back bit for bit (W = the oracle's
  values rounded to the activations' dtype); random activations match the
  oracle chain (decode, MatMul in that dtype) within the float path's
  tolerance |got - ref| <= 1e-2 |ref| + u sum_k |a w| (u = 2^-11 FLOAT16,
  2^-8 BFLOAT16)."""
import numpy as np
import pytest
import torch

from awq_gptq_cases import awq_fixture, awq_pack, gptq_fixture, gptq_pack
from test_gpu_float import T, assert_close, tensor_bits

pytestmark = pytest.mark.gpu

OUTS = [("FLOAT", torch.float32), ("FLOAT16", torch.float16), ("BFLOAT16", torch.bfloat16), ("DOUBLE", torch.float64)]


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _rounded(values, name, oracle):
    """The oracle's FLOAT values as the output dtype stores them (as comparable arrays)."""
    if name == "FLOAT":
        return values.view(np.uint32)
    if name == "DOUBLE":
        return values.astype(np.float64).view(np.uint64)
    if name == "FLOAT16":
        return oracle.f32_to_f16_bits(values)
    return oracle.f32_to_bf16_bits(values)


def _got(y, name):
    a = y.cpu()
    if name == "FLOAT":
        return a.numpy().view(np.uint32)
    if name == "DOUBLE":
        return a.numpy().view(np.uint64)
    return a.view(torch.int16).numpy().view(np.uint16)


def _f32(a):
    return a.float().numpy() if isinstance(a, torch.Tensor) else np.asarray(a).astype(np.float32)


# ---- dense decode -------------------------------------------------------------

@pytest.mark.parametrize("variant", ["gemm", "gemv", "gemv_fast", "llm-awq"])
@pytest.mark.parametrize("group_size", [-1, 64, 128])
@pytest.mark.parametrize("out", OUTS, ids=[o[0] for o in OUTS])
def test_awq_decode_reference_fixtures(olamd, oracle, dev, variant, group_size, out):
    fx = awq_fixture(variant, group_size)
    _, _, values = oracle.awq_decode(variant, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), 128, 8, group_size)
    code = getattr(olamd, out[0])
    y = olamd.dequantize_awq(variant, *(T(fx[k], dev) for k in ("qweight", "qzeros", "scales")), 128, 8, group_size,
                             output_dtype=code)
    assert np.array_equal(_got(y, out[0]), _rounded(values, out[0], oracle))


@pytest.mark.parametrize("variant,K,N,group,scale_dt", [
    ("gemm", 4096, 512, 128, "f16"), ("gemm", 1024, 264, 64, "bf16"), ("gemv", 2048, 136, 32, "f16"),
    ("gemv", 1536, 40, 512, "f16"), ("gemm8", 768, 96, 128, "f16"), ("gemm8", 512, 64, -1, "bf16")])
def test_awq_decode_packed(olamd, oracle, dev, variant, K, N, group, scale_dt):
    rng = np.random.default_rng(K + N)
    bits = 8 if variant == "gemm8" else 4
    eff = K if group == -1 else group
    groups = K // eff
    codes = rng.integers(0, 1 << bits, (K, N))
    zeros = rng.integers(0, 1 << bits, (groups, N))
    s32 = rng.uniform(0.002, 0.05, (groups, N)).astype(np.float32)
    scales = torch.from_numpy(s32).to(torch.bfloat16) if scale_dt == "bf16" else s32.astype(np.float16)
    pk = awq_pack(variant, codes, zeros, scales if scale_dt == "f16" else scales.float().numpy(), group)
    if scale_dt == "bf16":
        pk["scales"] = scales
    name = "gemm" if variant == "gemm8" else variant
    _, _, values = oracle.awq_decode(name, pk["qweight"], pk["qzeros"], _f32(pk["scales"]), K, N, group, bits=bits)
    for oname, _ in OUTS:
        y = olamd.dequantize_awq(name, T(pk["qweight"], dev), T(pk["qzeros"], dev),
                                 pk["scales"].to(dev) if scale_dt == "bf16" else T(pk["scales"], dev), K, N, group,
                                 bits=bits, output_dtype=getattr(olamd, oname))
        assert np.array_equal(_got(y, oname), _rounded(values, oname, oracle)), (variant, oname)


GPTQ_FIXTURES = [(f, b, w) for f in ("gptq", "gptq_v2", "gptq_p") for b in range(2, 9)
                 for w in (1, 2, 4, 8) if (f == "gptq_p" or b not in (5, 6, 7))
                 and (w == 4 or not (f == "gptq_p" or b in (3, 5, 6, 7)))]


@pytest.mark.parametrize("fmt,bits,width", GPTQ_FIXTURES)
def test_gptq_decode_reference_fixtures(olamd, oracle, dev, fmt, bits, width):
    fx = gptq_fixture(bits, fmt, width)
    _, _, values = oracle.gptq_decode(fmt, bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), fx["g_idx"], 32, 32,
                                      16)
    for oname, _ in OUTS:
        y = olamd.dequantize_gptq(fmt, *(T(fx[k], dev) for k in ("qweight", "qzeros", "scales", "g_idx")), 32, 32,
                                  bits, 16, output_dtype=getattr(olamd, oname))
        assert np.array_equal(_got(y, oname), _rounded(values, oname, oracle)), oname


GPTQ_PACKED = [("gptq_v2", 4, 4, 4096, 256, 128, "f16", False), ("gptq", 4, 4, 2048, 96, 64, "f16", True),
               ("gptq", 3, 4, 1024, 128, 128, "f16", False), ("gptq_v2", 2, 2, 512, 72, 32, "f32", True),
               ("gptq_p", 5, 4, 512, 64, 128, "f16", False), ("gptq_p", 6, 4, 256, 96, -1, "bf16", False),
               ("gptq_p", 7, 4, 384, 32, 64, "f16", True), ("gptq_v2", 8, 8, 512, 40, 128, "f32", False),
               ("gptq_p", 3, 4, 256, 64, 32, "f16", False), ("gptq_v2", 4, 1, 200, 24, 48, "f16", False)]


def _gptq_weight(fmt, bits, width, K, N, group, scale_dt, act_order, seed):
    rng = np.random.default_rng(seed)
    planar = bits in (5, 6, 7) or (fmt == "gptq_p" and bits == 3)
    eff = K if group == -1 else group
    groups = -(-K // eff)
    maxq = (1 << bits) - 1
    codes = rng.integers(0, maxq + 1, (K, N))
    zeros = rng.integers(1, maxq + 1, (groups, N)) if fmt == "gptq" else rng.integers(0, maxq + 1, (groups, N))
    qw, qz = gptq_pack(codes, zeros - 1 if fmt == "gptq" else zeros, bits, width, planar)
    s32 = rng.uniform(0.002, 0.05, (groups, N)).astype(np.float32)
    scales = {"f16": s32.astype(np.float16), "f32": s32,
              "bf16": torch.from_numpy(s32).to(torch.bfloat16)}[scale_dt]
    g_idx = np.arange(K) // eff
    if act_order:
        g_idx = rng.permutation(g_idx)
    return dict(qweight=qw, qzeros=qz, scales=scales, g_idx=g_idx.astype(np.int32))


def _dev(x, dev):
    return x.to(dev) if isinstance(x, torch.Tensor) else T(x, dev)


@pytest.mark.parametrize("fmt,bits,width,K,N,group,scale_dt,act_order", GPTQ_PACKED)
def test_gptq_decode_packed(olamd, oracle, dev, fmt, bits, width, K, N, group, scale_dt, act_order):
    fx = _gptq_weight(fmt, bits, width, K, N, group, scale_dt, act_order, K * N + bits)
    _, _, values = oracle.gptq_decode(fmt, bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), fx["g_idx"], K, N,
                                      group)
    for oname, _ in OUTS:
        y = olamd.dequantize_gptq(fmt, *(_dev(fx[k], dev) for k in ("qweight", "qzeros", "scales", "g_idx")), K, N,
                                  bits, group, output_dtype=getattr(olamd, oname))
        assert np.array_equal(_got(y, oname), _rounded(values, oname, oracle)), oname


# ---- prepared weights on the fused DequantizeLinear -> MatMul ------------------

def _one_hot_rows(olamd, oracle, dev, prep, w_bits, K, act_dt, rows):
    a = np.zeros((len(rows), K), np.uint16)
    a[np.arange(len(rows)), rows] = 0x3F80 if act_dt == torch.bfloat16 else 0x3C00  # 1.0
    y = olamd.matmul_nbits(T(a.view(np.int16), dev).view(act_dt), prep)
    assert np.array_equal(tensor_bits(y), w_bits[rows]), "rows of W"


def _w_bits(values_nk, act_dt, oracle):
    w = np.ascontiguousarray(values_nk.T)  # [K, N]
    return oracle.f32_to_bf16_bits(w) if act_dt == torch.bfloat16 else oracle.f32_to_f16_bits(w)


@pytest.mark.parametrize("variant,K,N,group,scale_dt", [
    ("gemm", 1024, 96, 128, "f16"), ("gemm", 512, 40, 64, "bf16"), ("gemv", 768, 72, 32, "f16"),
    ("gemv", 256, 24, -1, "f16"), ("gemm8", 512, 64, 128, "f16"), ("gemm8", 256, 36, 64, "bf16")])
def test_awq_prepared_one_hot_rows(olamd, oracle, dev, variant, K, N, group, scale_dt):
    rng = np.random.default_rng(7 * K + N)
    bits = 8 if variant == "gemm8" else 4
    eff = K if group == -1 else group
    groups = K // eff
    codes = rng.integers(0, 1 << bits, (K, N))
    zeros = rng.integers(0, 1 << bits, (groups, N))
    s32 = rng.uniform(0.002, 0.05, (groups, N)).astype(np.float32)
    pk = awq_pack(variant, codes, zeros, s32.astype(np.float16), group)
    if scale_dt == "bf16":
        pk["scales"] = torch.from_numpy(s32).to(torch.bfloat16)
    name = "gemm" if variant == "gemm8" else variant
    _, _, values = oracle.awq_decode(name, pk["qweight"], pk["qzeros"], _f32(pk["scales"]), K, N, group, bits=bits)
    act = torch.bfloat16 if scale_dt == "bf16" else torch.float16
    prep = olamd.prepare_awq(name, T(pk["qweight"], dev), T(pk["qzeros"], dev), _dev(pk["scales"], dev), K, N, group,
                             bits=bits)
    _one_hot_rows(olamd, oracle, dev, prep, _w_bits(values, act, oracle), K, act,
                  [0, 1, 2, 31, min(eff, K - 3), K // 2 + 3, K - 2, K - 1])


@pytest.mark.parametrize("fmt,bits,width,K,N,group,scale_dt", [
    ("gptq_v2", 4, 4, 1024, 128, 128, "f16"), ("gptq", 4, 4, 512, 48, 32, "f16"), ("gptq", 2, 4, 512, 64, 64, "f16"),
    ("gptq_v2", 3, 4, 256, 64, 128, "f32"), ("gptq_p", 5, 4, 512, 64, 128, "f16"), ("gptq_p", 6, 4, 256, 32, -1, "bf16"),
    ("gptq_p", 7, 4, 256, 96, 64, "f16"), ("gptq", 8, 8, 384, 40, 128, "f16"), ("gptq_v2", 8, 2, 256, 20, 64, "bf16"),
    ("gptq_p", 3, 4, 256, 64, 32, "f16")])
def test_gptq_prepared_one_hot_rows(olamd, oracle, dev, fmt, bits, width, K, N, group, scale_dt):
    fx = _gptq_weight(fmt, bits, width, K, N, group, scale_dt, False, 3 * K + N + bits)
    _, _, values = oracle.gptq_decode(fmt, bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), fx["g_idx"], K, N,
                                      group)
    act = torch.bfloat16 if scale_dt == "bf16" else torch.float16
    prep = olamd.prepare_gptq(fmt, *(_dev(fx[k], dev) for k in ("qweight", "qzeros", "scales", "g_idx")), K, N, bits,
                              group)
    eff = K if group == -1 else group
    _one_hot_rows(olamd, oracle, dev, prep, _w_bits(values, act, oracle), K, act,
                  [0, 1, 2, 31, min(eff, K - 3), K // 2 + 3, K - 2, K - 1])


@pytest.mark.parametrize("M", [1, 8, 24])
def test_awq_gemm_llama_shape_random(olamd, oracle, dev, M):
    """AWQ gemm, 4 bits, group 128, fp16: [M, 4096] x [4096, 11008] (the decode
    GEMV shape of configuration 3 for M <= 16, the GEMM path above)."""
    K, N, group = 4096, 11008, 128
    rng = np.random.default_rng(M)
    codes = rng.integers(0, 16, (K, N))
    zeros = rng.integers(0, 16, (K // group, N))
    scales = rng.uniform(0.002, 0.02, (K // group, N)).astype(np.float16)
    pk = awq_pack("gemm", codes, zeros, scales, group)
    _, _, values = oracle.awq_decode("gemm", pk["qweight"], pk["qzeros"], _f32(pk["scales"]), K, N, group)
    w_bits = _w_bits(values, torch.float16, oracle)
    prep = olamd.prepare_awq("gemm", pk["qweight"], pk["qzeros"], pk["scales"], K, N, group)  # host payloads
    a = oracle.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    y = olamd.matmul_nbits(T(a.view(np.int16), dev).view(torch.float16), prep)
    ref = oracle.matmul_half(a, w_bits, oracle.FLOAT16, nthreads=8)
    mag = np.abs(oracle.f16_bits_to_f32(a).astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64))
    assert_close(tensor_bits(y), ref, mag, "f16", oracle, f"awq gemm M={M}")


@pytest.mark.parametrize("fmt,bits,scale_dt,M", [("gptq", 4, "f16", 4), ("gptq_p", 6, "f16", 24),
                                                 ("gptq_v2", 8, "bf16", 8), ("gptq_v2", 3, "f32", 2)])
def test_gptq_random_vs_oracle_chain(olamd, oracle, dev, fmt, bits, scale_dt, M):
    K, N, group = 1024, 352, 128
    fx = _gptq_weight(fmt, bits, 4, K, N, group, scale_dt, False, M + bits)
    _, _, values = oracle.gptq_decode(fmt, bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), fx["g_idx"], K, N,
                                      group)
    act = torch.bfloat16 if scale_dt == "bf16" else torch.float16
    dt, code = ("bf16", oracle.BFLOAT16) if act == torch.bfloat16 else ("f16", oracle.FLOAT16)
    w_bits = _w_bits(values, act, oracle)
    prep = olamd.prepare_gptq(fmt, *(_dev(fx[k], dev) for k in ("qweight", "qzeros", "scales", "g_idx")), K, N, bits,
                              group)
    rng = np.random.default_rng(M)
    a32 = rng.standard_normal((M, K)).astype(np.float32)
    a = oracle.f32_to_bf16_bits(a32) if dt == "bf16" else oracle.f32_to_f16_bits(a32)
    y = olamd.matmul_nbits(T(a.view(np.int16), dev).view(act), prep)
    ref = oracle.matmul_half(a, w_bits, code)
    dec = oracle.bf16_bits_to_f32 if dt == "bf16" else oracle.f16_bits_to_f32
    mag = np.abs(dec(a).astype(np.float64)) @ np.abs(dec(w_bits).astype(np.float64))
    assert_close(tensor_bits(y), ref, mag, dt, oracle, f"{fmt} {bits} {scale_dt} M={M}")


def test_unsupported_preparations(olamd, oracle, dev):
    fast = awq_fixture("gemv_fast", 64)
    with pytest.raises(olamd.Unsupported, match="float zero terms"):
        olamd.prepare_awq("gemv_fast", fast["qweight"], fast["qzeros"], fast["scales"], 128, 8, 64)
    fx = gptq_fixture(4)  # the reference fixture's g_idx is k % 2
    with pytest.raises(olamd.Unsupported, match="act-order"):
        olamd.prepare_gptq("gptq_v2", fx["qweight"], fx["qzeros"], fx["scales"], fx["g_idx"], 32, 32, 4, 16)
    part = _gptq_weight("gptq_v2", 4, 4, 200, 24, 64, "f16", False, 5)
    with pytest.raises(olamd.Unsupported, match="partial last group"):
        olamd.prepare_gptq("gptq_v2", part["qweight"], part["qzeros"], part["scales"], part["g_idx"], 200, 24, 4, 64)
