"""bitsandbytes weights on the GPU against the oracle (oracle.bnb_*, pinned
by bitsandbytes' own outputs in test_oracle_bnb.py).

- onnxl_amd_dequantize_bitsandbytes: every value bit for bit in FLOAT,
  FLOAT16 and BFLOAT16 on the reference's golden cases (bitsandbytes 0.50.2)
  and fixtures, and on larger random nf4 / fp4 / int8 weights (every block
  size, nested statistics, partial last blocks, rows that do not divide
  8); the reference's error messages for invalid tables, absmax and
  nonfinite reconstructions.
- onnxl_amd_prepare_bitsandbytes, then onnxl_amd_bitsandbytes_matmul (the
  fused GEMV for FLOAT16 nf4 / fp4 at M <= 4, the decoded weight and the
  MFMA GEMM otherwise): one-hot activations read every weight back bit for
  bit; random activations match the oracle chain (decode to the dtype, then
  MatMul(a, W^T)) within the float path's tolerance |got - ref| <= 1e-2 |ref|
  + u sum_k |a w| (u = 2^-11 FLOAT16, 2^-8 BFLOAT16)."""
import ctypes

import numpy as np
import pytest
import torch

from test_gpu_float import T, assert_close, tensor_bits
from test_oracle_bnb import _cases, _cc_fixture, golden_case

pytestmark = pytest.mark.gpu

DTYPES = [(1, torch.float32), (10, torch.float16), (16, torch.bfloat16)]


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _weight(olamd, dev, fmt, rows, cols, block, kw):
    """An olamd.BnbWeight on the device from oracle-style arguments."""
    qm = kw.get("quant_map")
    nested = kw.get("nested_absmax") is not None
    return olamd.BnbWeight(fmt, rows, cols, T(kw["codes"].reshape(-1), dev), T(kw["absmax"], dev),
                           None if qm is None else T(qm, dev), block,
                           T(kw["nested_absmax"], dev) if nested else None,
                           T(kw["nested_map"], dev) if nested else None, 256 if nested else 0,
                           kw.get("offset", 0.0))


def _bits(t):
    return t.cpu().numpy().view(np.uint32) if t.dtype == torch.float32 else tensor_bits(t)


def _expect(oracle, fmt, rows, cols, block, kw, code):
    args = {k: v for k, v in kw.items() if k != "quant_map"}
    rc, ref = oracle.bnb_reconstruct(fmt, rows, cols, block, **args, out_dtype=code)
    assert rc == 0
    return ref.view(np.uint32) if code == 1 else ref


@pytest.mark.parametrize("code,tdt", DTYPES)
@pytest.mark.parametrize("name", [c["name"] for c in _cases()])
def test_golden_decode(olamd, oracle, dev, name, code, tdt):
    c = next(c for c in _cases() if c["name"] == name)
    fmt, rows, cols, block, kw, expected = golden_case(c)
    w = _weight(olamd, dev, fmt, rows, cols, block, kw)
    got = olamd.dequantize_bitsandbytes(w, code)
    if code == 1:
        assert np.array_equal(_bits(got), expected.view(np.uint32)), name
    assert np.array_equal(_bits(got), _expect(oracle, fmt, rows, cols, block, kw, code)), name


@pytest.mark.parametrize("nested", [False, True])
def test_cc_fixture_decode(olamd, oracle, dev, nested):
    codes, kw = _cc_fixture(nested)
    kw = dict(kw, codes=codes, quant_map=oracle.bnb_table("nf4"))
    w = _weight(olamd, dev, "nf4", 3, 11, 32, kw)
    for code, _ in DTYPES:
        assert np.array_equal(_bits(olamd.dequantize_bitsandbytes(w, code)), _expect(oracle, "nf4", 3, 11, 32, kw, code))


def _random_weight(oracle, rng, fmt, rows, cols, block, nested):
    if fmt == "int8":
        return dict(codes=rng.integers(0, 256, rows * cols).astype(np.uint8),
                    absmax=rng.uniform(0.1, 8.0, rows).astype(np.float32))
    count = rows * cols
    blocks = -(-count // block)
    kw = dict(codes=rng.integers(0, 256, (count + 1) // 2).astype(np.uint8), quant_map=oracle.bnb_table(fmt))
    if nested:
        kw.update(absmax=rng.integers(0, 256, blocks).astype(np.uint8),
                  nested_absmax=rng.uniform(0.01, 0.1, -(-blocks // 256)).astype(np.float32),
                  nested_map=np.sort(rng.uniform(-1, 1, 256)).astype(np.float32), offset=0.05)
    else:
        kw.update(absmax=rng.uniform(0.001, 0.1, blocks).astype(np.float32))
    return kw


_SHAPES = [("nf4", 64, 4096, 64, False), ("nf4", 37, 333, 32, True), ("fp4", 128, 1024, 4096, False),
           ("fp4", 5, 7000, 128, True), ("nf4", 300, 512, 256, True), ("int8", 61, 77, 0, False),
           ("int8", 256, 1024, 0, False)]


@pytest.mark.parametrize("fmt,rows,cols,block,nested", _SHAPES)
def test_random_decode(olamd, oracle, dev, fmt, rows, cols, block, nested):
    rng = np.random.default_rng(rows * 31 + cols + block)
    kw = _random_weight(oracle, rng, fmt, rows, cols, block, nested)
    w = _weight(olamd, dev, fmt, rows, cols, block, kw)
    for code, _ in DTYPES:
        assert np.array_equal(_bits(olamd.dequantize_bitsandbytes(w, code)),
                              _expect(oracle, fmt, rows, cols, block, kw, code)), (fmt, code)


def _raises(olamd, fn, message):
    with pytest.raises(olamd.InvalidArgument) as e:
        fn()
    assert message in str(e.value), str(e.value)


def test_errors(olamd, oracle, dev):
    rng = np.random.default_rng(5)
    kw = _random_weight(oracle, rng, "nf4", 4, 64, 64, False)
    bad = dict(kw, absmax=kw["absmax"].copy())
    bad["absmax"][2] = -1.0
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(_weight(olamd, dev, "nf4", 4, 64, 64, bad), 10),
            "bitsandbytes nonfinite table or invalid absmax.")
    bad = dict(kw, quant_map=oracle.bnb_table("fp4"))
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(_weight(olamd, dev, "nf4", 4, 64, 64, bad), 10),
            "bitsandbytes noncanonical NF4/FP4 table.")
    bad = dict(kw, absmax=np.full(4, 1e5, np.float32))  # fine in FLOAT and BFLOAT16, past FLOAT16
    w = _weight(olamd, dev, "nf4", 4, 64, 64, bad)
    olamd.dequantize_bitsandbytes(w, 1)
    olamd.dequantize_bitsandbytes(w, 16)
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(w, 10), "bitsandbytes nonfinite reconstruction.")
    _raises(olamd, lambda: olamd.prepare_bitsandbytes(w, 10), "bitsandbytes nonfinite reconstruction.")
    olamd.prepare_bitsandbytes(w, 16)
    nk = _random_weight(oracle, rng, "nf4", 4, 64, 64, True)
    nk["nested_absmax"] = np.array([3e38], np.float32)
    nk["nested_map"] = np.full(256, 2.0, np.float32)
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(_weight(olamd, dev, "nf4", 4, 64, 64, nk), 1),
            "bitsandbytes nonfinite reconstruction.")
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(_weight(olamd, dev, "nf4", 4, 64, 48, kw), 1),
            "bitsandbytes unsupported four-bit state.")
    short = dict(kw, absmax=kw["absmax"][:3])
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(_weight(olamd, dev, "nf4", 4, 64, 64, short), 1),
            "bitsandbytes invalid tensor type, shape or byte extent: weight_absmax.")
    ik = _random_weight(oracle, rng, "int8", 3, 5, 0, False)
    ik["absmax"][1] = np.nan
    _raises(olamd, lambda: olamd.dequantize_bitsandbytes(_weight(olamd, dev, "int8", 3, 5, 0, ik), 1),
            "bitsandbytes nonfinite table or invalid absmax.")


def _chain(oracle, fmt, rows, cols, block, kw, a_bits, dt):
    code = 10 if dt == "f16" else 16
    w_bits = _expect(oracle, fmt, rows, cols, block, kw, code)
    ref = oracle.matmul_half(a_bits, np.ascontiguousarray(w_bits.T), code)
    dec = oracle.f16_bits_to_f32 if dt == "f16" else oracle.bf16_bits_to_f32
    mag = np.abs(dec(a_bits).astype(np.float64)) @ np.abs(dec(w_bits).astype(np.float64)).T
    return w_bits, ref, mag


_MM = [("nf4", 1, 11008 // 4, 4096, 64, False, "f16"), ("fp4", 2, 512, 2048, 128, True, "f16"),
       ("nf4", 3, 37, 1024, 32, False, "f16"), ("nf4", 4, 200, 4096, 4096, True, "f16"),
       ("nf4", 5, 96, 512, 64, False, "f16"), ("fp4", 16, 64, 256, 32, False, "f16"),
       ("nf4", 2, 96, 512, 64, True, "bf16"), ("int8", 3, 70, 200, 0, False, "f16"),
       ("int8", 8, 64, 128, 0, False, "bf16"), ("nf4", 1, 33, 96, 32, False, "f16")]


@pytest.mark.parametrize("fmt,M,rows,cols,block,nested,dt", _MM)
def test_fused_matmul_vs_chain(olamd, oracle, dev, fmt, M, rows, cols, block, nested, dt):
    rng = np.random.default_rng(M * 1000 + rows + cols + block)
    kw = _random_weight(oracle, rng, fmt, rows, cols, block, nested)
    w = olamd.prepare_bitsandbytes(_weight(olamd, dev, fmt, rows, cols, block, kw), 10 if dt == "f16" else 16)
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    a = torch.from_numpy(rng.standard_normal((M, cols)).astype(np.float32)).to(dev, tdt)
    got = tensor_bits(olamd.bitsandbytes_matmul(a, w))
    _, ref, mag = _chain(oracle, fmt, rows, cols, block, kw, tensor_bits(a), dt)
    assert_close(got, ref, mag, dt, oracle, f"bitsandbytes {fmt} {M}x{rows}x{cols} {dt}")


@pytest.mark.parametrize("fmt,M,block", [("nf4", 4, 64), ("fp4", 4, 32), ("nf4", 8, 128)])
def test_fused_matmul_one_hot_rows_all_k(olamd, oracle, dev, fmt, M, block):
    """Every weight read back: row m of a is coef_m at k0 + m, so y[m, n] =
    coef_m * W[n, k0 + m] exactly (coef +1 / -2)."""
    rows, cols = 48, 512
    rng = np.random.default_rng(block + M)
    kw = _random_weight(oracle, rng, fmt, rows, cols, block, True)
    w = olamd.prepare_bitsandbytes(_weight(olamd, dev, fmt, rows, cols, block, kw), 10)
    w_f = oracle.f16_bits_to_f32(_expect(oracle, fmt, rows, cols, block, kw, 10))
    coef = np.where(np.arange(M) % 2 == 0, 1.0, -2.0).astype(np.float32)
    for k0 in range(0, cols, M):
        a = np.zeros((M, cols), np.float32)
        a[np.arange(M), k0 + np.arange(M)] = coef
        y = olamd.bitsandbytes_matmul(torch.from_numpy(a).to(dev, torch.float16), w)
        want = oracle.f32_to_f16_bits((w_f[:, k0:k0 + M].T * coef[:, None]) + np.float32(0.0))
        assert np.array_equal(tensor_bits(y), want), f"{fmt} one-hot rows {k0}"
