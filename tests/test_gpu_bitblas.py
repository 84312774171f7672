"""BitBLAS row-packed weights on the GPU against the oracle
(oracle.bitblas_reconstruct, pinned by the upstream packer's outputs and the
reference test's fixture in test_oracle_bitblas.py).

- onnxl_amd_dequantize_bitblas: the reference's 13 golden cases reproduce
  their SHA-256 digests in FLOAT and match the oracle bit for bit in FLOAT,
  FLOAT16, BFLOAT16 and DOUBLE (FLOAT16 overflow raising the reference's
  error where the oracle reports it); the C++ fixture; random weights of
  every bit width and group size, symmetric GPTQ and not, from host and
  device inputs; the scale and output-range errors.
- onnxl_amd_prepare_bitblas, then the fused DequantizeLinear -> MatMul
  call (axis 0): one-hot activations read every weight back bit for bit;
  random activations match the oracle chain (decode in A's dtype, then
  MatMul(a, W^T)) within |got - ref| <= 1e-2 |ref| + u sum_k |a w|
  (u = 2^-11 FLOAT16), on the GEMV and GEMM paths, 4-bit (tiled UINT4) and
  wider (UINT8) codes."""
import hashlib

import numpy as np
import pytest
import torch

from test_gpu_float import T, assert_close, tensor_bits
from test_oracle_bitblas import bitblas_cases, case_id, cc_fixture, golden_args, signed

pytestmark = pytest.mark.gpu

DTYPES = [1, 10, 16, 11]


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _bits(t):
    a = t.cpu().numpy() if isinstance(t, torch.Tensor) and t.dtype in (torch.float32, torch.float64) else None
    if a is not None:
        return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)
    return tensor_bits(t)


def _ref_bits(a, code):
    return a.view(np.uint32) if code == 1 else (a.view(np.uint64) if code == 11 else a)


def _on(x, dev, host):
    if x is None or np.size(x) == 0:
        return None
    return np.ascontiguousarray(x) if host else T(x, dev)


def _raises(olamd, fn, message):
    with pytest.raises(olamd.InvalidArgument) as e:
        fn()
    assert message in str(e.value), str(e.value)


def _check_all(olamd, oracle, dev, m, k, n, g, bits, sym, qw, sc, qz, host=False, what=""):
    for code in DTYPES:
        rc, ref, _ = oracle.bitblas_reconstruct(k, n, g, bits, signed(m, sym), qw, sc, qz, out_dtype=code)
        args = (m, _on(qw, dev, host), _on(sc, dev, host), _on(qz, dev, host), k, n, bits, g, sym, code)
        if rc == 4:
            _raises(olamd, lambda: olamd.dequantize_bitblas(*args), "Dequantization output dtype overflow.")
            continue
        assert rc == 0
        got = olamd.dequantize_bitblas(*args)
        assert np.array_equal(_bits(got), _ref_bits(ref, code)), (what, code)


@pytest.mark.parametrize("c", bitblas_cases(), ids=case_id)
def test_golden_decode(olamd, oracle, dev, c):
    m, k, n, g, bits, sym, qw, sc, qz = golden_args(c)
    got = olamd.dequantize_bitblas(m, T(qw, dev), T(sc, dev), _on(qz, dev, False), k, n, bits, g, sym, 1)
    assert hashlib.sha256(got.cpu().numpy().astype("<f4").tobytes()).hexdigest() == c["expected_sha256"]
    _check_all(olamd, oracle, dev, m, k, n, g, bits, sym, qw, sc, qz, what=case_id(c))


@pytest.mark.parametrize("symmetric", [False, True])
def test_cc_fixture_decode(olamd, oracle, dev, symmetric):
    qw, sc, qz = cc_fixture(symmetric)
    _check_all(olamd, oracle, dev, "gptq", 32, 32, -1, 2, symmetric, qw, sc, qz)


def pack_rows(codes, bits):
    """Unsigned codes [rows, count] -> int8 [rows, count * bits / 8], each row
    a little-endian bit stream (the row packer's layout)."""
    rows, count = codes.shape
    out = np.zeros((rows, count * bits // 8), np.uint8)
    for i in range(count):
        bit = i * bits
        v = codes[:, i].astype(np.uint32) << (bit % 8)
        out[:, bit // 8] |= (v & 0xFF).astype(np.uint8)
        if bit % 8 + bits > 8:
            out[:, bit // 8 + 1] |= (v >> 8).astype(np.uint8)
    return out.view(np.int8)


def _random(rng, method, k, n, bits, group, sym, extremes=False):
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint8)
    groups = k // (k if group == -1 else group)
    sc = rng.uniform(0.001, 0.05, (n, groups)).astype(np.float16)
    if extremes:
        sc.reshape(-1)[:3] = [2.0 ** -24, 65504.0, 1.0]
    qz = None if signed(method, sym) else pack_rows(rng.integers(0, 1 << bits, (groups, n)).astype(np.uint8), bits)
    return pack_rows(codes, bits), sc, qz


_SHAPES = [("gptq", 4096, 256, 4, 128, False, False), ("gptq", 1024, 128, 8, 64, True, True),
           ("gptq", 512, 96, 2, -1, True, False), ("awq", 768, 80, 3, 128, False, True),
           ("awq", 256, 48, 5, 32, False, False), ("awq", 256, 64, 6, 256, True, False),
           ("awq", 128, 16, 7, -1, False, True)]


@pytest.mark.parametrize("m,k,n,bits,g,sym,host", _SHAPES)
def test_random_decode(olamd, oracle, dev, m, k, n, bits, g, sym, host):
    rng = np.random.default_rng(k + n + bits)
    qw, sc, qz = _random(rng, m, k, n, bits, g, sym, extremes=True)
    _check_all(olamd, oracle, dev, m, k, n, g, bits, sym, qw, sc, qz, host=host, what=(m, bits))


def test_errors(olamd, oracle, dev):
    rng = np.random.default_rng(9)
    qw, sc, qz = _random(rng, "gptq", 256, 64, 4, 128, False)
    bad = sc.copy()
    bad[5, 1] = np.nan
    _raises(olamd, lambda: olamd.dequantize_bitblas("gptq", T(qw, dev), T(bad, dev), T(qz, dev), 256, 64, 4, 128),
            "BitBLAS nonfinite or nonpositive scale.")
    bad[5, 1] = -0.0
    _raises(olamd, lambda: olamd.prepare_bitblas("gptq", T(qw, dev), T(bad, dev), T(qz, dev), 256, 64, 4, 128),
            "BitBLAS nonfinite or nonpositive scale.")
    big = np.full_like(sc, 65504.0)
    olamd.dequantize_bitblas("gptq", T(qw, dev), T(big, dev), T(qz, dev), 256, 64, 4, 128, False, 16)
    if oracle.bitblas_reconstruct(256, 64, 128, 4, False, qw, big, qz, out_dtype=10)[0] == 4:
        _raises(olamd, lambda: olamd.dequantize_bitblas("gptq", T(qw, dev), T(big, dev), T(qz, dev), 256, 64, 4, 128,
                                                        False, 10), "Dequantization output dtype overflow.")


def _chain(oracle, k, n, g, bits, sgn, qw, sc, qz, a_bits):
    rc, w_bits, _ = oracle.bitblas_reconstruct(k, n, g, bits, sgn, qw, sc, qz, out_dtype=10)
    assert rc == 0
    ref = oracle.matmul_half(a_bits, np.ascontiguousarray(w_bits.T), 10)
    mag = np.abs(oracle.f16_bits_to_f32(a_bits).astype(np.float64)) @ \
        np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64)).T
    return w_bits, ref, mag


@pytest.mark.parametrize("M,m,k,n,bits,g,sym", [(1, "gptq", 4096, 512, 4, 128, False), (8, "gptq", 2048, 256, 4, 64, True),
                                                (3, "awq", 1024, 128, 3, 128, False), (40, "gptq", 512, 256, 8, 128, False),
                                                (5, "awq", 512, 64, 6, 32, False), (24, "gptq", 256, 64, 2, -1, True)])
def test_prepared_matmul_vs_chain(olamd, oracle, dev, M, m, k, n, bits, g, sym):
    rng = np.random.default_rng(M + k + n + bits)
    qw, sc, qz = _random(rng, m, k, n, bits, g, sym)
    p = olamd.prepare_bitblas(m, T(qw, dev), T(sc, dev), _on(qz, dev, False), k, n, bits, g, sym)
    a = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(dev, torch.float16)
    got = tensor_bits(olamd.matmul_nbits(a, p))
    _, ref, mag = _chain(oracle, k, n, g, bits, signed(m, sym), qw, sc, qz, tensor_bits(a))
    assert_close(got, ref, mag, "f16", oracle, f"bitblas {m} {bits}-bit {M}x{k}x{n}")


@pytest.mark.parametrize("M,m,bits,sym", [(4, "gptq", 4, False), (4, "gptq", 4, True), (8, "awq", 7, False)])
def test_prepared_matmul_one_hot_rows_all_k(olamd, oracle, dev, M, m, bits, sym):
    """Every weight read back: row r of a is coef_r at k0 + r, so y[r, n] =
    coef_r * W[n, k0 + r] exactly (coef +1 / -2)."""
    k, n, g = 256, 48 if m == "awq" else 64, 64
    rng = np.random.default_rng(M + bits)
    qw, sc, qz = _random(rng, m, k, n, bits, g, sym)
    p = olamd.prepare_bitblas(m, T(qw, dev), T(sc, dev), _on(qz, dev, False), k, n, bits, g, sym)
    rc, w_bits, _ = oracle.bitblas_reconstruct(k, n, g, bits, signed(m, sym), qw, sc, qz, out_dtype=10)
    assert rc == 0
    w_f = oracle.f16_bits_to_f32(w_bits)
    coef = np.where(np.arange(M) % 2 == 0, 1.0, -2.0).astype(np.float32)
    for k0 in range(0, k, M):
        a = np.zeros((M, k), np.float32)
        a[np.arange(M), k0 + np.arange(M)] = coef
        y = olamd.matmul_nbits(torch.from_numpy(a).to(dev, torch.float16), p)
        want = w_f[:, k0:k0 + M].T * coef[:, None]
        assert np.array_equal(tensor_bits(y), oracle.f32_to_f16_bits(want + np.float32(0.0))), (m, bits, k0)


def test_prepared_fp16_scales_widened_for_bf16_activations(olamd, oracle, dev):
    """With BFLOAT16 activations the adapter widens the prepared FLOAT16
    scales to FLOAT and runs DequantizeLinear in FLOAT with a Cast to
    BFLOAT16: every weight is then the reference's BFLOAT16 rounding of the
    FLOAT value (Dequantize with dtype = BFLOAT16), read back bit for bit
    through one-hot rows."""
    k, n, g, bits, M = 256, 64, 64, 4, 4
    rng = np.random.default_rng(21)
    qw, sc, qz = _random(rng, "gptq", k, n, bits, g, False)
    p = olamd.prepare_bitblas("gptq", T(qw, dev), T(sc, dev), T(qz, dev), k, n, bits, g)
    wide = p.scale.storage[: p.scale.desc.size_bytes].view(torch.float16).float().contiguous()
    rc, w_bits, _ = oracle.bitblas_reconstruct(k, n, g, bits, False, qw, sc, qz, out_dtype=16)
    assert rc == 0
    w_f = oracle.bf16_bits_to_f32(w_bits)
    coef = np.where(np.arange(M) % 2 == 0, 1.0, -2.0).astype(np.float32)
    for k0 in range(0, k, M):
        a = np.zeros((M, k), np.float32)
        a[np.arange(M), k0 + np.arange(M)] = coef
        y = olamd.dequantize_linear_matmul(torch.from_numpy(a).to(dev, torch.bfloat16), p.weight,
                                           wide.view(k // g, n), p.zero_point, 0, 16, x_shape=(k, n))
        want = (w_f[:, k0:k0 + M].T * coef[:, None]).astype(np.float32) + np.float32(0.0)
        assert np.array_equal(tensor_bits(y), (want.view(np.uint32) >> 16).astype(np.uint16)), k0
