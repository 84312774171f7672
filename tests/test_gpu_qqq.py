"""QQQ weights on the GPU against the oracle (oracle.qqq_reconstruct, pinned
by the upstream packer's outputs and the reference test's fixtures in
test_oracle_qqq.py).

- onnxl_amd_dequantize_qqq: the reference's golden cases reproduce their
  SHA-256 digests in FLOAT, and every value matches the oracle bit for bit in
  FLOAT, FLOAT16, BFLOAT16 and DOUBLE on the golden cases, the C++ fixtures
  and larger random weights (both permutation orders, signed zeros, ties,
  saturation, subnormal and large scales), from host and device inputs; the
  reference's error messages in its order.
- onnxl_amd_prepare_qqq, then the fused DequantizeLinear -> MatMul call:
  one-hot activations read every weight back bit for bit (so the prepared
  INT4 / INT8 operand times its scale is the chain's weight exactly); random
  activations match the oracle chain (decode in A's dtype, then MatMul(a,
  W^T)) within |got - ref| <= 1e-2 |ref| + u sum_k |a w| (u = 2^-11 FLOAT16,
  2^-8 BFLOAT16), on the GEMV (M <= 16) and GEMM paths."""
import hashlib

import numpy as np
import pytest
import torch

from test_gpu_float import T, assert_close, tensor_bits
from test_oracle_qqq import fixture, golden_tensors, pack_codes, qqq_cases

pytestmark = pytest.mark.gpu

DTYPES = [(1, torch.float32), (10, torch.float16), (16, torch.bfloat16), (11, torch.float64)]


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _bits(t):
    if t.dtype == torch.float32:
        return t.cpu().numpy().view(np.uint32)
    if t.dtype == torch.float64:
        return t.cpu().numpy().view(np.uint64)
    return tensor_bits(t)


def _ref_bits(a, code):
    return a.view(np.uint32) if code == 1 else (a.view(np.uint64) if code == 11 else a)


def _on(x, dev, host):
    if x is None or np.size(x) == 0:
        return None
    return np.ascontiguousarray(x) if host else T(x, dev)


def _check_all_dtypes(olamd, oracle, dev, k, n, g, B, sc, sg, host=False, what=""):
    for code, _ in DTYPES:
        rc, ref, _ = oracle.qqq_reconstruct(k, n, g, B, sc, sg, out_dtype=code)
        args = (k, n, g, _on(B, dev, host), _on(sc, dev, host), _on(sg, dev, host), code)
        if rc == 4:  # a value past FLOAT16 / BFLOAT16: WriteFloat's error
            _raises(olamd, lambda: olamd.dequantize_qqq(*args), "Dequantization output dtype overflow.")
            continue
        assert rc == 0
        got = olamd.dequantize_qqq(*args)
        if host:
            got = torch.from_numpy(got) if isinstance(got, np.ndarray) else got
        assert np.array_equal(_bits(got), _ref_bits(ref, code)), (what, code)


@pytest.mark.parametrize("name", [c["name"] for c in qqq_cases()])
def test_golden_decode(olamd, oracle, dev, name):
    c = next(c for c in qqq_cases() if c["name"] == name)
    k, n, g, B, sc, sg = golden_tensors(c)
    got = olamd.dequantize_qqq(k, n, g, T(B, dev), T(sc, dev), _on(sg, dev, False), 1)
    assert hashlib.sha256(got.cpu().numpy().astype("<f4").tobytes()).hexdigest() == c["expected_sha256"], name
    _check_all_dtypes(olamd, oracle, dev, k, n, g, B, sc, sg, what=name)


@pytest.mark.parametrize("k,n,group", [(64, 64, -1), (128, 320, 128), (256, 128, 128), (384, 320, 128)])
def test_cc_fixture_decode(olamd, oracle, dev, k, n, group):
    _, B, sc, sg = fixture(k, n, group)
    _check_all_dtypes(olamd, oracle, dev, k, n, group, B, sc, sg, what=(k, n, group))


def _random(rng, k, n, grouped, extremes=False):
    codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
    B = pack_codes(codes, k, n, grouped)
    sc = rng.uniform(0.001, 0.05, (1, n)).astype(np.float32)
    sg = rng.uniform(0.5, 20.0, (k // 128, n)).astype(np.float16) if grouped else np.zeros(0, np.float16)
    if extremes:
        sc[0, :4] = [0.0, -0.0, np.finfo(np.float32).smallest_subnormal, 3.0e4]
        if grouped:
            sg[0, :6] = [0.0, -0.0, 0.5, 1.5, 65504.0, 2.0 ** -24]
    return codes, B, sc, sg


@pytest.mark.parametrize("k,n,grouped,host", [(1024, 512, False, False), (4096, 256, True, False),
                                              (640, 192, True, True), (128, 128, False, True)])
def test_random_decode(olamd, oracle, dev, k, n, grouped, host):
    rng = np.random.default_rng(k + n)
    _, B, sc, sg = _random(rng, k, n, grouped, extremes=True)
    _check_all_dtypes(olamd, oracle, dev, k, n, 128 if grouped else -1, B, sc, sg, host=host, what=(k, n))


def _raises(olamd, fn, message, cls=None):
    with pytest.raises(cls or olamd.InvalidArgument) as e:
        fn()
    assert message in str(e.value), str(e.value)


def test_errors(olamd, oracle, dev):
    rng = np.random.default_rng(3)
    _, B, sc, sg = _random(rng, 256, 64, True)
    dq = lambda sc_, sg_, code=1, k=256, g=128, B_=B: olamd.dequantize_qqq(k, 64, g, T(B_, dev), T(sc_, dev),
                                                                          _on(sg_, dev, False), code)
    bad = sc.copy()
    bad[0, 7] = -1.0
    badg = sg.copy()
    badg[1, 2] = np.nan
    _raises(olamd, lambda: dq(bad, badg), "QQQ nonfinite or negative channel scale.")
    _raises(olamd, lambda: dq(sc, badg), "QQQ nonfinite or negative group scale.")
    assert oracle.qqq_reconstruct(256, 64, 128, B, sc, badg)[0] == 2
    big = np.full((1, 64), 3e37, np.float32)
    _raises(olamd, lambda: dq(big, sg), "QQQ FLOAT reconstruction overflow.")
    mid = np.full((1, 64), 1e4, np.float32)
    dq(mid, sg, 16)
    _raises(olamd, lambda: dq(mid, sg, 10), "Dequantization output dtype overflow.")
    _raises(olamd, lambda: olamd.prepare_qqq(256, 64, 128, T(B, dev), T(mid, dev), T(sg, dev), 10),
            "Dequantization output dtype overflow.")
    olamd.prepare_qqq(256, 64, 128, T(B, dev), T(mid, dev), T(sg, dev), 16)
    _raises(olamd, lambda: dq(sc, sg, k=96), "QQQ requires four-bit, unpadded dimensions divisible by 64")
    _raises(olamd, lambda: dq(sc, sg, g=64), "QQQ requires four-bit, unpadded dimensions divisible by 64")
    _raises(olamd, lambda: olamd.dequantize_qqq(192, 64, 128, T(B[:12], dev), T(sc, dev), T(sg[:1], dev), 1),
            "QQQ incomplete 128-element group.")
    _raises(olamd, lambda: dq(sc, sg[:1]), "QQQ invalid tensor type, shape or byte extent: s_group.")
    _raises(olamd, lambda: dq(sc, sg, B_=B[:8]), "QQQ invalid tensor type, shape or byte extent: B.")
    _raises(olamd, lambda: dq(sc.reshape(-1), sg), "QQQ invalid tensor type, shape or byte extent: s_channel.")
    # a per-channel weight whose 16 x channel scale overflows: decodes, has no fused operand
    zero = pack_codes(np.zeros((64, 64), np.uint8), 64, 64, False)
    huge = np.full((1, 64), 3e38, np.float32)
    y = olamd.dequantize_qqq(64, 64, -1, T(zero, dev), T(huge, dev), None, 1)
    assert not y.any()
    _raises(olamd, lambda: olamd.prepare_qqq(64, 64, -1, T(zero, dev), T(huge, dev), None, 10),
            "16 x a channel scale overflows FLOAT", olamd.Unsupported)


def _chain(oracle, k, n, g, B, sc, sg, a_bits, code):
    rc, w_bits, _ = oracle.qqq_reconstruct(k, n, g, B, sc, sg, out_dtype=code)
    assert rc == 0
    ref = oracle.matmul_half(a_bits, np.ascontiguousarray(w_bits.T), code)
    dec = oracle.f16_bits_to_f32 if code == 10 else oracle.bf16_bits_to_f32
    mag = np.abs(dec(a_bits).astype(np.float64)) @ np.abs(dec(w_bits).astype(np.float64)).T
    return w_bits, ref, mag


@pytest.mark.parametrize("M,k,n,grouped,dt", [(1, 4096, 1024, False, "f16"), (8, 2048, 512, True, "f16"),
                                              (3, 1024, 256, True, "bf16"), (40, 512, 384, False, "f16"),
                                              (64, 1024, 256, True, "f16"), (16, 256, 128, False, "bf16")])
def test_prepared_matmul_vs_chain(olamd, oracle, dev, M, k, n, grouped, dt):
    rng = np.random.default_rng(M * 100 + k + n)
    _, B, sc, sg = _random(rng, k, n, grouped)
    code = 10 if dt == "f16" else 16
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    p = olamd.prepare_qqq(k, n, 128 if grouped else -1, T(B, dev), T(sc, dev), _on(sg, dev, False), code)
    a = torch.from_numpy(rng.standard_normal((M, k)).astype(np.float32)).to(dev, tdt)
    got = tensor_bits(olamd.qqq_matmul(a, p))
    _, ref, mag = _chain(oracle, k, n, 128 if grouped else -1, B, sc, sg, tensor_bits(a), code)
    assert_close(got, ref, mag, dt, oracle, f"qqq {M}x{k}x{n} grouped={grouped} {dt}")


@pytest.mark.parametrize("M,grouped", [(4, False), (4, True), (24, True)])
def test_prepared_matmul_one_hot_rows_all_k(olamd, oracle, dev, M, grouped):
    """Every weight read back: row m of a is coef_m at k0 + m, so y[m, n] =
    coef_m * W[n, k0 + m] exactly (coef +1 / -2)."""
    k, n = 256, 64
    rng = np.random.default_rng(M + grouped)
    _, B, sc, sg = _random(rng, k, n, grouped, extremes=True)
    sc[0, 3] = 1.0  # keep every value inside FLOAT16
    g = 128 if grouped else -1
    p = olamd.prepare_qqq(k, n, g, T(B, dev), T(sc, dev), _on(sg, dev, False), 10)
    rc, w_bits, _ = oracle.qqq_reconstruct(k, n, g, B, sc, sg, out_dtype=10)
    assert rc == 0
    w_f = oracle.f16_bits_to_f32(w_bits)
    coef = np.where(np.arange(M) % 2 == 0, 1.0, -2.0).astype(np.float32)
    for k0 in range(0, k, M):
        m = min(M, k - k0)
        a = np.zeros((M, k), np.float32)
        a[np.arange(m), k0 + np.arange(m)] = coef[:m]
        y = olamd.qqq_matmul(torch.from_numpy(a).to(dev, torch.float16), p)
        want = np.zeros((M, n), np.float32)
        want[:m] = w_f[:, k0:k0 + m].T * coef[:m, None]
        assert np.array_equal(tensor_bits(y), oracle.f32_to_f16_bits(want + np.float32(0.0))), (grouped, k0)
