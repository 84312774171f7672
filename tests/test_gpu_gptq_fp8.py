"""GPTQModel FP8 weights on the GPU against the oracle
(oracle.gptq_fp8_reconstruct, pinned by the reference test's fixtures in
test_oracle_gptq_fp8.py): onnxl_amd_dequantize_gptqmodel_fp8 bit for bit in
FLOAT, FLOAT16, BFLOAT16 and DOUBLE on the fixtures, on every code of every
FP8 subtype, and on random weights per tensor, per row and in blocks, from
host and device inputs; the reference's errors in its order."""
import numpy as np
import pytest
import torch

from test_gpu_float import T, tensor_bits
from test_oracle_gptq_fp8 import CC_METHODS, SUBTYPES, cc_fixture

pytestmark = pytest.mark.gpu

DTYPES = [1, 10, 16, 11]


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _bits(t):
    if t.dtype in (torch.float32, torch.float64):
        a = t.cpu().numpy()
        return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)
    return tensor_bits(t)


def _ref_bits(a, code):
    return a.view(np.uint32) if code == 1 else (a.view(np.uint64) if code == 11 else a)


def _raises(olamd, fn, message):
    with pytest.raises(olamd.InvalidArgument) as e:
        fn()
    assert message in str(e.value), str(e.value)


def _check(olamd, oracle, dev, codes, code_type, scales, method, block=(), host=False):
    for out in DTYPES:
        rc, ref = oracle.gptq_fp8_reconstruct(codes, code_type, scales, method, block or (1, 1), out_dtype=out)
        w = np.ascontiguousarray(codes) if host else T(codes, dev)
        s = np.array(scales, copy=True) if host else torch.from_numpy(np.array(scales, copy=True)).to(dev)  # keeps []
        call = lambda: olamd.dequantize_gptqmodel_fp8(w, s, method, block, code_type, out)
        if rc:
            _raises(olamd, call, oracle.GPTQ_FP8_ERRORS[rc])
            continue
        assert np.array_equal(_bits(call()), _ref_bits(ref, out)), (method, block, code_type, out)


@pytest.mark.parametrize("method,block", CC_METHODS)
def test_cc_fixture_decode(olamd, oracle, dev, method, block):
    codes, scales = cc_fixture(method, block)
    _check(olamd, oracle, dev, codes, 17, scales, method, block)


@pytest.mark.parametrize("code_type", [t for t, _, _ in SUBTYPES])
def test_every_code_of_every_subtype(olamd, oracle, dev, code_type):
    codes = np.arange(256, dtype=np.uint8).reshape(16, 16)
    scales = np.linspace(1.0, 4.0, 16).astype(np.float32)
    nan = {17: [0x7F, 0xFF], 18: [0x80], 19: [0x7D, 0x7E, 0x7F, 0xFD, 0xFE, 0xFF], 20: [0x80], 24: [0xFF]}[code_type]
    if code_type == 19:  # E5M2 infinities too: every nonfinite code replaced, then checked alone
        nan = nan + [0x7C, 0xFC]
    clean = codes.copy()
    clean[np.isin(clean, nan)] = 0
    _check(olamd, oracle, dev, clean, code_type, scales, "row")
    bad = clean.copy()
    bad[3, 5] = nan[0]
    _check(olamd, oracle, dev, bad, code_type, scales, "row")


@pytest.mark.parametrize("n,k,method,block,code_type,host", [(256, 512, "block", (128, 128), 17, False),
                                                             (96, 384, "row", (), 19, True),
                                                             (64, 200, "tensor", (), 18, False),
                                                             (48, 96, "block", (16, 32), 20, True)])
def test_random_decode(olamd, oracle, dev, n, k, method, block, code_type, host):
    rng = np.random.default_rng(n + k)
    codes = rng.integers(0, 256, (n, k)).astype(np.uint8)
    codes[np.isin(codes, [0x7F, 0xFF, 0x80, 0x7C, 0x7D, 0x7E, 0xFC, 0xFD, 0xFE])] = 0x11
    shape = () if method == "tensor" else ((n,) if method == "row" else (n // block[0], k // block[1]))
    scales = rng.uniform(0.05, 2.0, shape).astype(np.float32)
    _check(olamd, oracle, dev, codes, code_type, scales, method, block, host=host)


def test_errors(olamd, oracle, dev):
    codes, scales = cc_fixture("row")
    bad = scales.copy()
    bad[1] = -1.0
    nan = codes.copy()
    nan[0, 0] = 0x7F
    _raises(olamd, lambda: olamd.dequantize_gptqmodel_fp8(T(nan, dev), T(bad, dev), "row", (), 17),
            "GPTQModel FP8 inverse scales must be finite and positive.")
    _raises(olamd, lambda: olamd.dequantize_gptqmodel_fp8(T(nan, dev), T(scales, dev), "row", (), 17),
            "GPTQModel FP8 nonfinite weight or reconstruction.")
    _raises(olamd, lambda: olamd.dequantize_gptqmodel_fp8(T(codes, dev), T(scales, dev), "block", (3, 2), 17),
            "GPTQModel FP8 requires divisible two-axis blocks.")
    _raises(olamd, lambda: olamd.dequantize_gptqmodel_fp8(T(codes, dev), T(scales, dev), "row", (2, 2), 17),
            "GPTQModel FP8 non-block scaling forbids weight_block_size.")
    _raises(olamd, lambda: olamd.dequantize_gptqmodel_fp8(T(codes, dev), T(scales, dev), "row", (), 3),
            "GPTQModel FP8 unsupported scalar format.")
    _raises(olamd, lambda: olamd.dequantize_gptqmodel_fp8(T(codes, dev), T(scales[:3], dev), "row", (), 17),
            "GPTQModel FP8 invalid tensor dtype, shape or byte extent.")
