"""The GPTQModel FP8 oracle (oracle.c, orc_gptq_fp8_reconstruct) pinned by
the fixtures of unittests/cc/onnx_core/runtime/test_gptqmodel_fp8.cc:

- the 4 x 4 E4M3FN weight with rows 0x38 0xBC 0x40 0xB0 (1, -1.5, 2, -0.5)
  over inverse scales per tensor, per row and in (1, 2), (2, 1), (2, 2),
  (4, 4) blocks: every value is fp32(decoded / scale), bit for bit;
- every FP8 subtype's scalar fixtures (E4M3FN, E4M3FNUZ, E5M2, E5M2FNUZ,
  E8M0: 0x7F 0x80 0x7E 0x00 = 1, 2, 0.5, 2^-127), divided by 0.3, signed
  zeros kept;
- CheckData's errors (scales zero, negative, infinite or NaN; a NaN code;
  an overflowing quotient) and WriteFloat's FLOAT16 range."""
import numpy as np
import pytest

import oracle as orc

ROW = [0x38, 0xBC, 0x40, 0xB0]
DECODED = np.array([1.0, -1.5, 2.0, -0.5], np.float32)


def cc_fixture(method, block=()):
    codes = np.array([ROW] * 4, np.uint8)
    if method == "tensor":
        scales = np.array(0.3, np.float32)  # shape []
    elif method == "row":
        scales = np.array([0.3, 1.3, 3.0, 7.0], np.float32)
    else:
        rows, cols = 4 // block[0], 4 // block[1]
        scales = (np.arange(rows * cols, dtype=np.float32) + 1) * np.float32(0.3)
        scales = scales.reshape(rows, cols)
    return codes, scales


CC_METHODS = [("tensor", ()), ("row", ()), ("block", (1, 2)), ("block", (2, 1)), ("block", (2, 2)), ("block", (4, 4))]


@pytest.mark.parametrize("method,block", CC_METHODS)
def test_cc_exact_bytes_inverse_scales_and_two_axis_grouping(oracle, method, block):
    codes, scales = cc_fixture(method, block)
    rc, out = oracle.gptq_fp8_reconstruct(codes, 17, scales, method, block or (1, 1))
    assert rc == 0
    flat = scales.reshape(-1)
    for n in range(4):
        for k in range(4):
            idx = 0 if method == "tensor" else (n if method == "row" else
                                                 (n // block[0]) * (4 // block[1]) + k // block[1])
            want = np.float32(DECODED[k] / flat[idx])
            assert out[n, k].view(np.uint32) == want.view(np.uint32), (method, block, n, k)


SUBTYPES = [(17, [0x38, 0xBC, 0x00, 0x80], [1.0, -1.5, 0.0, -0.0]),
            (18, [0x40, 0xC4, 0x00, 0x38], [1.0, -1.5, 0.0, 0.5]),
            (19, [0x3C, 0xBE, 0x00, 0x80], [1.0, -1.5, 0.0, -0.0]),
            (20, [0x40, 0xC2, 0x00, 0x3C], [1.0, -1.5, 0.0, 0.5]),
            (24, [0x7F, 0x80, 0x7E, 0x00], [1.0, 2.0, 0.5, 2.0 ** -127])]


@pytest.mark.parametrize("code_type,codes,decoded", SUBTYPES)
def test_cc_subtypes_and_signed_zero(oracle, code_type, codes, decoded):
    rc, out = oracle.gptq_fp8_reconstruct(np.array([codes], np.uint8), code_type, np.array([0.3], np.float32),
                                          "tensor")
    assert rc == 0
    want = (np.array(decoded, np.float32) / np.float32(0.3)).astype(np.float32)
    assert np.array_equal(out.reshape(-1).view(np.uint32), want.view(np.uint32))


def test_e8m0_decode_every_code(oracle):
    for c in range(256):
        got = np.float32(oracle.lib().orc_f8e8m0_to_f32(c))
        if c == 255:
            assert np.isnan(got) and got.view(np.uint32) == 0x7FC00000
        else:
            assert got == np.float32(2.0 ** (c - 127)), c


def test_checks_and_errors(oracle):
    codes, scales = cc_fixture("row")
    for bad in (0.0, -0.3, np.inf, np.nan):
        s = scales.copy()
        s[2] = bad
        assert oracle.gptq_fp8_reconstruct(codes, 17, s, "row")[0] == 1, bad
    nan_code = codes.copy()
    nan_code[1, 1] = 0x7F  # E4M3FN NaN
    assert oracle.gptq_fp8_reconstruct(nan_code, 17, scales, "row")[0] == 2
    tiny = np.full(4, 1e-38, np.float32)  # 448 / 1e-38 overflows FLOAT
    big = np.full((4, 4), 0x7E, np.uint8)  # 448
    assert oracle.gptq_fp8_reconstruct(big, 17, tiny, "row")[0] == 2
    small = np.full(4, 1e-3, np.float32)  # 448 000: fits FLOAT and BFLOAT16, not FLOAT16
    assert oracle.gptq_fp8_reconstruct(big, 17, small, "row")[0] == 0
    assert oracle.gptq_fp8_reconstruct(big, 17, small, "row", out_dtype=orc.BFLOAT16)[0] == 0
    assert oracle.gptq_fp8_reconstruct(big, 17, small, "row", out_dtype=orc.FLOAT16)[0] == 4
