"""The MX / NVFP4 weight oracle (oracle.c, orc_mx_reconstruct) pinned by the
reference's own fixtures and by closed forms:

- MXFP4, unittests/cc/onnx_core/runtime/test_quantization.cc:260-443: the
  level table packed low nibble first at scale 127, the all-ones row at 125,
  the scale-rounding boundary rows at 127 / 128, signed zeros, the 2^-127
  scale byte 0, the row-major [2, 64] groups, a NaN scale and an
  overflowing 254-scaled code rejected;
- MXFP6 E2M3, :454-565: the 48 f8 01 triplets, the scale-threshold rows
  (codes 24 / 31 over scales 125 ... 252), every one of the 64 codes over
  scales 127 and 0 (2^-127), and code 8 at 254 = 2^127;
- NVFP4, unittests/python/backend/test_nvfp4_weights.py:35-160: the level
  table over local scales 0x38 / 0x3A, the row groups over a global scale
  of 2, the calibrated 448 / 112 over 224 fixture and the fp32 division
  order 1.5 * fp32(2^-9 / 7);
- MXFP8 (no fixture in the reference's tests): every E4M3FN code times a
  power of two equals float64's exact product (ldexp), NaN codes and
  overflow rejected in order.
A mistake in the nibble order, the 6-bit offsets, the E8M0 bias or the
NVFP4 division order fails one of these."""
import math

import numpy as np
import pytest

LEVELS = [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]


def _f32(vals):
    return np.array(vals, np.float32)


def _same(a, b):
    """Bit for bit, except that the fixtures' -0.0 and 0.0 compare equal (the
    reference's ExpectValues compares values; its signbit checks are
    separate tests)."""
    a, b = np.asarray(a, np.float32).reshape(-1), np.asarray(b, np.float32).reshape(-1)
    assert a.shape == b.shape
    a, b = a + np.float32(0), b + np.float32(0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (a, b)


def test_mxfp4_level_table_and_unit_row(oracle):
    packed = np.array([0x10, 0x32, 0x54, 0x76, 0x90, 0xba, 0xdc, 0xfe] * 2, np.uint8)
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 1, 32, packed, np.array([127], np.uint8))
    assert rc == 0
    _same(v, LEVELS * 2)
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 1, 32, np.full(16, 0x66, np.uint8), np.array([125], np.uint8))
    assert rc == 0
    _same(v, [1.0] * 32)


@pytest.mark.parametrize("scale,packed,maximum", [(127, [0xf7, 0xa2, 0xc4, 0xd5], 6.0),
                                                  (128, [0xe6, 0x91, 0xa2, 0xb3], 8.0)])
def test_mxfp4_scale_rounding_boundary(oracle, scale, packed, maximum):
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 1, 32, np.array(packed + [0] * 12, np.uint8),
                                        np.array([scale], np.uint8))
    assert rc == 0
    _same(v, [maximum, -maximum, 1, -1, 2, -2, 3, -3] + [0] * 24)


def test_mxfp4_signed_zeros_and_scale_extremes(oracle):
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 1, 32, np.array([0x20, 0x42, 0x64, 0x86, 0x70] + [0] * 11, np.uint8),
                                        np.array([127], np.uint8))
    assert rc == 0 and math.copysign(1, v[0, 7]) < 0 and math.copysign(1, v[0, 8]) > 0
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 1, 32, np.array([7] + [0] * 15, np.uint8), np.array([0], np.uint8))
    assert rc == 0 and v[0, 0] == np.float32(6.0 * 2.0 ** -127)
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 1, 32, np.array([7] + [0] * 15, np.uint8), np.array([252], np.uint8))
    assert rc == 0 and np.isfinite(v[0, 0])


def test_mxfp4_row_major_groups(oracle):
    packed = np.repeat(np.array([0x66, 0xee, 0x66, 0x66], np.uint8), 16)
    rc, _, _, v = oracle.mx_reconstruct("mxfp4", 2, 64, packed, np.array([125, 128, 126, 129], np.uint8))
    assert rc == 0
    _same(v, np.repeat(_f32([1, -8, 2, 16]), 32))


def test_mxfp4_rejections(oracle):
    rc, g, _, _ = oracle.mx_reconstruct("mxfp4", 1, 32, np.zeros(16, np.uint8), np.array([255], np.uint8))
    assert (rc, g) == (1, 0)
    assert oracle.mx_error("mxfp4", rc, g, -1) == "MXFP4 WEIGHT E8M0 scale is NaN in group 0."
    packed = np.zeros(16, np.uint8)
    packed[0] = 0x77
    rc, g, e, _ = oracle.mx_reconstruct("mxfp4", 1, 32, packed, np.array([254], np.uint8))
    assert (rc, g, e) == (5, 0, 0)


def _write6(codes):
    out = np.zeros(len(codes) * 6 // 8, np.uint8)
    for i, c in enumerate(codes):
        bit = 6 * i
        out[bit // 8] |= (c << (bit % 8)) & 0xff
        if bit % 8 > 2:
            out[bit // 8 + 1] |= c >> (8 - bit % 8)
    return out


def test_mxfp6_pinned_packing(oracle):
    packed = np.array([0x48, 0xf8, 0x01] * 8, np.uint8)
    rc, _, _, v = oracle.mx_reconstruct("mxfp6_e2m3", 1, 32, packed, np.array([127], np.uint8))
    assert rc == 0
    _same(v, [1, -.125, 7.5, 0] * 8)
    assert np.array_equal(_write6([8, 0x21, 31, 0] * 8), packed)


def test_mxfp6_scale_threshold_rows(oracle):
    scales = np.array([125, 126, 126, 127, 127, 128, 0, 252], np.uint8)
    codes = [24, 31, 31, 24, 31, 24, 0, 31]
    packed = np.concatenate([_write6([c] * 32) for c in codes])
    rc, _, _, v = oracle.mx_reconstruct("mxfp6_e2m3", 4, 64, packed, scales)
    assert rc == 0
    want = [1, 3.75, 3.75, 4, 7.5, 8, 0, math.ldexp(7.5, 125)]
    _same(v, np.repeat(_f32(want), 32))


def test_mxfp6_every_code_and_scale_extremes(oracle):
    packed = _write6(list(range(64)))
    rc, _, _, v = oracle.mx_reconstruct("mxfp6_e2m3", 2, 32, packed, np.array([127, 0], np.uint8))
    assert rc == 0
    for i in range(64):
        sign = -1.0 if i & 0x20 else 1.0
        e, m = (i >> 3) & 3, i & 7
        mag = m / 8.0 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 1)
        want = np.float32(sign * mag * (1.0 if i < 32 else 2.0 ** -127))
        assert v.reshape(-1)[i].view(np.uint32) == want.view(np.uint32), i
    rc, _, _, v = oracle.mx_reconstruct("mxfp6_e2m3", 1, 32, _write6([8] + [0] * 31), np.array([254], np.uint8))
    assert rc == 0 and v[0, 0] == np.float32(2.0 ** 127)
    rc, g, _, _ = oracle.mx_reconstruct("mxfp6_e2m3", 1, 32, _write6([8] * 32), np.array([255], np.uint8))
    assert (rc, g) == (1, 0)
    rc, g, e, _ = oracle.mx_reconstruct("mxfp6_e2m3", 1, 32, _write6([0, 16] + [0] * 30), np.array([254], np.uint8))
    assert (rc, g, e) == (5, 0, 1)


def test_nvfp4_fixtures(oracle):
    packed = np.array([0x20, 0x42, 0x64, 0x76, 0xA8, 0xCA, 0xEC, 0xFE] * 2, np.uint8)
    rc, _, _, v = oracle.mx_reconstruct("nvfp4", 1, 32, packed, np.array([0x38, 0x3A], np.uint8), 1.0)
    assert rc == 0
    _same(v[0, :16], [0, 1, 1, 2, 2, 4, 4, 6, -0.0, -1, -1, -2, -2, -4, -4, -6])
    rc, _, _, v = oracle.mx_reconstruct("nvfp4", 1, 16, np.full(8, 0x11, np.uint8), np.array([0x38], np.uint8), 1.0)
    assert rc == 0
    _same(v, [0.5] * 16)
    packed = np.repeat(np.array([0x77, 0x55, 0x33, 0x22], np.uint8), 8)
    rc, _, _, v = oracle.mx_reconstruct("nvfp4", 2, 32, packed, np.array([0x38, 0x40, 0x48, 0x50], np.uint8), 2.0)
    want = np.full((2, 32), 3, np.float32)
    want[1, 16:] = 4
    assert rc == 0
    _same(v, want)
    packed = np.array([0x10, 0x32, 0x54, 0x76, 0x90, 0xBA, 0xDC, 0xFE] * 2, np.uint8)
    rc, _, _, v = oracle.mx_reconstruct("nvfp4", 1, 32, packed, np.array([0x7E, 0x6E], np.uint8), 224.0)
    assert rc == 0
    _same(v, np.concatenate([_f32(LEVELS) * 2, _f32(LEVELS) * 0.5]))
    rc, _, _, v = oracle.mx_reconstruct("nvfp4", 1, 16, np.full(8, 0x33, np.uint8), np.array([0x01], np.uint8), 7.0)
    eff = np.float32(np.float32(2.0 ** -9) / np.float32(7))
    assert rc == 0
    _same(v, np.full(16, np.float32(1.5) * eff, np.float32))


def test_nvfp4_rejections_in_order(oracle):
    z = np.zeros(8, np.uint8)
    # a zero quotient (step 3) cannot occur: the smallest local scale 2^-9
    # over the largest global scale is 2^-137, a nonzero fp32 subnormal
    for scales, glob, want in (([0x38, 0x00], 1.0, (1, 1)), ([0x38], float("nan"), (1, 0)),
                               ([0x38], -1.0, (1, 0)), ([0x7E], 1e-40, (2, 0)), ([0x01], 3e38, (0, -1))):
        s = np.array(scales, np.uint8)
        rc, g, _, _ = oracle.mx_reconstruct("nvfp4", 1, 16 * len(scales), np.zeros(8 * len(scales), np.uint8), s,
                                            glob)
        assert (rc, g) == want, (scales, glob)
    assert z.sum() == 0


def test_mxfp8_every_code_times_powers_of_two(oracle):
    codes = np.arange(256, dtype=np.uint8)
    codes = codes[(codes & 0x7f) != 0x7f]
    codes = np.concatenate([codes, codes[:2]])[:256 - 2]  # 254 codes
    codes = np.concatenate([codes, np.zeros(2, np.uint8)]).reshape(8, 32)
    for e in (0, 1, 100, 127, 130, 200):
        rc, _, _, v = oracle.mx_reconstruct("mxfp8", 8, 32, codes, np.full(8, e, np.uint8))
        assert rc == 0
        for c, got in zip(codes.reshape(-1), v.reshape(-1)):
            sign = -1.0 if c & 0x80 else 1.0
            ex, m = (int(c) >> 3) & 15, int(c) & 7
            mag = m * 2.0 ** -9 if ex == 0 else (1 + m / 8.0) * 2.0 ** (ex - 7)
            want = np.float32(sign * math.ldexp(mag, (e if e else 0) - 127))
            assert got.view(np.uint32) == want.view(np.uint32), (c, e)


def test_mxfp8_rejections_in_order(oracle):
    codes = np.full((2, 32), 0x38, np.uint8)
    codes[1, 5] = 0x7F
    codes[1, 3] = 0x7E  # 448 at 2^127 overflows before the NaN code
    rc, g, e, _ = oracle.mx_reconstruct("mxfp8", 2, 32, codes, np.array([127, 254], np.uint8))
    assert (rc, g, e) == (5, 1, 3)
    rc, g, e, _ = oracle.mx_reconstruct("mxfp8", 2, 32, codes, np.array([127, 127], np.uint8))
    assert (rc, g, e) == (4, 1, 5)
    rc, g, _, _ = oracle.mx_reconstruct("mxfp8", 2, 32, codes, np.array([127, 255], np.uint8))
    assert (rc, g) == (1, 1)
    assert oracle.mx_error("mxfp8", 4, 1, 5) == "MXFP8 E4M3FN weight must not be NaN."


def test_output_range(oracle):
    rc, _, _, _ = oracle.mx_reconstruct("mxfp4", 1, 32, np.full(16, 0x77, np.uint8), np.array([150], np.uint8),
                                        out_dtype=10)
    assert rc == 6
