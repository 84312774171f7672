"""CPU checks of the oracle's QuantizeLinear and DynamicQuantizeLinear
(oracle/oracle.c, restating kq/kernel_quantizelinear.cc and
kq/kernel_dynamicquantizelinear.cc): the known answers the reference's own
tests hold (tests/golden/reference_known_answers.json), and a numpy float32
closed form (IEEE true division, np.rint ties-to-even, saturation) over random
inputs in every scale layout and output type."""
import zlib
from fractions import Fraction

import numpy as np
import pytest

DT = {"float": 1, "uint8": 2, "int8": 3, "uint16": 4, "int16": 5, "float16": 10, "float8e4m3fn": 17,
      "uint4": 21, "int4": 22}
NP = {"uint8": np.uint8, "int8": np.int8, "uint16": np.uint16, "int16": np.int16, "float8e4m3fn": np.uint8}
RANGE = {"uint8": (0, 255), "int8": (-128, 127), "uint16": (0, 65535), "int16": (-32768, 32767),
         "uint4": (0, 15), "int4": (-8, 7)}


def _values(oracle, vals, dtype, shape):
    a = np.array(vals, np.float32).reshape(shape)
    return oracle.f32_to_f16_bits(a) if dtype == "float16" else a


def _zp_storage(oracle, zp, y_dtype, shape):
    if y_dtype in ("uint4", "int4"):
        return oracle.pack_int4(np.array(zp).reshape(-1))
    if y_dtype == "float8e4m3fn":
        return oracle.f32_to_f8e4m3fn_bits(np.array(zp, np.float32)).reshape(shape)
    return np.array(zp, NP[y_dtype]).reshape(shape)


def _unpack4(y, n, signed):
    nib = np.stack([y & 15, y >> 4], axis=1).reshape(-1)[:n].astype(np.int32)
    return np.where(nib >= 8, nib - 16, nib) if signed else nib


def test_quantize_known_answers(oracle, golden):
    for c in golden["quantize_linear"]:
        x = _values(oracle, c["x"], c["x_dtype"], c["x_shape"])
        s = _values(oracle, c["scale"], c["scale_dtype"], c["scale_shape"])
        zp = None if c["zp"] is None else _zp_storage(oracle, c["zp"], c["y_dtype"], c["zp_shape"])
        y = oracle.quantize_linear(x, DT[c["x_dtype"]], s, DT[c["scale_dtype"]], DT[c["y_dtype"]], zp, c["axis"])
        if c["y_dtype"] in ("uint4", "int4"):
            got = _unpack4(y, x.size, c["y_dtype"] == "int4").tolist()
        else:
            got = y.reshape(-1).astype(np.int64).tolist()
        assert got == c["y"], c["name"]
        if "y_values" in c:
            assert oracle.f8e4m3fn_bits_to_f32(y).tolist() == c["y_values"], c["name"]


def _closed_form(oracle, x32, s32_full, z_full, y_dtype):
    q = (x32 / s32_full).astype(np.float32)
    if y_dtype == "float8e4m3fn":
        return oracle.f32_to_f8e4m3fn_bits((q + z_full).astype(np.float32))
    lo, hi = RANGE[y_dtype]
    return np.clip(np.rint(q) + z_full, lo, hi).astype(np.int64)


@pytest.mark.parametrize("y_dtype", ["uint8", "int8", "uint16", "int16", "uint4", "int4", "float8e4m3fn"])
@pytest.mark.parametrize("layout", ["tensor", "axis", "blocked"])
@pytest.mark.parametrize("x_dtype", ["float", "float16"])
def test_quantize_closed_form_random(oracle, y_dtype, layout, x_dtype):
    rng = np.random.default_rng(zlib.crc32(repr((y_dtype, layout, x_dtype)).encode()))
    shape, axis = (6, 64), 1 if layout != "blocked" else 1
    xv = (rng.standard_normal(shape) * rng.choice([3.0, 40.0, 300.0])).astype(np.float32)
    x = oracle.f32_to_f16_bits(xv) if x_dtype == "float16" else xv
    x32 = oracle.f16_bits_to_f32(x) if x_dtype == "float16" else xv
    if layout == "tensor":
        s_shape = ()
    elif layout == "axis":
        s_shape = (shape[axis],)
    else:
        s_shape = (6, 64 // 16)
    sv = rng.uniform(0.05, 2.0, s_shape).astype(np.float32)
    s = oracle.f32_to_f16_bits(sv) if x_dtype == "float16" else sv
    s32 = oracle.f16_bits_to_f32(s) if x_dtype == "float16" else sv
    lo, hi = RANGE.get(y_dtype, (-4, 4))
    zv = rng.integers(lo // 2 if lo < 0 else 0, hi // 2 + 1, s_shape) if y_dtype != "float8e4m3fn" \
        else rng.choice([0.0, 1.0, -2.0, 0.5], s_shape).astype(np.float32)
    zv = np.asarray(zv).reshape(s_shape)
    zp = _zp_storage(oracle, zv, y_dtype, s_shape)
    z32 = oracle.f8e4m3fn_bits_to_f32(zp).reshape(s_shape) if y_dtype == "float8e4m3fn" else zv.astype(np.float32)
    if layout == "tensor":
        s_full, z_full = s32.reshape(()), z32.reshape(())
    elif layout == "axis":
        s_full, z_full = s32.reshape(1, -1), z32.reshape(1, -1)
    else:
        s_full, z_full = np.repeat(s32, 16, axis=1), np.repeat(z32, 16, axis=1)
    for with_zp in (True, False):
        y = oracle.quantize_linear(x, DT[x_dtype], s, DT[x_dtype], DT[y_dtype], zp if with_zp else None, axis)
        want = _closed_form(oracle, x32, np.broadcast_to(s_full, shape), np.broadcast_to(z_full if with_zp else
                            np.float32(0), shape), y_dtype)
        if y_dtype in ("uint4", "int4"):
            got = _unpack4(y, x32.size, y_dtype == "int4").reshape(shape)
        else:
            got = y.astype(np.int64) if y_dtype != "float8e4m3fn" else y
        assert np.array_equal(got, want), (y_dtype, layout, x_dtype, with_zp)


def test_quantize_ties_nan_and_saturation(oracle):
    """Ties go to even before the zero point is added; NaN lands as 0 (the
    x86-64 conversion of the reference build); infinities saturate."""
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, np.nan, np.inf, -np.inf], np.float32)
    s = np.array([1.0], np.float32).reshape(())
    for y_dtype, zp_val, want in (("uint8", 10, [10, 12, 12, 10, 8, 0, 255, 0]),
                                  ("int8", 0, [0, 2, 2, 0, -2, 0, 127, -128]),
                                  ("int16", 0, [0, 2, 2, 0, -2, 0, 32767, -32768])):
        zp = np.array(zp_val, NP[y_dtype]).reshape(())
        y = oracle.quantize_linear(x, 1, s, 1, DT[y_dtype], zp, 1)
        assert y.astype(np.int64).tolist() == want, y_dtype


def test_dynamic_quantize_known_answers(oracle, golden):
    for c in golden["dynamic_quantize_linear"]:
        x = np.array(c["x"], np.float32).reshape(c["x_shape"])
        y, sc, zp = oracle.dynamic_quantize_linear(x)
        assert abs(float(sc) - c["scale"]) <= c["scale_tol"], c["name"]
        assert int(zp) == c["zp"], c["name"]
        assert y.reshape(-1).tolist() == c["y"], c["name"]
    for v in golden["dynamic_quantize_linear_rejects"]["values"]:
        with pytest.raises(ValueError):
            oracle.dynamic_quantize_linear(np.array([0.0, float(v)], np.float32))
    with pytest.raises(ValueError):
        oracle.dynamic_quantize_linear(np.zeros(0, np.float32))


@pytest.mark.parametrize("spread", [(0.0, 1.0), (-3.0, 1.0), (5.0, 0.1), (-7.0, 0.01), (0.0, 1e-30)])
def test_dynamic_quantize_closed_form_random(oracle, spread):
    rng = np.random.default_rng(int(abs(spread[0]) * 100 + spread[1] * 1000) % 9973)
    x = (spread[0] + spread[1] * rng.standard_normal(3000)).astype(np.float32)
    y, sc, zp = oracle.dynamic_quantize_linear(x)
    mn, mx = min(np.float32(0), x.min()), max(np.float32(0), x.max())
    rng_ = np.float32(mx - mn)
    want_sc = np.float32(1) if rng_ == 0 else np.float32(rng_ / np.float32(255))
    want_zp = int(np.clip(np.rint(np.float32(-mn) / want_sc), 0, 255))
    assert np.float32(sc) == want_sc and int(zp) == want_zp
    want = np.clip(np.rint(x / want_sc) + np.float32(want_zp), 0, 255).astype(np.uint8)
    assert np.array_equal(y, want)


def test_fp8_nan_sign_follows_x86(oracle):
    """FLOAT8E4M3FN keeps the fp32 NaN's sign (0x7f / 0xff).  On x86-64, where
    the reference is built, an invalid operation (0/0, inf/inf) returns the
    negative "real indefinite" QNaN 0xffc00000, and a NaN operand is returned
    as it is (the destination operand when both are NaN: x for x / scale; for
    the commutative quotient + zero point gcc -O2 puts the zero point there).
    The oracle runs on the same instruction set, and the GPU kernel restates
    the rule."""
    x = np.array([0.0, np.inf, np.nan, -np.nan, 1.0], np.float32)
    zp = np.zeros(1, np.uint8).reshape(())
    for sv, want in ((0.0, [0xff, 0x7e, 0x7f, 0xff, 0x7e]), (np.inf, [0x00, 0xff, 0x7f, 0xff, 0x00])):
        y = oracle.quantize_linear(x, 1, np.array(sv, np.float32), 1, DT["float8e4m3fn"], zp, 1)
        assert y.tolist() == want, sv
    nan_zp = np.array(0x7f, np.uint8).reshape(())
    y = oracle.quantize_linear(np.array([1.0, -np.nan], np.float32), 1, np.array(1.0, np.float32), 1,
                               DT["float8e4m3fn"], nan_zp, 1)
    assert y.tolist() == [0x7f, 0x7f]


# ---- the float and 2-bit output types ---------------------------------------
# Codes per type and whether the type is FNUZ (no negative zero, one NaN).
FLOAT_CODES = {18: (256, True), 19: (256, False), 20: (256, True), 23: (16, False), 27: (64, False),
               28: (64, False)}


def _table(oracle, dtype):
    """Decoded value of every code (the decoders are pinned against numpy's
    fp16, the formats' maxima and subnormal steps in test_oracle_codecs)."""
    n, _ = FLOAT_CODES[dtype]
    bits = {16: 4, 64: 6}.get(n, 8)
    raw = np.arange(n, dtype=np.uint8) if bits == 8 else oracle.pack_bits(np.arange(n), bits)
    return oracle.dq_decode(raw, dtype, n).astype(np.float64)


def _nearest(oracle, dtype, v):
    """Brute-force nearest finite code to v among the codes of v's sign (the
    FNUZ types' single zero included), exact rational distances, ties to the
    even code; what every encoder of the reference computes, stated without
    its bit manipulations."""
    n, fnuz = FLOAT_CODES[dtype]
    vals = _table(oracle, dtype)
    sign_bit = {256: 0x80, 16: 8, 64: 0x20}[n]
    neg = np.signbit(np.float32(v))
    best = None
    for c in range(n):
        if not np.isfinite(vals[c]):
            continue
        if fnuz:
            if c != 0 and bool(c & sign_bit) != neg:
                continue
        elif bool(c & sign_bit) != neg:
            continue
        d = abs(Fraction(float(v)) - Fraction(vals[c]))
        if best is None or d < best[0] or (d == best[0] and c % 2 == 0 and best[1] % 2 == 1):
            best = (d, c)
    return best[1]


@pytest.mark.parametrize("dtype", sorted(FLOAT_CODES))
def test_float_encoders_round_trip(oracle, dtype):
    """Every finite code decodes and encodes back to itself; the E5M2
    infinities saturate to the largest finite code."""
    n, _ = FLOAT_CODES[dtype]
    vals = _table(oracle, dtype).astype(np.float32)
    codes = oracle.float_code(vals, dtype)
    for c in range(n):
        if np.isnan(vals[c]):
            continue
        want = (c & 0x80) | 0x7B if np.isinf(vals[c]) else c
        assert codes[c] == want, (dtype, c, vals[c])


@pytest.mark.parametrize("dtype", sorted(FLOAT_CODES))
def test_float_encoders_nearest_even(oracle, dtype):
    """Midpoints of adjacent codes (ties, exact in fp32), points just either
    side of them, random values across the range and beyond it: the nearest
    code by brute force, ties to the even code, saturation past the
    largest."""
    vals = np.unique(_table(oracle, dtype)[np.isfinite(_table(oracle, dtype))])
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    probes = [mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))]
    rng = np.random.default_rng(dtype)
    top = float(vals.max())
    probes.append((rng.uniform(-1.5, 1.5, 300) * top).astype(np.float32))
    probes.append((rng.standard_normal(200) * float(vals[vals > 0].min()) * 4).astype(np.float32))
    probes.append(np.array([top * 1.01, -top * 4, 1e30, -1e-30, 1e-30, -0.0, 0.0], np.float32))
    x = np.concatenate(probes)
    got = oracle.float_code(x, dtype)
    want = [_nearest(oracle, dtype, v) for v in x]
    bad = [(float(v), int(g), int(w)) for v, g, w in zip(x, got, want) if g != w]
    assert not bad, bad[:8]


def test_float_encoders_specials(oracle):
    """NaN: 0x80 for the FNUZ types, sign|0x7e for E5M2 (cast_float8.cc:
    214-262), 0 for FLOAT4E2M1 and FLOAT6 (cast_helper.cc:168-246);
    infinities saturate."""
    x = np.array([np.nan, -np.nan, np.inf, -np.inf], np.float32)
    assert oracle.float_code(x, 18).tolist() == [0x80, 0x80, 0x7F, 0xFF]
    assert oracle.float_code(x, 19).tolist() == [0x7E, 0xFE, 0x7B, 0xFB]
    assert oracle.float_code(x, 20).tolist() == [0x80, 0x80, 0x7F, 0xFF]
    assert oracle.float_code(x, 23).tolist() == [0, 0, 7, 15]
    assert oracle.float_code(x, 27).tolist() == [0, 0, 0x1F, 0x3F]
    assert oracle.float_code(x, 28).tolist() == [0, 0, 0x1F, 0x3F]


def test_quantize_float6_and_float4_known_answers(oracle):
    """The reference's own answers: QuantizeAndDequantizeLinearFloat6
    (unittests/cc/onnx_extensions/kernels/kernels/test_kernels_quantization.cc:
    136-154) and the FLOAT4E2M1 signed-zero case without a zero point
    (unittests/cc/onnx_extensions/backend_test/cases/test_cases_quantization.cc:
    271-287)."""
    x = np.array([-1.0, -0.5, 0.0, 1.0, 2.0], np.float32)
    one = np.array(1.0, np.float32)
    for dtype, want in ((27, [40, 9, 32, 16]), (28, [44, 10, 48, 16])):
        y = oracle.quantize_linear(x, 1, one, 1, dtype, np.zeros(1, np.uint8), 0)
        assert y.tolist() == want, dtype
    y = oracle.quantize_linear(np.array([-0.0, 0.0], np.float32), 1, one, 1, 23, None, 0)
    assert y.tolist() == [0x08]
    # a zero point of +0 turns -0 into +0 (-0 + 0 = +0)
    y = oracle.quantize_linear(np.array([-0.0, 0.0], np.float32), 1, one, 1, 23, np.zeros(1, np.uint8), 0)
    assert y.tolist() == [0x00]


@pytest.mark.parametrize("dtype", [25, 26])
def test_quantize_int2_closed_form(oracle, dtype):
    """UINT2 / INT2 (kq/kernel_quantizelinear.cc:202-224): rint(x / scale) +
    zero point saturated to 0..3 / -2..1, packed four per byte from the low
    bits; per axis with a zero point per row."""
    rng = np.random.default_rng(dtype)
    x = (rng.standard_normal((5, 13)) * 3).astype(np.float32)
    x[0, :4] = [0.5, 1.5, -0.5, -2.5]  # ties
    s = rng.uniform(0.5, 2.0, 5).astype(np.float32)
    lo, hi = (0, 3) if dtype == 25 else (-2, 1)
    z = rng.integers(lo, hi + 1, 5)
    y = oracle.quantize_linear(x, 1, s, 1, dtype, oracle.pack_bits(z & 3, 2), 0)
    q = (x / s[:, None]).astype(np.float32)
    want = np.clip(np.rint(q) + z[:, None], lo, hi).astype(np.int64) & 3
    assert y.tolist() == oracle.pack_bits(want.reshape(-1), 2).tolist()
