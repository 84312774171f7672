"""CPU checks of the oracle's QuantizeLinear and DynamicQuantizeLinear
(oracle/oracle.c, restating kq/kernel_quantizelinear.cc and
kq/kernel_dynamicquantizelinear.cc): the known answers the reference's own
tests hold (tests/golden/reference_known_answers.json), and a numpy float32
closed form (IEEE true division, np.rint ties-to-even, saturation) over random
inputs in every scale layout and output type."""
import zlib

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
