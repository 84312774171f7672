"""Pins the oracle's scalar codecs and RNG against independent implementations
(numpy float16, torch bfloat16 / float8_e4m3fn) and closed forms, exhaustively
where the code space is small."""
import numpy as np
import pytest
import torch


def _bits32(x):
    return np.asarray(x, np.float32).view(np.uint32)


def test_f16_decode_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_bits_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(_bits32(got[~nan]), _bits32(ref[~nan]))
    # NaN keeps sign and payload: sign | 0x7f800000 | man << 13
    c = codes[nan].astype(np.uint32)
    want = ((c & 0x8000) << 16) | 0x7F800000 | ((c & 0x3FF) << 13)
    assert np.array_equal(_bits32(got[nan]), want)


def _f16_probe_set():
    """Every fp16 value, every midpoint between neighbours, the midpoints
    +-1 fp32 ulp, plus random fp32 bit patterns over the whole range."""
    finite = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = np.unique(finite[np.isfinite(finite)].astype(np.float64))
    mids = (finite[1:] + finite[:-1]) / 2.0
    mids32 = mids.astype(np.float32)
    up = np.nextafter(mids32, np.float32(np.inf))
    dn = np.nextafter(mids32, np.float32(-np.inf))
    rng = np.random.default_rng(0)
    rnd = rng.integers(0, 2**32, size=1 << 21, dtype=np.uint64).astype(np.uint32).view(np.float32)
    extra = np.array([65504.0, 65519.99, 65520.0, 65536.0, 1e30, -1e30, np.inf, -np.inf, 0.0, -0.0,
                      2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001, 2.0**-26, 1e-45], np.float32)
    return np.concatenate([finite.astype(np.float32), mids32, up, dn, rnd, extra])


def test_f16_encode_matches_numpy_rne(oracle):
    x = _f16_probe_set()
    x = x[~np.isnan(x)]
    got = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f16_encode_nan_is_quiet_with_sign(oracle):
    x = np.array([0x7F800001, 0x7FC00000, 0xFFFFFFFF, 0xFF800001], np.uint32).view(np.float32)
    got = oracle.f32_to_f16_bits(x)
    assert list(got) == [0x7E00, 0x7E00, 0xFE00, 0xFE00]


def test_bf16_codecs_match_torch(oracle):
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    u = (hi[:, None] | lows[None, :]).reshape(-1)
    x = u.view(np.float32)
    got = oracle.f32_to_bf16_bits(x)
    nan = np.isnan(x)
    ref = torch.from_numpy(x[~nan].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[~nan], ref)
    # NaN: upper half with the quiet bit forced
    assert np.array_equal(got[nan], ((u[nan] >> 16) | 0x40).astype(np.uint16))
    dec = oracle.bf16_bits_to_f32(np.arange(65536, dtype=np.uint16))
    assert np.array_equal(_bits32(dec), np.arange(65536, dtype=np.uint32) << 16)


def _e4m3_closed_form(c):
    s = -1.0 if c & 0x80 else 1.0
    e, m = (c >> 3) & 0xF, c & 7
    if e == 15 and m == 7:
        return np.nan
    if e == 0:
        return s * m / 8.0 * 2.0**-6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def test_f8_decode_exhaustive(oracle):
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.f8e4m3fn_bits_to_f32(codes)
    want = np.array([_e4m3_closed_form(int(c)) for c in codes])
    ref_t = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(want)
    assert np.array_equal(got[~nan], want[~nan].astype(np.float32))
    assert np.array_equal(got[~nan], ref_t[~nan])
    assert np.isnan(got[nan]).all() and nan.sum() == 2
    assert _bits32(got[[0x7F]])[0] == 0x7FC00000 and _bits32(got[[0xFF]])[0] == 0xFFC00000


def test_f8_encode_rne_saturating(oracle):
    vals = np.array([_e4m3_closed_form(c) for c in range(0x7F)])  # 0 .. 448, ascending
    # every representable value round-trips
    for sgn in (1.0, -1.0):
        x = (sgn * vals).astype(np.float32)
        codes = oracle.f32_to_f8e4m3fn_bits(x)
        assert np.array_equal(codes & 0x7F, np.arange(0x7F, dtype=np.uint8))
        if sgn < 0:
            assert (codes[1:] & 0x80).all()
    # midpoints tie to the even code, +-1 ulp goes to the near side
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    lo = np.arange(0x7E, dtype=np.uint8)
    assert np.array_equal(oracle.f32_to_f8e4m3fn_bits(mids), np.where(lo % 2 == 0, lo, lo + 1))
    assert np.array_equal(oracle.f32_to_f8e4m3fn_bits(np.nextafter(mids, np.float32(0))), lo)
    assert np.array_equal(oracle.f32_to_f8e4m3fn_bits(np.nextafter(mids, np.float32(1e9))), lo + 1)
    # torch (non-saturating RNE) agrees below the saturation region
    rng = np.random.default_rng(1)
    r = (rng.standard_normal(1 << 18) * rng.choice([1e-3, 1.0, 100.0], 1 << 18)).astype(np.float32)
    r = r[np.abs(r) < 464.0]
    ref = torch.from_numpy(r.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.f32_to_f8e4m3fn_bits(r), ref)
    # saturation and specials
    x = np.array([464.0, 480.0, 1e6, np.inf, -np.inf, -500.0, np.nan, 2.0**-10, 2.0**-10 * 1.01,
                  1e-40], np.float32)
    assert list(oracle.f32_to_f8e4m3fn_bits(x)) == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE, 0x7F, 0x00,
                                                     0x01, 0x00]


def test_f8_reference_known_answers(oracle):
    # rk tests: {0, .5, 1, 448, -104} encode then decode exactly (test_kernels_quantization.cc:350-368)
    v = np.array([0.0, 0.5, 1.0, 448.0, -104.0], np.float32)
    assert np.array_equal(oracle.f8e4m3fn_bits_to_f32(oracle.f32_to_f8e4m3fn_bits(v)), v)


def test_splitmix64_published_vectors(oracle):
    # canonical SplitMix64 (Vigna), state 0: first outputs
    assert oracle.splitmix64(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_rng_samplers(oracle):
    u = oracle.rand_uniform(0, 4)
    assert u[0] == (0xE220A8397B1DCDAF >> 11) / 2.0**53
    r = oracle.rand_int(0, 256, 5, 100000)
    assert r.min() == 0 and r.max() == 255 and abs(r.mean() - 127.5) < 1.0
    r = oracle.rand_int(-4, 5, 7, 100000)
    assert set(np.unique(r)) == set(range(-4, 5))
    # rejection sampling: with span 3 the first draw is accepted unless >= 2^64 - (2^64 % 3)
    x = oracle.splitmix64(9, 1)[0]
    assert oracle.rand_int(0, 3, 9, 1)[0] == x % 3
    n = oracle.randn(3, 200000)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1.0) < 0.01 and np.abs(n).max() <= 6.0
    with pytest.raises(ValueError):
        oracle.rand_int(3, 3, 0, 1)


# ---- the further DequantizeLinear inputs (cast_float8.cc, cast_helper.cc,
# cast_sub_byte.h), pinned by numpy's fp16 (E5M2 is its top byte), the
# formats' published maxima and subnormal steps, and hand-packed bytes ------

def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_float8e5m2_is_the_fp16_top_byte(oracle):
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.dq_decode(codes, oracle.FLOAT8E5M2, 256)
    half = (codes.astype(np.uint16) << 8).view(np.float16).astype(np.float32)
    special = {124: 0x7F800000, 252: 0xFF800000, 125: 0x7FC00000, 126: 0x7FC00000, 127: 0x7FC00000,
               253: 0xFFC00000, 254: 0xFFC00000, 255: 0xFFC00000}
    for c in range(256):
        if c in special:
            assert _bits(got[c]) == special[c], c
        else:
            assert _bits(got[c]) == _bits(half[c]), c
    assert got[0x7B] == 57344.0 and got[1] == 2.0 ** -16


@pytest.mark.parametrize("dtype,bias,mbits,maxv,tiny", [("FLOAT8E4M3FNUZ", 8, 3, 240.0, 2.0 ** -10),
                                                         ("FLOAT8E5M2FNUZ", 16, 2, 57344.0, 2.0 ** -17)])
def test_float8_fnuz(oracle, dtype, bias, mbits, maxv, tiny):
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.dq_decode(codes, getattr(oracle, dtype), 256)
    eb = 7 - mbits
    for c in range(256):
        if c == 0x80:
            assert _bits(got[c]) == 0xFFC00000  # the only NaN
            continue
        e, m = (c >> mbits) & ((1 << eb) - 1), c & ((1 << mbits) - 1)
        mag = m * 2.0 ** (1 - bias - mbits) if e == 0 else (1 + m / 2 ** mbits) * 2.0 ** (e - bias)
        assert got[c] == (-mag if c & 0x80 else mag), c
    assert np.nanmax(got) == maxv and got[1] == tiny and _bits(got[0]) == 0


def test_float4e2m1_and_float6(oracle):
    # FLOAT4E2M1: the OCP MX element values; two per byte, low nibble first
    packed = oracle.pack_int4(np.arange(16))
    assert oracle.dq_decode(packed, oracle.FLOAT4E2M1, 16).tolist() == [
        0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    # FLOAT6E2M3 / FLOAT6E3M2: the OCP MX maxima 7.5 / 28 and subnormal steps 1/8 / 1/16
    raw = oracle.pack_bits(np.arange(64), 6)
    for dtype, maxv, step, mb in (("FLOAT6E2M3", 7.5, 0.125, 3), ("FLOAT6E3M2", 28.0, 0.0625, 2)):
        v = oracle.dq_decode(raw, getattr(oracle, dtype), 64)
        assert v[31] == maxv and v[63] == -maxv and v[1] == step and v[32] == 0.0 and np.signbit(v[32])
        pos = v[:32]
        assert np.all(np.diff(pos) > 0)                         # monotone magnitudes
        assert np.array_equal(pos[:(1 << mb)], step * np.arange(1 << mb))  # evenly spaced subnormals
        assert np.array_equal(v[32:], -pos)


def test_two_and_six_bit_packing(oracle):
    # four 2-bit elements per byte from the low bits; INT2 is two's complement
    assert oracle.dq_decode(np.array([0b11100100], np.uint8), oracle.UINT2, 4).tolist() == [0, 1, 2, 3]
    assert oracle.dq_decode(np.array([0b11100100], np.uint8), oracle.INT2, 4).tolist() == [0, 1, -2, -1]
    # six-bit elements as one little-endian bit stream: codes 1, 2, 3, 4 -> 0x103081
    raw = np.array([0x81, 0x30, 0x10], np.uint8)
    assert np.array_equal(oracle.pack_bits([1, 2, 3, 4], 6), raw)
    assert oracle.dq_decode(raw, oracle.FLOAT6E3M2, 4).tolist() == [0.0625, 0.125, 0.1875, 0.25]
