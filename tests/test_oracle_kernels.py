"""Pins the oracle's kernels: the reference's own known-answer vectors
(tests/golden/reference_known_answers.json) plus independent numpy closed
forms and brute force on random small inputs, including broadcasting."""
import numpy as np
import pytest

NP = {"uint8": np.uint8, "int8": np.int8, "uint16": np.uint16, "int16": np.int16}


def test_matmul_integer_known_answers(oracle, golden):
    for c in golden["matmul_integer"]:
        a = np.array(c["a"], NP[c["a_dtype"]]).reshape(c["a_shape"])
        b = np.array(c["b"], NP[c["b_dtype"]]).reshape(c["b_shape"])
        za = None if c["a_zp"] is None else c["a_zp"]["values"]
        zb = None if c["b_zp"] is None else c["b_zp"]["values"]
        y = oracle.matmul_integer(a, b, za, zb)
        assert list(y.shape) == c["y_shape"], c["name"]
        assert y.reshape(-1).tolist() == c["y"], c["name"]


def test_matmul_shape_rules(oracle, golden):
    for c in golden["matmul_shapes"]:
        assert list(oracle.matmul_output_shape(c["a_shape"], c["b_shape"])) == c["y_shape"]
    with pytest.raises(ValueError):
        oracle.matmul_output_shape([2, 3], [4, 2])
    with pytest.raises(ValueError):
        oracle.matmul_output_shape([2, 2, 3], [3, 3, 4])


def _np_mmi(a, b, za, zb):
    """numpy int64 brute force of Y = (A - za[:,None]) @ (B - zb[None,:])."""
    a2 = a.astype(np.int64)
    b2 = b.astype(np.int64)
    za = np.asarray(za, np.int64).reshape(-1)
    zb = np.asarray(zb, np.int64).reshape(-1)
    if a.ndim == 1:
        a2 = a2[None, :]
    if b.ndim == 1:
        b2 = b2[:, None]
    a2 = a2 - (za[:, None] if za.size > 1 else (za[0] if za.size else 0))
    b2 = b2 - (zb[None, :] if zb.size > 1 else (zb[0] if zb.size else 0))
    y = np.matmul(a2, b2)
    if a.ndim == 1:
        y = y[..., 0, :]
    if b.ndim == 1:
        y = y[..., 0]
    return y


@pytest.mark.parametrize("a_shape,b_shape", [
    ((5, 7), (7, 3)), ((2, 4, 9), (2, 9, 6)), ((3, 1, 4, 8), (5, 8, 2)), ((1, 6, 5), (3, 5, 4)),
    ((7,), (7, 3)), ((4, 7), (7,)), ((6,), (6,)), ((2, 3, 17, 33), (1, 33, 19)), ((0, 4), (4, 3)),
])
@pytest.mark.parametrize("dt", [(np.uint8, np.int8), (np.int8, np.int8), (np.uint8, np.uint8),
                                (np.int8, np.uint8)])
def test_matmul_integer_brute_force(oracle, a_shape, b_shape, dt):
    rng = np.random.default_rng(len(a_shape) * 7 + len(b_shape))
    ia, ib = np.iinfo(dt[0]), np.iinfo(dt[1])
    a = rng.integers(ia.min, ia.max + 1, a_shape).astype(dt[0])
    b = rng.integers(ib.min, ib.max + 1, b_shape).astype(dt[1])
    M = a_shape[-2] if len(a_shape) > 1 else 1
    N = b_shape[-1] if len(b_shape) > 1 else 1
    for za, zb in [([0], [0]), ([int(rng.integers(ia.min, ia.max + 1))], [int(rng.integers(ib.min, ib.max + 1))]),
                   (rng.integers(ia.min, ia.max + 1, M), rng.integers(ib.min, ib.max + 1, N))]:
        y = oracle.matmul_integer(a, b, za, zb)
        ref = _np_mmi(a, b, za, zb)
        assert y.shape == ref.shape
        assert np.array_equal(y.astype(np.int64), ref)


def _np_qlinear(a, a_s, za, b, b_s, zb, y_s, zy, out_dt):
    acc = np.matmul(a.astype(np.int64) - za, b.astype(np.int64) - zb)
    cs = np.float32(np.float32(a_s) * np.float32(b_s)) / np.float32(y_s)
    v = np.rint(acc.astype(np.float32) * np.float32(cs)).astype(np.float32) + np.float32(zy)
    info = np.iinfo(out_dt)
    return np.clip(v, info.min, info.max).astype(out_dt)


def test_qlinear_known_answers(oracle, golden):
    for c in golden["qlinear_matmul"]:
        dt = NP[c["dtype"]]
        a = np.array(c["a"], dt).reshape(c["a_shape"])
        b = np.array(c["b"], dt).reshape(c["b_shape"])
        y = oracle.qlinear_matmul(a, c["a_scale"], c["a_zp"], b, c["b_scale"], c["b_zp"],
                                  c["y_scale"], c["y_zp"])
        assert y.reshape(-1).tolist() == c["y"], c["name"]


def test_qlinear_int8_and_fp16_scale_variants(oracle, golden):
    """cases_qlinearmatmul.cc:118-247: the INT8 variant shifts every input by
    -127; fp16 scales give the same output for these inputs."""
    c = golden["qlinear_matmul"][0]
    a = (np.array(c["a"]) - 127).astype(np.int8).reshape(2, 4)
    b = (np.array(c["b"]) - 127).astype(np.int8).reshape(4, 3)
    y = oracle.qlinear_matmul(a, 0.0066, 113 - 127, b, 0.00705, 114 - 127, 0.0107, 118 - 127)
    ref = _np_qlinear(a, 0.0066, -14, b, 0.00705, -13, 0.0107, -9, np.int8)
    assert np.array_equal(y, ref)
    # 255 - 127 = 128 wraps to -128 in the INT8 tensor (cases_qlinearmatmul.cc:49-56);
    # the result is the INT8 output listed at cases_qlinearmatmul.cc:229-230.
    assert y.reshape(-1).tolist() == [41, -12, -9, 1, -75, -128]
    h = lambda v: float(np.float16(v))
    au = np.array(c["a"], np.uint8).reshape(2, 4)
    bu = np.array(c["b"], np.uint8).reshape(4, 3)
    yh = oracle.qlinear_matmul(au, h(0.0066), 113, bu, h(0.00705), 114, h(0.0107), 118)
    assert yh.reshape(-1).tolist() == c["y"]
    # 3-D: the 2-D case stacked twice along a batch dimension
    a3 = np.stack([au, au])
    b3 = np.stack([bu, bu])
    y3 = oracle.qlinear_matmul(a3, 0.0066, 113, b3, 0.00705, 114, 0.0107, 118)
    assert y3.reshape(2, -1).tolist() == [c["y"], c["y"]]


@pytest.mark.parametrize("dt", [np.uint8, np.int8])
def test_qlinear_closed_form_random(oracle, dt):
    rng = np.random.default_rng(11)
    info = np.iinfo(dt)
    for shape_a, shape_b in [((17, 64), (64, 23)), ((3, 5, 40), (40, 9)), ((2, 1, 8, 16), (3, 16, 4))]:
        a = rng.integers(info.min, info.max + 1, shape_a).astype(dt)
        b = rng.integers(-128, 128, shape_b).astype(np.int8)
        for _ in range(3):
            a_s, b_s, y_s = rng.uniform(0.001, 0.05, 3)
            za = int(rng.integers(info.min, info.max + 1))
            zb = int(rng.integers(-128, 128))
            zy = int(rng.integers(info.min, info.max + 1))
            y = oracle.qlinear_matmul(a, a_s, za, b, b_s, zb, y_s, zy, y_dtype=3 if dt == np.int8 else 2)
            ref = _np_qlinear(a, a_s, za, b, b_s, zb, y_s, zy, dt)
            assert np.array_equal(y, ref)


def _x_raw(c, oracle):
    dt = c["x_dtype"]
    if dt == "float8e4m3fn":
        return oracle.f32_to_f8e4m3fn_bits(c["x_float"]), oracle.FLOAT8E4M3FN
    if dt in ("int4", "uint4"):
        return oracle.pack_int4(c["x"]), oracle.INT4 if dt == "int4" else oracle.UINT4
    code = {"uint8": oracle.UINT8, "int8": oracle.INT8, "uint16": oracle.UINT16, "int16": oracle.INT16}[dt]
    return np.array(c["x"], NP[dt]), code


def _zp_raw(c, oracle, x_code):
    if c["zp"] is None:
        return None
    v = c["zp"]["values"]
    if x_code in (oracle.INT4, oracle.UINT4):
        return oracle.pack_int4(v)
    return np.array(v, NP[c["x_dtype"]])


def test_dequantize_known_answers(oracle, golden):
    for c in golden["dequantize_linear"]:
        x, code = _x_raw(c, oracle)
        if c["scale_dtype"] == "float16":
            sc = (np.array(c["scale_bits"], np.uint16) if "scale_bits" in c
                  else np.array(c["scale_float"], np.float16).view(np.uint16))
            sdt = oracle.FLOAT16
        else:
            sc, sdt = np.array(c["scale"], np.float32), oracle.FLOAT
        sc = sc.reshape(c["scale_shape"])
        y = oracle.dequantize_linear(x, code, c["x_shape"], sc, sdt, _zp_raw(c, oracle, code), c["axis"])
        if "y_bits" in c:
            assert y.reshape(-1).tolist() == c["y_bits"], c["name"]
        elif sdt == oracle.FLOAT16:
            assert y.view(np.float16).astype(np.float32).reshape(-1).tolist() == c["y"], c["name"]
        else:
            assert y.reshape(-1).tolist() == [float(v) for v in c["y"]], c["name"]


def _np_dq(q, scale_f32, zp, axis, blocked_shape=None):
    """numpy closed form: expand scale/zp with np.repeat (upstream ONNX
    reference formulation) and compute (q - zp) * s in float32."""
    if blocked_shape is None:
        shp = [1] * q.ndim
        shp[axis] = -1
        s = scale_f32.reshape(shp)
        z = zp.reshape(shp).astype(np.float32)
    else:
        rep = q.shape[axis] // blocked_shape[axis]
        s = np.repeat(scale_f32.reshape(blocked_shape), rep, axis=axis)
        z = np.repeat(zp.reshape(blocked_shape).astype(np.float32), rep, axis=axis)
    return ((q.astype(np.float32) - z) * s).astype(np.float32)


@pytest.mark.parametrize("kind", ["uint8", "int8", "int4", "uint4", "fp8"])
def test_dequantize_closed_form_random(oracle, kind):
    rng = np.random.default_rng(5)
    K, N, bs = 64, 24, 16
    if kind == "fp8":
        codes = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal((K, N)).astype(np.float32))
        q = oracle.f8e4m3fn_bits_to_f32(codes)
        raw, code, zpq = codes, oracle.FLOAT8E4M3FN, None
    elif kind in ("int4", "uint4"):
        lo, hi = (-8, 8) if kind == "int4" else (0, 16)
        q = rng.integers(lo, hi, (K, N))
        raw, code = oracle.pack_int4(q), (oracle.INT4 if kind == "int4" else oracle.UINT4)
        zpq = rng.integers(lo, hi, (K // bs, N))
    else:
        dt = NP[kind]
        info = np.iinfo(dt)
        q = rng.integers(info.min, info.max + 1, (K, N)).astype(dt)
        raw, code = q, (oracle.UINT8 if kind == "uint8" else oracle.INT8)
        zpq = rng.integers(info.min, info.max + 1, (K // bs, N)).astype(dt)
    # blocked along K (axis 0), float16 scales -> float16 output
    s16 = rng.uniform(0.002, 0.02, (K // bs, N)).astype(np.float16)
    zraw = None if zpq is None else (oracle.pack_int4(zpq) if code in (oracle.INT4, oracle.UINT4) else zpq)
    y = oracle.dequantize_linear(raw, code, (K, N), s16.view(np.uint16), oracle.FLOAT16, zraw, 0)
    z = np.zeros((K // bs, N)) if zpq is None else zpq
    ref = _np_dq(np.asarray(q), s16.astype(np.float32), np.asarray(z), 0, (K // bs, N))
    assert np.array_equal(y, ref.astype(np.float16).view(np.uint16))
    # per-axis along N (axis 1), float32 scales -> float32 output
    s32 = rng.uniform(0.005, 0.05, N).astype(np.float32)
    zpn = None if zpq is None else zpq[0]
    zraw = None if zpn is None else (oracle.pack_int4(zpn) if code in (oracle.INT4, oracle.UINT4) else zpn)
    y = oracle.dequantize_linear(raw, code, (K, N), s32, oracle.FLOAT, zraw, 1)
    ref = _np_dq(np.asarray(q), s32, np.zeros(N) if zpn is None else np.asarray(zpn), 1)
    assert np.array_equal(y, ref)


def test_matmul_half_known_answer_and_bound(oracle, golden):
    c = golden["matmul_half"][0]
    for dt, tol in ((oracle.FLOAT16, c["tol_float16"]), (oracle.BFLOAT16, c["tol_bfloat16"])):
        enc = oracle.f32_to_f16_bits if dt == oracle.FLOAT16 else oracle.f32_to_bf16_bits
        dec = oracle.f16_bits_to_f32 if dt == oracle.FLOAT16 else oracle.bf16_bits_to_f32
        y = oracle.matmul_half(enc(np.array(c["a"]).reshape(2, 3)), enc(np.array(c["b"]).reshape(3, 2)), dt)
        assert np.abs(dec(y).reshape(-1) - np.array(c["y"])).max() <= tol
    # random: |oracle - float64| within the fp32-accumulation + final-rounding bound
    rng = np.random.default_rng(3)
    a = rng.standard_normal((9, 300)).astype(np.float32)
    b = rng.standard_normal((300, 13)).astype(np.float32)
    ab, bb = oracle.f32_to_bf16_bits(a), oracle.f32_to_bf16_bits(b)
    y = oracle.bf16_bits_to_f32(oracle.matmul_half(ab, bb, oracle.BFLOAT16))
    exact = oracle.bf16_bits_to_f32(ab).astype(np.float64) @ oracle.bf16_bits_to_f32(bb).astype(np.float64)
    mag = np.abs(oracle.bf16_bits_to_f32(ab)).astype(np.float64) @ np.abs(oracle.bf16_bits_to_f32(bb)).astype(np.float64)
    assert np.all(np.abs(y - exact) <= 2.0**-8 * np.abs(exact) + 300 * 2.0**-24 * mag + 1e-30)
    # k-sequential fp32 accumulation: bit-equal to an explicit numpy float32 loop
    yf = oracle.matmul_f32(a[:2, :50], b[:50, :3])
    ref = np.zeros((2, 3), np.float32)
    for k in range(50):
        ref = (ref + (a[:2, k:k + 1] * b[k:k + 1, :3]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(yf, ref)
    # thread split does not change the result
    assert np.array_equal(oracle.matmul_f32(a, b, nthreads=4), oracle.matmul_f32(a, b))
