"""C-ABI host logic without a GPU: the library loads, exports every symbol the
header declares, and reproduces the reference kernels' validation (same
checks and message text) before touching the device.  Calls whose arguments
are valid stop at NOT_INITIALIZED (no GPU here): no kernel runs on the CPU."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    with open(os.path.join(ROOT, "include", "onnxl_amd.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(onnxl_amd_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol(olamd):
    names = _header_functions()
    assert len(names) >= 11
    L = olamd.lib()
    for n in names:
        assert hasattr(L, n), n
    assert L.onnxl_amd_version().startswith(b"onnxl_amd")


def test_library_carries_gfx950_code_objects():
    with open(os.path.join(ROOT, "onnx-light_amd", "libonnxl_amd.so"), "rb") as f:
        blob = f.read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def _call(olamd, fn, *args):
    rc = getattr(olamd.lib(), fn)(*args)
    return rc, olamd.lib().onnxl_amd_last_error().decode()


def test_matmul_integer_validation(olamd):
    d = olamd.describe
    a = np.zeros((4, 3), np.uint8)
    b = np.zeros((3, 2), np.uint8)
    y = np.zeros((4, 2), np.int32)
    cases = [
        ((np.zeros((4, 3), np.int32), b, None, None, y), "A must be INT8 or UINT8."),  # :2268-2276
        ((a, np.zeros((3, 2), np.float32), None, None, y), "B must be INT8 or UINT8."),
        ((a, b, None, None, np.zeros((4, 2), np.float32)), "output dtype must be INT32."),
        ((a, np.zeros((4, 2), np.uint8), None, None, y), "incompatible inner dimensions."),
        ((a, b, None, None, np.zeros((4, 3), np.int32)), "preallocated output has invalid shape."),
        ((a, b, np.zeros(1, np.int8), None, y), "'a_zero_point' dtype must match its data input."),
        ((a, b, np.zeros((2, 2), np.uint8), None, y), "'a_zero_point' must be a scalar or a 1-D tensor."),
        ((a, b, np.zeros(3, np.uint8), None, y), "'a_zero_point' must be a scalar, a one-element 1-D"),
        ((a, b, None, np.zeros(4, np.uint8), y), "'b_zero_point' must be a scalar, a one-element 1-D"),
        ((np.zeros((2, 4, 3), np.uint8), np.zeros((3, 3, 2), np.uint8), None, None,
          np.zeros((3, 4, 2), np.int32)), "not broadcast-compatible on batch dimensions."),
    ]
    for args, msg in cases:
        rc, err = _call(olamd, "onnxl_amd_matmul_integer", *[d(t) for t in args], None)
        assert rc == olamd.INVALID_ARGUMENT, (msg, err)
        assert err.startswith("[onnx-light] kernel::MatMulInteger")
        assert msg in err, (msg, err)
    # rank-0 input
    rc, err = _call(olamd, "onnxl_amd_matmul_integer", d(np.zeros((), np.uint8)), d(b), d(None), d(None),
                    d(y), None)
    assert rc == olamd.INVALID_ARGUMENT and "rank-0 inputs are not accepted." in err
    # valid arguments stop at the device
    rc, _ = _call(olamd, "onnxl_amd_matmul_integer", d(a), d(b), d(np.array([1, 2, 3, 4], np.uint8)),
                  d(np.array(3, np.uint8)), d(y), None)
    assert rc == olamd.NOT_INITIALIZED


def test_qlinear_validation(olamd):
    d = olamd.describe
    a = np.zeros((2, 4), np.uint8)
    b = np.zeros((4, 3), np.int8)
    f = lambda v: np.array(v, np.float32)
    u = lambda v: np.array(v, np.uint8)
    s = lambda v: np.array(v, np.int8)
    y = np.zeros((2, 3), np.uint8)
    base = [a, f(0.1), u(1), b, f(0.2), s(0), f(0.3), u(2), y]

    def run(**over):
        args = list(base)
        for k, v in over.items():
            args[int(k[1:])] = v
        return _call(olamd, "onnxl_amd_qlinear_matmul", *[d(t) for t in args], None)

    rc, err = run(i0=np.zeros((2, 4), np.int16))
    assert rc == olamd.INVALID_ARGUMENT and "a must be INT8 or UINT8." in err
    rc, err = run(i2=s(1))
    assert rc == olamd.INVALID_ARGUMENT and "a_zero_point dtype must match a." in err
    rc, err = run(i5=u(1))
    assert rc == olamd.INVALID_ARGUMENT and "b_zero_point dtype must match b." in err
    rc, err = run(i7=np.array(1, np.int32))
    assert rc == olamd.INVALID_ARGUMENT and "y_zero_point must be INT8 or UINT8." in err
    rc, err = run(i8=np.zeros((2, 3), np.int8))
    assert rc == olamd.INVALID_ARGUMENT and "output dtype must match y_zero_point." in err
    rc, err = run(i1=np.array([0.1, 0.2], np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "'a_scale' must be a scalar." in err
    rc, err = run(i4=np.array(1, np.int32))
    assert rc == olamd.INVALID_ARGUMENT and "'b_scale' must be a FLOAT or FLOAT16 scalar" in err
    rc, err = run(i6=f(0.0))
    assert rc == olamd.INVALID_ARGUMENT and "y_scale must be non-zero." in err  # :264
    rc, err = run(i8=np.zeros((3, 2), np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "preallocated output has invalid shape." in err
    rc, err = run()
    assert rc == olamd.NOT_INITIALIZED
    # FLOAT16 scales are accepted (bits 0x2e66 ~ 0.1)
    rc, err = run(i1=np.array(0x2E66, np.uint16), i4=np.array(0x2E66, np.uint16))
    assert rc == olamd.INVALID_ARGUMENT  # uint16 is not a scale dtype
    h = np.array(0.1, np.float16)
    rc, _ = _call(olamd, "onnxl_amd_qlinear_matmul", d(a), d(h), d(u(1)), d(b), d(h), d(s(0)), d(h),
                  d(u(2)), d(y), None)
    assert rc == olamd.NOT_INITIALIZED


def test_qlinear_accepts_sums_past_int32(olamd):
    """Past K * max|a-za| * max|b-zb| = 2^31 the call is valid (the int64
    kernel takes it): without a device it gets as far as the launch."""
    d = olamd.describe
    K = 70000  # 70000 * 255 * 255 > 2^31
    a = np.zeros((1, K), np.uint8)
    b = np.zeros((K, 1), np.uint8)
    rc, err = _call(olamd, "onnxl_amd_qlinear_matmul", d(a), d(np.array(1, np.float32)),
                    d(np.array(0, np.uint8)), d(b), d(np.array(1, np.float32)),
                    d(np.array(0, np.uint8)), d(np.array(1, np.float32)), d(np.array(0, np.uint8)),
                    d(np.zeros((1, 1), np.uint8)), None)
    assert rc == olamd.NOT_INITIALIZED, err


def test_dequantize_validation(olamd):
    d = olamd.describe
    x = np.zeros((2, 3), np.uint8)
    sc = np.array([1.0, 2.0, 3.0], np.float32)
    y = np.zeros((2, 3), np.float32)
    L = olamd.lib()

    def run(x=x, s=sc, z=None, axis=1, y=y):
        rc = L.onnxl_amd_dequantize_linear(d(x), d(s), d(z), axis, d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    rc, err = run(s=np.array([1.0, 2.0], np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "x_scale element count must equal axis dimension." in err
    rc, err = run(z=np.zeros(3, np.int8))
    assert rc == olamd.INVALID_ARGUMENT and "x_zero_point data_type must match x." in err
    rc, err = run(axis=2)
    assert rc == olamd.INVALID_ARGUMENT and "axis out of range." in err
    rc, err = run(axis=-1)  # the reference does not normalise negative axes
    assert rc == olamd.INVALID_ARGUMENT and "axis out of range." in err
    rc, err = run(y=np.zeros((2, 3), np.float16))
    assert rc == olamd.INVALID_ARGUMENT and "output dtype must match x_scale." in err
    rc, err = run(s=np.array(1.0, np.float32), y=np.zeros((2, 3), np.float16))
    assert rc == olamd.INVALID_ARGUMENT and "output (no x_zero_point) dtype must match x_scale." in err
    rc, err = run(s=np.array(1.0, np.float32), z=np.zeros(2, np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "x_zero_point must be a scalar (per-tensor" in err
    rc, err = run(s=np.array([1, 2, 3], np.int32))
    assert rc == olamd.INVALID_ARGUMENT and "x_scale must be FLOAT or FLOAT16." in err
    rc, err = run(x=np.zeros((2, 3), np.float32), s=np.array(1.0, np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "unsupported data type 1" in err  # :295-309
    rc, err = run(s=np.ones((2, 2), np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "blocked x_scale dimension must divide" in err
    rc, err = run(s=np.ones((1, 3), np.float32))  # dim 0 differs and is not the axis
    assert rc == olamd.INVALID_ARGUMENT and "may only differ from x along the quantization axis" in err
    rc, err = run(x=np.zeros((4, 6), np.uint8), s=np.ones((2, 3), np.float32), y=np.zeros((4, 6), np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "may only differ from x along the quantization axis" in err
    rc, err = run(z=np.zeros(2, np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "must have the same shape" in err
    rc, err = run(y=np.zeros((3, 2), np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "preallocated output shape must match x shape." in err
    rc, _ = run()
    assert rc == olamd.NOT_INITIALIZED
    # every input dtype the reference decodes reaches the device step; FLOAT8E8M0 is not one of them
    for dt in (18, 19, 20, 23, 25, 26, 27, 28):
        rc = L.onnxl_amd_dequantize_linear(d(np.zeros(8, np.uint8), dt, (2, 3)), d(np.array(1.0, np.float32)),
                                           d(None), 1, d(y), None)
        assert rc == olamd.NOT_INITIALIZED, dt
    rc = L.onnxl_amd_dequantize_linear(d(x, 24), d(np.array(1.0, np.float32)), d(None), 1, d(y), None)
    err = L.onnxl_amd_last_error().decode()
    assert rc == olamd.INVALID_ARGUMENT and "unsupported data type 24, kernel::DequantizeLinear: only" in err


def test_matmul_shape_rules(olamd, golden):
    for c in golden["matmul_shapes"]:
        assert list(olamd.matmul_shape(c["a_shape"], c["b_shape"])) == c["y_shape"]
    with pytest.raises(olamd.InvalidArgument):
        olamd.matmul_shape((2, 3), (4, 2))


def test_not_initialized_before_device_work(olamd):
    with pytest.raises(olamd.DeviceError):
        olamd.matmul_integer(np.zeros((2, 2), np.uint8), np.zeros((2, 2), np.uint8),
                             out=np.zeros((2, 2), np.int32))


def test_quantize_validation(olamd):
    """kq/kernel_quantizelinear.cc:485-941: dispatch on zero point /
    output_dtype / UINT8 default, and the same messages."""
    d = olamd.describe
    x = np.zeros((2, 3), np.float32)
    sc = np.array([1.0, 2.0, 3.0], np.float32)
    L = olamd.lib()

    def run(x=x, s=sc, z=None, axis=1, odt=0, y=np.zeros((2, 3), np.uint8), ydt=None, zdt=None):
        rc = L.onnxl_amd_quantize_linear(d(x), d(s), d(z, zdt), axis, odt,
                                         d(y, ydt, None if ydt is None else (2, 3)), None)
        return rc, L.onnxl_amd_last_error().decode()

    rc, err = run(s=sc)  # per-axis scale with neither zero point nor output_dtype
    assert rc == olamd.INVALID_ARGUMENT and "y_scale must be a scalar (per-tensor quantization)." in err
    rc, err = run(x=np.zeros((2, 3), np.int32), s=np.array(1.0, np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "x must be FLOAT or FLOAT16." in err
    rc, err = run(z=np.zeros(3, np.int32), y=np.zeros((2, 3), np.int32))
    assert rc == olamd.INVALID_ARGUMENT and "unsupported data type 6" in err
    rc, err = run(z=np.zeros(3, np.int8))
    assert rc == olamd.INVALID_ARGUMENT and "output data_type must match y_zero_point." in err
    rc, err = run(z=np.zeros(3, np.uint8), axis=2)
    assert rc == olamd.INVALID_ARGUMENT and "axis out of range." in err
    rc, _ = run(z=np.zeros(3, np.uint8), axis=-1)  # Run normalises negative axes (:928-930)
    assert rc == olamd.NOT_INITIALIZED
    rc, err = run(z=np.zeros(2, np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "y_scale and y_zero_point must have the same shape." in err
    rc, err = run(s=np.ones(2, np.float32), z=np.zeros(2, np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "y_scale element count must equal axis dimension." in err
    rc, err = run(s=np.ones((2, 2), np.float32), odt=olamd.UINT8)
    assert rc == olamd.INVALID_ARGUMENT and "blocked y_scale dimension must divide" in err
    rc, err = run(s=np.ones((1, 3), np.float32), odt=olamd.UINT8)
    assert rc == olamd.INVALID_ARGUMENT and "may only differ from x along the quantization axis" in err
    rc, err = run(odt=olamd.INT8)
    assert rc == olamd.INVALID_ARGUMENT and "output data_type must match output_dtype." in err
    rc, err = run(odt=olamd.INT4, y=np.zeros(3, np.uint8), ydt=olamd.INT4)  # symmetric per-axis: 8/16-bit only
    assert rc == olamd.INVALID_ARGUMENT and "unsupported output dtype." in err
    rc, err = run(z=np.zeros(3, np.uint8), y=np.zeros((3, 2), np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "preallocated output shape must match x shape." in err
    rc, err = run(s=np.array(1.0, np.float32), z=np.zeros(2, np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "y_zero_point must be a scalar" in err
    rc, err = run(s=np.array(1.0, np.float32), y=np.zeros((2, 3), np.int8))
    assert rc == olamd.INVALID_ARGUMENT
    rc, _ = run(z=np.zeros(3, np.uint8))
    assert rc == olamd.NOT_INITIALIZED
    rc, _ = run(s=np.array(1.0, np.float32))
    assert rc == olamd.NOT_INITIALIZED
    # the fp8 variants, FLOAT4E2M1, UINT2 / INT2 and FLOAT6 with a zero point
    # (packed sizes: 6 elements in 6, 3, 2 and 5 bytes) pass validation
    for dt, nbytes in ((18, 6), (19, 6), (20, 6), (23, 3), (25, 2), (26, 2), (27, 5), (28, 5)):
        rc, err = run(s=np.array(1.0, np.float32), z=np.zeros(1, np.uint8), zdt=dt,
                      y=np.zeros(nbytes, np.uint8), ydt=dt)
        assert rc == olamd.NOT_INITIALIZED, (dt, err)
    # without one: FLOAT4E2M1 and FLOAT6 per tensor only (:485-532)
    for dt, nbytes in ((23, 3), (27, 5), (28, 5)):
        rc, _ = run(s=np.array(1.0, np.float32), odt=dt, y=np.zeros(nbytes, np.uint8), ydt=dt)
        assert rc == olamd.NOT_INITIALIZED, dt
        rc, err = run(odt=dt, y=np.zeros(nbytes, np.uint8), ydt=dt)
        assert rc == olamd.INVALID_ARGUMENT and "unsupported output dtype." in err, dt
    for dt in (18, 25):
        rc, err = run(s=np.array(1.0, np.float32), odt=dt, y=np.zeros(6, np.uint8), ydt=dt)
        assert rc == olamd.INVALID_ARGUMENT and "unsupported output dtype." in err, dt
    rc, err = run(s=np.array(1.0, np.float32), z=np.zeros(1, np.uint8), zdt=24, y=np.zeros(6, np.uint8), ydt=24)
    assert rc == olamd.INVALID_ARGUMENT and "unsupported data type 24" in err


def test_dynamic_quantize_validation(olamd):
    """kq/kernel_dynamicquantizelinear.cc:57-77."""
    d = olamd.describe
    L = olamd.lib()
    x = np.zeros((2, 3), np.float32)

    def run(x=x, y=np.zeros((2, 3), np.uint8), s=np.zeros((), np.float32), z=np.zeros((), np.uint8)):
        rc = L.onnxl_amd_dynamic_quantize_linear(d(x), d(y), d(s), d(z), None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(x=x.astype(np.float16)), "x must be FLOAT."),
                    (dict(y=np.zeros((2, 3), np.int8)), "y must be UINT8."),
                    (dict(y=np.zeros((3, 2), np.uint8)), "y shape must match x shape."),
                    (dict(s=np.zeros((), np.float16)), "y_scale must be FLOAT."),
                    (dict(s=np.zeros(1, np.float32)), "y_scale must be a scalar FLOAT."),
                    (dict(z=np.zeros((), np.int8)), "y_zero_point must be UINT8."),
                    (dict(z=np.zeros(1, np.uint8)), "y_zero_point must be a scalar UINT8."),
                    (dict(x=np.zeros(0, np.float32), y=np.zeros(0, np.uint8)), "x must be non-empty.")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    rc, _ = run()
    assert rc == olamd.NOT_INITIALIZED


def test_conv_validation(olamd):
    """nn/kernel_conv_integer.cc:24-201 and kq/kernel_qlinearconv.cc:53-238."""
    d = olamd.describe
    L = olamd.lib()
    x = np.zeros((1, 4, 5, 5), np.uint8)
    w = np.zeros((6, 2, 3, 3), np.uint8)
    ok_attrs = dict(group=2, pads=[1, 1, 1, 1])

    def ci(x=x, w=w, xz=None, wz=None, y=None, **kw):
        a = olamd.conv_attrs(**(kw or ok_attrs))
        y = np.zeros((1, 6, 5, 5), np.int32) if y is None else y
        rc = L.onnxl_amd_conv_integer(d(x), d(w), d(xz), d(wz), ctypes.byref(a), d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(kernel_shape=[3]), "'kernel_shape' size must match input spatial rank."),
                    (dict(strides=[1, 1, 1]), "'strides' size must match input spatial rank."),
                    (dict(pads=[1, 1]), "'pads' size must be 2 * spatial rank."),
                    (dict(auto_pad=7), "'auto_pad' must be NOTSET/SAME_UPPER/SAME_LOWER/VALID."),
                    (dict(group=3, pads=[1, 1, 1, 1]), "x.shape[1] must equal w.shape[1] * group.")):
        rc, err = ci(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    rc, err = ci(x=np.zeros((1, 4, 5, 5), np.int32))
    assert rc == olamd.INVALID_ARGUMENT and "x must be INT8 or UINT8." in err
    rc, err = ci(xz=np.zeros(1, np.int8))
    assert rc == olamd.INVALID_ARGUMENT and "x_zero_point dtype must match x." in err
    rc, err = ci(wz=np.zeros(4, np.uint8))
    assert rc == olamd.INVALID_ARGUMENT and "w_zero_point must be a scalar or 1-D of length M." in err
    rc, err = ci(y=np.zeros((1, 6, 5, 5), np.float32))
    assert rc == olamd.INVALID_ARGUMENT and "preallocated output must be INT32." in err
    rc, err = ci(y=np.zeros((1, 6, 3, 3), np.int32))
    assert rc == olamd.INVALID_ARGUMENT and "preallocated output shape mismatch." in err
    rc, _ = ci(xz=np.zeros((), np.uint8), wz=np.zeros(6, np.uint8))
    assert rc == olamd.NOT_INITIALIZED

    f = lambda v: np.array(v, np.float32)

    def qc(ws=f(1.0), wz=np.zeros((), np.uint8), xs=f(0.5), ys=f(2.0), yz=np.zeros((), np.uint8), B=None,
           y=None, xz=np.zeros((), np.uint8)):
        a = olamd.conv_attrs(**ok_attrs)
        y = np.zeros((1, 6, 5, 5), yz.dtype) if y is None else y
        rc = L.onnxl_amd_qlinear_conv(d(x), d(xs), d(xz), d(w), d(ws), d(wz), d(ys), d(yz), d(B),
                                      ctypes.byref(a), d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(ys=f(0.0)), "y_scale must be non-zero."),
                    (dict(xs=f([1.0, 2.0])), "'x_scale' and 'y_scale' must be scalar."),
                    (dict(ws=f([1.0, 2.0])), "'w_scale' must be scalar or length-M."),
                    (dict(wz=np.zeros(2, np.uint8)), "'w_zero_point' must be scalar or length-M."),
                    (dict(B=np.zeros(6, np.int64)), "B must be INT32."),
                    (dict(B=np.zeros(5, np.int32)), "B must be 1-D with length M."),
                    (dict(xz=np.zeros(2, np.uint8)), "'x_zero_point' must be a scalar."),
                    (dict(yz=np.zeros((), np.int8), y=np.zeros((1, 6, 5, 5), np.uint8)),
                     "output dtype must match y_zero_point."),
                    (dict(xs=np.array(0.5, np.float16)), "scale must be FLOAT for the reference kernel.")):
        rc, err = qc(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    rc, _ = qc(ws=f(np.ones(6)), wz=np.zeros(6, np.uint8), B=np.zeros(6, np.int32))
    assert rc == olamd.NOT_INITIALIZED
    assert olamd.conv_shape((2, 3, 9, 8), (4, 3, 3, 3), olamd.conv_attrs(strides=[2, 2])) == (2, 4, 4, 3)


def test_dequantize_packed_validation(olamd):
    """onnx_core/runtime/dequantize_packed.cc:296-343."""
    d = olamd.describe
    L = olamd.lib()

    def run(x=np.zeros(36, np.uint8), fmt=b"gguf:q4_0", shape=(2, 32), odt=olamd.FLOAT, y=None):
        y = np.zeros(shape, np.float32) if y is None else y
        dims = (ctypes.c_int64 * olamd.MAX_RANK)(*shape)
        rc = L.onnxl_amd_dequantize_packed(d(x), fmt, dims, len(shape), odt, d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(fmt=b"gguf:Q4_0"), "unsupported format 'gguf:Q4_0'."),
                    (dict(odt=6), "output_dtype must be FLOAT, FLOAT16, BFLOAT16 or DOUBLE."),
                    (dict(shape=(2, 31), y=np.zeros((2, 31), np.float32)), "last dimension must contain complete blocks."),
                    (dict(x=np.zeros(36, np.int8)), "x must be a one-dimensional UINT8 tensor."),
                    (dict(x=np.zeros(35, np.uint8)), "packed input length must match exactly.")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    rc, _ = run()
    assert rc == olamd.NOT_INITIALIZED
    # the codebook profiles pass validation as the others do (the device work
    # then needs onnxl_amd_init)
    for fmt, size in ((b"gguf:iq2_xxs", 66), (b"gguf:iq2_xs", 74), (b"gguf:iq2_s", 82), (b"gguf:iq3_xxs", 98),
                      (b"gguf:iq3_s", 110), (b"gguf:iq1_s", 50), (b"gguf:iq1_m", 56)):
        rc, _ = run(x=np.zeros(size, np.uint8), fmt=fmt, shape=(256,), y=np.zeros(256, np.float32))
        assert rc == olamd.NOT_INITIALIZED, fmt
        rc, err = run(x=np.zeros(size + 1, np.uint8), fmt=fmt, shape=(256,), y=np.zeros(256, np.float32))
        assert rc == olamd.INVALID_ARGUMENT and "packed input length must match exactly." in err, fmt


def test_awq_validation(olamd):
    """The AWQ format's checks and messages (onnx_core/runtime/awq.cc:64-118
    Geometry, :156-183 CheckParameter, :232-245 CheckReconstruction, :263-268
    tensor checks) on host payloads; valid arguments stop at NOT_INITIALIZED."""
    import torch
    from awq_gptq_cases import awq_fixture
    L = olamd.lib()
    d = olamd.describe

    def run(variant="gemm", fx=None, K=128, N=8, bits=4, group=64, y=None, **over):
        fx = dict(awq_fixture(variant if variant in ("gemm", "gemv", "gemv_fast", "llm-awq") else "gemm", 64)
                  if fx is None else fx)
        fx.update(over)
        y = np.zeros((N, K), np.float32) if y is None else y
        rc = L.onnxl_amd_dequantize_awq(variant.encode(), d(fx["qweight"]), d(fx["qzeros"]), d(fx["scales"]), K, N,
                                        bits, group, d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(K=0), "AWQ requires positive dimensions, supported bits and group_axis=1."),
                    (dict(bits=8, variant="gemv"), "AWQ requires positive dimensions, supported bits and group_axis=1."),
                    (dict(variant="marlin"), "AWQ unsupported variant."),
                    (dict(group=0), "AWQ unsupported group size."),
                    (dict(group=48), "AWQ requires complete groups."),
                    (dict(N=12), "AWQ GEMM requires complete INT32 words and FP16/BF16 scales."),
                    (dict(scales=np.ones((2, 8), np.float32)),
                     "AWQ GEMM requires complete INT32 words and FP16/BF16 scales."),
                    (dict(qweight=np.zeros((128, 2), np.int32)), "AWQ invalid tensor type, shape or byte extent: qweight."),
                    (dict(qzeros=np.zeros((2, 1), np.int64)), "AWQ invalid tensor type, shape or byte extent: qzeros."),
                    (dict(y=np.zeros((8, 128), np.int32)), "Quantization requires FLOAT, DOUBLE, FLOAT16 or BFLOAT16.")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    gemv = awq_fixture("gemv", 64)
    for kw, msg in ((dict(group=8), "AWQ invalid effective group size."),
                    (dict(scales=gemv["scales"].astype(np.float32)), "AWQ GEMV requires FLOAT16 parameters."),
                    (dict(K=132, group=-1), "AWQ GEMV requires K divisible by eight.")):
        rc, err = run("gemv", gemv, **kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    rc, err = run("gemv_fast", awq_fixture("gemv_fast", 64), K=96, group=32)
    assert rc == olamd.INVALID_ARGUMENT and "AWQ GEMV_FAST requires K divisible by 64 and N by four." in err
    rc, err = run("llm-awq", awq_fixture("llm-awq", 64), qzeros=np.zeros((16, 8), np.float32))
    assert "AWQ invalid tensor type, shape or byte extent: scaled_zeros." in err
    # value checks: nonfinite anywhere, nonpositive where used (the gemv padding is not used)
    fx = awq_fixture("gemm", 64)
    bad = fx["scales"].copy()
    bad[1, 3] = np.inf
    assert "AWQ nonfinite parameter." in run(scales=bad)[1]
    bad = fx["scales"].copy()
    bad[0, 0] = 0
    assert "AWQ nonpositive used scale." in run(scales=bad)[1]
    sc = gemv["scales"].copy()
    sc[:, 2:] = -3  # padding groups
    assert run("gemv", gemv, scales=sc)[0] == olamd.NOT_INITIALIZED
    terms = awq_fixture("gemv_fast", 64)
    tz = terms["qzeros"].copy()
    tz[5, 1] = np.nan
    assert "AWQ nonfinite parameter." in run("gemv_fast", terms, qzeros=tz)[1]
    # BFLOAT16 scales: the FLOAT reconstruction must stay finite
    big = torch.full((2, 8), 3.0e38, dtype=torch.bfloat16)
    assert "AWQ FLOAT reconstruction overflow." in run(scales=big)[1]
    # FLOAT16 output: values that round past 65504 (15 * 8192 here)
    sc = fx["scales"].copy()
    sc[0, 1] = 8192
    y16 = np.zeros((8, 128), np.float16)
    assert "Dequantization output dtype overflow." in run(scales=sc, y=y16)[1]
    assert run(scales=sc)[0] == olamd.NOT_INITIALIZED  # FLOAT output holds it
    # valid arguments reach the device step; prepare checks its output buffers first
    assert run()[0] == olamd.NOT_INITIALIZED
    o = [olamd.Tensor() for _ in range(3)]
    rc = L.onnxl_amd_prepare_awq(b"gemm", d(fx["qweight"]), d(fx["qzeros"]), d(fx["scales"]), 128, 8, 4, 64,
                                 *(ctypes.byref(t) for t in o), None)
    assert rc == olamd.INVALID_ARGUMENT and "prepare_awq: weight holds 0 bytes, needs 1024" in L.onnxl_amd_last_error().decode()
    w, s, z = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert L.onnxl_amd_prepare_awq_size(b"gemv", 4096, 11008, 4, 128, olamd.FLOAT16, ctypes.byref(w),
                                        ctypes.byref(s), ctypes.byref(z)) == olamd.OK
    assert (s.value, z.value) == (32 * 11008 * 2, 32 * 11008 // 2) and w.value >= 4096 * 11008 // 2
    assert L.onnxl_amd_prepare_awq_size(b"gemm", 256, 64, 8, 128, olamd.BFLOAT16, ctypes.byref(w),
                                        ctypes.byref(s), ctypes.byref(z)) == olamd.OK
    assert (w.value, s.value, z.value) == (256 * 64, 2 * 64 * 4, 2 * 64)


def test_gptq_validation(olamd):
    """The GPTQ format's checks and messages (onnx_core/runtime/gptq.cc:67-123
    Geometry, :230-253 CheckData, :158-166 tensor checks)."""
    from awq_gptq_cases import gptq_fixture
    L = olamd.lib()
    d = olamd.describe

    def run(fmt="gptq_v2", bits=4, width=4, K=32, N=32, group=16, fx=None, y=None, **over):
        fx = dict(gptq_fixture(bits, fmt if fmt in ("gptq", "gptq_v2", "gptq_p") else "gptq_v2", width)
                  if fx is None else fx)
        fx.update(over)
        y = np.zeros((N, K), np.float32) if y is None else y
        rc = L.onnxl_amd_dequantize_gptq(fmt.encode(), d(fx["qweight"]), d(fx["qzeros"]), d(fx["scales"]),
                                         d(fx["g_idx"]), K, N, bits, group, d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    fx4 = gptq_fixture(4)
    for kw, msg in ((dict(fmt="gptq_v3"), "GPTQ unsupported format."),
                    (dict(bits=9, fx=fx4), "GPTQ invalid dimensions, bits or group axis."),
                    (dict(group=-2), "GPTQ invalid group size."),
                    (dict(qweight=fx4["qweight"].astype(np.uint8)), "GPTQ unsupported packed word dtype."),
                    (dict(fmt="gptq_p", width=2, fx=gptq_fixture(4, "gptq_v2", 2)),
                     "GPTQ planar checkpoint format requires INT32 words."),
                    (dict(bits=5, fx=fx4), "GPTQ five-, six- and seven-bit codes require the gptq_p format."),
                    (dict(bits=3, K=48, fx=gptq_fixture(3)),
                     "GPTQ three-bit and planar layouts require INT32 and 32-code blocks."),
                    (dict(scales=fx4["scales"].astype(np.float64)), "GPTQ unsupported scales dtype."),
                    (dict(qzeros=fx4["qzeros"][:1]), "GPTQ invalid tensor type, shape or byte extent: qzeros."),
                    (dict(g_idx=fx4["g_idx"].astype(np.int64)), "GPTQ invalid tensor type, shape or byte extent: g_idx."),
                    (dict(g_idx=np.full(32, 2, np.int32)), "GPTQ invalid group map index."),
                    (dict(scales=np.zeros((2, 32), np.float16)), "GPTQ nonfinite or nonpositive scale.")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    # v1 all-ones zero fields are ambiguous (test_gptq.cc:314-330)
    v1 = gptq_fixture(4, "gptq")
    rc, err = run("gptq", fx=v1, qzeros=np.full_like(v1["qzeros"], -1))
    assert "GPTQ v1 all-ones zero field has ambiguous upstream conversion semantics." in err
    assert run("gptq", fx=v1)[0] == olamd.NOT_INITIALIZED
    # FLOAT scales: the FLOAT reconstruction must stay finite
    big = np.full((2, 32), 3.0e37, np.float32)
    assert "GPTQ FLOAT reconstruction overflow." in run(scales=big)[1]
    # every format, bit width and word width of the reference's fixtures passes the checks
    for fmt in ("gptq", "gptq_v2", "gptq_p"):
        for bits in range(2, 9):
            if fmt != "gptq_p" and bits in (5, 6, 7):
                continue
            for width in ((4,) if fmt == "gptq_p" or bits in (3, 5, 6, 7) else (1, 2, 4, 8)):
                assert run(fmt, bits, width)[0] == olamd.NOT_INITIALIZED, (fmt, bits, width)
    w, s, z = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert L.onnxl_amd_prepare_gptq_size(b"gptq_p", 4096, 4096, 6, 128, olamd.INT32, olamd.FLOAT,
                                         ctypes.byref(w), ctypes.byref(s), ctypes.byref(z)) == olamd.OK
    assert (w.value, s.value, z.value) == (4096 * 4096, 32 * 4096 * 4, 32 * 4096)


def test_qqq_validation(olamd):
    """The QQQ format's geometry and tensor checks and messages
    (onnx_core/runtime/qqq.cc:38-56 Geometry, :136-141 CheckTensor) on host
    payloads; valid arguments stop at NOT_INITIALIZED.  CheckData's scale and
    overflow errors need the device (test_gpu_qqq.py)."""
    L = olamd.lib()
    d = olamd.describe
    k, n = 256, 64
    B = np.zeros((k // 16, 2 * n), np.int32)
    sc = np.ones((1, n), np.float32)
    sg = np.ones((k // 128, n), np.float16)

    def run(k=k, n=n, group=128, bits=4, B=B, sc=sc, sg=sg, y=None):
        y = np.zeros((n, k), np.float32) if y is None else y
        rc = L.onnxl_amd_dequantize_qqq(k, n, group, bits, d(B), d(sc), d(sg), d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    geo = "QQQ requires four-bit, unpadded dimensions divisible by 64 and group -1/128."
    for kw, msg in ((dict(k=96), geo), (dict(n=0), geo), (dict(bits=8), geo), (dict(group=64), geo),
                    (dict(k=192, B=B[:12], sg=sg[:1]), "QQQ incomplete 128-element group."),
                    (dict(B=B.astype(np.int64)), "QQQ invalid tensor type, shape or byte extent: B."),
                    (dict(B=B[:8]), "QQQ invalid tensor type, shape or byte extent: B."),
                    (dict(sc=sc.reshape(-1)), "QQQ invalid tensor type, shape or byte extent: s_channel."),
                    (dict(sc=sc.astype(np.float16)), "QQQ invalid tensor type, shape or byte extent: s_channel."),
                    (dict(sg=sg[:1]), "QQQ invalid tensor type, shape or byte extent: s_group."),
                    (dict(sg=None), "QQQ invalid tensor type, shape or byte extent: s_group."),
                    (dict(group=-1), "QQQ invalid tensor type, shape or byte extent: s_group."),
                    (dict(k=32768, n=16384, B=None), "QQQ logical FLOAT weights exceed max_bytes."),
                    (dict(y=np.zeros((n, k), np.int32)), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16."),
                    (dict(y=np.zeros((k, n), np.float32)), "QQQ: y must be [out_features, in_features]")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    assert run()[0] == olamd.NOT_INITIALIZED
    # per channel (and group 128 with k == 128): s_group empty or absent
    assert run(group=-1, sg=np.zeros(0, np.float16))[0] == olamd.NOT_INITIALIZED
    assert run(group=-1, sg=None)[0] == olamd.NOT_INITIALIZED
    assert run(k=128, B=B[:8], sg=None, y=np.zeros((n, 128), np.float32))[0] == olamd.NOT_INITIALIZED
    w, s = ctypes.c_int64(), ctypes.c_int64()
    assert L.onnxl_amd_prepare_qqq_size(4096, 11008, 128, 4, ctypes.byref(w), ctypes.byref(s)) == olamd.OK
    assert (w.value, s.value) == (4096 * 11008, 11008 * 4)
    assert L.onnxl_amd_prepare_qqq_size(4096, 11008, -1, 4, ctypes.byref(w), ctypes.byref(s)) == olamd.OK
    assert w.value == 4096 * 11008 // 2


def test_bitblas_validation(olamd):
    """BitBLAS's geometry and tensor checks and messages (onnx_core/runtime/
    bitblas.cc:38-84 Geometry, :101-106 CheckTensor) on host payloads; valid
    arguments stop at NOT_INITIALIZED.  CheckScales runs on the host copy of
    the scales before any device work."""
    L = olamd.lib()
    d = olamd.describe
    K, N = 64, 32
    qw = np.zeros((N, K // 8 * 4), np.int8)
    sc = np.ones((N, 2), np.float16)
    qz = np.zeros((2, N // 8 * 4), np.int8)

    def run(method="gptq", qw=qw, sc=sc, qz=qz, K=K, N=N, bits=4, group=32, sym=0, y=None):
        y = np.zeros((N, K), np.float32) if y is None else y
        rc = L.onnxl_amd_dequantize_bitblas(method.encode(), d(qw), d(sc), d(qz), K, N, bits, group, sym, d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    dims = "BitBLAS row-packed checkpoint requires aligned, unpadded dimensions."
    for kw, msg in ((dict(sc=None), "BitBLAS missing scales."),
                    (dict(method="marlin"), "BitBLAS requires an explicit GPTQ/AWQ originating method."),
                    (dict(K=48), dims), (dict(N=16), dims), (dict(N=0), dims),
                    (dict(bits=3), "BitBLAS unsupported bit width for the originating method."),
                    (dict(bits=9, method="awq"), "BitBLAS unsupported bit width for the originating method."),
                    (dict(group=16), "BitBLAS unsupported group size."),
                    (dict(K=96, group=64), "BitBLAS incomplete group."),
                    (dict(sc=sc.astype(np.float32)), "BitBLAS row-packed checkpoint reader requires FP16 scales."),
                    (dict(qw=qw[:16]), "BitBLAS invalid tensor type, shape or extent: qweight."),
                    (dict(sc=sc[:, :1]), "BitBLAS invalid tensor type, shape or extent: scales."),
                    (dict(qz=None), "BitBLAS invalid tensor type, shape or extent: qzeros."),
                    (dict(sym=1), "BitBLAS invalid tensor type, shape or extent: qzeros."),
                    (dict(sc=np.zeros((N, 2), np.float16)), "BitBLAS nonfinite or nonpositive scale."),
                    (dict(sc=-sc), "BitBLAS nonfinite or nonpositive scale.")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    assert run()[0] == olamd.NOT_INITIALIZED
    assert run(sym=1, qz=None)[0] == olamd.NOT_INITIALIZED  # symmetric GPTQ: no qzeros
    assert run(method="awq", sym=1, N=16, qw=qw[:16], sc=sc[:16], qz=qz[:, :8])[0] == olamd.NOT_INITIALIZED
    w, s, z = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert L.onnxl_amd_prepare_bitblas_size(b"awq", 4096, 11008, 6, 128, 0, ctypes.byref(w), ctypes.byref(s),
                                            ctypes.byref(z)) == olamd.OK
    assert (w.value, s.value, z.value) == (4096 * 11008, 32 * 11008 * 2, 32 * 11008)


def test_gptqmodel_fp8_validation(olamd):
    """GPTQModel FP8's geometry and tensor checks and messages
    (onnx_core/runtime/gptqmodel_fp8.cc:58-101 Geometry, :246-254 the
    import's tensor check) on host payloads; valid arguments stop at
    NOT_INITIALIZED."""
    L = olamd.lib()
    d = olamd.describe
    w = np.zeros((4, 8), np.uint8)
    s = np.ones(4, np.float32)

    def run(method="row", block=(), w=w, s=s, code=17, n=4, k=8, y=None):
        y = np.zeros((n, k), np.float32) if y is None else y
        blk = (ctypes.c_int64 * 2)(*block) if block else None
        rc = L.onnxl_amd_dequantize_gptqmodel_fp8(k, n, method.encode(), blk, len(block), d(w, code), d(s), d(y),
                                                  None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(n=0), "GPTQModel FP8 requires nonempty [N,K] weights and positive max_bytes."),
                    (dict(n=1 << 14, k=1 << 15), "GPTQModel FP8 logical FLOAT weights exceed max_bytes."),
                    (dict(code=3), "GPTQModel FP8 unsupported scalar format."),
                    (dict(method="block", block=(0, 2)), "GPTQModel FP8 invalid weight_block_size."),
                    (dict(block=(2, 2)), "GPTQModel FP8 non-block scaling forbids weight_block_size."),
                    (dict(method="block", block=(3, 2)), "GPTQModel FP8 requires divisible two-axis blocks."),
                    (dict(method="channel"), "GPTQModel FP8 requires divisible two-axis blocks."),
                    (dict(s=s[:3]), "GPTQModel FP8 invalid tensor dtype, shape or byte extent."),
                    (dict(method="tensor"), "GPTQModel FP8 invalid tensor dtype, shape or byte extent."),
                    (dict(w=w[:2]), "GPTQModel FP8 invalid tensor dtype, shape or byte extent."),
                    (dict(y=np.zeros((4, 8), np.int8)), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    assert run()[0] == olamd.NOT_INITIALIZED
    assert run(method="tensor", s=np.ones((), np.float32))[0] == olamd.NOT_INITIALIZED
    assert run(method="block", block=(2, 4), s=np.ones((2, 2), np.float32))[0] == olamd.NOT_INITIALIZED
    for code in (18, 19, 20, 24):
        assert run(code=code)[0] == olamd.NOT_INITIALIZED


def test_vptq_validation(olamd):
    """VPTQ's layout and tensor checks and messages (onnx_core/runtime/
    vptq.cc:52-129 Layout, :359-367 the import's tensor checks) on the
    reference's golden fixture; valid arguments stop at NOT_INITIALIZED."""
    from test_oracle_vptq import vptq_cases, _arr
    L = olamd.lib()
    f = next(f for f in vptq_cases() if f["name"] == "combined_float16_norm0_perm_tails")
    tensors = {k: _arr(v) for k, v in f["tensors"].items()}

    def run(params=None, t=None, y=None, dtype=10):
        cfg = olamd.VptqConfig.of(dict(f["parameters"], **(params or {})))
        tt = dict(tensors, **(t or {}))
        y = np.zeros((cfg.out_features, cfg.in_features), np.float32) if y is None else y
        descs = [olamd.describe(tt.get(n), dtype if n not in ("indices", "outlier_indices", "perm") and
                                tt.get(n) is not None else None) for n in olamd.VPTQ_TENSORS]
        rc = L.onnxl_amd_dequantize_vptq(ctypes.byref(cfg), *descs, olamd.describe(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    for kw, msg in ((dict(params=dict(in_features=0)), "VPTQ invalid positive dimension."),
                    (dict(params=dict(num_centroids=[5, 1])), "VPTQ unsupported codebook or outlier residual"),
                    (dict(params=dict(num_res_centroids=[-1, 1])), "VPTQ unsupported codebook or outlier residual"),
                    (dict(dtype=11), "VPTQ unsupported codebook dtype."),
                    (dict(params=dict(npercent=100.0)), "VPTQ invalid constructor metadata."),
                    (dict(params=dict(norm_dim=2)), "VPTQ invalid constructor metadata."),
                    (dict(params=dict(vector_lens=[-1, 3])), "VPTQ unusable outlier codebook."),
                    (dict(params=dict(group_num=2)), "VPTQ grouping knobs must be mutually exclusive."),
                    (dict(params=dict(group_size=-1, group_num=99)), "VPTQ empty groups."),
                    (dict(t={"indices": tensors["indices"][:2]}), "VPTQ invalid tensor type, shape or bytes: indices."),
                    (dict(t={"perm": None}), "VPTQ missing tensor perm."),
                    (dict(t={"weight_bias": tensors["weight_bias"][:3]}),
                     "VPTQ invalid tensor type, shape or bytes: weight_bias."),
                    (dict(y=np.zeros((7, 17), np.int8)), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16."),
                    (dict(y=np.zeros((17, 7), np.float32)), "VPTQ: y must be [out_features, in_features]")):
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw, err)
    assert run()[0] == olamd.NOT_INITIALIZED


def test_mx_weights_validation(olamd):
    """The MX / NVFP4 imports' checks and messages (quantization.cc:2099-2118,
    2193-2229, 2279-2298: matrix, packed columns, Geometry, the two tensors)
    on host payloads, in that order; valid arguments stop at
    NOT_INITIALIZED."""
    L = olamd.lib()
    d = olamd.describe

    def run(fmt, w, s, code=None, scode=None, y=None, g=1.0):
        rows = w.shape[0] if w.ndim else 1
        y = np.zeros((rows, 32), np.float32) if y is None else y
        rc = L.onnxl_amd_dequantize_mx_weights(fmt.encode(), d(w, code), d(s, scode), g, d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    u8 = np.uint8
    cases = [
        ("mxfp4", np.zeros(16, u8), np.zeros((1, 1), u8), None, None, "MXFP4 WEIGHT packed weights must be a matrix."),
        ("mxfp4", np.zeros((1, 0), u8), np.zeros((1, 1), u8), None, None, "MXFP4 WEIGHT packed columns overflow."),
        ("mxfp4", np.zeros((1, 8), u8), np.zeros((1, 1), u8), None, None,
         "MXFP4 WEIGHT requires positive [rows,cols] with cols divisible by 32."),
        ("mxfp4", np.zeros((0, 16), u8), np.zeros((0, 1), u8), None, None,
         "MXFP4 WEIGHT requires positive [rows,cols] with cols divisible by 32."),
        ("mxfp4", np.zeros((1, 16), np.int8), np.zeros((1, 1), u8), None, None,
         "Invalid MXFP4 WEIGHT tensor type, shape or storage."),
        ("mxfp4", np.zeros((1, 16), u8), np.zeros((1, 2), u8), None, None,
         "Invalid MXFP4 WEIGHT tensor type, shape or storage."),
        ("nvfp4", np.zeros((1, 16), u8), np.zeros((1, 2), u8), None, None,
         "Invalid NVFP4 WEIGHT tensor type, shape or storage."),
        ("nvfp4", np.zeros((1, 12), u8), np.zeros((1, 2), u8), None, 17,
         "NVFP4 WEIGHT requires positive [rows,cols] with cols divisible by 16."),
        ("mxfp8", np.zeros(32, u8), np.zeros((1, 1), u8), 17, None, "MXFP8 weights must be a matrix."),
        ("mxfp8", np.zeros((1, 32), u8), np.zeros((1, 1), u8), None, None, "Invalid MX tensor type, shape or storage."),
        ("mxfp8", np.zeros((1, 48), u8), np.zeros((1, 1), u8), 17, None,
         "MXFP8 requires positive [rows,cols] with cols divisible by 32."),
        ("mxfp6_e2m3", np.zeros((1, 25), u8), np.zeros((1, 1), u8), None, None, "Invalid MXFP6 E2M3 packed columns."),
        ("mxfp6_e2m3", np.zeros((1, 24), u8), np.zeros((1, 1), np.int8), None, None,
         "Invalid MX tensor type, shape or storage."),
    ]
    for fmt, w, s, code, scode, msg in cases:
        rc, err = run(fmt, w, s, code, scode)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (fmt, w.shape, err)
    rc, err = run("mxfp5", np.zeros((1, 16), u8), np.zeros((1, 1), u8))
    assert rc == olamd.UNSUPPORTED and "unknown format" in err
    for fmt, w, s, code, scode in (("mxfp4", np.zeros((1, 16), u8), np.zeros((1, 1), u8), None, None),
                                   ("mxfp6_e2m3", np.zeros((1, 24), u8), np.zeros((1, 1), u8), None, None),
                                   ("mxfp8", np.zeros((1, 32), u8), np.zeros((1, 1), u8), 17, None),
                                   ("nvfp4", np.zeros((1, 16), u8), np.zeros((1, 2), u8), None, 17)):
        rc, err = run(fmt, w, s, code, scode)
        assert rc == olamd.NOT_INITIALIZED, (fmt, err)


def test_exl3_validation(olamd):
    """EXL3's Validate checks and messages (exl3.cc:136-165: trellis
    dimensions, Geometry, the codebook count, each tensor then its scales'
    finiteness, the marker) on host payloads, in that order; valid arguments
    stop at NOT_INITIALIZED."""
    L = olamd.lib()
    d = olamd.describe
    tr = np.zeros((8, 8, 48), np.int16)
    suh, svh = np.ones(128, np.float16), np.ones(128, np.float16)
    mcg = np.array(0xCBAC1FED, np.uint32).view(np.int32).reshape(())
    mul1 = np.array(0x83DCD12D, np.uint32).view(np.int32).reshape(())

    def run(t=tr, u=suh, v=svh, m1=None, m2=None):
        y = np.zeros((t.shape[0] * 16 if t.ndim == 3 else 1, t.shape[1] * 16 if t.ndim == 3 else 1), np.float32)
        rc = L.onnxl_amd_dequantize_exl3(d(t), d(u), d(v), d(m1), d(m2), d(y), None)
        return rc, L.onnxl_amd_last_error().decode()

    inf = suh.copy()
    inf[3] = np.float16(np.inf)
    cases = [(dict(t=np.zeros((8, 8), np.int16)), "EXL3 invalid trellis dimensions."),
             (dict(t=np.zeros((8, 8, 17), np.int16)), "EXL3 invalid trellis dimensions."),
             (dict(t=np.zeros((4, 8, 48), np.int16)), "EXL3 dimensions must be positive multiples of 128."),
             (dict(t=np.zeros((8, 8, 0), np.int16)), "EXL3 unsupported trellis rate."),
             (dict(t=np.zeros((8, 8, 144), np.int16)), "EXL3 unsupported trellis rate."),
             (dict(t=np.zeros((2048, 2048, 16), np.int16)), "EXL3 logical FLOAT weights exceed max_bytes."),
             (dict(m1=mcg, m2=mul1), "EXL3 unexpected side tensors or conflicting codebooks."),
             (dict(t=np.zeros((8, 8, 48), np.uint16)), "EXL3 invalid tensor type, shape or byte extent."),
             (dict(u=inf, v=svh[:5]), "EXL3 nonfinite scale."),
             (dict(v=svh[:5]), "EXL3 invalid tensor type, shape or byte extent."),
             (dict(u=suh.astype(np.float32)), "EXL3 invalid tensor type, shape or byte extent."),
             (dict(m1=np.array(mcg ^ 1)), "EXL3 invalid codebook marker."),
             (dict(m2=mcg), "EXL3 invalid codebook marker.")]
    for kw, msg in cases:
        rc, err = run(**kw)
        assert rc == olamd.INVALID_ARGUMENT and msg in err, (kw.keys(), err)
    for kw in (dict(), dict(m1=mcg), dict(m2=mul1)):
        rc, err = run(**kw)
        assert rc == olamd.NOT_INITIALIZED, err
