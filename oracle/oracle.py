"""numpy front end of the C oracle (``oracle/liboracle.so``).

Test infrastructure only: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the parity checker / CPU
baseline.  The shipped library never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FLOAT, UINT8, INT8, UINT16, INT16, INT32 = 1, 2, 3, 4, 5, 6
FLOAT16, BFLOAT16, FLOAT8E4M3FN, UINT4, INT4 = 10, 16, 17, 21, 22
FLOAT8E4M3FNUZ, FLOAT8E5M2, FLOAT8E5M2FNUZ, FLOAT4E2M1, UINT2, INT2, FLOAT6E2M3, FLOAT6E3M2 = (
    18, 19, 20, 23, 25, 26, 27, 28)

_NP_OF = {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, INT32: np.int32,
          FLOAT: np.float32, FLOAT16: np.uint16, BFLOAT16: np.uint16, FLOAT8E4M3FN: np.uint8,
          INT4: np.uint8, UINT4: np.uint8}

_lib = None


def build() -> None:
    """Compiles liboracle.so with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64P = ctypes.POINTER(ctypes.c_int64)


class VptqConfig(ctypes.Structure):
    """orc_vptq_config (oracle.h)."""
    _fields_ = [("k", ctypes.c_int64), ("n", ctypes.c_int64), ("bits", ctypes.c_int64),
                ("vector_lens", ctypes.c_int64 * 2), ("num_centroids", ctypes.c_int64 * 2),
                ("num_res_centroids", ctypes.c_int64 * 2), ("npercent", ctypes.c_double),
                ("group_size", ctypes.c_int64), ("group_num", ctypes.c_int64), ("enable_norm", ctypes.c_int32),
                ("norm_dim", ctypes.c_int32), ("enable_perm", ctypes.c_int32), ("dtype", ctypes.c_int32)]


def _declare(L):
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f32_to_f16.argtypes = [ctypes.c_float]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_f32_to_f8e4m3fn.restype = ctypes.c_uint8
    L.orc_f32_to_f8e4m3fn.argtypes = [ctypes.c_float]
    L.orc_f8e4m3fn_to_f32.restype = ctypes.c_float
    L.orc_f8e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
    L.orc_f32_to_float_code.restype = ctypes.c_uint8
    L.orc_f32_to_float_code.argtypes = [ctypes.c_float, ctypes.c_int]
    for name in ("orc_f32_to_f16_n", "orc_f16_to_f32_n", "orc_f32_to_bf16_n", "orc_bf16_to_f32_n",
                 "orc_f32_to_f8e4m3fn_n", "orc_f8e4m3fn_to_f32_n"):
        getattr(L, name).restype = None
        getattr(L, name).argtypes = [P, ctypes.c_int64, P]
    L.orc_splitmix64_next.restype = ctypes.c_uint64
    L.orc_splitmix64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.orc_rand_uniform.restype = None
    L.orc_rand_uniform.argtypes = [ctypes.c_uint64, ctypes.c_int64, P]
    L.orc_rand_int.restype = ctypes.c_int
    L.orc_rand_int.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int64, P]
    L.orc_randn.restype = None
    L.orc_randn.argtypes = [ctypes.c_uint64, ctypes.c_int64, P]
    L.orc_matmul_output_shape.restype = ctypes.c_int
    L.orc_matmul_output_shape.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P,
                                          ctypes.POINTER(ctypes.c_int)]
    L.orc_matmul_integer.restype = ctypes.c_int
    L.orc_matmul_integer.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P,
                                     ctypes.c_int, P, ctypes.c_int64, P, ctypes.c_int64, P]
    L.orc_qlinear_matmul.restype = ctypes.c_int
    L.orc_qlinear_matmul.argtypes = [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int32,
                                     ctypes.c_float, P, ctypes.c_int, P, ctypes.c_int,
                                     ctypes.c_int32, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_int32, ctypes.c_int, P, ctypes.c_int64,
                                     ctypes.c_int64]
    L.orc_dequantize_linear.restype = ctypes.c_int
    L.orc_dequantize_linear.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P,
                                        ctypes.c_int, P, ctypes.c_int64, P]
    L.orc_quantize_linear.restype = ctypes.c_int
    L.orc_quantize_linear.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P,
                                      ctypes.c_int, P, ctypes.c_int, ctypes.c_int64, P]
    L.orc_dynamic_quantize_linear.restype = ctypes.c_int
    L.orc_dynamic_quantize_linear.argtypes = [P, ctypes.c_int64, P, P, P]
    L.orc_conv_geometry.restype = ctypes.c_int
    L.orc_conv_geometry.argtypes = [P, ctypes.c_int, P, P, P, P, P, ctypes.c_int, P, P, P, P, P]
    L.orc_conv_integer.restype = ctypes.c_int
    L.orc_conv_integer.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P, P, P,
                                   ctypes.c_int64, ctypes.c_int64, P, P, P, P, ctypes.c_int, P]
    L.orc_qlinear_conv.restype = ctypes.c_int
    L.orc_qlinear_conv.argtypes = [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_float, ctypes.c_int32,
                                   P, ctypes.c_int, P, P, ctypes.c_int64, P, ctypes.c_int64,
                                   ctypes.c_float, ctypes.c_int32, ctypes.c_int, P, ctypes.c_int64,
                                   P, P, P, P, ctypes.c_int, P]
    L.orc_packed_block_bytes.restype = ctypes.c_int
    L.orc_packed_block_bytes.argtypes = [ctypes.c_int]
    L.orc_packed_block_values.restype = ctypes.c_int
    L.orc_packed_block_values.argtypes = [ctypes.c_int]
    L.orc_dequantize_packed.restype = ctypes.c_int
    L.orc_dequantize_packed.argtypes = [ctypes.c_int, P, ctypes.c_int64, P]
    L.orc_matmul_f32.restype = ctypes.c_int
    L.orc_matmul_f32.argtypes = [P, P, ctypes.c_int, P, P, ctypes.c_int, P, ctypes.c_int64,
                                 ctypes.c_int64, ctypes.c_int]
    L.orc_ort_nbits_decode.restype = ctypes.c_int
    L.orc_ort_nbits_decode.argtypes = [P, P, ctypes.c_int, P, P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                       ctypes.c_int64, P]
    L.orc_dq_decode_n.restype = None
    L.orc_dq_decode_n.argtypes = [P, ctypes.c_int, ctypes.c_int64, P]
    L.orc_awq_decode.restype = ctypes.c_int
    L.orc_awq_decode.argtypes = [ctypes.c_int, ctypes.c_int, P, P, P, P, ctypes.c_int64, ctypes.c_int64,
                                 ctypes.c_int64, ctypes.c_int64, P, P, P]
    L.orc_gptq_decode.restype = ctypes.c_int
    L.orc_gptq_decode.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P, ctypes.c_int64,
                                  ctypes.c_int64, ctypes.c_int64, P, P, P]
    L.orc_bnb_table.restype = ctypes.c_float
    L.orc_bnb_table.argtypes = [ctypes.c_int, ctypes.c_int]
    L.orc_bnb_check.restype = ctypes.c_int
    L.orc_bnb_check.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                ctypes.c_float, P, P, P, P]
    L.orc_vptq_reconstruct.restype = ctypes.c_int
    L.orc_vptq_reconstruct.argtypes = [ctypes.POINTER(VptqConfig), P, P, P, P, P, P, P, P, ctypes.c_int, P]
    L.orc_f8e8m0_to_f32.restype = ctypes.c_float
    L.orc_f8e8m0_to_f32.argtypes = [ctypes.c_uint8]
    L.orc_exl3_reconstruct.restype = ctypes.c_int
    L.orc_exl3_reconstruct.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    L.orc_mx_reconstruct.restype = ctypes.c_int
    L.orc_mx_reconstruct.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                     ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64),
                                     ctypes.POINTER(ctypes.c_int64)]
    L.orc_gptq_fp8_reconstruct.restype = ctypes.c_int
    L.orc_gptq_fp8_reconstruct.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int64, ctypes.c_int64, P, P, ctypes.c_int, P]
    L.orc_bitblas_reconstruct.restype = ctypes.c_int
    L.orc_bitblas_reconstruct.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                          P, P, P, ctypes.c_int, P, P]
    L.orc_qqq_position.restype = ctypes.c_int64
    L.orc_qqq_position.argtypes = [ctypes.c_int64] * 5
    L.orc_qqq_scale_position.restype = ctypes.c_int64
    L.orc_qqq_scale_position.argtypes = [ctypes.c_int64, ctypes.c_int]
    L.orc_qqq_reconstruct.restype = ctypes.c_int
    L.orc_qqq_reconstruct.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, P, P, P, ctypes.c_int, P, P]
    L.orc_bnb_reconstruct.restype = ctypes.c_int
    L.orc_bnb_reconstruct.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                      ctypes.c_float, P, P, P, P, ctypes.c_int, P]
    L.orc_grouped_matmul.restype = ctypes.c_int
    L.orc_grouped_matmul.argtypes = [ctypes.c_int, P, ctypes.c_int64, ctypes.c_int64, P, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int, P, ctypes.c_int64, P, P]
    L.orc_matmul_half.restype = ctypes.c_int
    L.orc_matmul_half.argtypes = [P, P, ctypes.c_int, P, P, ctypes.c_int, ctypes.c_int, P,
                                  ctypes.c_int64, ctypes.c_int64, ctypes.c_int]


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(P)


def _shape(shape):
    return np.ascontiguousarray(np.array(list(shape) or [0], dtype=np.int64))


# ---- codecs -----------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_ptr(x), x.size, _ptr(out))
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(_ptr(h), h.size, _ptr(out))
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_ptr(x), x.size, _ptr(out))
    return out


def bf16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_n(_ptr(h), h.size, _ptr(out))
    return out


def f32_to_f8e4m3fn_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.uint8)
    lib().orc_f32_to_f8e4m3fn_n(_ptr(x), x.size, _ptr(out))
    return out


def f8e4m3fn_bits_to_f32(c) -> np.ndarray:
    c = np.ascontiguousarray(np.asarray(c, dtype=np.uint8))
    out = np.empty(c.shape, np.float32)
    lib().orc_f8e4m3fn_to_f32_n(_ptr(c), c.size, _ptr(out))
    return out


# ---- RNG --------------------------------------------------------------------

def splitmix64(seed: int, n: int) -> list[int]:
    s = ctypes.c_uint64(seed)
    return [lib().orc_splitmix64_next(ctypes.byref(s)) for _ in range(n)]


def rand_uniform(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float64)
    lib().orc_rand_uniform(seed, n, _ptr(out))
    return out


def rand_int(low: int, high: int, seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int64)
    if lib().orc_rand_int(low, high, seed, n, _ptr(out)) != 0:
        raise ValueError("high must be greater than low.")
    return out


def randn(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float64)
    lib().orc_randn(seed, n, _ptr(out))
    return out


def pack_int4(values) -> np.ndarray:
    """Packs 4-bit values (flat order, low nibble = even index) into bytes."""
    v = np.asarray(values, dtype=np.int64).reshape(-1) & 0xF
    if v.size % 2:
        v = np.concatenate([v, np.zeros(1, np.int64)])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


# ---- kernels ----------------------------------------------------------------

def matmul_output_shape(a_shape, b_shape):
    a_s, b_s = _shape(a_shape), _shape(b_shape)
    out = np.zeros(40, np.int64)
    r = ctypes.c_int(0)
    rc = lib().orc_matmul_output_shape(_ptr(a_s), len(a_shape), _ptr(b_s), len(b_shape),
                                       _ptr(out), ctypes.byref(r))
    if rc:
        raise ValueError(f"matmul shape error {rc}")
    return tuple(int(d) for d in out[: r.value])


def matmul_integer(a: np.ndarray, b: np.ndarray, a_zp=None, b_zp=None) -> np.ndarray:
    """MatMulInteger with zero points given as int arrays (1 or M / 1 or N values)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    ad = INT8 if a.dtype == np.int8 else UINT8
    bd = INT8 if b.dtype == np.int8 else UINT8
    za = np.ascontiguousarray(np.asarray([0] if a_zp is None else a_zp, np.int32).reshape(-1))
    zb = np.ascontiguousarray(np.asarray([0] if b_zp is None else b_zp, np.int32).reshape(-1))
    out_shape = matmul_output_shape(a.shape, b.shape)
    y = np.empty(out_shape, np.int32)
    rc = lib().orc_matmul_integer(_ptr(a), ad, _ptr(_shape(a.shape)), a.ndim, _ptr(b), bd,
                                  _ptr(_shape(b.shape)), b.ndim, _ptr(za), za.size, _ptr(zb),
                                  zb.size, _ptr(y))
    if rc:
        raise ValueError(f"matmul_integer error {rc}")
    return y


def qlinear_matmul(a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, y_dtype=None,
                   rows=None) -> np.ndarray:
    """QLinearMatMul; y dtype defaults to the dtype of the y zero point (u8 or s8)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    ad = INT8 if a.dtype == np.int8 else UINT8
    bd = INT8 if b.dtype == np.int8 else UINT8
    yd = y_dtype if y_dtype is not None else ad
    out_shape = matmul_output_shape(a.shape, b.shape)
    y = np.zeros(out_shape, np.int8 if yd == INT8 else np.uint8)
    r0, r1 = (0, -1) if rows is None else rows
    rc = lib().orc_qlinear_matmul(_ptr(a), ad, _ptr(_shape(a.shape)), a.ndim, int(a_zp),
                                  float(a_scale), _ptr(b), bd, _ptr(_shape(b.shape)), b.ndim,
                                  int(b_zp), float(b_scale), float(y_scale), int(y_zp), yd,
                                  _ptr(y), r0, r1)
    if rc:
        raise ValueError(f"qlinear_matmul error {rc}")
    return y


def dequantize_linear(x: np.ndarray, x_dtype: int, x_shape, scale: np.ndarray, scale_dtype: int,
                      zp=None, axis: int = 1) -> np.ndarray:
    """DequantizeLinear.  x holds the raw storage (bytes for 4-bit types);
    scale holds FLOAT values or FLOAT16 bit patterns; the output follows the
    scale dtype (float32 array, or uint16 FLOAT16 bits)."""
    x = np.ascontiguousarray(x)
    scale = np.ascontiguousarray(scale)
    zp_arr = None if zp is None else np.ascontiguousarray(zp)
    n = int(np.prod(x_shape)) if len(x_shape) else 1
    y = np.empty(tuple(x_shape), np.uint16 if scale_dtype == FLOAT16 else np.float32)
    s_shape = scale.shape
    rc = lib().orc_dequantize_linear(_ptr(x), x_dtype, _ptr(_shape(x_shape)), len(x_shape),
                                     _ptr(scale), scale_dtype, _ptr(_shape(s_shape)),
                                     len(s_shape), None if zp_arr is None else _ptr(zp_arr),
                                     axis, _ptr(y))
    if rc:
        raise ValueError(f"dequantize_linear error {rc}")
    assert y.size == n
    return y


def quantize_linear(x: np.ndarray, x_dtype: int, scale: np.ndarray, scale_dtype: int, y_dtype: int,
                    zp=None, axis: int = 1) -> np.ndarray:
    """QuantizeLinear.  x holds FLOAT values or FLOAT16 bit patterns (its shape
    is x's shape); scale likewise; zp holds the raw storage of the y dtype
    (bytes for 4-bit types).  Returns the raw y storage: a uint8 / int8 /
    uint16 / int16 / fp8-bits uint8 array of x's shape, or the packed bytes
    of the sub-byte types."""
    x = np.ascontiguousarray(x)
    scale = np.ascontiguousarray(scale)
    zp_arr = None if zp is None else np.ascontiguousarray(zp)
    n = x.size
    sub = {UINT4: 4, INT4: 4, FLOAT4E2M1: 4, UINT2: 2, INT2: 2, FLOAT6E2M3: 6, FLOAT6E3M2: 6}
    if y_dtype in sub:
        y = np.zeros((n * sub[y_dtype] + 7) // 8, np.uint8)
    else:
        y = np.empty(x.shape, {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16,
                               FLOAT8E4M3FN: np.uint8, FLOAT8E4M3FNUZ: np.uint8, FLOAT8E5M2: np.uint8,
                               FLOAT8E5M2FNUZ: np.uint8}[y_dtype])
    rc = lib().orc_quantize_linear(_ptr(x), x_dtype, _ptr(_shape(x.shape)), x.ndim, _ptr(scale),
                                   scale_dtype, _ptr(_shape(scale.shape)), scale.ndim,
                                   None if zp_arr is None else _ptr(zp_arr), y_dtype, axis, _ptr(y))
    if rc:
        raise ValueError(f"quantize_linear error {rc}")
    return y


def dynamic_quantize_linear(x: np.ndarray):
    """DynamicQuantizeLinear of a FLOAT array: (y uint8, scale, zero point).
    Raises ValueError for an empty or non-finite x, as the reference does."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint8)
    sc = np.zeros(1, np.float32)
    zp = np.zeros(1, np.uint8)
    rc = lib().orc_dynamic_quantize_linear(_ptr(x), x.size, _ptr(y), _ptr(sc), _ptr(zp))
    if rc:
        raise ValueError("kernel::DynamicQuantizeLinear: x must be non-empty and finite")
    return y, sc[0], zp[0]


def matmul_f32(a: np.ndarray, b: np.ndarray, rows=None, nthreads=1) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    y = np.zeros(matmul_output_shape(a.shape, b.shape), np.float32)
    r0, r1 = (0, -1) if rows is None else rows
    rc = lib().orc_matmul_f32(_ptr(a), _ptr(_shape(a.shape)), a.ndim, _ptr(b),
                              _ptr(_shape(b.shape)), b.ndim, _ptr(y), r0, r1, nthreads)
    if rc:
        raise ValueError(f"matmul error {rc}")
    return y


def matmul_half(a_bits: np.ndarray, b_bits: np.ndarray, dtype: int, rows=None,
                nthreads=1) -> np.ndarray:
    """fp16 / bf16 MatMul on bit patterns (uint16 arrays); returns uint16 bits."""
    a = np.ascontiguousarray(a_bits, dtype=np.uint16)
    b = np.ascontiguousarray(b_bits, dtype=np.uint16)
    y = np.zeros(matmul_output_shape(a.shape, b.shape), np.uint16)
    r0, r1 = (0, -1) if rows is None else rows
    rc = lib().orc_matmul_half(_ptr(a), _ptr(_shape(a.shape)), a.ndim, _ptr(b),
                               _ptr(_shape(b.shape)), b.ndim, dtype, _ptr(y), r0, r1, nthreads)
    if rc:
        raise ValueError(f"matmul_half error {rc}")
    return y


DOUBLE = 11


def ort_nbits_decode(B: np.ndarray, scales: np.ndarray, zero_points, K: int, N: int, bits: int,
                     block: int) -> np.ndarray:
    """ORT MatMulNBits value -> float64 [K, N] = (code - zp) * scale.  B uint8
    [N, groups, blob]; scales float [N, groups] (values); zero_points None,
    uint8 packed codes [N, ceil(groups * bits / 8)], or float [N, groups]."""
    B = np.ascontiguousarray(B, dtype=np.uint8)
    sc = np.ascontiguousarray(scales, dtype=np.float64)
    out = np.zeros((K, N), np.float64)
    kind, zc, zv = 0, None, None
    if zero_points is not None:
        zp = np.asarray(zero_points)
        if zp.dtype == np.uint8:
            kind, zc = 1, np.ascontiguousarray(zp)
        else:
            kind, zv = 2, np.ascontiguousarray(zp, dtype=np.float64)
    rc = lib().orc_ort_nbits_decode(_ptr(B), _ptr(sc), kind, None if zc is None else _ptr(zc),
                                    None if zv is None else _ptr(zv), K, N, bits, block, _ptr(out))
    if rc:
        raise ValueError(f"ort_nbits_decode error {rc}")
    return out


def grouped_matmul(x: np.ndarray, w: np.ndarray, indices: np.ndarray, bias=None, transB: int = 0,
                   dtype: int = FLOAT) -> np.ndarray:
    """GroupedMatMul: x [M, K], w [G, K, N] (or [G, N, K] with transB), indices
    [M, S] -> y [M, S, N].  FLOAT16 / BFLOAT16 tensors are uint16 bit arrays."""
    np_t = {FLOAT: np.float32, DOUBLE: np.float64, FLOAT16: np.uint16, BFLOAT16: np.uint16}[dtype]
    x = np.ascontiguousarray(x, dtype=np_t)
    w = np.ascontiguousarray(w, dtype=np_t)
    idx = np.ascontiguousarray(indices, dtype=np.int64)
    M, K = x.shape
    G = w.shape[0]
    N = w.shape[1] if transB else w.shape[2]
    S = idx.shape[1]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np_t)
    y = np.zeros((M, S, N), np_t)
    rc = lib().orc_grouped_matmul(dtype, _ptr(x), M, K, _ptr(w), G, N, 1 if transB else 0, _ptr(idx), S,
                                  None if b is None else _ptr(b), _ptr(y))
    if rc == 5:
        raise ValueError("group index must be in [0,G)")
    if rc:
        raise ValueError(f"grouped_matmul error {rc}")
    return y


# ---- ConvInteger / QLinearConv ----------------------------------------------

AUTO_PAD = {"NOTSET": 0, "SAME_UPPER": 1, "SAME_LOWER": 2, "VALID": 3}


def _opt(v):
    return None if v is None else _shape(v)


def conv_geometry(x_shape, w_shape, kernel_shape=None, strides=None, pads=None, dilations=None,
                  auto_pad="NOTSET"):
    """(kernel, strides, dilations, resolved pads, output spatial sizes) as the
    reference resolves them; raises ValueError where it rejects."""
    sr = len(x_shape) - 2
    outs = [np.zeros(max(sr, 1) * (2 if i == 3 else 1), np.int64) for i in range(5)]
    args = [_opt(v) for v in (kernel_shape, strides, pads, dilations)]
    rc = lib().orc_conv_geometry(_ptr(_shape(x_shape)), len(x_shape), _ptr(_shape(w_shape)),
                                 *[None if a is None else _ptr(a) for a in args], AUTO_PAD[auto_pad],
                                 *[_ptr(o) for o in outs])
    if rc:
        raise ValueError("conv attributes rejected")
    return tuple(tuple(int(v) for v in o) for o in outs)


def _conv_args(x, w, group, kernel_shape, strides, pads, dilations, auto_pad):
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    geo = conv_geometry(x.shape, w.shape, kernel_shape, strides, pads, dilations, auto_pad)
    out_shape = (x.shape[0], w.shape[0]) + geo[4]
    attrs = [_opt(v) for v in (kernel_shape, strides, pads, dilations)]
    return x, w, out_shape, attrs


def conv_integer(x, x_dtype, w, w_dtype, x_zp=None, w_zp=None, group=1, kernel_shape=None, strides=None,
                 pads=None, dilations=None, auto_pad="NOTSET"):
    """ConvInteger on raw int8 / uint8 storage: int32 output (wrapping)."""
    x, w, out_shape, attrs = _conv_args(x, w, group, kernel_shape, strides, pads, dilations, auto_pad)
    xz = None if x_zp is None else np.ascontiguousarray(x_zp).reshape(-1)
    wz = None if w_zp is None else np.ascontiguousarray(w_zp).reshape(-1)
    y = np.zeros(out_shape, np.int32)
    rc = lib().orc_conv_integer(_ptr(x), x_dtype, _ptr(_shape(x.shape)), x.ndim, _ptr(w), w_dtype,
                                _ptr(_shape(w.shape)), None if xz is None else _ptr(xz),
                                None if wz is None else _ptr(wz), 0 if wz is None else wz.size, group,
                                *[None if a is None else _ptr(a) for a in attrs], AUTO_PAD[auto_pad],
                                _ptr(y))
    if rc:
        raise ValueError(f"conv_integer error {rc}")
    return y


def qlinear_conv(x, x_dtype, x_scale, x_zp, w, w_dtype, w_scale, w_zp, y_scale, y_zp, y_dtype, bias=None,
                 group=1, kernel_shape=None, strides=None, pads=None, dilations=None, auto_pad="NOTSET"):
    """QLinearConv on raw storage; scales are float32 values (w_scale and w_zp
    scalar or length M), bias int32 length M or None."""
    x, w, out_shape, attrs = _conv_args(x, w, group, kernel_shape, strides, pads, dilations, auto_pad)
    ws = np.ascontiguousarray(np.asarray(w_scale, np.float32).reshape(-1))
    wz = np.ascontiguousarray(np.asarray(w_zp).reshape(-1).astype(_NP_OF[w_dtype]))
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias, np.int32).reshape(-1))
    y = np.zeros(out_shape, np.int8 if y_dtype == INT8 else np.uint8)
    rc = lib().orc_qlinear_conv(_ptr(x), x_dtype, _ptr(_shape(x.shape)), x.ndim, float(np.float32(x_scale)),
                                int(x_zp), _ptr(w), w_dtype, _ptr(_shape(w.shape)), _ptr(ws), ws.size,
                                _ptr(wz), wz.size, float(np.float32(y_scale)), int(y_zp),
                                int(y_dtype == INT8), None if b is None else _ptr(b), group,
                                *[None if a is None else _ptr(a) for a in attrs], AUTO_PAD[auto_pad],
                                _ptr(y))
    if rc:
        raise ValueError(f"qlinear_conv error {rc}")
    return y


# ---- DequantizePacked (the GGUF profiles without codebooks) ------------------

GGUF_TYPES = {"gguf:q4_0": 2, "gguf:q4_1": 3, "gguf:q5_0": 6, "gguf:q5_1": 7, "gguf:q8_0": 8,
              "gguf:q8_1": 9, "gguf:iq4_nl": 20, "gguf:q4_k": 12, "gguf:q6_k": 14,
              "gguf:q2_k": 10, "gguf:q3_k": 11, "gguf:q5_k": 13, "gguf:q8_k": 15, "gguf:iq4_xs": 23,
              "gguf:tq1_0": 34, "gguf:tq2_0": 35, "gguf:mxfp4": 39, "gguf:nvfp4": 40, "gguf:q1_0": 41,
              "gguf:q2_0": 42, "gguf:iq2_xxs": 16, "gguf:iq2_xs": 17, "gguf:iq3_xxs": 18, "gguf:iq1_s": 19,
              "gguf:iq3_s": 21, "gguf:iq2_s": 22, "gguf:iq1_m": 29}


def packed_block_bytes(fmt: str) -> int:
    return lib().orc_packed_block_bytes(GGUF_TYPES[fmt])


def packed_block_values(fmt: str) -> int:
    return lib().orc_packed_block_values(GGUF_TYPES[fmt])


def dequantize_packed(x: np.ndarray, fmt: str, shape, output_dtype: int = FLOAT) -> np.ndarray:
    """FLOAT values (float32 array of `shape`), or FLOAT16 / BFLOAT16 bit
    patterns (uint16) / DOUBLE values converted from them."""
    x = np.ascontiguousarray(x, dtype=np.uint8)
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, np.float32)
    rc = lib().orc_dequantize_packed(GGUF_TYPES[fmt], _ptr(x), n // packed_block_values(fmt), _ptr(out))
    if rc:
        raise ValueError(f"dequantize_packed error {rc}")
    out = out.reshape(shape)
    if output_dtype == FLOAT16:
        return f32_to_f16_bits(out)
    if output_dtype == BFLOAT16:
        return f32_to_bf16_bits(out)
    if output_dtype == 11:  # DOUBLE
        return out.astype(np.float64)
    return out


# ---- AWQ and GPTQ weights (awq.cc:185-247, gptq.cc:166-228) ------------------

AWQ_VARIANTS = {"gemm": 0, "gemv": 1, "gemv_fast": 2, "llm-awq": 2}
GPTQ_FORMATS = {"gptq": 0, "gptq_v2": 1, "gptq_p": 2}


def awq_decode(variant: str, qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, K: int, N: int,
               group: int, bits: int = 4):
    """AWQ weight -> (codes uint8 [N, K], zeros uint8 [N, groups], FLOAT values
    float32 [N, K]).  qweight / qzeros in the variant's integer layout (for
    gemv_fast / llm-awq, qzeros is the float zero-term array [padded, N]);
    scales float values in the variant's layout ([groups, N] gemm, [N, padded]
    gemv, [padded, N] gemv_fast / llm-awq)."""
    v = AWQ_VARIANTS[variant]
    qw = np.ascontiguousarray(qweight)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    eff = K if group == -1 else group
    groups = K // eff
    padded = sc.shape[1] if v == 1 else 0
    if v == 2:
        zt = np.ascontiguousarray(qzeros, dtype=np.float32)
        qz = np.zeros(1, np.uint32)
    else:
        qz = np.ascontiguousarray(qzeros)
        zt = np.zeros(1, np.float32)
    codes = np.empty((N, K), np.uint8)
    zeros = np.zeros((N, groups), np.uint8)
    out = np.empty((N, K), np.float32)
    rc = lib().orc_awq_decode(v, bits, _ptr(qw), _ptr(qz), _ptr(zt), _ptr(sc), K, N, group, padded, _ptr(codes),
                              _ptr(zeros), _ptr(out))
    if rc:
        raise ValueError(f"awq_decode error {rc}")
    return codes, zeros, out


def gptq_decode(fmt: str, bits: int, qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
                g_idx: np.ndarray, K: int, N: int, group: int):
    """GPTQ weight -> (codes uint8 [N, K], zeros int16 [N, groups], FLOAT
    values float32 [N, K]).  qweight / qzeros integer words (their itemsize is
    the word width); scales float values [groups, N]; g_idx int32 [K]."""
    qw = np.ascontiguousarray(qweight)
    qz = np.ascontiguousarray(qzeros)
    assert qw.dtype.itemsize == qz.dtype.itemsize
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    gi = np.ascontiguousarray(g_idx, dtype=np.int32)
    eff = K if group == -1 else group
    groups = -(-K // eff)
    codes = np.empty((N, K), np.uint8)
    zeros = np.empty((N, groups), np.int16)
    out = np.empty((N, K), np.float32)
    lib().orc_gptq_decode(GPTQ_FORMATS[fmt], bits, qw.dtype.itemsize, _ptr(qw), _ptr(qz), _ptr(sc), _ptr(gi), K, N,
                          group, _ptr(codes), _ptr(zeros), _ptr(out))
    return codes, zeros, out


# ---- sub-byte and further float8 DequantizeLinear inputs ---------------------

def dq_decode(raw: np.ndarray, dtype: int, n: int) -> np.ndarray:
    """The n decoded float32 elements of a DequantizeLinear input buffer of
    `dtype` (packed storage for the sub-byte types)."""
    raw = np.ascontiguousarray(raw)
    out = np.empty(n, np.float32)
    lib().orc_dq_decode_n(_ptr(raw), dtype, n, _ptr(out))
    return out


def float_code(values, dtype: int) -> np.ndarray:
    """QuantizeLinear's float encoders element by element: fp32 values ->
    FLOAT8E4M3FN / FNUZ / E5M2 / E5M2FNUZ bytes, FLOAT4E2M1 or FLOAT6 codes."""
    v = np.asarray(values, np.float32).reshape(-1)
    return np.array([lib().orc_f32_to_float_code(float(f), dtype) for f in v], np.uint8)


def pack_bits(codes, bits: int) -> np.ndarray:
    """Codes of `bits` bits (2, 4 or 6) as the packed little-endian bit stream
    of ONNX sub-byte tensors: element i at bits i * bits onwards."""
    codes = np.asarray(codes, np.uint64).reshape(-1)
    n = codes.size
    out = np.zeros((n * bits + 7) // 8 + 1, np.uint8)
    for i, c in enumerate(codes.tolist()):
        bit = i * bits
        v = (int(c) & ((1 << bits) - 1)) << (bit % 8)
        out[bit // 8] |= v & 0xFF
        out[bit // 8 + 1] |= (v >> 8) & 0xFF
    return out[:(n * bits + 7) // 8].copy()


# ---- bitsandbytes weights (nf4 / fp4 / int8) ---------------------------------

BNB_FORMATS = {"nf4": 0, "fp4": 1, "int8": 2}
BNB_ERRORS = {2: "bitsandbytes nonfinite reconstruction.", 3: "bitsandbytes nonfinite table or invalid absmax.",
              4: "bitsandbytes noncanonical NF4/FP4 table."}


def bnb_table(fmt: str) -> np.ndarray:
    """The format's 16 code values (nf4 / fp4) as float32."""
    return np.array([lib().orc_bnb_table(BNB_FORMATS[fmt], j) for j in range(16)], np.float32)


def _f32(x):
    return np.zeros(1, np.float32) if x is None else np.ascontiguousarray(x, dtype=np.float32)


def bnb_check(fmt: str, rows: int, cols: int, block: int, absmax, quant_map=None, nested_absmax=None,
              nested_map=None, offset: float = 0.0) -> int:
    """The side-tensor checks: 0, or the key of BNB_ERRORS.  absmax float32
    (or uint8 codes with nested_absmax / nested_map)."""
    nested = nested_absmax is not None
    am = np.ascontiguousarray(absmax)
    return lib().orc_bnb_check(BNB_FORMATS[fmt], rows, cols, block, int(nested), offset, _ptr(am), _ptr(_f32(quant_map)),
                               _ptr(_f32(nested_absmax)), _ptr(_f32(nested_map)))


def bnb_reconstruct(fmt: str, rows: int, cols: int, block: int, codes, absmax, nested_absmax=None, nested_map=None,
                    offset: float = 0.0, out_dtype: int = FLOAT):
    """(rc, values [rows, cols]): float32 for FLOAT, uint16 bits for FLOAT16 /
    BFLOAT16; rc 2 is the reference's nonfinite-reconstruction error."""
    nested = nested_absmax is not None
    cd = np.ascontiguousarray(codes).view(np.uint8)
    am = np.ascontiguousarray(absmax)
    out = np.zeros((rows, cols), np.float32 if out_dtype == FLOAT else np.uint16)
    rc = lib().orc_bnb_reconstruct(BNB_FORMATS[fmt], rows, cols, block, int(nested), offset, _ptr(cd), _ptr(am),
                                   _ptr(_f32(nested_absmax)), _ptr(_f32(nested_map)), out_dtype, _ptr(out))
    return rc, out


# ---- QQQ weights (four-bit, group -1 / 128) ------------------------------------

QQQ_ERRORS = {1: "QQQ nonfinite or negative channel scale.", 2: "QQQ nonfinite or negative group scale.",
              3: "QQQ FLOAT reconstruction overflow.", 4: "Dequantization output dtype overflow."}


def qqq_position(k: int, n: int, group: int, n_index: int, k_index: int) -> int:
    """Nibble index of code (n_index, k_index) in the packed words."""
    return lib().orc_qqq_position(k, n, group, n_index, k_index)


def qqq_scale_position(index: int, channel: bool) -> int:
    """Storage index of logical channel scale `index` (or group-scale index)."""
    return lib().orc_qqq_scale_position(index, int(channel))


def qqq_reconstruct(k: int, n: int, group: int, words, s_channel, s_group, out_dtype: int = FLOAT):
    """(rc, values [n, k], codes [n, k]): float32 (FLOAT), float64 (DOUBLE) or
    uint16 bits (FLOAT16 / BFLOAT16); rc is 0 or a key of QQQ_ERRORS.  words:
    the int32 B tensor; s_channel float32 [1, n]; s_group float16 [k/128, n]
    (or empty)."""
    w = np.ascontiguousarray(words).view(np.uint8)
    sc = np.ascontiguousarray(s_channel, dtype=np.float32)
    sg = np.ascontiguousarray(s_group).view(np.uint16) if np.size(s_group) else np.zeros(1, np.uint16)
    dt = {FLOAT: np.float32, DOUBLE: np.float64}.get(out_dtype, np.uint16)
    out = np.zeros((n, k), dt)
    codes = np.zeros((n, k), np.uint8)
    rc = lib().orc_qqq_reconstruct(k, n, group, _ptr(w), _ptr(sc), _ptr(sg), out_dtype, _ptr(out), _ptr(codes))
    return rc, out, codes


# ---- BitBLAS row-packed weights ------------------------------------------------

BITBLAS_ERRORS = {1: "BitBLAS nonfinite or nonpositive scale.", 4: "Dequantization output dtype overflow."}


def bitblas_reconstruct(k: int, n: int, group: int, bits: int, signed_codes: bool, qweight, scales, qzeros=None,
                        out_dtype: int = FLOAT):
    """(rc, values [n, k], raw codes [n, k]) of a BitBLAS row-packed weight:
    qweight int8 [n, k * bits / 8], scales float16 [n, groups], qzeros int8
    [groups, n * bits / 8] (None for symmetric GPTQ codes)."""
    qw = np.ascontiguousarray(qweight).view(np.uint8)
    sc = np.ascontiguousarray(scales).view(np.uint16)
    qz = np.zeros(1, np.uint8) if qzeros is None or np.size(qzeros) == 0 else np.ascontiguousarray(qzeros).view(np.uint8)
    dt = {FLOAT: np.float32, DOUBLE: np.float64}.get(out_dtype, np.uint16)
    out = np.zeros((n, k), dt)
    codes = np.zeros((n, k), np.uint8)
    rc = lib().orc_bitblas_reconstruct(k, n, group, bits, int(signed_codes), _ptr(qw), _ptr(sc), _ptr(qz), out_dtype,
                                       _ptr(out), _ptr(codes))
    return rc, out, codes


# ---- GPTQModel FP8 weights -------------------------------------------------------

GPTQ_FP8_METHODS = {"tensor": 0, "row": 1, "block": 2}
GPTQ_FP8_ERRORS = {1: "GPTQModel FP8 inverse scales must be finite and positive.",
                   2: "GPTQModel FP8 nonfinite weight or reconstruction.", 4: "Dequantization output dtype overflow."}


def gptq_fp8_reconstruct(codes, code_type: int, scales, method: str, block=(1, 1), out_dtype: int = FLOAT):
    """(rc, values [n, k]) of FP8 codes [n, k] over FLOAT inverse scales."""
    c = np.ascontiguousarray(codes).view(np.uint8)
    n, k = c.shape
    s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    dt = {FLOAT: np.float32, DOUBLE: np.float64}.get(out_dtype, np.uint16)
    out = np.zeros((n, k), dt)
    rc = lib().orc_gptq_fp8_reconstruct(n, k, code_type, GPTQ_FP8_METHODS[method], block[0], block[1], _ptr(c),
                                        _ptr(s), out_dtype, _ptr(out))
    return rc, out


# ---- EXL3 weights ----------------------------------------------------------------------

EXL3_ERRORS = {1: "EXL3 nonfinite reconstruction.", 4: "Dequantization output dtype overflow."}


def exl3_reconstruct(trellis, suh, svh, book: int = 0, out_dtype: int = FLOAT):
    """(rc, values [k, n]) of an EXL3 weight: trellis int16 [k / 16, n / 16,
    16 * bits], suh / svh binary16 [k] / [n], book 0 3INST, 1 MCG, 2 MUL1."""
    t = np.ascontiguousarray(trellis).view(np.uint16)
    k, n, bits = t.shape[0] * 16, t.shape[1] * 16, t.shape[2] // 16
    u = np.ascontiguousarray(suh).view(np.uint16)
    v = np.ascontiguousarray(svh).view(np.uint16)
    dt = {FLOAT: np.float32, DOUBLE: np.float64}.get(out_dtype, np.uint16)
    out = np.zeros((k, n), dt)
    rc = lib().orc_exl3_reconstruct(k, n, bits, book, _ptr(t), _ptr(u), _ptr(v), out_dtype, _ptr(out))
    return rc, out


# ---- MX and NVFP4 weights -----------------------------------------------------------

MX_FORMATS = {"mxfp4": 0, "mxfp6_e2m3": 1, "mxfp8": 2, "nvfp4": 3}


def mx_error(fmt: str, rc: int, group: int, element: int) -> str:
    """The reference's message for orc_mx_reconstruct's failure `rc`
    (quantization.cc:1322-1342, 1458-1470, 1591-1600, 1700-1707, RoundFloat
    :41-45, WriteFloat :184-201)."""
    if rc == 6:
        return "Dequantization output dtype overflow."
    if fmt == "mxfp4":
        return {1: f"MXFP4 WEIGHT E8M0 scale is NaN in group {group}.",
                5: f"MXFP4 WEIGHT reconstruction overflow or nonfinite value in group {group}, element {element}."}[rc]
    if fmt == "nvfp4":
        return {1: f"NVFP4 WEIGHT scales must be positive and finite in group {group}.",
                2: f"NVFP4 WEIGHT effective scale overflow or nonfinite value in group {group}.",
                3: f"NVFP4 WEIGHT effective scale rounds to zero in group {group}.",
                5: f"NVFP4 WEIGHT reconstruction overflow or nonfinite value in group {group}, element {element}."}[rc]
    if fmt == "mxfp8":
        return {1: "MXFP8 E8M0 scale must not be NaN.", 4: "MXFP8 E4M3FN weight must not be NaN.",
                5: "FLOAT reconstruction overflow or nonfinite value."}[rc]
    return {1: "MXFP6 E2M3 E8M0 scale byte 255 is invalid.", 5: "FLOAT reconstruction overflow or nonfinite value."}[rc]


def mx_reconstruct(fmt: str, rows: int, cols: int, codes, scales, global_scale: float = 0.0,
                   out_dtype: int = FLOAT):
    """(rc, group, element, values [rows, cols]) of an MX / NVFP4 weight."""
    c = np.ascontiguousarray(codes).view(np.uint8).reshape(-1)
    s = np.ascontiguousarray(scales).view(np.uint8).reshape(-1)
    dt = {FLOAT: np.float32, DOUBLE: np.float64}.get(out_dtype, np.uint16)
    out = np.zeros((rows, cols), dt)
    g, e = ctypes.c_int64(), ctypes.c_int64()
    rc = lib().orc_mx_reconstruct(MX_FORMATS[fmt], rows * cols, _ptr(c), _ptr(s), float(global_scale), out_dtype,
                                  _ptr(out), ctypes.byref(g), ctypes.byref(e))
    return rc, g.value, e.value, out


# ---- VPTQ weights ------------------------------------------------------------------

VPTQ_ERRORS = {1: "VPTQ index exceeds codebook.", 2: "VPTQ outlier index exceeds codebook.",
               3: "VPTQ invalid permutation.", 5: "Dequantization produced a nonfinite value.",
               4: "Dequantization output dtype overflow."}


def vptq_config(params: dict, dtype: int, bits: int = 4) -> VptqConfig:
    """A VptqConfig from the checkpoint parameters (the reference fixture's names)."""
    c = VptqConfig()
    c.k, c.n, c.bits = params["in_features"], params["out_features"], bits
    for name in ("vector_lens", "num_centroids", "num_res_centroids"):
        getattr(c, name)[0], getattr(c, name)[1] = params[name]
    c.npercent = params["npercent"]
    c.group_size, c.group_num = params["group_size"], params["group_num"]
    c.enable_norm, c.norm_dim, c.enable_perm = int(params["enable_norm"]), params["norm_dim"], int(params["enable_perm"])
    c.dtype = dtype
    return c


def vptq_reconstruct(cfg: VptqConfig, tensors: dict, out_dtype: int = FLOAT):
    """(rc, values [n, k]); tensors by the checkpoint's names, codebooks as
    float32 arrays or uint16 bit patterns of the codebook dtype."""
    def arr(name, dt):
        t = tensors.get(name)
        return np.zeros(1, dt) if t is None else np.ascontiguousarray(t).view(dt)
    cb = np.float32 if cfg.dtype == FLOAT else np.uint16
    dt = {FLOAT: np.float32, DOUBLE: np.float64}.get(out_dtype, np.uint16)
    out = np.zeros((cfg.n, cfg.k), dt)
    rc = lib().orc_vptq_reconstruct(ctypes.byref(cfg), _ptr(arr("indices", np.uint32)),
                                    _ptr(arr("centroids.weight", cb)), _ptr(arr("res_centroids.weight", cb)),
                                    _ptr(arr("outlier_centroids.weight", cb)), _ptr(arr("outlier_indices", np.int32)),
                                    _ptr(arr("weight_scale", cb)), _ptr(arr("weight_bias", cb)),
                                    _ptr(arr("perm", np.int32)), out_dtype, _ptr(out))
    return rc, out
