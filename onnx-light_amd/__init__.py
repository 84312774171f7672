"""Python front end of the MI355X quantized-matmul kernels.

Mirrors the onnx-light reference kernel classes for this path
(``kernel::MatMulInteger``, ``kernel::QLinearMatMul``,
``kernel::DequantizeLinear``, ``kernel::MatMul``) with the same argument
meaning and error behaviour: validation failures raise :class:`InvalidArgument`
(a ``ValueError``, the reference raises ``std::invalid_argument``) with the
reference's message text.  Every call goes through the C ABI of
``libonnxl_amd.so`` (``include/onnxl_amd.h``); there is no CPU fallback: if the
library is missing, :func:`lib` raises.

Tensors are ``torch.Tensor`` objects (CUDA tensors are used in place, CPU
tensors are staged by the library) or numpy arrays (host).  4-bit tensors are
passed as packed ``uint8`` storage together with ``dtype=INT4/UINT4`` and the
logical ``shape``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libonnxl_amd.so")
MAX_RANK = 8

# ONNX TensorProto.DataType codes.
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64 = 1, 2, 3, 4, 5, 6, 7
FLOAT16, DOUBLE, BFLOAT16, FLOAT8E4M3FN, UINT4, INT4 = 10, 11, 16, 17, 21, 22

OK, INVALID_ARGUMENT, UNSUPPORTED, DEVICE_ERROR, NOT_INITIALIZED = 0, 1, 2, 3, 4
DEVICE, HOST = 0, 1
LAYOUT_ONNX, LAYOUT_TILED_INT4 = 0, 1


class InvalidArgument(ValueError):
    """The reference kernel would raise std::invalid_argument."""


class Unsupported(NotImplementedError):
    """Valid for the reference, but this input has no GPU kernel."""


class DeviceError(RuntimeError):
    """HIP runtime failure, or the library was not initialised."""


class Tensor(ctypes.Structure):
    """onnxl_amd_tensor (include/onnxl_amd.h)."""
    _fields_ = [("data_type", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("dims", ctypes.c_int64 * MAX_RANK), ("data", ctypes.c_void_p),
                ("size_bytes", ctypes.c_int64), ("location", ctypes.c_int32),
                ("layout", ctypes.c_int32)]


TP = ctypes.POINTER(Tensor)
_lib = None


def build() -> str:
    """Compiles libonnxl_amd.so in place (hipcc, gfx950)."""
    subprocess.run(["make", "-s", "-C", HERE, "-j8"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded C ABI library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run onnx_light_amd.build() (make -C onnx-light_amd)")
        L = ctypes.CDLL(LIB_PATH)
        L.onnxl_amd_init.argtypes = [ctypes.c_int]
        L.onnxl_amd_shutdown.argtypes = []
        L.onnxl_amd_last_error.restype = ctypes.c_char_p
        L.onnxl_amd_version.restype = ctypes.c_char_p
        L.onnxl_amd_matmul_shape.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                             ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                             ctypes.POINTER(ctypes.c_int64),
                                             ctypes.POINTER(ctypes.c_int32)]
        L.onnxl_amd_matmul_integer.argtypes = [TP, TP, TP, TP, TP, ctypes.c_void_p]
        L.onnxl_amd_qlinear_matmul.argtypes = [TP] * 9 + [ctypes.c_void_p]
        L.onnxl_amd_dequantize_linear.argtypes = [TP, TP, TP, ctypes.c_int64, TP, ctypes.c_void_p]
        L.onnxl_amd_matmul.argtypes = [TP, TP, TP, ctypes.c_void_p]
        L.onnxl_amd_cast.argtypes = [TP, ctypes.c_int32, TP, ctypes.c_void_p]
        L.onnxl_amd_grouped_matmul.argtypes = [TP, TP, TP, TP, ctypes.c_int64, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_linear_grouped_matmul.argtypes = [TP, TP, TP, TP, ctypes.c_int64, ctypes.c_int32,
                                                                 TP, TP, ctypes.c_int64, TP, ctypes.c_void_p]
        I64 = ctypes.c_int64
        L.onnxl_amd_prepare_matmul_nbits_size.argtypes = [I64, I64, I64, I64, ctypes.c_int, ctypes.POINTER(I64),
                                                          ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.onnxl_amd_prepare_matmul_nbits.argtypes = [TP, TP, TP, I64, I64, I64, I64, ctypes.POINTER(Tensor),
                                                     ctypes.POINTER(Tensor), ctypes.POINTER(Tensor), ctypes.c_void_p]
        PT = ctypes.POINTER(Tensor)
        I32 = ctypes.c_int32
        CS = ctypes.c_char_p
        L.onnxl_amd_prepare_awq_size.argtypes = [CS, I64, I64, I64, I64, I32, ctypes.POINTER(I64),
                                                 ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.onnxl_amd_prepare_awq.argtypes = [CS, TP, TP, TP, I64, I64, I64, I64, PT, PT, PT, ctypes.c_void_p]
        L.onnxl_amd_dequantize_awq.argtypes = [CS, TP, TP, TP, I64, I64, I64, I64, TP, ctypes.c_void_p]
        L.onnxl_amd_prepare_gptq_size.argtypes = [CS, I64, I64, I64, I64, I32, I32, ctypes.POINTER(I64),
                                                  ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.onnxl_amd_prepare_gptq.argtypes = [CS, TP, TP, TP, TP, I64, I64, I64, I64, PT, PT, PT, ctypes.c_void_p]
        L.onnxl_amd_dequantize_gptq.argtypes = [CS, TP, TP, TP, TP, I64, I64, I64, I64, TP, ctypes.c_void_p]
        F32 = ctypes.c_float
        L.onnxl_amd_dequantize_bitsandbytes.argtypes = [I32, I64, I64, I64, I64, F32, TP, TP, TP, TP, TP, TP,
                                                        ctypes.c_void_p]
        L.onnxl_amd_prepare_bitsandbytes_size.argtypes = [I32, I64, I64, I64, ctypes.POINTER(I64)]
        L.onnxl_amd_prepare_bitsandbytes.argtypes = [I32, I64, I64, I64, I64, F32, TP, TP, TP, TP, TP, I32, PT,
                                                     ctypes.c_void_p]
        L.onnxl_amd_bitsandbytes_matmul.argtypes = [TP, I32, I64, I64, I64, TP, TP, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_qqq.argtypes = [I64, I64, I64, I64, TP, TP, TP, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_gptqmodel_fp8.argtypes = [I64, I64, CS, ctypes.POINTER(I64), I32, TP, TP, TP,
                                                         ctypes.c_void_p]
        L.onnxl_amd_transpose_2d.argtypes = [TP, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_exl3.argtypes = [TP, TP, TP, TP, TP, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_mx_weights.argtypes = [CS, TP, TP, F32, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_vptq.argtypes = [ctypes.POINTER(VptqConfig), TP, TP, TP, TP, TP, TP, TP, TP, TP,
                                                ctypes.c_void_p]
        L.onnxl_amd_dequantize_bitblas.argtypes = [CS, TP, TP, TP, I64, I64, I64, I64, I32, TP, ctypes.c_void_p]
        L.onnxl_amd_prepare_bitblas_size.argtypes = [CS, I64, I64, I64, I64, I32, ctypes.POINTER(I64),
                                                     ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.onnxl_amd_prepare_bitblas.argtypes = [CS, TP, TP, TP, I64, I64, I64, I64, I32, PT, PT, PT,
                                                ctypes.c_void_p]
        L.onnxl_amd_prepare_qqq_size.argtypes = [I64, I64, I64, I64, ctypes.POINTER(I64), ctypes.POINTER(I64)]
        L.onnxl_amd_prepare_qqq.argtypes = [I64, I64, I64, I64, TP, TP, TP, I32, PT, PT, ctypes.c_void_p]
        L.onnxl_amd_dequantize_linear_matmul.argtypes = [TP, TP, TP, TP, ctypes.c_int64,
                                                         ctypes.c_int32, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_linear_matmul_noalloc.argtypes = [TP, TP, TP, TP, ctypes.c_int64,
                                                                 ctypes.c_int32, TP, ctypes.c_void_p]
        L.onnxl_amd_quantize_linear.argtypes = [TP, TP, TP, ctypes.c_int64, ctypes.c_int32, TP,
                                                ctypes.c_void_p]
        L.onnxl_amd_dynamic_quantize_linear.argtypes = [TP, TP, TP, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_packed.argtypes = [TP, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                                                  ctypes.c_int32, ctypes.c_int64, TP, ctypes.c_void_p]
        L.onnxl_amd_dequantize_packed_matmul.argtypes = [TP, TP, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                                                         ctypes.c_int32, TP, ctypes.c_void_p]
        CA = ctypes.POINTER(ConvAttrs)
        L.onnxl_amd_conv_shape.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                           ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, CA,
                                           ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32)]
        L.onnxl_amd_conv_integer.argtypes = [TP, TP, TP, TP, CA, TP, ctypes.c_void_p]
        L.onnxl_amd_qlinear_conv.argtypes = [TP] * 9 + [CA, TP, ctypes.c_void_p]
        L.onnxl_amd_prepare_weight_size.argtypes = [TP, ctypes.POINTER(ctypes.c_int64)]
        L.onnxl_amd_prepare_weight.argtypes = [TP, TP, ctypes.c_void_p]
        L.onnxl_amd_synchronize.argtypes = [ctypes.c_void_p]
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc == OK:
        return
    msg = lib().onnxl_amd_last_error().decode(errors="replace")
    if rc == INVALID_ARGUMENT:
        raise InvalidArgument(msg)
    if rc == UNSUPPORTED:
        raise Unsupported(msg)
    raise DeviceError(f"status {rc}: {msg}")


def init(device: int = 0) -> None:
    _check(lib().onnxl_amd_init(device))


def shutdown() -> None:
    _check(lib().onnxl_amd_shutdown())


def synchronize(stream=None) -> None:
    _check(lib().onnxl_amd_synchronize(stream))


# ---- descriptors ------------------------------------------------------------

def _torch():
    import torch
    return torch


_TORCH_CODES = None


def _torch_code(dt):
    global _TORCH_CODES
    if _TORCH_CODES is None:
        torch = _torch()
        _TORCH_CODES = {torch.float32: FLOAT, torch.uint8: UINT8, torch.int8: INT8,
                        torch.int16: INT16, torch.int32: INT32, torch.int64: INT64,
                        torch.float16: FLOAT16, torch.float64: DOUBLE, torch.bfloat16: BFLOAT16,
                        torch.float8_e4m3fn: FLOAT8E4M3FN, torch.uint16: UINT16}
    return _TORCH_CODES[dt]


_NP_CODES = {np.dtype(np.float32): FLOAT, np.dtype(np.uint8): UINT8, np.dtype(np.int8): INT8,
             np.dtype(np.uint16): UINT16, np.dtype(np.int16): INT16, np.dtype(np.int32): INT32,
             np.dtype(np.int64): INT64, np.dtype(np.float16): FLOAT16, np.dtype(np.float64): DOUBLE}


def describe(t, dtype: int | None = None, shape=None) -> Tensor:
    """Builds an onnxl_amd_tensor for a torch tensor / numpy array / None.

    ``dtype`` overrides the element type (4-bit types, FLOAT16 bits held in
    uint16 arrays, ...); ``shape`` overrides the logical shape."""
    if isinstance(t, PreparedWeight):
        return t.desc
    d = Tensor()
    if t is None:
        d.rank = -1
        return d
    if isinstance(t, np.ndarray):
        arr = t if t.flags["C_CONTIGUOUS"] else np.ascontiguousarray(t).reshape(t.shape)
        d.data_type = dtype if dtype is not None else _NP_CODES[arr.dtype]
        d.data = arr.ctypes.data if arr.nbytes else None
        d.size_bytes = arr.nbytes
        d.location = HOST
        d._keep = arr
        shp = arr.shape if shape is None else tuple(shape)
    else:
        torch = _torch()
        if not t.is_contiguous():
            raise InvalidArgument("tensors passed to the C ABI must be contiguous")
        d.data_type = dtype if dtype is not None else _torch_code(t.dtype)
        d.data = t.data_ptr() if t.numel() else None
        d.size_bytes = t.numel() * t.element_size()
        d.location = DEVICE if t.is_cuda else HOST
        d._keep = t
        shp = tuple(t.shape) if shape is None else tuple(shape)
        del torch
    if len(shp) > MAX_RANK:
        raise InvalidArgument(f"rank {len(shp)} above {MAX_RANK}")
    d.rank = len(shp)
    for i, s in enumerate(shp):
        d.dims[i] = int(s)
    return d


class PreparedWeight:
    """A constant INT4 / UINT4 weight in the tiled device layout written by
    onnxl_amd_prepare_weight: `storage` holds the bytes, `desc` the descriptor
    (layout LAYOUT_TILED_INT4) that stands for the weight in later calls."""

    def __init__(self, storage, desc: Tensor):
        self.storage = storage
        self.desc = desc
        self.shape = tuple(desc.dims[i] for i in range(desc.rank))
        self.is_cuda = True
        self.device = storage.device


def prepare_weight(x, x_dtype: int, x_shape=None) -> PreparedWeight:
    """Session-time preparation of a constant 4-bit weight x [K, N] (packed
    uint8 storage in the ONNX layout) for dequantize_linear_matmul."""
    torch = _torch()
    d = describe(x, x_dtype, _shape_of(x, x_shape))
    n = ctypes.c_int64(0)
    _check(lib().onnxl_amd_prepare_weight_size(ctypes.byref(d), ctypes.byref(n)))
    dev = x.device if (not isinstance(x, np.ndarray) and x.is_cuda) else torch.device("cuda", torch.cuda.current_device())
    storage = torch.empty(max(n.value, 1), dtype=torch.uint8, device=dev)
    out = describe(storage)
    _check(lib().onnxl_amd_prepare_weight(ctypes.byref(d), ctypes.byref(out),
                                          ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    out._keep = storage
    return PreparedWeight(storage, out)


class PreparedNbits:
    """A packed-checkpoint weight prepared for the fused DequantizeLinear ->
    MatMul kernels (onnxl_amd_prepare_matmul_nbits / _awq / _gptq): weight,
    scale and zero point (None without zero points), each a PreparedWeight
    (device storage + descriptor)."""

    def __init__(self, weight, scale, zero_point, K, N):
        self.weight, self.scale, self.zero_point = weight, scale, zero_point
        self.shape = (K, N)


def prepare_matmul_nbits(B, scales, zero_points, K: int, N: int, bits: int, block_size: int) -> PreparedNbits:
    """Session-time preparation of an ORT MatMulNBits weight: B uint8 [N,
    groups, block_size * bits / 8], scales FLOAT16 [N, groups], zero_points
    None or packed uint8 codes [N, ceil(groups * bits / 8)]."""
    torch = _torch()
    has_zp = zero_points is not None
    wb, sb, zb = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
    _check(lib().onnxl_amd_prepare_matmul_nbits_size(K, N, bits, block_size, int(has_zp), ctypes.byref(wb),
                                                      ctypes.byref(sb), ctypes.byref(zb)))
    dev = torch.device("cuda", torch.cuda.current_device())
    bufs = [torch.empty(max(n.value, 16), dtype=torch.uint8, device=dev) for n in (wb, sb, zb)]
    descs = [describe(b) for b in bufs]
    _check(lib().onnxl_amd_prepare_matmul_nbits(describe(B), describe(scales, FLOAT16), describe(zero_points), K, N,
                                                bits, block_size, ctypes.byref(descs[0]), ctypes.byref(descs[1]),
                                                ctypes.byref(descs[2]),
                                                ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    for d, b in zip(descs, bufs):
        d._keep = b
    zp = PreparedWeight(bufs[2], descs[2]) if has_zp else None
    return PreparedNbits(PreparedWeight(bufs[0], descs[0]), PreparedWeight(bufs[1], descs[1]), zp, K, N)


def matmul_nbits(a, prepared: PreparedNbits, out=None):
    """MatMul(a, W) for a prepared weight W [K, N] through the fused
    DequantizeLinear -> MatMul entry point (blocked scales, axis 0); FLOAT
    scales take a Cast to a's dtype."""
    cast_to = _torch_code(a.dtype) if prepared.scale.desc.data_type == FLOAT else 0
    return dequantize_linear_matmul(a, prepared.weight, prepared.scale, prepared.zero_point, 0, cast_to,
                                    x_shape=prepared.shape, out=out)


def _prepared_triplet(sizes, run) -> tuple:
    torch = _torch()
    dev = torch.device("cuda", torch.cuda.current_device())
    bufs = [torch.empty(max(n.value, 16), dtype=torch.uint8, device=dev) for n in sizes]
    descs = [describe(b) for b in bufs]
    _check(run(*(ctypes.byref(d) for d in descs), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    for d, b in zip(descs, bufs):
        d._keep = b
    return tuple(PreparedWeight(b, d) for b, d in zip(bufs, descs))


def _scale_code(scales) -> int:
    if isinstance(scales, np.ndarray) and scales.dtype == np.uint16:
        raise InvalidArgument("pass FLOAT16 / BFLOAT16 scales as float16 arrays or torch tensors")
    return _NP_CODES[scales.dtype] if isinstance(scales, np.ndarray) else _torch_code(scales.dtype)


def prepare_awq(variant: str, qweight, qzeros, scales, K: int, N: int, group_size: int, bits: int = 4) -> PreparedNbits:
    """onnxl_amd_prepare_awq: an AWQ checkpoint (awq.cc layouts) as the fused
    kernels' UINT4 / UINT8 weight, zero points and scales."""
    sizes = [ctypes.c_int64(0) for _ in range(3)]
    _check(lib().onnxl_amd_prepare_awq_size(variant.encode(), K, N, bits, group_size, _scale_code(scales),
                                            *(ctypes.byref(x) for x in sizes)))
    w, s, z = _prepared_triplet(sizes, lambda pw, ps, pz, st: lib().onnxl_amd_prepare_awq(
        variant.encode(), describe(qweight), describe(qzeros), describe(scales), K, N, bits, group_size, pw, ps, pz,
        st))
    return PreparedNbits(w, s, z, K, N)


def prepare_gptq(fmt: str, qweight, qzeros, scales, g_idx, K: int, N: int, bits: int,
                 group_size: int) -> PreparedNbits:
    """onnxl_amd_prepare_gptq: a GPTQ checkpoint (gptq.cc layouts) as the
    fused kernels' UINT4 / UINT8 weight, zero points and scales."""
    sizes = [ctypes.c_int64(0) for _ in range(3)]
    word = _NP_CODES[qweight.dtype] if isinstance(qweight, np.ndarray) else _torch_code(qweight.dtype)
    _check(lib().onnxl_amd_prepare_gptq_size(fmt.encode(), K, N, bits, group_size, word, _scale_code(scales),
                                             *(ctypes.byref(x) for x in sizes)))
    w, s, z = _prepared_triplet(sizes, lambda pw, ps, pz, st: lib().onnxl_amd_prepare_gptq(
        fmt.encode(), describe(qweight), describe(qzeros), describe(scales), describe(g_idx), K, N, bits,
        group_size, pw, ps, pz, st))
    return PreparedNbits(w, s, z, K, N)



def _decode_out(K, N, output_dtype, like, out):
    torch = _torch()
    if out is None:
        tdt = {FLOAT: torch.float32, FLOAT16: torch.float16, BFLOAT16: torch.bfloat16,
               DOUBLE: torch.float64}.get(output_dtype, torch.float32)
        out = _empty((N, K), tdt, _device_of(*like))
    return out


def dequantize_awq(variant: str, qweight, qzeros, scales, K: int, N: int, group_size: int, bits: int = 4,
                   output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_awq: the AWQ weight as [N, K] values."""
    out = _decode_out(K, N, output_dtype, (qweight, qzeros, scales), out)
    _check(lib().onnxl_amd_dequantize_awq(variant.encode(), describe(qweight), describe(qzeros), describe(scales),
                                          K, N, bits, group_size, describe(out),
                                          _stream_of(qweight, qzeros, scales, out)))
    return out


BNB_FORMATS = {"nf4": 0, "fp4": 1, "int8": 2}
# bitsandbytes' nf4 table (the canonical weight_quant_map), float32
BNB_NF4_TABLE = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                          -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                          0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
                          0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], np.float32)


class BnbWeight:
    """A bitsandbytes weight (bitsandbytes.cc) of logical shape [rows, cols]
    = [out_features, in_features]: the tensors of its checkpoint and the
    numbers of its quant state.  fmt "nf4" / "fp4": weight uint8 packed codes,
    absmax float32 [blocks] (or uint8 codes with nested_absmax and
    nested_quant_map, nested_block 256, nested_offset), quant_map float32
    [16]; "int8": weight int8 [rows, cols], absmax the row maxima
    (weight_scb)."""

    def __init__(self, fmt, rows, cols, weight, absmax, quant_map=None, block=0, nested_absmax=None,
                 nested_quant_map=None, nested_block=0, nested_offset=0.0):
        self.fmt, self.rows, self.cols, self.block = fmt, rows, cols, block
        self.weight, self.absmax, self.quant_map = weight, absmax, quant_map
        self.nested_absmax, self.nested_quant_map = nested_absmax, nested_quant_map
        self.nested_block, self.nested_offset = nested_block, nested_offset
        self.scales = None  # set by prepare_bitsandbytes

    def args(self):
        code = UINT8 if self.fmt != "int8" else INT8
        return (BNB_FORMATS[self.fmt], self.rows, self.cols, self.block, self.nested_block,
                ctypes.c_float(self.nested_offset), describe(self.weight, code), describe(self.absmax),
                describe(self.quant_map), describe(self.nested_absmax), describe(self.nested_quant_map))

    def tensors(self):
        return (self.weight, self.absmax, self.quant_map, self.nested_absmax, self.nested_quant_map)


def dequantize_bitsandbytes(w: BnbWeight, output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_bitsandbytes: the weight as [rows, cols] values."""
    out = _decode_out(w.cols, w.rows, output_dtype, w.tensors(), out)
    _check(lib().onnxl_amd_dequantize_bitsandbytes(*w.args(), describe(out), _stream_of(*w.tensors(), out)))
    return out


def prepare_bitsandbytes(w: BnbWeight, reconstruction_dtype: int = FLOAT16) -> BnbWeight:
    """onnxl_amd_prepare_bitsandbytes: the checks and the resolved per-block
    scales (device float32), kept on w for bitsandbytes_matmul."""
    torch = _torch()
    n = ctypes.c_int64(0)
    _check(lib().onnxl_amd_prepare_bitsandbytes_size(BNB_FORMATS[w.fmt], w.rows, w.cols, w.block, ctypes.byref(n)))
    dev = torch.device("cuda", torch.cuda.current_device())
    storage = torch.empty(max(n.value // 4, 4), dtype=torch.float32, device=dev)
    d = describe(storage)
    _check(lib().onnxl_amd_prepare_bitsandbytes(*w.args(), reconstruction_dtype, ctypes.byref(d),
                                                ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    w.scales = storage[: n.value // 4]
    return w


def bitsandbytes_matmul(a, w: BnbWeight, out=None):
    """onnxl_amd_bitsandbytes_matmul: MatMul(a, Transpose(Dequantize(w)))
    with w prepared for a's dtype."""
    if w.scales is None:
        raise InvalidArgument("bitsandbytes_matmul: prepare_bitsandbytes the weight first")
    if out is None:
        out = _empty(tuple(a.shape[:-1]) + (w.rows,), a.dtype, _device_of(a))
    code = UINT8 if w.fmt != "int8" else INT8
    _check(lib().onnxl_amd_bitsandbytes_matmul(describe(a), BNB_FORMATS[w.fmt], w.rows, w.cols, w.block,
                                               describe(w.weight, code), describe(w.scales), describe(out),
                                               _stream_of(a, w.weight, out)))
    return out


class VptqConfig(ctypes.Structure):
    """onnxl_amd_vptq_config: the VPTQ constructor metadata the layout uses."""
    _fields_ = [("in_features", ctypes.c_int64), ("out_features", ctypes.c_int64), ("bits", ctypes.c_int64),
                ("vector_lens", ctypes.c_int64 * 2), ("num_centroids", ctypes.c_int64 * 2),
                ("num_res_centroids", ctypes.c_int64 * 2), ("npercent", ctypes.c_double),
                ("group_size", ctypes.c_int64), ("group_num", ctypes.c_int64), ("enable_norm", ctypes.c_int32),
                ("norm_dim", ctypes.c_int32), ("enable_perm", ctypes.c_int32)]

    @classmethod
    def of(cls, params: dict, bits: int = 4):
        c = cls()
        c.in_features, c.out_features, c.bits = params["in_features"], params["out_features"], bits
        for name in ("vector_lens", "num_centroids", "num_res_centroids"):
            getattr(c, name)[0], getattr(c, name)[1] = params[name]
        c.npercent = params["npercent"]
        c.group_size, c.group_num = params["group_size"], params["group_num"]
        c.enable_norm, c.norm_dim = int(params["enable_norm"]), params["norm_dim"]
        c.enable_perm = int(params["enable_perm"])
        return c


VPTQ_TENSORS = ("indices", "centroids.weight", "res_centroids.weight", "outlier_centroids.weight",
                "outlier_indices", "weight_scale", "weight_bias", "perm")


def dequantize_vptq(config: VptqConfig, tensors: dict, codebook_dtype: int, output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_vptq: a VPTQ weight (tensors by the checkpoint's
    names; BFLOAT16 / FLOAT16 codebooks may be uint16 bit patterns, typed by
    codebook_dtype) as [out_features, in_features] values."""
    out = _decode_out(config.in_features, config.out_features, output_dtype, tuple(tensors.values()), out)
    cb = {"centroids.weight", "res_centroids.weight", "outlier_centroids.weight", "weight_scale", "weight_bias"}
    descs = [describe(tensors.get(n), codebook_dtype if n in cb and tensors.get(n) is not None else None)
             for n in VPTQ_TENSORS]
    _check(lib().onnxl_amd_dequantize_vptq(ctypes.byref(config), *descs, describe(out),
                                           _stream_of(*tensors.values(), out)))
    return out


def dequantize_gptqmodel_fp8(weight, weight_scale_inv, method: str, block=(), code: int | None = None,
                             output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_gptqmodel_fp8: FP8 codes [N, K] (`code` the FP8
    data_type when `weight` holds raw uint8 bytes) over FLOAT inverse scales
    (method "tensor", "row" or "block" with block (b0, b1)) as [N, K]."""
    n, k = _shape_of(weight)
    out = _decode_out(k, n, output_dtype, (weight, weight_scale_inv), out)
    blk = (ctypes.c_int64 * 2)(*block) if block else None
    _check(lib().onnxl_amd_dequantize_gptqmodel_fp8(k, n, method.encode(), blk, len(block),
                                                    describe(weight, code), describe(weight_scale_inv),
                                                    describe(out), _stream_of(weight, weight_scale_inv, out)))
    return out


def transpose_2d(x, out=None):
    """onnxl_amd_transpose_2d: Transpose(x, perm=[1, 0]) of a 2-D tensor."""
    torch = _torch()
    if out is None:
        dt = torch.from_numpy(x[:0]).dtype if isinstance(x, np.ndarray) else x.dtype
        out = _empty(tuple(x.shape)[::-1], dt, _device_of(x))
    _check(lib().onnxl_amd_transpose_2d(describe(x), describe(out), _stream_of(x, out)))
    return out


def dequantize_exl3(trellis, suh, svh, mcg=None, mul1=None, output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_exl3: an EXL3 weight (trellis int16 [k / 16,
    n / 16, 16 * bits], suh / svh float16 [k] / [n], the optional int32
    codebook marker mcg or mul1) as [k, n] values."""
    d0, d1, _ = _shape_of(trellis)
    out = _decode_out(d1 * 16, d0 * 16, output_dtype, (trellis, suh, svh), out)
    _check(lib().onnxl_amd_dequantize_exl3(describe(trellis), describe(suh), describe(svh), describe(mcg),
                                           describe(mul1), describe(out), _stream_of(trellis, suh, svh, out)))
    return out


MX_FORMATS = ("mxfp4", "mxfp6_e2m3", "mxfp8", "nvfp4")


def dequantize_mx_weights(fmt: str, weight, weight_scale, global_scale: float = 0.0, code: int | None = None,
                          scale_code: int | None = None, output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_mx_weights: an MX / NVFP4 weight (`fmt` one of
    MX_FORMATS; `code` / `scale_code` the data_types when the tensors hold raw
    uint8 bytes: FLOAT8E4M3FN for the mxfp8 weight and the nvfp4 scales) as
    [rows, cols] values."""
    rows, wcols = _shape_of(weight)
    cols = wcols if fmt == "mxfp8" else (wcols // 3 * 4 if fmt == "mxfp6_e2m3" else wcols * 2)
    out = _decode_out(cols, rows, output_dtype, (weight, weight_scale), out)
    _check(lib().onnxl_amd_dequantize_mx_weights(fmt.encode(), describe(weight, code),
                                                 describe(weight_scale, scale_code), float(global_scale),
                                                 describe(out), _stream_of(weight, weight_scale, out)))
    return out


def dequantize_bitblas(method: str, qweight, scales, qzeros, K: int, N: int, bits: int, group_size: int,
                       symmetric: bool = False, output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_bitblas: a BitBLAS row-packed weight (bitblas.cc;
    qweight int8 [N, K * bits / 8], scales float16 [N, groups], qzeros int8
    [groups, N * bits / 8] or None for symmetric GPTQ) as [N, K] values."""
    out = _decode_out(K, N, output_dtype, (qweight, scales), out)
    _check(lib().onnxl_amd_dequantize_bitblas(method.encode(), describe(qweight), describe(scales), describe(qzeros),
                                              K, N, bits, group_size, int(symmetric), describe(out),
                                              _stream_of(qweight, scales, out)))
    return out


def prepare_bitblas(method: str, qweight, scales, qzeros, K: int, N: int, bits: int, group_size: int,
                    symmetric: bool = False) -> PreparedNbits:
    """onnxl_amd_prepare_bitblas: the fused kernels' UINT4 / UINT8 weight,
    zero points and FLOAT16 scales (matmul_nbits multiplies with them)."""
    sizes = [ctypes.c_int64(0) for _ in range(3)]
    _check(lib().onnxl_amd_prepare_bitblas_size(method.encode(), K, N, bits, group_size, int(symmetric),
                                                *(ctypes.byref(x) for x in sizes)))
    w, s, z = _prepared_triplet(sizes, lambda pw, ps, pz, st: lib().onnxl_amd_prepare_bitblas(
        method.encode(), describe(qweight), describe(scales), describe(qzeros), K, N, bits, group_size,
        int(symmetric), pw, ps, pz, st))
    return PreparedNbits(w, s, z, K, N)


def dequantize_qqq(k: int, n: int, group_size: int, B, s_channel, s_group=None, output_dtype: int = FLOAT,
                   out=None, bits: int = 4):
    """onnxl_amd_dequantize_qqq: a QQQ weight (qqq.cc: in_features k,
    out_features n, B int32 [k / 16, 2n], s_channel float32 [1, n], s_group
    float16 [k / 128, n] or None) as [n, k] values."""
    out = _decode_out(k, n, output_dtype, (B, s_channel), out)
    _check(lib().onnxl_amd_dequantize_qqq(k, n, group_size, bits, describe(B), describe(s_channel),
                                          describe(s_group), describe(out), _stream_of(B, s_channel, out)))
    return out


def prepare_qqq(k: int, n: int, group_size: int, B, s_channel, s_group=None, dtype: int = FLOAT16,
                bits: int = 4) -> PreparedNbits:
    """onnxl_amd_prepare_qqq: the fused kernels' weight (tiled INT4 per
    channel, INT8 grouped) and FLOAT per-column scale, after the format's
    checks in `dtype`; qqq_matmul multiplies with it."""
    sizes = [ctypes.c_int64(0) for _ in range(2)]
    _check(lib().onnxl_amd_prepare_qqq_size(k, n, group_size, bits, *(ctypes.byref(x) for x in sizes)))
    w, s = _prepared_triplet(sizes, lambda pw, ps, st: lib().onnxl_amd_prepare_qqq(
        k, n, group_size, bits, describe(B), describe(s_channel), describe(s_group), dtype, pw, ps, st))
    return PreparedNbits(w, s, None, k, n)


def qqq_matmul(a, prepared: PreparedNbits, out=None):
    """MatMul(a, Transpose(Dequantize(Q, dtype = a's dtype))) for a QQQ weight
    prepared by prepare_qqq: the fused DequantizeLinear -> Cast -> MatMul
    entry point with the per-column scale (axis 1)."""
    return dequantize_linear_matmul(a, prepared.weight, prepared.scale, None, 1, _torch_code(a.dtype),
                                    x_shape=prepared.shape, out=out)


def dequantize_gptq(fmt: str, qweight, qzeros, scales, g_idx, K: int, N: int, bits: int, group_size: int,
                    output_dtype: int = FLOAT, out=None):
    """onnxl_amd_dequantize_gptq: the GPTQ weight as [N, K] values."""
    out = _decode_out(K, N, output_dtype, (qweight, qzeros, scales, g_idx), out)
    _check(lib().onnxl_amd_dequantize_gptq(fmt.encode(), describe(qweight), describe(qzeros), describe(scales),
                                           describe(g_idx), K, N, bits, group_size, describe(out),
                                           _stream_of(qweight, qzeros, scales, g_idx, out)))
    return out


class ConvAttrs(ctypes.Structure):
    """onnxl_amd_conv_attrs: the reference's Attributes of ConvInteger /
    QLinearConv (empty lists are the absent attributes)."""
    _fields_ = [("n_kernel_shape", ctypes.c_int32), ("n_strides", ctypes.c_int32),
                ("n_pads", ctypes.c_int32), ("n_dilations", ctypes.c_int32),
                ("kernel_shape", ctypes.c_int64 * 3), ("strides", ctypes.c_int64 * 3),
                ("pads", ctypes.c_int64 * 6), ("dilations", ctypes.c_int64 * 3),
                ("group", ctypes.c_int64), ("auto_pad", ctypes.c_int32)]


AUTO_PAD = {"NOTSET": 0, "SAME_UPPER": 1, "SAME_LOWER": 2, "VALID": 3}


def conv_attrs(kernel_shape=None, strides=None, pads=None, dilations=None, group=1,
               auto_pad="NOTSET") -> ConvAttrs:
    a = ConvAttrs()
    for name, vals, cap in (("kernel_shape", kernel_shape, 3), ("strides", strides, 3),
                            ("pads", pads, 6), ("dilations", dilations, 3)):
        vals = list(vals or [])
        if len(vals) > cap:
            raise Unsupported(f"'{name}' with {len(vals)} entries: at most 3 spatial dimensions")
        setattr(a, "n_" + name, len(vals))
        arr = getattr(a, name)
        for i, v in enumerate(vals):
            arr[i] = int(v)
    a.group = int(group)
    a.auto_pad = AUTO_PAD[auto_pad] if isinstance(auto_pad, str) else int(auto_pad)
    return a


def _stream_of(*ts):
    for t in ts:
        if isinstance(t, PreparedWeight):
            continue
        if t is not None and not isinstance(t, np.ndarray) and t.is_cuda:
            return ctypes.c_void_p(_torch().cuda.current_stream(t.device).cuda_stream)
    return None


def _device_of(*ts):
    for t in ts:
        if isinstance(t, PreparedWeight):
            return t.device
        if t is not None and not isinstance(t, np.ndarray) and t.is_cuda:
            return t.device
    return "cpu"


def _describe_zp(zp, x_dtype, x_scale):
    """Zero point descriptor: sub-byte zero points (4-, 2- and 6-bit types)
    are packed storage whose logical shape is the scale's shape."""
    if zp is None:
        return describe(None)
    if x_dtype in (INT4, UINT4, 23, 25, 26, 27, 28):
        return describe(zp, x_dtype, tuple(x_scale.shape))
    return describe(zp, x_dtype)


def matmul_shape(a_shape, b_shape) -> tuple:
    a = (ctypes.c_int64 * MAX_RANK)(*a_shape)
    b = (ctypes.c_int64 * MAX_RANK)(*b_shape)
    out = (ctypes.c_int64 * MAX_RANK)()
    r = ctypes.c_int32(0)
    _check(lib().onnxl_amd_matmul_shape(a, len(a_shape), b, len(b_shape), out,
                                        ctypes.byref(r)))
    return tuple(out[i] for i in range(r.value))


def _shape_of(t, shape=None):
    return tuple(shape) if shape is not None else tuple(t.shape)


def _empty(shape, torch_dtype, device):
    return _torch().empty(shape, dtype=torch_dtype, device=device)


# ---- kernels (reference operator() overloads) ------------------------------

def matmul_integer(a, b, a_zero_point=None, b_zero_point=None, out=None):
    """kernel::MatMulInteger (km/kernel_matmul_integer.cc:212-234)."""
    torch = _torch()
    if out is None:
        out = _empty(matmul_shape(_shape_of(a), _shape_of(b)), torch.int32, _device_of(a, b))
    da, db = describe(a), describe(b)
    dza, dzb, dy = describe(a_zero_point), describe(b_zero_point), describe(out)
    _check(lib().onnxl_amd_matmul_integer(da, db, dza, dzb, dy, _stream_of(a, b, out)))
    return out


def qlinear_matmul(a, a_scale, a_zero_point, b, b_scale, b_zero_point, y_scale, y_zero_point,
                   out=None):
    """kernel::QLinearMatMul (kq/kernel_qlinearmatmul.cc:221-267); output dtype
    follows y_zero_point."""
    torch = _torch()
    if out is None:
        ydt = y_zero_point.dtype
        if isinstance(y_zero_point, np.ndarray):
            ydt = torch.int8 if ydt == np.int8 else torch.uint8
        out = _empty(matmul_shape(_shape_of(a), _shape_of(b)), ydt, _device_of(a, b))
    ds = [describe(t) for t in (a, a_scale, a_zero_point, b, b_scale, b_zero_point, y_scale,
                                y_zero_point, out)]
    _check(lib().onnxl_amd_qlinear_matmul(*ds, _stream_of(a, b, out)))
    return out


def dequantize_linear(x, x_scale, x_zero_point=None, axis: int = 1, x_dtype=None, x_shape=None,
                      out=None):
    """kernel::DequantizeLinear (kq/kernel_dequantizelinear.cc:332-693); the
    output dtype follows x_scale (FLOAT or FLOAT16)."""
    torch = _torch()
    shape = _shape_of(x, x_shape)
    if out is None:
        odt = x_scale.dtype
        if isinstance(x_scale, np.ndarray):
            odt = torch.float16 if x_scale.dtype == np.float16 else torch.float32
        out = _empty(shape, odt, _device_of(x))
    dx = describe(x, x_dtype, shape)
    dz = _describe_zp(x_zero_point, x_dtype, x_scale)
    _check(lib().onnxl_amd_dequantize_linear(dx, describe(x_scale), dz, axis, describe(out),
                                             _stream_of(x, out)))
    return out


def matmul(a, b, out=None):
    """kernel::MatMul for FLOAT16 / BFLOAT16 (km/kernel_matmul.cc:181-258)."""
    if out is None:
        out = _empty(matmul_shape(_shape_of(a), _shape_of(b)), a.dtype, _device_of(a, b))
    _check(lib().onnxl_amd_matmul(describe(a), describe(b), describe(out), _stream_of(a, b, out)))
    return out


def grouped_matmul(input, weights, group_indices, bias=None, transB: int = 0, out=None, check: bool = True):
    """kernel::GroupedMatMul (math/kernel_grouped_matmul.cc:48-103) for FLOAT16
    / BFLOAT16: out[m, s] = input[m] @ W[group_indices[m, s]] (+ bias).  With
    device-resident indices and ``check``, an index outside [0, G) raises
    InvalidArgument before the launch, as the reference does (one
    synchronisation); without ``check`` such a pair's row comes out NaN."""
    torch = _torch()
    M, S = (int(d) for d in _shape_of(group_indices))
    G = int(_shape_of(weights)[0])
    N = int(_shape_of(weights)[1 if transB else 2])
    if check and isinstance(group_indices, torch.Tensor) and group_indices.is_cuda and group_indices.numel():
        if bool(((group_indices < 0) | (group_indices >= G)).any()):
            raise InvalidArgument("kernel::GroupedMatMul group index must be in [0,G).")
    if out is None:
        out = _empty((M, S, N), input.dtype, _device_of(input, weights))
    _check(lib().onnxl_amd_grouped_matmul(describe(input), describe(weights), describe(group_indices),
                                          describe(bias), int(transB), describe(out),
                                          _stream_of(input, weights, group_indices, out)))
    return out


def dequantize_linear_grouped_matmul(input, x, x_scale, group_indices, x_zero_point=None, axis: int = 1,
                                     cast_to: int = 0, bias=None, transB: int = 0, x_dtype=None, x_shape=None,
                                     out=None):
    """Fused GroupedMatMul(input, [Cast](DequantizeLinear(x, x_scale,
    x_zero_point, axis)), group_indices, bias, transB): quantized MoE experts
    x [G, K, N] ([G, N, K] with transB)."""
    shape = _shape_of(x, x_shape)
    M, S = (int(d) for d in _shape_of(group_indices))
    N = int(shape[1 if transB else 2])
    if out is None:
        out = _empty((M, S, N), input.dtype, _device_of(input, x))
    dz = _describe_zp(x_zero_point, x_dtype, x_scale)
    _check(lib().onnxl_amd_dequantize_linear_grouped_matmul(describe(input), describe(x, x_dtype, shape),
                                                            describe(x_scale), dz, axis, cast_to,
                                                            describe(group_indices), describe(bias), int(transB),
                                                            describe(out),
                                                            _stream_of(input, x, group_indices, out)))
    return out


def cast(x, to: int, out=None):
    """FLOAT -> FLOAT16 / BFLOAT16 Cast (ext/kernels/kernels/tensor/kernel_cast.cc:360-370)."""
    torch = _torch()
    if out is None:
        out = _empty(_shape_of(x), torch.bfloat16 if to == BFLOAT16 else torch.float16,
                     _device_of(x))
    _check(lib().onnxl_amd_cast(describe(x), to, describe(out), _stream_of(x, out)))
    return out


def dequantize_linear_matmul(a, x, x_scale, x_zero_point=None, axis: int = 1, cast_to: int = 0,
                             x_dtype=None, x_shape=None, out=None):
    """Fused MatMul(a, [Cast](DequantizeLinear(x, x_scale, x_zero_point, axis)))."""
    shape = _shape_of(x, x_shape)
    if out is None:
        out = _empty(matmul_shape(_shape_of(a), shape), a.dtype, _device_of(a, x))
    dz = _describe_zp(x_zero_point, x_dtype, x_scale)
    _check(lib().onnxl_amd_dequantize_linear_matmul(describe(a), describe(x, x_dtype, shape),
                                                    describe(x_scale), dz, axis, cast_to,
                                                    describe(out), _stream_of(a, x, out)))
    return out


def dequantize_linear_matmul_noalloc(a, x, x_scale, x_zero_point=None, axis: int = 1, cast_to: int = 0,
                                     x_dtype=None, x_shape=None, out=None):
    """dequantize_linear_matmul through the no-allocation entry point: device
    tensors only, scratch from the library's fixed per-device array."""
    shape = _shape_of(x, x_shape)
    if out is None:
        out = _empty(matmul_shape(_shape_of(a), shape), a.dtype, _device_of(a, x))
    dz = _describe_zp(x_zero_point, x_dtype, x_scale)
    _check(lib().onnxl_amd_dequantize_linear_matmul_noalloc(describe(a), describe(x, x_dtype, shape),
                                                            describe(x_scale), dz, axis, cast_to,
                                                            describe(out), _stream_of(a, x, out)))
    return out


def _code_of(t):
    if isinstance(t, np.ndarray):
        return _NP_CODES[t.dtype]
    return _torch_code(t.dtype)


def quantize_linear(x, y_scale, y_zero_point=None, axis: int = 1, output_dtype: int = 0,
                    y_dtype=None, out=None):
    """kernel::QuantizeLinear with the node dispatch of QuantizeLinear::Run
    (kq/kernel_quantizelinear.cc:917-941): the output dtype is y_zero_point's
    (``y_dtype`` names it for packed sub-byte and uint8-held fp8 zero
    points), else output_dtype, else UINT8.  Sub-byte outputs (UINT4, INT4,
    FLOAT4E2M1, UINT2, INT2, FLOAT6E2M3, FLOAT6E3M2) are returned as packed
    uint8 storage (element i at bits i * bits onwards), FLOAT8E4M3FN as
    torch.float8_e4m3fn, the other fp8 types as their uint8 bits."""
    torch = _torch()
    shape = _shape_of(x)
    if y_dtype is None:
        y_dtype = (_code_of(y_zero_point) if y_zero_point is not None
                   else output_dtype if output_dtype else UINT8)
    n = int(np.prod(shape, dtype=np.int64))
    if out is None:
        bits = {INT4: 4, UINT4: 4, 23: 4, 25: 2, 26: 2, 27: 6, 28: 6}.get(y_dtype)
        if bits:
            out = _empty(((n * bits + 7) // 8,), torch.uint8, _device_of(x))
        else:
            tdt = {UINT8: torch.uint8, INT8: torch.int8, UINT16: torch.uint16, INT16: torch.int16,
                   FLOAT8E4M3FN: torch.float8_e4m3fn}.get(y_dtype, torch.uint8)
            out = _empty(shape, tdt, _device_of(x))
    dy = describe(out, y_dtype, shape)
    dz = _describe_zp(y_zero_point, y_dtype, y_scale)
    _check(lib().onnxl_amd_quantize_linear(describe(x), describe(y_scale), dz, axis, output_dtype,
                                           dy, _stream_of(x, out)))
    return out


def dynamic_quantize_linear(x, out=None, check: bool = True):
    """kernel::DynamicQuantizeLinear (kq/kernel_dynamicquantizelinear.cc:
    57-121): returns (y, y_scale, y_zero_point).  The library reports
    non-finite input through y_scale = NaN (finite input never gives a NaN
    scale: the range is >= 0, an infinite range gives an infinite scale);
    with ``check`` the scale is read back (a synchronisation) and such input
    raises InvalidArgument with the reference's message."""
    torch = _torch()
    dev = _device_of(x)
    y, y_scale, y_zp = out if out is not None else (
        _empty(_shape_of(x), torch.uint8, dev), _empty((), torch.float32, dev),
        _empty((), torch.uint8, dev))
    _check(lib().onnxl_amd_dynamic_quantize_linear(describe(x), describe(y), describe(y_scale),
                                                   describe(y_zp), _stream_of(x, y)))
    if check and bool(torch.isnan(y_scale).item()):
        raise InvalidArgument("kernel::DynamicQuantizeLinear: x elements must be finite.")
    return y, y_scale, y_zp


def dequantize_packed(x, format: str, shape, output_dtype: int = FLOAT, out=None):
    """kernel::DequantizePacked (kq/kernel_dequantize_packed.cc:11-28): decodes
    the packed UINT8 vector x into `shape` values of output_dtype."""
    torch = _torch()
    shape = tuple(int(d) for d in shape)
    if out is None:
        tdt = {FLOAT: torch.float32, FLOAT16: torch.float16, BFLOAT16: torch.bfloat16,
               DOUBLE: torch.float64}.get(output_dtype, torch.float32)
        out = _empty(shape, tdt, _device_of(x))
    dims = (ctypes.c_int64 * MAX_RANK)(*shape)
    _check(lib().onnxl_amd_dequantize_packed(describe(x), format.encode(), dims, len(shape), output_dtype,
                                             describe(out), _stream_of(x, out)))
    return out


def dequantize_packed_matmul(a, x, format: str, shape, out=None):
    """Fused a @ DequantizePacked(x, format, shape=[N, K], FLOAT16)^T."""
    torch = _torch()
    N, K = (int(d) for d in shape)
    if out is None:
        out = _empty((a.shape[0], N), torch.float16, _device_of(a, x))
    dims = (ctypes.c_int64 * MAX_RANK)(N, K)
    _check(lib().onnxl_amd_dequantize_packed_matmul(describe(a), describe(x), format.encode(), dims, 2,
                                                    describe(out), _stream_of(a, x, out)))
    return out


def conv_shape(x_shape, w_shape, attrs: ConvAttrs) -> tuple:
    xs = (ctypes.c_int64 * MAX_RANK)(*x_shape)
    ws = (ctypes.c_int64 * MAX_RANK)(*w_shape)
    out = (ctypes.c_int64 * MAX_RANK)()
    r = ctypes.c_int32(0)
    _check(lib().onnxl_amd_conv_shape(xs, len(x_shape), ws, len(w_shape), ctypes.byref(attrs), out,
                                      ctypes.byref(r)))
    return tuple(out[i] for i in range(r.value))


def conv_integer(x, w, x_zero_point=None, w_zero_point=None, out=None, **attrs):
    """kernel::ConvInteger (nn/kernel_conv_integer.cc:152-304); attrs are
    kernel_shape, strides, pads, dilations, group, auto_pad."""
    torch = _torch()
    a = conv_attrs(**attrs)
    if out is None:
        out = _empty(conv_shape(_shape_of(x), _shape_of(w), a), torch.int32, _device_of(x, w))
    _check(lib().onnxl_amd_conv_integer(describe(x), describe(w), describe(x_zero_point),
                                        describe(w_zero_point), ctypes.byref(a), describe(out),
                                        _stream_of(x, w, out)))
    return out


def qlinear_conv(x, x_scale, x_zero_point, w, w_scale, w_zero_point, y_scale, y_zero_point, B=None,
                 out=None, **attrs):
    """kernel::QLinearConv (kq/kernel_qlinearconv.cc:146-340); the output
    dtype follows y_zero_point."""
    torch = _torch()
    a = conv_attrs(**attrs)
    if out is None:
        ydt = y_zero_point.dtype
        if isinstance(y_zero_point, np.ndarray):
            ydt = torch.int8 if ydt == np.int8 else torch.uint8
        out = _empty(conv_shape(_shape_of(x), _shape_of(w), a), ydt, _device_of(x, w))
    ds = [describe(t) for t in (x, x_scale, x_zero_point, w, w_scale, w_zero_point, y_scale,
                                y_zero_point, B)]
    _check(lib().onnxl_amd_qlinear_conv(*ds, ctypes.byref(a), describe(out), _stream_of(x, w, out)))
    return out


class MatMulInteger:
    """Kernel-class mirror of kernel::MatMulInteger."""
    name = "onnxl_amd:GPU:ai.onnx:MatMulInteger"

    def __call__(self, a, b, a_zero_point=None, b_zero_point=None, out=None):
        return matmul_integer(a, b, a_zero_point, b_zero_point, out)


class QLinearMatMul:
    """Kernel-class mirror of kernel::QLinearMatMul."""
    name = "onnxl_amd:GPU:ai.onnx:QLinearMatMul"

    def __call__(self, a, a_scale, a_zero_point, b, b_scale, b_zero_point, y_scale, y_zero_point,
                 out=None):
        return qlinear_matmul(a, a_scale, a_zero_point, b, b_scale, b_zero_point, y_scale,
                              y_zero_point, out)


class DequantizeLinear:
    """Kernel-class mirror of kernel::DequantizeLinear (axis defaults to 1 as
    in DequantizeLinear::Run, kq/kernel_dequantizelinear.cc:705)."""
    name = "onnxl_amd:GPU:ai.onnx:DequantizeLinear"

    def __call__(self, x, x_scale, x_zero_point=None, axis=1, x_dtype=None, x_shape=None, out=None):
        return dequantize_linear(x, x_scale, x_zero_point, axis, x_dtype, x_shape, out)


class MatMul:
    """Kernel-class mirror of kernel::MatMul (FLOAT16 / BFLOAT16 inputs)."""
    name = "onnxl_amd:GPU:ai.onnx:MatMul"

    def __call__(self, a, b, out=None):
        return matmul(a, b, out)


class DequantizePacked:
    """Kernel-class mirror of kernel::DequantizePacked (default ONNX domain,
    onnx-light opset 29; kernel_dispatch_table.cc:147)."""
    name = "onnxl_amd:GPU:ai.onnx:DequantizePacked"

    def __call__(self, x, format, shape, output_dtype=FLOAT, out=None):
        return dequantize_packed(x, format, shape, output_dtype, out)


class ConvInteger:
    """Kernel-class mirror of kernel::ConvInteger."""
    name = "onnxl_amd:GPU:ai.onnx:ConvInteger"

    def __call__(self, x, w, x_zero_point=None, w_zero_point=None, out=None, **attrs):
        return conv_integer(x, w, x_zero_point, w_zero_point, out, **attrs)


class QLinearConv:
    """Kernel-class mirror of kernel::QLinearConv."""
    name = "onnxl_amd:GPU:ai.onnx:QLinearConv"

    def __call__(self, x, x_scale, x_zero_point, w, w_scale, w_zero_point, y_scale, y_zero_point, B=None,
                 out=None, **attrs):
        return qlinear_conv(x, x_scale, x_zero_point, w, w_scale, w_zero_point, y_scale, y_zero_point, B, out,
                            **attrs)


class QuantizeLinear:
    """Kernel-class mirror of kernel::QuantizeLinear (axis defaults to 1 as in
    QuantizeLinear::Run, kq/kernel_quantizelinear.cc:927)."""
    name = "onnxl_amd:GPU:ai.onnx:QuantizeLinear"

    def __call__(self, x, y_scale, y_zero_point=None, axis=1, output_dtype=0, y_dtype=None,
                 out=None):
        return quantize_linear(x, y_scale, y_zero_point, axis, output_dtype, y_dtype, out)


class DynamicQuantizeLinear:
    """Kernel-class mirror of kernel::DynamicQuantizeLinear."""
    name = "onnxl_amd:GPU:ai.onnx:DynamicQuantizeLinear"

    def __call__(self, x, out=None, check=True):
        return dynamic_quantize_linear(x, out, check)


class DequantizeLinearMatMul:
    """Kernel of the fused node that the DequantizeLinear -> [Cast] -> MatMul
    rewrite (``patterns.DequantizeLinearMatMulPattern``) produces: inputs
    (A, W, scale[, zero_point]), attributes axis and cast_to.  No reference
    kernel: it computes kernel::DequantizeLinear, kernel::Cast and
    kernel::MatMul in one pass."""
    name = "onnxl_amd:GPU:ai.rt.amd:DequantizeLinearMatMul"

    def __call__(self, a, x, x_scale, x_zero_point=None, axis=1, cast_to=0, x_dtype=None, x_shape=None,
                 out=None):
        return dequantize_linear_matmul(a, x, x_scale, x_zero_point, axis, cast_to, x_dtype, x_shape, out)


class DequantizePackedMatMul:
    """Kernel of the fused node that the DequantizePacked -> Transpose ->
    MatMul rewrite (``patterns.DequantizePackedMatMulPattern``) produces:
    inputs (A, x), attributes format and shape = [N, K].  No reference
    kernel: it computes kernel::DequantizePacked (FLOAT16), the transpose and
    kernel::MatMul in one pass."""
    name = "onnxl_amd:GPU:ai.rt.amd:DequantizePackedMatMul"

    def __call__(self, a, x, format, shape, out=None):
        return dequantize_packed_matmul(a, x, format, shape, out)


class GroupedMatMul:
    """Kernel-class mirror of kernel::GroupedMatMul (transB defaults to 0 as
    in GroupedMatMul::Run, math/kernel_grouped_matmul.cc:105-114)."""
    name = "onnxl_amd:GPU:ai.onnx:GroupedMatMul"

    def __call__(self, input, weights, group_indices, bias=None, transB=0, out=None):
        return grouped_matmul(input, weights, group_indices, bias, transB, out)


class DequantizeLinearGroupedMatMul:
    """Kernel of the fused node that the DequantizeLinear -> [Cast] ->
    GroupedMatMul rewrite (``patterns.DequantizeLinearGroupedMatMulPattern``)
    produces: inputs (input, x, scale, zero_point or None, group_indices[,
    bias]), attributes axis, cast_to and transB.  No reference kernel: it
    computes kernel::DequantizeLinear, kernel::Cast and kernel::GroupedMatMul
    in one pass."""
    name = "onnxl_amd:GPU:ai.rt.amd:DequantizeLinearGroupedMatMul"

    def __call__(self, input, x, x_scale, x_zero_point, group_indices, bias=None, axis=1, cast_to=0, transB=0,
                 x_dtype=None, x_shape=None, out=None):
        return dequantize_linear_grouped_matmul(input, x, x_scale, group_indices, x_zero_point, axis, cast_to, bias,
                                                transB, x_dtype, x_shape, out)


# Dispatch keys "<domain>:<op_type>" as the reference table uses them
# (core/runtime/kernels/kernel_dispatch_table.h:148-164).
KERNELS = {"ai.onnx:MatMulInteger": MatMulInteger, "ai.onnx:QLinearMatMul": QLinearMatMul,
           "ai.onnx:DequantizeLinear": DequantizeLinear, "ai.onnx:MatMul": MatMul,
           "ai.onnx:QuantizeLinear": QuantizeLinear,
           "ai.onnx:DynamicQuantizeLinear": DynamicQuantizeLinear,
           "ai.onnx:ConvInteger": ConvInteger, "ai.onnx:QLinearConv": QLinearConv,
           "ai.onnx:DequantizePacked": DequantizePacked,
           "ai.onnx:GroupedMatMul": GroupedMatMul,
           "ai.rt.amd:DequantizeLinearMatMul": DequantizeLinearMatMul,
           "ai.rt.amd:DequantizePackedMatMul": DequantizePackedMatMul,
           "ai.rt.amd:DequantizeLinearGroupedMatMul": DequantizeLinearGroupedMatMul}


class Prepared:
    """A C-ABI call with its descriptors built once (what a session adapter
    keeps per node): calling it re-runs the kernel on the same buffers."""

    def __init__(self, fn_name: str, descs: list, extra: tuple, stream):
        self._fn_name = fn_name
        self._fn = getattr(lib(), fn_name)
        self._descs = descs
        self._args = [ctypes.byref(d) if isinstance(d, Tensor) else d for d in descs]
        self._extra = extra
        self._stream = stream

    def __call__(self) -> None:
        _check(self._fn(*self._args, self._stream))

    def on(self, stream) -> "Prepared":
        """The same call launched on `stream` (a torch stream or a raw
        hipStream_t handle), e.g. the stream a HIP graph is captured on."""
        handle = getattr(stream, "cuda_stream", stream)
        return Prepared(self._fn_name, self._descs, self._extra, ctypes.c_void_p(handle))


def prepare(fn_name: str, *tensors, descs=None, **kw):
    """Prepared call of `onnxl_amd_<fn_name>`: tensors are described in order
    (None = absent); `descs` overrides individual descriptors by position and
    scalar (non-tensor) arguments are passed through unchanged."""
    out = []
    for i, t in enumerate(tensors):
        if descs and i in descs:
            out.append(descs[i])
        elif isinstance(t, (int, float)) and not isinstance(t, bool):
            out.append(t)
        else:
            out.append(describe(t))
    return Prepared("onnxl_amd_" + fn_name, out, (), _stream_of(*[t for t in tensors
                                                                  if not isinstance(t, (int, float))]))
