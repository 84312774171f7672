"""Benchmark of the MI355X quantized-matmul kernels (one GPU).

Default workload (the JSON line's `value`): configuration 2, QLinearMatMul
prefill u8[2048,4096] x s8[4096,4096] -> u8[2048,4096], int8 MFMA.  A step is
one QLinearMatMul over device-resident inputs; `value` is whole-job TOPS
(2*M*N*K ops / time per step).

Timing: after W untimed warm-up calls, K calls of the C-ABI entry point are
captured once into a HIP graph and the graph is replayed once untimed; the
timed region is one replay of exactly K steps, bracketed by synchronisations
and by HIP events on the replay stream.  `ms_per_step` is its wall time / K,
`kernel_ms_mean` its event time / K (the per-launch kernel time that
`roofline.achieved` divides the algorithmic work by).  The same K calls made
one by one from Python (validation and launch on the host each step) are
reported as `host_path_ms_per_step`.  `cpu_baseline` times the serial CPU
oracle (a restatement of the reference kernel, single core as the reference
runs it) on a bounded row sample.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2|c3|c3_onnx_layout|c3_stream_ceiling|
                   c4|c5|q8|dql|qconv|pk|pkgemv|pkgemv8|pkgemv_q2k|pkgemv_q3k|pkgemv_q4k|pkgemv_q5k|
                   pkgemv_q6k|pkgemv_iq4xs|awq|bnb|moe|moe_fp8]
                  [--no-extra] [--no-cpu-baseline]

The other configurations (3, 4, 5) and the quantizers in front of the
integer GEMMs (QuantizeLinear `q8`, DynamicQuantizeLinear `dql`, both on
configuration 2's fp32 activation), a QLinearConv layer (`qconv`), a
GGUF q4_0 weight decode (`pk`), the fused q4_0 / q8_0 / q2_k / q3_k / q4_k /
q5_k / q6_k / iq4_xs GEMVs (`pkgemv`, `pkgemv8`, `pkgemv_q2k`, `pkgemv_q3k`,
`pkgemv_q4k`, `pkgemv_q5k`, `pkgemv_q6k`, `pkgemv_iq4xs`), an AWQ gemm 4-bit
checkpoint prepared for the fused decode GEMV (`awq`), a bitsandbytes nf4
weight prepared for its fused GEMV (`bnb`) and a Mixtral-shaped
MoE GroupedMatMul (`moe`), the same with fp8 experts fused through
DequantizeLinear -> Cast (`moe_fp8`) are timed too and
reported under `extra` unless --no-extra is given.  `c3_stream_ceiling` is a plain streaming read of configuration 3's
25,604,096 bytes with the same replica rotation (libonnxl_amd_bench.so): the
rate a kernel that only reads those bytes reaches, beside which the GEMV's
own rate is read.

HBM-bound lines rotate buffer replicas totalling more than 512 MB, so each
launch misses the 256 MB Infinity Cache.  `cpu_baseline` (configurations 2,
3, 4 and 5, and `moe`) times the CPU oracle as the reference runs: MatMulInteger,
QLinearMatMul and DequantizeLinear on one core, MatMul and Cast on the
physical cores of the process's CPU set; it reports `nproc` and the physical
core count.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "int8/fp8 GEMM TOPS + GEMV GB/s (% of MI355X roofline), 1 GPU"
PEAK = {"hbm_GBps": 8000.0, "int8_TOPs": 5000.0, "bf16_TFLOPs": 2500.0, "fp8_TFLOPs": 5000.0}


def load_package():
    if "onnx_light_amd" in sys.modules:
        return sys.modules["onnx_light_amd"]
    path = os.path.join(ROOT, "onnx-light_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location("onnx_light_amd", path,
                                                  submodule_search_locations=[os.path.dirname(path)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["onnx_light_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


class Workload:
    """One configuration: inputs on the GPU, a prepared call per replica."""
    name = ""
    unit = ""
    dtype = ""
    bound = ""
    work = 0.0     # algorithmic ops/flops (mfma) or bytes (hbm) per launch
    nbytes = 0     # algorithmic HBM bytes per launch

    def step(self, i):
        self.calls[i % len(self.calls)]()


def make_c2(olamd, dev, k_depth=0):
    """Configuration 2.  `k_depth` > 0 replaces K = 4096 by that depth (the
    same distributions, drawn on the GPU): the K sweep that splits the GEMM's
    time into a per-K-step and a fixed per-launch part."""
    import importlib
    import torch
    syn = importlib.import_module("onnx_light_amd.synth")
    M, K, N = 2048, 4096, 4096
    w = Workload()
    w.key, w.unit, w.dtype, w.bound = "c2", "TOPS", "int8", "mfma"
    if k_depth:
        K = k_depth
        x = syn.config_inputs(2, scale=1 / 2048)  # the scalars
        g = torch.Generator(device=dev)
        g.manual_seed(K)
        a = torch.randint(0, 256, (M, K), dtype=torch.uint8, device=dev, generator=g)
        b = torch.randint(-128, 128, (K, N), dtype=torch.int8, device=dev, generator=g)
        w.name = (f"C2 shape at K = {K}: QLinearMatMul u8[2048,{K}] x s8[{K},4096] -> u8[2048,4096] "
                  f"(a_zp=128, b_zp=0, y_zp=128)")
    else:
        x = syn.config_inputs(2)
        a, b = _t(x["a"], dev), _t(x["b"], dev)
        w.name = "C2 QLinearMatMul prefill u8[2048,4096] x s8[4096,4096] -> u8[2048,4096] (a_zp=128, b_zp=0, y_zp=128)"
    w.work = 2.0 * M * N * K
    w.nbytes = M * K + K * N + M * N
    y = torch.empty((M, N), dtype=torch.uint8, device=dev)
    w.calls = [olamd.prepare("qlinear_matmul", a, x["a_scale"], x["a_zp"], b, x["b_scale"], x["b_zp"],
                             x["y_scale"], x["y_zp"], y)]
    w.inputs = x
    return w


def make_c3(olamd, dev, replicas, prepared=True):
    """Configuration 3.  `prepared`: the weight is given in the tiled layout
    written once by onnxl_amd_prepare_weight (the session-time preparation of
    a constant weight; the dequantisation itself still runs in every call),
    else in the ONNX packing."""
    import importlib
    import torch
    syn = importlib.import_module("onnx_light_amd.synth")
    x = syn.config_inputs(3)
    w = Workload()
    w.name = ("C3 decode GEMV fp16[8,4096] x DequantizeLinear(int4[4096,11008], block 32 on K, fp16 "
              "scales) -> fp16[8,11008], weight " + ("prepared (tiled layout)" if prepared else "in the ONNX packing"))
    w.key, w.unit, w.dtype, w.bound = "c3", "GB/s", "fp16 x int4 (fp32 accumulate)", "hbm"
    if not prepared:
        w.key = "c3_onnx_layout"
    K, N = x["w_shape"]
    w.nbytes = K * N // 2 + (K // 32) * N * 2 + 8 * K * 2 + 8 * N * 2
    w.work = float(w.nbytes)
    a = _t(x["a"], dev)
    w.calls = []
    for _ in range(replicas):
        wq = _t(x["w"], dev)
        sc = _t(x["scale"], dev)
        y = torch.empty((8, N), dtype=torch.float16, device=dev)
        if prepared:
            pw = olamd.prepare_weight(wq, olamd.INT4, (K, N))
            del wq
            w.calls.append(olamd.prepare("dequantize_linear_matmul", a, pw, sc, None, 0, 0, y))
        else:
            w.calls.append(olamd.prepare("dequantize_linear_matmul", a, wq, sc, None, 0, 0, y,
                                         descs={1: olamd.describe(wq, olamd.INT4, (K, N))}))
    w.inputs = x
    return w


def make_c4(olamd, dev):
    import importlib
    import torch
    syn = importlib.import_module("onnx_light_amd.synth")
    xt = syn.config4_torch(dev)  # drawn on the GPU, equal to config_inputs(4)
    x = {"a_bits": xt["a"].view(torch.int16).cpu().numpy().view(np.uint16), "w": xt["w"].cpu().numpy(),
         "scale": xt["scale"].cpu().numpy(), "axis": 1}
    w = Workload()
    w.name = ("C4 fp8 per-axis prefill bf16[4096,4096] x Cast(bf16, DequantizeLinear(fp8e4m3fn"
              "[4096,14336], fp32 per-column scale)) -> bf16[4096,14336]")
    w.key, w.unit, w.dtype, w.bound = "c4", "TFLOPS", "bf16 (fp32 accumulate)", "mfma"
    M, K, N = 4096, 4096, 14336
    w.work = 2.0 * M * N * K
    w.nbytes = M * K * 2 + K * N + N * 4 + M * N * 2
    a, wq, sc = xt["a"], xt["w"], xt["scale"]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    w.calls = [olamd.prepare("dequantize_linear_matmul", a, wq, sc, None, 1, olamd.BFLOAT16, y,
                             descs={1: olamd.describe(wq, olamd.FLOAT8E4M3FN)})]
    w.inputs = x
    return w


def make_c5(olamd, dev, replicas):
    import importlib
    import torch
    syn = importlib.import_module("onnx_light_amd.synth")
    x = syn.config_inputs(5)
    w = Workload()
    w.name = ("C5 batched MatMulInteger s8[32,512,64] x s8[32,64,512], per-row / per-column int8 "
              "zero points -> i32[32,512,512]")
    w.key, w.unit, w.dtype, w.bound = "c5", "GB/s", "int8 (int32 accumulate)", "hbm"
    w.nbytes = 32 * 512 * 64 * 2 + 1024 + 32 * 512 * 512 * 4
    w.work = float(w.nbytes)
    a, b = _t(x["a"], dev), _t(x["b"], dev)
    za, zb = _t(x["a_zp"], dev), _t(x["b_zp"], dev)
    w.calls = []
    for _ in range(replicas):
        y = torch.empty((32, 512, 512), dtype=torch.int32, device=dev)
        w.calls.append(olamd.prepare("matmul_integer", a, b, za, zb, y))
    w.inputs = x
    return w


def make_qconv(olamd, dev):
    """QLinearConv u8[32,256,28,28] x s8[256,256,3,3], pads 1, per-channel
    w_scale and bias -> u8[32,256,28,28]: im2col + int8 MFMA GEMM +
    requantization.  Work 2*N*M*P*K with K = 256*9, P = 28*28."""
    import torch
    w = Workload()
    w.name = ("QLinearConv u8[32,256,28,28] x s8[256,256,3,3] pads 1, per-channel w_scale, bias "
              "-> u8[32,256,28,28]")
    w.key, w.unit, w.dtype, w.bound = "qconv", "TOPS", "int8 (int32 accumulate)", "mfma"
    N, C, H, W, M = 32, 256, 28, 28, 256
    K, P = C * 9, H * W
    w.work = 2.0 * N * M * P * K
    w.nbytes = N * C * H * W + M * K + N * M * P
    rng = np.random.default_rng(21)
    x = _t(rng.integers(0, 256, (N, C, H, W)).astype(np.uint8), dev)
    wt = _t(rng.integers(-128, 128, (M, C, 3, 3)).astype(np.int8), dev)
    ws = _t(rng.uniform(0.0005, 0.002, M).astype(np.float32), dev)
    bias = _t(rng.integers(-30000, 30000, M).astype(np.int32), dev)
    y = torch.empty((N, M, H, W), dtype=torch.uint8, device=dev)
    a = olamd.conv_attrs(pads=[1, 1, 1, 1])
    descs = [olamd.describe(t) for t in (x, np.array(0.02, np.float32), np.array(128, np.uint8), wt, ws,
                                         np.array(0, np.int8), np.array(0.8, np.float32),
                                         np.array(120, np.uint8), bias)]
    w.calls = [olamd.Prepared("onnxl_amd_qlinear_conv", descs + [ctypes.byref(a), olamd.describe(y)],
                              (a, x, wt, ws, bias, y), olamd._stream_of(x))]
    return w


def make_pk(olamd, dev, replicas):
    """DequantizePacked gguf:q4_0 [14336, 4096] -> FLOAT16: 18 bytes in and
    64 bytes out per 32 values."""
    import torch
    w = Workload()
    w.name = "DequantizePacked gguf:q4_0 [14336,4096] -> float16"
    w.key, w.unit, w.dtype, w.bound = "pk", "GB/s", "q4_0 -> f16 (fp32 decode)", "hbm"
    n = 14336 * 4096
    w.nbytes = n // 32 * 18 + n * 2
    w.work = float(w.nbytes)
    rng = np.random.default_rng(31)
    blocks = rng.integers(0, 256, (n // 32, 18)).astype(np.uint8)
    blocks[:, 1] = rng.integers(0x20, 0x30, n // 32)  # fp16 scales of moderate size
    w.calls = []
    for _ in range(replicas):
        x = _t(blocks.reshape(-1), dev)
        y = torch.empty((14336, 4096), dtype=torch.float16, device=dev)
        dims = (ctypes.c_int64 * olamd.MAX_RANK)(14336, 4096)
        w.calls.append(olamd.Prepared("onnxl_amd_dequantize_packed",
                                      [olamd.describe(x), b"gguf:q4_0", dims, 2, olamd.FLOAT16, olamd.describe(y)],
                                      (x, y, dims), olamd._stream_of(x)))
    return w


PKGEMV_KEYS = {"q4_0": "pkgemv", "q8_0": "pkgemv8", "q2_k": "pkgemv_q2k", "q3_k": "pkgemv_q3k",
               "q4_k": "pkgemv_q4k", "q5_k": "pkgemv_q5k", "q6_k": "pkgemv_q6k", "iq4_xs": "pkgemv_iq4xs"}
PK_BLOCK = {"q4_0": (32, 18), "q8_0": (32, 34), "q2_k": (256, 84), "q3_k": (256, 110), "q4_k": (256, 144),
            "q5_k": (256, 176), "q6_k": (256, 210), "iq4_xs": (256, 136)}  # values, bytes
PK_D_AT = {"q2_k": 80, "q3_k": 108, "q6_k": 208}  # byte offset of the fp16 d (else 0)


def make_pkgemv(olamd, dev, replicas, fmt="q4_0"):
    """Fused GEMV y[1, 14336] = a[1, 4096] @ DequantizePacked(gguf:<fmt>,
    [14336, 4096], FLOAT16)^T: the weight's bytes per block (PK_BLOCK)
    dominate."""
    import torch
    w = Workload()
    per, block_bytes = PK_BLOCK[fmt]
    w.name = f"GEMV fp16[1,4096] x DequantizePacked(gguf:{fmt} [14336,4096])^T -> fp16[1,14336]"
    w.key = PKGEMV_KEYS[fmt]
    w.unit, w.dtype, w.bound = "GB/s", "f16 (fp32 accumulate)", "hbm"
    N, K = 14336, 4096
    w.nbytes = N * K // per * block_bytes + K * 2 + N * 2
    w.work = float(w.nbytes)
    rng = np.random.default_rng(41)
    blocks = rng.integers(0, 256, (N * K // per, block_bytes)).astype(np.uint8)
    at = PK_D_AT.get(fmt, 0)  # the fp16 d
    d = np.float16(rng.uniform(0.001, 0.05, N * K // per)).view(np.uint16)
    blocks[:, at], blocks[:, at + 1] = d & 255, d >> 8
    if fmt in ("q2_k", "q4_k", "q5_k"):  # dmin follows d
        m = np.float16(rng.uniform(0.001, 0.05, N * K // per)).view(np.uint16)
        blocks[:, at + 2], blocks[:, at + 3] = m & 255, m >> 8
    a = _t(np.float16(rng.standard_normal((1, K))), dev)
    w.calls = []
    for _ in range(replicas):
        x = _t(blocks.reshape(-1), dev)
        y = torch.empty((1, N), dtype=torch.float16, device=dev)
        dims = (ctypes.c_int64 * olamd.MAX_RANK)(N, K)
        w.calls.append(olamd.Prepared("onnxl_amd_dequantize_packed_matmul",
                                      [olamd.describe(a), olamd.describe(x), f"gguf:{fmt}".encode(), dims, 2,
                                       olamd.describe(y)],
                                      (a, x, y, dims), olamd._stream_of(x)))
    return w


def make_bnb(olamd, dev, replicas):
    """bitsandbytes nf4 (block 64, nested statistics) weight of configuration
    3's shape [11008, 4096], prepared once (checks, resolved block scales),
    then the fused GEMV fp16[1,4096] x W^T -> fp16[1,11008] per call: the
    codes and the scales dominate.  Random codes are valid nf4 codes."""
    import torch
    w = Workload()
    rows, cols, block = 11008, 4096, 64
    w.name = ("bitsandbytes nf4 (block 64, nested statistics) fp16[1,4096] x W[11008,4096]^T -> fp16[1,11008], "
              "weight prepared once (resolved block scales)")
    w.key, w.unit, w.dtype, w.bound = "bnb", "GB/s", "fp16 x nf4 (fp32 accumulate)", "hbm"
    blocks = rows * cols // block
    w.nbytes = rows * cols // 2 + blocks * 4 + cols * 2 + rows * 2
    w.work = float(w.nbytes)
    rng = np.random.default_rng(47)
    table = olamd.BNB_NF4_TABLE
    a = _t(np.float16(rng.standard_normal((1, cols))), dev)
    w.calls = []
    for _ in range(replicas):
        codes = _t(rng.integers(0, 256, rows * cols // 2).astype(np.uint8), dev)
        absmax = _t(rng.integers(0, 256, blocks).astype(np.uint8), dev)
        nested = _t(np.float32(rng.uniform(0.01, 0.1, -(-blocks // 256))), dev)
        nmap = _t(np.sort(np.float32(rng.uniform(-1, 1, 256))), dev)
        bw = olamd.prepare_bitsandbytes(olamd.BnbWeight("nf4", rows, cols, codes, absmax, _t(table, dev), block,
                                                        nested, nmap, 256, 0.05), olamd.FLOAT16)
        y = torch.empty((1, rows), dtype=torch.float16, device=dev)
        w.calls.append(olamd.Prepared("onnxl_amd_bitsandbytes_matmul",
                                      [olamd.describe(a), 0, rows, cols, block, olamd.describe(codes, olamd.UINT8),
                                       olamd.describe(bw.scales), olamd.describe(y)],
                                      (a, codes, bw.scales, y), olamd._stream_of(codes)))
    return w


def make_awq(olamd, dev, replicas):
    """AWQ gemm checkpoint (4 bits, group 128) of configuration 3's weight
    shape, prepared once by onnxl_amd_prepare_awq, then the fused decode GEMV
    fp16[8,4096] x W[4096,11008] -> fp16[8,11008] per call.  Random qweight /
    qzeros words are valid codes; scales fp16."""
    import torch
    w = Workload()
    K, N, group = 4096, 11008, 128
    w.name = ("AWQ gemm 4-bit (group 128) fp16[8,4096] x W[4096,11008] -> fp16[8,11008], weight prepared once "
              "into the fused DequantizeLinear -> MatMul operands")
    w.key, w.unit, w.dtype, w.bound = "awq", "GB/s", "fp16 x uint4 (fp32 accumulate)", "hbm"
    groups = K // group
    w.nbytes = K * N // 2 + groups * N * 2 + groups * N // 2 + 8 * K * 2 + 8 * N * 2
    w.work = float(w.nbytes)
    rng = np.random.default_rng(43)
    a = _t(np.float16(rng.standard_normal((8, K))), dev)
    w.calls = []
    for _ in range(replicas):
        qweight = _t(rng.integers(-2**31, 2**31, (K, N // 8), dtype=np.int64).astype(np.int32), dev)
        qzeros = _t(rng.integers(-2**31, 2**31, (groups, N // 8), dtype=np.int64).astype(np.int32), dev)
        scales = _t(np.float16(rng.uniform(0.002, 0.02, (groups, N))), dev)
        prep = olamd.prepare_awq("gemm", qweight, qzeros, scales, K, N, group)
        del qweight, qzeros, scales
        y = torch.empty((8, N), dtype=torch.float16, device=dev)
        w.calls.append(olamd.prepare("dequantize_linear_matmul", a, prep.weight, prep.scale, prep.zero_point, 0, 0,
                                     y))
    return w


def make_q8(olamd, dev, replicas):
    """QuantizeLinear of configuration 2's activation: fp32[2048,4096] -> u8
    with a scalar scale and zero point (the producer of QLinearMatMul's A)."""
    import torch
    w = Workload()
    w.name = "QuantizeLinear fp32[2048,4096] -> u8, scalar scale and zero point"
    w.key, w.unit, w.dtype, w.bound = "q8", "GB/s", "f32 -> u8", "hbm"
    n = 2048 * 4096
    w.nbytes = n * 4 + n + 4 + 1
    w.work = float(w.nbytes)
    g = torch.Generator(device=dev).manual_seed(11)
    sc = torch.tensor(0.031, device=dev)
    zp = torch.tensor(128, dtype=torch.uint8, device=dev)
    w.calls = []
    for _ in range(replicas):
        x = torch.randn((2048, 4096), generator=g, device=dev) * 4
        y = torch.empty((2048, 4096), dtype=torch.uint8, device=dev)
        w.calls.append(olamd.prepare("quantize_linear", x, sc, zp, 1, 0, y))
    return w


def make_dql(olamd, dev, replicas):
    """DynamicQuantizeLinear of configuration 2's activation: fp32[2048,4096]
    -> u8 plus scale and zero point.  The scale depends on all of x before any
    element is quantized, so x is read twice (min/max pass, quantize pass):
    algorithmic bytes 2 * 4n + n."""
    import torch
    w = Workload()
    w.name = "DynamicQuantizeLinear fp32[2048,4096] -> u8, scale, zero point"
    w.key, w.unit, w.dtype, w.bound = "dql", "GB/s", "f32 -> u8", "hbm"
    n = 2048 * 4096
    w.nbytes = 2 * n * 4 + n + 5
    w.work = float(w.nbytes)
    g = torch.Generator(device=dev).manual_seed(12)
    w.calls = []
    for _ in range(replicas):
        x = torch.randn((2048, 4096), generator=g, device=dev) * 3 + 0.5
        y = torch.empty((2048, 4096), dtype=torch.uint8, device=dev)
        s = torch.empty((), device=dev)
        z = torch.empty((), dtype=torch.uint8, device=dev)
        w.calls.append(olamd.prepare("dynamic_quantize_linear", x, y, s, z))
    return w


class _StreamCall:
    """One streaming read of `nbytes` at `ptr` (libonnxl_amd_bench.so, read
    design `variant`), with the `on(stream)` interface of a prepared call."""

    def __init__(self, lib, ptr, nbytes, sink, stream=None, variant=0):
        self.lib, self.ptr, self.nbytes, self.sink, self.stream = lib, ptr, nbytes, sink, stream
        self.variant = variant

    def __call__(self):
        rc = self.lib.onnxl_amd_bench_stream_read_v(ctypes.c_void_p(self.ptr), ctypes.c_int64(self.nbytes),
                                                    ctypes.c_void_p(self.sink), self.stream, self.variant)
        if rc:
            raise RuntimeError(f"stream read failed ({rc})")

    def on(self, stream):
        handle = getattr(stream, "cuda_stream", stream)
        return _StreamCall(self.lib, self.ptr, self.nbytes, self.sink, ctypes.c_void_p(handle), self.variant)


def make_moe(olamd, dev):
    """GroupedMatMul, the MoE expert contraction of a Mixtral-8x7B-shaped
    layer: 4096 tokens x top-2 of 8 experts, hidden 4096 -> 14336, bf16,
    weights in the [G, N, K] layout (transB = 1).  Routing: two distinct
    experts per token drawn uniformly (device generator, fixed seed)."""
    import torch
    M, S, G, K, N = 4096, 2, 8, 4096, 14336
    w = Workload()
    w.name = ("MoE GroupedMatMul bf16[4096,4096] x experts bf16[8,14336,4096] (transB=1), top-2 routing "
              "-> bf16[4096,2,14336]")
    w.key, w.unit, w.dtype, w.bound = "moe", "TFLOPS", "bf16 (fp32 accumulate)", "mfma"
    w.work = 2.0 * M * S * K * N
    w.nbytes = M * K * 2 + G * N * K * 2 + M * S * 8 + M * S * N * 2
    g = torch.Generator(device=dev).manual_seed(29)
    x = (torch.randn((M, K), device=dev, generator=g) * 0.5).to(torch.bfloat16)
    wt = (torch.randn((G, N, K), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    idx = torch.rand((M, G), device=dev, generator=g).argsort(dim=1)[:, :S].contiguous()  # distinct experts
    y = torch.empty((M, S, N), dtype=torch.bfloat16, device=dev)
    w.calls = [olamd.prepare("grouped_matmul", x, wt, idx, None, 1, y)]
    w.inputs = {"x": x, "w": wt, "idx": idx}
    return w


def make_moe_fp8(olamd, dev):
    """The same Mixtral-8x7B-shaped expert contraction with quantized
    experts: DequantizeLinear(fp8e4m3fn experts [8, 4096, 14336], fp32 scale
    per (expert, column) [8, 1, 14336]) -> Cast(bf16) -> GroupedMatMul, fused
    (onnxl_amd_dequantize_linear_grouped_matmul, fp8 codes as the matrix
    cores' B operand).  Same tokens, routing and flops as `moe`."""
    import torch
    M, S, G, K, N = 4096, 2, 8, 4096, 14336
    w = Workload()
    w.name = ("MoE DequantizeLinear(fp8e4m3fn experts [8,4096,14336], fp32 scale [8,1,14336]) -> Cast(bf16) -> "
              "GroupedMatMul bf16[4096,4096], top-2 routing -> bf16[4096,2,14336], fused")
    w.key, w.unit, w.dtype, w.bound = "moe_fp8", "TFLOPS", "bf16 x fp8 (fp32 accumulate)", "mfma"
    w.work = 2.0 * M * S * K * N
    w.nbytes = M * K * 2 + G * K * N + G * N * 4 + M * S * 8 + M * S * N * 2
    g = torch.Generator(device=dev).manual_seed(29)
    x = (torch.randn((M, K), device=dev, generator=g) * 0.5).to(torch.bfloat16)
    codes = torch.randn((G, K, N), device=dev, generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
    scale = torch.rand((G, 1, N), device=dev, generator=g) * 0.02 + 0.002
    idx = torch.rand((M, G), device=dev, generator=g).argsort(dim=1)[:, :S].contiguous()  # distinct experts
    y = torch.empty((M, S, N), dtype=torch.bfloat16, device=dev)
    w.calls = [olamd.prepare("dequantize_linear_grouped_matmul", x, codes, scale, None, 1, olamd.BFLOAT16, idx, None,
                             0, y, descs={1: olamd.describe(codes, olamd.FLOAT8E4M3FN)})]
    return w


STREAM_VARIANTS = {0: "one pass, 4 16-byte loads in flight per lane", 1: "one pass, 8 loads in flight per lane",
                   2: "one pass, 16 loads in flight per lane",
                   3: "persistent, 4 workgroups per CU looping, 4 loads in flight per lane",
                   4: "one pass, 8 non-temporal loads in flight per lane"}


def make_stream(olamd, dev, replicas, nbytes, key, name, variant=0):
    """A plain read of `nbytes` per launch over `replicas` buffers with read
    design `variant` (STREAM_VARIANTS): the streaming ceiling for a
    bandwidth-bound kernel of that byte count."""
    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "onnx-light_amd", "libonnxl_amd_bench.so"))
    lib.onnxl_amd_bench_stream_blocks_v.argtypes = [ctypes.c_int64, ctypes.c_int]
    lib.onnxl_amd_bench_stream_read_v.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_int]
    w = Workload()
    w.name = f"{name}; read design: {STREAM_VARIANTS[variant]}"
    w.key, w.unit, w.dtype, w.bound = key, "GB/s", "u8 (read only)", "hbm"
    w.nbytes = nbytes
    w.work = float(nbytes)
    w.variant = variant
    sink = torch.empty(lib.onnxl_amd_bench_stream_blocks_v(nbytes, variant) * 256, dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    w.bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev, generator=g) for _ in range(replicas)]
    w.sink = sink
    w.calls = [_StreamCall(lib, b.data_ptr(), nbytes, sink.data_ptr(), olamd._stream_of(b), variant)
               for b in w.bufs]
    return w


def best_stream(olamd, dev, replicas, nbytes, key, name, steps, warmup):
    """The fastest of the read designs (by HIP-event kernel time) and its
    timings: the ceiling is the best plain read of these bytes, not one
    design's."""
    best = None
    for variant in STREAM_VARIANTS:
        w = make_stream(olamd, dev, replicas, nbytes, key, name, variant)
        timing = time_workload(w, steps, warmup)
        if best is None or timing[1] < best[1][1]:
            best = (w, timing)
        else:
            del w
    return best


def replicas_for(nbytes, floor=512 << 20):
    """Buffer replicas whose total exceeds `floor` (the MALL is 256 MB)."""
    return max(2, floor // nbytes + 1)


def cpu_topology():
    """(logical CPUs in this process's CPU set, physical cores among them)."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f1, open(base + "core_id") as f2:
                cores.add((f1.read().strip(), f2.read().strip()))
        except OSError:
            cores.add(("cpu", str(c)))
    return len(cpus), len(cores)


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    orc.lib()
    return orc


def _median_time(fn, runs=3, budget_s=20.0):
    fn()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < runs and (not times or time.perf_counter() - t_start < budget_s):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times), len(times)


def _threaded(fn, n, nthreads):
    """fn(lo, hi) over [0, n) split into nthreads slices (the oracle's C code
    releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor
    step = (n + nthreads - 1) // nthreads
    with ThreadPoolExecutor(nthreads) as ex:
        list(ex.map(lambda lo: fn(lo, min(n, lo + step)), range(0, n, step)))


def cpu_baseline_c3(x):
    """The reference chain on the host: DequantizeLinear (serial, INT4 ->
    FLOAT16) then the fp16 MatMul (promote/demote serial, the product on the
    physical cores), the whole job, median of 3."""
    orc = _oracle()
    nproc, phys = cpu_topology()
    K, N = x["w_shape"]
    sbits = x["scale"].view(np.uint16)
    a = x["a"].view(np.uint16)

    def job():
        w = orc.dequantize_linear(x["w"], orc.INT4, (K, N), sbits, orc.FLOAT16, None, 0)
        orc.matmul_half(a, w, orc.FLOAT16, nthreads=phys)

    t, runs = _median_time(job)
    nbytes = K * N // 2 + (K // 32) * N * 2 + 8 * K * 2 + 8 * N * 2
    return {"value": round(nbytes / t / 1e9, 4), "unit": "GB/s", "cores": phys, "kind": "port",
            "sample": f"the whole job, median of {runs}: serial oracle DequantizeLinear (int4 -> fp16) then "
                      f"oracle fp16 MatMul on {phys} threads ({t:.3f} s per job)",
            "nproc": nproc, "physical_cores": phys}


def cpu_baseline_c4(x):
    """The reference chain on the host: DequantizeLinear (serial, fp8 ->
    FLOAT), Cast FLOAT -> BFLOAT16 (parallel), bf16 MatMul (promote serial,
    product on the physical cores).  The MatMul is timed on two row samples
    and fitted as fixed + per-row cost, then extrapolated to the 4096 rows."""
    orc = _oracle()
    nproc, phys = cpu_topology()
    K, N = x["w"].shape
    a = x["a_bits"]
    t_dq, _ = _median_time(lambda: orc.dequantize_linear(x["w"], orc.FLOAT8E4M3FN, (K, N), x["scale"], orc.FLOAT,
                                                         None, 1), runs=1)
    wf = orc.dequantize_linear(x["w"], orc.FLOAT8E4M3FN, (K, N), x["scale"], orc.FLOAT, None, 1).reshape(-1)
    wb = np.empty(wf.size, np.uint16)

    def cast(lo, hi):
        wb[lo:hi] = orc.f32_to_bf16_bits(wf[lo:hi])

    t_cast, _ = _median_time(lambda: _threaded(cast, wf.size, phys), runs=1)
    wb = wb.reshape(K, N)
    r1, r2 = 8, 40
    t1, _ = _median_time(lambda: orc.matmul_half(a, wb, orc.BFLOAT16, rows=(0, r1), nthreads=phys), runs=2)
    t2, _ = _median_time(lambda: orc.matmul_half(a, wb, orc.BFLOAT16, rows=(0, r2), nthreads=phys), runs=2)
    per_row = max(0.0, (t2 - t1) / (r2 - r1))
    fixed = max(0.0, t1 - per_row * r1)
    job = t_dq + t_cast + fixed + per_row * a.shape[0]
    return {"value": round(2.0 * a.shape[0] * K * N / job / 1e12, 6), "unit": "TFLOPS", "cores": phys,
            "kind": "port",
            "sample": f"serial oracle DequantizeLinear ({t_dq:.2f} s) + Cast on {phys} threads ({t_cast:.2f} s) + "
                      f"oracle bf16 MatMul on {phys} threads timed at {r1} and {r2} rows and extrapolated as "
                      f"{fixed:.2f} s + {per_row * 1e3:.1f} ms/row to {a.shape[0]} rows ({job:.1f} s per job)",
            "nproc": nproc, "physical_cores": phys}


def cpu_baseline_c5(x):
    """Serial oracle MatMulInteger (int32 accumulate, one core as the
    reference), the whole job, median of 3."""
    orc = _oracle()
    nproc, phys = cpu_topology()
    t, runs = _median_time(lambda: orc.matmul_integer(x["a"], x["b"], x["a_zp"], x["b_zp"]))
    nbytes = 32 * 512 * 64 * 2 + 1024 + 32 * 512 * 512 * 4
    return {"value": round(nbytes / t / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the whole job, median of {runs}: serial oracle MatMulInteger ({t:.3f} s per job)",
            "nproc": nproc, "physical_cores": phys}


def cpu_baseline_moe(x):
    """Oracle GroupedMatMul (bf16, in-order fp32 sums, one core as the
    reference) on the first 4 tokens of the job (8 expert rows), extrapolated
    per routed row to the 8192 of the job."""
    orc = _oracle()
    nproc, phys = cpu_topology()
    rows = 4
    xs = x["x"][:rows].view(__import__("torch").int16).cpu().numpy().view(np.uint16)
    ws = x["w"].view(__import__("torch").int16).cpu().numpy().view(np.uint16)
    idx = x["idx"][:rows].cpu().numpy()
    t, runs = _median_time(lambda: orc.grouped_matmul(xs, ws, idx, None, 1, orc.BFLOAT16), runs=2)
    M, S = x["idx"].shape
    G, N, K = x["w"].shape
    job = t * (M * S) / (rows * S)
    return {"value": round(2.0 * M * S * K * N / job / 1e12, 6), "unit": "TFLOPS", "cores": 1, "kind": "port",
            "sample": f"serial oracle GroupedMatMul on {rows} tokens ({rows * S} routed rows, {t:.2f} s, median "
                      f"of {runs}), extrapolated per row to {M * S} rows ({job:.0f} s per job)",
            "nproc": nproc, "physical_cores": phys}


def time_direct(w, steps, warmup):
    """Host path: one C-ABI call from Python per step (validation + launch),
    `steps` calls bracketed by synchronisations; ms per step by wall clock."""
    import torch
    for i in range(warmup):
        w.step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        w.step(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def time_graph(w, steps, warmup):
    """The timed region: `steps` calls captured once into a HIP graph (on a
    side stream), replayed once untimed, then once more bracketed by
    synchronisations and HIP events on the replay stream.  Returns the wall
    ms per step and the per-launch kernel time (event time / steps)."""
    import torch
    side = torch.cuda.Stream()
    calls = [c.on(side) for c in w.calls]
    with torch.cuda.stream(side):
        for i in range(warmup):
            calls[i % len(calls)]()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for i in range(steps):
            calls[i % len(calls)]()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern = e0.elapsed_time(e1) / steps
    del g
    return wall / steps * 1e3, kern


def time_workload(w, steps, warmup):
    host_ms = time_direct(w, steps, warmup)
    ms, kern = time_graph(w, steps, warmup)
    return ms, kern, host_ms


def cpu_baseline_c2(w, budget_s=20.0):
    """Serial oracle QLinearMatMul (the reference kernel restated, 1 core) on a
    row sample of configuration 2; median of repeated timed runs."""
    orc = _oracle()
    x = w.inputs
    rows = 40  # about 2.5 s per run on one core, 5 runs: 10-15 s of CPU work
    orc.qlinear_matmul(x["a"], x["a_scale"], 128, x["b"], x["b_scale"], 0, x["y_scale"], 128,
                       rows=(0, 2))  # warm-up
    times = []
    t_start = time.perf_counter()
    r0 = 0
    while len(times) < 5 and time.perf_counter() - t_start < budget_s:
        t = time.perf_counter()
        orc.qlinear_matmul(x["a"], x["a_scale"], 128, x["b"], x["b_scale"], 0, x["y_scale"], 128,
                           rows=(r0, r0 + rows))
        times.append(time.perf_counter() - t)
        r0 += rows
    sec_per_row = statistics.median(times) / rows
    ops = 2.0 * 2048 * 4096 * 4096
    full_s = sec_per_row * 2048
    return {"value": ops / full_s / 1e12, "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": f"{len(times)} timed runs of {rows} rows (of 2048) through the serial oracle "
                      f"QLinearMatMul (oracle/oracle.c, int64 accumulate, column-strided B), median, "
                      f"extrapolated linearly to the full 2048 rows ({full_s:.1f} s per job)",
            "nproc": cpu_topology()[0], "physical_cores": cpu_topology()[1]}


def roofline(w, kernel_ms, traffic):
    if w.bound == "mfma":
        int8 = w.key in ("c2", "qconv")
        peak = PEAK["int8_TOPs"] if int8 else PEAK["bf16_TFLOPs"]
        achieved = w.work / (kernel_ms * 1e-3) / 1e12
        unit = "TOP/s" if int8 else "TFLOP/s"
    else:
        peak = PEAK["hbm_GBps"]
        achieved = w.nbytes / (kernel_ms * 1e-3) / 1e9
        unit = "GB/s"
    out = {"bound": w.bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "traffic": traffic}
    if w.key == "c4":
        out["frac_of_fp8_peak"] = round(achieved / PEAK["fp8_TFLOPs"], 4)
    return out


def load_traffic(key):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(key, {}).get("hbm_bytes_per_launch")


def value_of(w, ms):
    if w.bound == "mfma":
        return w.work / (ms * 1e-3) / 1e12
    return w.nbytes / (ms * 1e-3) / 1e9


WORKLOADS = ("c2", "c3", "c3_onnx_layout", "c3_stream_ceiling", "c4", "c5", "q8", "dql", "qconv", "pk", "pkgemv",
             "pkgemv8", "pkgemv_q2k", "pkgemv_q3k", "pkgemv_q4k", "pkgemv_q5k", "pkgemv_q6k", "pkgemv_iq4xs", "awq", "bnb",
             "moe", "moe_fp8")
CPU_BASELINES = {"c3": cpu_baseline_c3, "c3_onnx_layout": cpu_baseline_c3, "c4": cpu_baseline_c4,
                 "c5": cpu_baseline_c5, "moe": cpu_baseline_moe}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2",
                    choices=list(WORKLOADS))
    ap.add_argument("--no-extra", dest="extra", action="store_false",
                    help="time only --workload (default: the other configurations too, under `extra`)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--replicas", type=int, default=0,
                    help="buffer replicas for HBM-bound configs (0 = enough to exceed 512 MB)")
    ap.add_argument("--k", type=int, default=0,
                    help="c2 only: time the configuration-2 shape at this K instead of 4096 (the K sweep "
                         "behind the per-K-step / per-launch cost split; implies --no-extra, no CPU baseline)")
    args = ap.parse_args()
    if args.k:
        if args.workload != "c2" or args.k % 64:
            ap.error("--k applies to --workload c2 with K a multiple of 64")
        args.extra, args.no_cpu_baseline = False, True
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the quantized-matmul kernels "
                                   "are single-device (see DESIGN.md for how they would shard)",
                          "n_gpus": args.gpus}))
        return 2

    import torch
    olamd = load_package()
    olamd.init(0)
    dev = torch.device("cuda:0")

    def build(key):
        if key == "c2":
            return make_c2(olamd, dev, args.k if key == args.workload else 0)
        if key == "c3":
            return make_c3(olamd, dev, args.replicas or 24)
        if key == "c3_onnx_layout":
            return make_c3(olamd, dev, args.replicas or 24, prepared=False)
        if key == "c4":
            return make_c4(olamd, dev)
        if key == "q8":
            return make_q8(olamd, dev, args.replicas or 14)
        if key == "dql":
            return make_dql(olamd, dev, args.replicas or 14)
        if key == "qconv":
            return make_qconv(olamd, dev)
        if key == "pk":
            return make_pk(olamd, dev, args.replicas or 4)
        if key == "pkgemv":
            return make_pkgemv(olamd, dev, args.replicas or replicas_for(14336 * 4096 // 32 * 18))
        if key == "pkgemv8":
            return make_pkgemv(olamd, dev, args.replicas or replicas_for(14336 * 4096 // 32 * 34), "q8_0")
        if key in PKGEMV_KEYS.values():
            fmt = next(f for f, k in PKGEMV_KEYS.items() if k == key)
            return make_pkgemv(olamd, dev, args.replicas or replicas_for(14336 * 4096 // 256 * PK_BLOCK[fmt][1]), fmt)
        if key == "awq":
            return make_awq(olamd, dev, args.replicas or 24)
        if key == "bnb":
            return make_bnb(olamd, dev, args.replicas or 24)
        if key == "moe":
            return make_moe(olamd, dev)
        if key == "moe_fp8":
            return make_moe_fp8(olamd, dev)
        return make_c5(olamd, dev, args.replicas or 16)

    def build_and_time(key, steps, warmup):
        """The workload and its (ms_per_step, kernel_ms_mean, host ms); the
        streaming ceiling is the fastest of its read designs."""
        if key == "c3_stream_ceiling":
            return best_stream(olamd, dev, args.replicas or 24, 25604096, key,
                               "streaming read of 25,604,096 bytes per launch (configuration 3's algorithmic "
                               "bytes), 24 replicas, the fastest of 5 read designs: the ceiling for the C3 GEMV",
                               steps, warmup)
        w = build(key)
        return w, time_workload(w, steps, warmup)

    w, (ms, kern_mean, host_ms) = build_and_time(args.workload, args.steps, args.warmup)
    line = {"metric": METRIC, "value": round(value_of(w, ms), 3), "unit": w.unit, "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": w.dtype,
            "data": "synthetic (SplitMix64 inputs of the reference's generator, device-resident)",
            "config": {"workload": w.name, "replicas": len(w.calls)},
            "kernel_ms_mean": round(kern_mean, 5),
            "host_path_ms_per_step": round(host_ms, 5),
            "roofline": roofline(w, kern_mean, load_traffic(w.key))}
    if args.extra:
        extra = {}
        for key in WORKLOADS:
            if key == args.workload:
                continue
            try:
                ew, (e_ms, e_mean, e_host) = build_and_time(key, max(20, args.steps // 4), max(3, args.warmup // 4))
                extra[key] = {"workload": ew.name, "value": round(value_of(ew, e_ms), 3), "unit": ew.unit,
                              "ms_per_step": round(e_ms, 5), "kernel_ms_mean": round(e_mean, 5),
                              "host_path_ms_per_step": round(e_host, 5),
                              "roofline": roofline(ew, e_mean, load_traffic(key))}
                if not args.no_cpu_baseline and key in CPU_BASELINES:
                    extra[key]["cpu_baseline"] = CPU_BASELINES[key](ew.inputs)
                del ew
                torch.cuda.empty_cache()
            except olamd.Unsupported as e:
                extra[key] = {"unsupported": str(e)}
        line["extra"] = extra
    if not args.no_cpu_baseline and args.workload == "c2":
        line["cpu_baseline"] = cpu_baseline_c2(w)
    elif not args.no_cpu_baseline and args.workload in CPU_BASELINES:
        line["cpu_baseline"] = CPU_BASELINES[args.workload](w.inputs)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
