"""The rewritten DequantizeLinear -> [Cast] -> MatMul node on the GPU
against the unfused chain (oracle), with the float path's tolerance."""
import importlib

import numpy as np
import pytest

from test_gpu_float import T, _chain_ref, assert_close, bits_tensor, dev, tensor_bits  # noqa: F401 (dev: fixture)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_rewritten_graph_runs_fused_kernel(olamd, oracle, dev, dt):
    pt = importlib.import_module("onnx_light_amd.patterns")
    M, K, N = 4, 512, 384
    rng = np.random.default_rng(17 if dt == "f16" else 18)
    a = oracle.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32)) if dt == "f16" else \
        oracle.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    x = rng.integers(-128, 128, (K, N)).astype(np.int8)
    s16 = dt == "f16"
    sc = rng.uniform(0.002, 0.02, (N,)).astype(np.float16 if s16 else np.float32)
    zp = rng.integers(0, 20, (N,)).astype(np.int8)
    Nd = pt.Node
    nodes = [Nd("DequantizeLinear", ["W", "s", "z"], ["Wd"], attrs={"axis": 1})]
    if not s16:
        nodes.append(Nd("Cast", ["Wd"], ["Wc"], attrs={"to": 16}))
    nodes.append(Nd("MatMul", ["A", nodes[-1].outputs[0]], ["Y"]))
    g = pt.Graph(nodes, {"W", "s", "z"}, ["A"], ["Y"],
                 {"W": (pt.INT8, (K, N)), "s": (pt.FLOAT16 if s16 else pt.FLOAT, (N,)), "z": (pt.INT8, (N,))})
    assert pt.optimize(g, [pt.create_registered_pattern("DequantizeLinearMatMulGpu")]) == 1
    (node,) = g.nodes
    feeds = {"A": bits_tensor(a, dt, dev), "W": T(x, dev), "s": T(sc, dev), "z": T(zp, dev)}
    kernel = olamd.KERNELS[f"{node.domain}:{node.op_type}"]()
    y = kernel(*[feeds[i] for i in node.inputs], **node.attrs)
    ref, mag = _chain_ref(oracle, a, x, oracle.INT8, K, N, sc, s16, zp, 1, "bf16", dt)
    assert_close(tensor_bits(y), ref, mag, dt, oracle, f"pattern {dt}")


@pytest.mark.parametrize("fmt,bpb", [("gguf:q4_0", 18), ("gguf:q8_0", 34)])
def test_rewritten_packed_graph_runs_fused_kernel(olamd, oracle, dev, fmt, bpb):
    """DequantizePacked -> Transpose -> MatMul rewritten into the fused node,
    run through the kernel table, against the oracle chain."""
    from test_gpu_packed import _block_weight
    pt = importlib.import_module("onnx_light_amd.patterns")
    M, N, K = 3, 200, 256
    rng = np.random.default_rng(len(fmt) + bpb)
    x = _block_weight(rng, N, K, bpb)
    a = np.float16(rng.standard_normal((M, K)))
    Nd = pt.Node
    g = pt.Graph([Nd("DequantizePacked", ["X"], ["Wd"], attrs={"format": fmt, "shape": [N, K], "output_dtype": 10}),
                  Nd("Transpose", ["Wd"], ["Wt"], attrs={"perm": [1, 0]}), Nd("MatMul", ["A", "Wt"], ["Y"])],
                 {"X"}, ["A"], ["Y"], {"A": (pt.FLOAT16, (M, K))})
    assert pt.optimize(g, [pt.create_registered_pattern("DequantizePackedMatMulGpu")]) == 1
    (node,) = g.nodes
    feeds = {"A": T(a, dev), "X": T(x, dev)}
    kernel = olamd.KERNELS[f"{node.domain}:{node.op_type}"]()
    y = kernel(*[feeds[i] for i in node.inputs], **node.attrs)
    w_bits = oracle.dequantize_packed(x, fmt, (N, K), 10)
    ref = oracle.matmul_half(a.view(np.uint16), np.ascontiguousarray(w_bits.T), 10)
    mag = np.abs(a.astype(np.float64)) @ np.abs(oracle.f16_bits_to_f32(w_bits).astype(np.float64)).T
    assert_close(tensor_bits(y), ref, mag, "f16", oracle, f"packed pattern {fmt}")


@pytest.mark.parametrize("fp8", [True, False])
def test_rewritten_grouped_graph_runs_fused_kernel(olamd, oracle, dev, fp8):
    """DequantizeLinear -> Cast -> GroupedMatMul over constant experts,
    rewritten into the fused node and run through the kernel table, against
    the oracle chain (fp8 experts on the scaled-sum path with the opt-in,
    INT8 experts with zero points on the dequantizing path)."""
    pt = importlib.import_module("onnx_light_amd.patterns")
    G, K, N, M, S = 4, 256, 128, 64, 2
    rng = np.random.default_rng(31 if fp8 else 32)
    x_bits = oracle.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    if fp8:
        codes = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(G * K * N).astype(np.float32)).reshape(G, K, N)
        wt, s_shape, zp = pt.FLOAT8E4M3FN, (G, 1, N), None
    else:
        codes = rng.integers(-128, 128, (G, K, N)).astype(np.int8)
        wt, s_shape = pt.INT8, (G, 1, N)
        zp = rng.integers(-5, 5, s_shape).astype(np.int8)
    sc = rng.uniform(0.005, 0.02, s_shape).astype(np.float32)
    idx = rng.integers(0, G, (M, S)).astype(np.int64)
    Nd = pt.Node
    nodes = [Nd("DequantizeLinear", ["W", "s"] + (["z"] if zp is not None else []), ["Wd"], attrs={"axis": 1}),
             Nd("Cast", ["Wd"], ["Wc"], attrs={"to": 16}), Nd("GroupedMatMul", ["X", "Wc", "I"], ["Y"])]
    info = {"W": (wt, (G, K, N)), "s": (pt.FLOAT, s_shape), "z": (wt, s_shape)}
    g = pt.Graph(nodes, {"W", "s", "z"}, ["X", "I"], ["Y"], info)
    p = pt.create_registered_pattern("DequantizeLinearGroupedMatMulGpu")
    p.fp8_scaled_sums = True
    assert pt.optimize(g, [p]) == 1
    (node,) = g.nodes
    feeds = {"X": bits_tensor(x_bits, "bf16", dev), "W": T(codes.view(np.uint8), dev), "s": T(sc, dev),
             "I": T(idx, dev), "z": None if zp is None else T(zp, dev), "": None}
    kernel = olamd.KERNELS[f"{node.domain}:{node.op_type}"]()
    y = kernel(*[feeds[i] for i in node.inputs], **node.attrs, x_dtype=wt, x_shape=(G, K, N))
    w = oracle.dequantize_linear(codes.view(np.uint8), wt, (G, K, N), sc, oracle.FLOAT,
                                 None if zp is None else zp.view(np.uint8), 1)
    wb = oracle.f32_to_bf16_bits(w)
    ref = oracle.grouped_matmul(x_bits, wb, idx, None, 0, oracle.BFLOAT16)
    xa = np.abs(oracle.bf16_bits_to_f32(x_bits).astype(np.float64))
    wa = np.abs(oracle.bf16_bits_to_f32(wb).astype(np.float64))
    mag = np.stack([np.einsum("mk,mkn->mn", xa, wa[idx[:, s]]) for s in range(S)], 1)
    # the fp8 path also skips each weight's bf16 rounding (2^-8 relative)
    assert_close(tensor_bits(y), ref, mag * (2.0 if fp8 else 1.0), "bf16", oracle, f"grouped pattern fp8={fp8}")
