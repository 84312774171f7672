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
