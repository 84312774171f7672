"""Prepared (tiled) INT4 / UINT4 weights: the tiled bytes against a numpy
restatement of the layout, and the fused DequantizeLinear -> MatMul on a
prepared weight against the oracle chain (same tolerance as the ONNX-layout
path: the dequantised weight is rounded exactly as the chain rounds it, only
the fp32 summation order differs)."""
import os
import zlib

import numpy as np
import pytest
import torch

from test_gpu_float import T, assert_close, bits_tensor, decode, tensor_bits, _chain_ref, _synth
from tiled_layout import tile_int4

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


@pytest.mark.parametrize("K,N,signed", [(128, 16, True), (4096, 11008, True), (200, 40, False),
                                        (96, 77, True), (1000, 130, False)])
def test_prepared_layout_matches_restatement(olamd, oracle, dev, K, N, signed):
    rng = np.random.default_rng(zlib.crc32(repr((K, N, signed)).encode()))
    q = rng.integers(-8, 8, K * N) if signed else rng.integers(0, 16, K * N)
    x = oracle.pack_int4(q)
    pw = olamd.prepare_weight(T(x, dev), olamd.INT4 if signed else olamd.UINT4, (K, N))
    torch.cuda.synchronize()
    got = pw.storage.cpu().numpy().view(np.uint32)
    ref = tile_int4(x, K, N, signed)
    assert got.size == ref.size
    assert np.array_equal(got, ref)
    assert pw.desc.layout == olamd.LAYOUT_TILED_INT4 and pw.shape == (K, N)


PREP_CASES = [
    # name, kind, M, K, N, scale mode, block, zp
    ("b32", "int4", 8, 4096, 2048, "blocked", 32, False),
    ("b32-zp", "uint4", 16, 2048, 400, "blocked", 32, True),
    ("b64-zp-signed", "int4", 5, 256, 136, "blocked", 64, True),
    ("b16", "uint4", 7, 1024, 512, "blocked", 16, False),
    ("b8-k200", "int4", 3, 200, 96, "blocked", 8, False),
    ("col-zp", "int4", 4, 512, 784, "col", None, True),
    ("col-n98", "uint4", 2, 384, 98, "col", None, False),
    ("tensor-zp", "int4", 1, 160, 48, "tensor", None, True),
    ("tensor-n77", "int4", 6, 136, 77, "tensor", None, False),
    ("m1-longk", "int4", 1, 8192, 256, "blocked", 128, False),
    ("wide-n", "int4", 8, 512, 9000, "blocked", 32, False),
    # 2 and 4 tiles per workgroup, a partial last tile, a partial last 128-row
    # group, scale blocks longer than a group
    ("b256-t2", "uint4", 2, 768, 4808, "blocked", 256, False),
    ("b8-k96-t4", "int4", 5, 96, 12808, "blocked", 8, False),
    ("b32-k224", "int4", 4, 224, 1040, "blocked", 32, False),
    ("b16-m16", "int4", 16, 384, 272, "blocked", 16, False),
    # M > 16: the general path dequantises the tiled weight, then the 16-bit MatMul
    ("general-m40", "int4", 40, 256, 80, "blocked", 32, True),
    ("general-m300", "uint4", 300, 128, 96, "col", None, False),
]


def _case_inputs(oracle, case):
    name, kind, M, K, N, smode, block, with_zp = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    a = oracle.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    lo, hi = (-8, 8) if kind == "int4" else (0, 16)
    x = oracle.pack_int4(rng.integers(lo, hi, K * N))
    code = oracle.INT4 if kind == "int4" else oracle.UINT4
    if smode == "blocked":
        s_shape, axis = (K // block, N), 0
    elif smode == "col":
        s_shape, axis = (N,), 1
    else:
        s_shape, axis = (), 1
    sc = rng.uniform(0.002, 0.02, s_shape).astype(np.float16)
    zp = None
    if with_zp:
        m = int(np.prod(s_shape)) if s_shape else 1
        zp = oracle.pack_int4(rng.integers(lo, hi, m))
    return a, x, code, sc, zp, axis


@pytest.mark.parametrize("case", PREP_CASES, ids=[c[0] for c in PREP_CASES])
def test_prepared_dq_matmul_vs_oracle(olamd, oracle, dev, case):
    name, kind, M, K, N = case[:5]
    a, x, code, sc, zp, axis = _case_inputs(oracle, case)
    pw = olamd.prepare_weight(T(x, dev), code, (K, N))
    y = olamd.dequantize_linear_matmul(bits_tensor(a, "f16", dev), pw, T(sc, dev),
                                       None if zp is None else T(zp, dev), axis=axis, x_dtype=code)
    ref, mag = _chain_ref(oracle, a, x, code, K, N, sc, True, zp, axis, None, "f16")
    assert_close(tensor_bits(y), ref, mag, "f16", oracle, f"prepared {name}")


def test_prepared_repeat_and_graph_replay(olamd, oracle, dev):
    """A prepared-weight call captured in a HIP graph: replays match the eager
    result bit for bit, with eager calls in between."""
    case = ("graph", "int4", 8, 4096, 2048, "blocked", 32, False)
    a, x, code, sc, zp, axis = _case_inputs(oracle, case)
    pw = olamd.prepare_weight(T(x, dev), code, (4096, 2048))
    at, st = bits_tensor(a, "f16", dev), T(sc, dev)
    y = torch.empty((8, 2048), dtype=torch.float16, device=dev)
    call = olamd.prepare("dequantize_linear_matmul", at, pw, st, None, axis, 0, y)
    call()
    torch.cuda.synchronize()
    ref = y.clone()
    side = torch.cuda.Stream()
    bound = call.on(side)
    with torch.cuda.stream(side):
        bound()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        bound()
    for rep in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
        call()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"eager after replay {rep}"


def test_config3_full_size_prepared(olamd, oracle, dev):
    fx = np.load(os.path.join(ROOT, "tests", "golden", "config_fixtures_float.npz"))
    x = _synth().config_inputs(3)
    K, N = x["w_shape"]
    a = x["a"].view(np.uint16)
    pw = olamd.prepare_weight(T(x["w"], dev), olamd.INT4, (K, N))
    y = olamd.dequantize_linear_matmul(bits_tensor(a, "f16", dev), pw, T(x["scale"], dev), None,
                                       axis=0, x_dtype=olamd.INT4)
    got = tensor_bits(y)
    rows = fx["c3_rows"]
    w = oracle.dequantize_linear(x["w"], oracle.INT4, (K, N), x["scale"].view(np.uint16), oracle.FLOAT16, None, 0)
    mag = np.abs(decode(a[rows], "f16", oracle)) @ np.abs(decode(w, "f16", oracle))
    assert_close(got[rows], fx["c3_y_bits"], mag, "f16", oracle, "config 3 prepared")
