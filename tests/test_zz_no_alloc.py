"""onnxl_amd_dequantize_linear_matmul_noalloc against the allocating entry
point it mirrors (same kernels, so the outputs must be bit-identical), through
the C ABI, on two calls in a row where the second input is smaller; plus the
host-side rejections (host payloads, scratch beyond the fixed array)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _int4_case(oracle, rng, M, K, N, block, zp, dev):
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(dev)
    x = torch.from_numpy(oracle.pack_int4(rng.integers(-8, 8, K * N))).to(dev)
    s = torch.from_numpy(rng.uniform(0.002, 0.02, (K // block, N)).astype(np.float16)).to(dev)
    z = torch.from_numpy(oracle.pack_int4(rng.integers(-8, 8, (K // block) * N))).to(dev) if zp else None
    return a, x, s, z


def _both(olamd, a, x, s, z, x_dtype, shape, axis, cast_to=0):
    ref = olamd.dequantize_linear_matmul(a, x, s, z, axis=axis, cast_to=cast_to, x_dtype=x_dtype, x_shape=shape)
    # the output buffer starts as garbage, so a kernel that skips a store shows
    got = torch.full_like(ref, float("nan"))
    olamd.dequantize_linear_matmul_noalloc(a, x, s, z, axis=axis, cast_to=cast_to, x_dtype=x_dtype,
                                           x_shape=shape, out=got)
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_int4_gemv_split_k(olamd, oracle, dev):
    """The ONNX-layout int4 GEMV splits K over workgroups: its partial sums and
    counters live in the fixed array.  C3's shape, then a smaller one."""
    rng = np.random.default_rng(7)
    cases = [(8, 4096, 11008, 32, False), (3, 1024, 2048, 64, True)]
    for M, K, N, block, zp in cases:
        print(f"noalloc int4 GEMV M={M} K={K} N={N} block={block} zp={zp}", flush=True)
        a, x, s, z = _int4_case(oracle, rng, M, K, N, block, zp, dev)
        ref, got = _both(olamd, a, x, s, z, olamd.INT4, (K, N), axis=0)
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16))


def test_noalloc_general_path_and_repeat(olamd, oracle, dev):
    """M > 16 takes the general path: the weight is dequantised into the fixed
    array, then multiplied.  Two calls in a row, the second smaller; then the
    GEMV again, so the counters are seen to be back at zero."""
    rng = np.random.default_rng(11)
    for M, K, N in [(40, 512, 1024), (20, 128, 96)]:
        print(f"noalloc general int8 M={M} K={K} N={N}", flush=True)
        a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(dev)
        x = torch.from_numpy(rng.integers(-128, 128, (K, N), dtype=np.int8)).to(dev)
        s = torch.from_numpy(rng.uniform(0.001, 0.01, (N,)).astype(np.float16)).to(dev)
        ref, got = _both(olamd, a, x, s, None, None, None, axis=1)
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16))
    for _ in range(2):
        a, x, s, z = _int4_case(oracle, rng, 5, 2048, 4096, 32, True, dev)
        ref, got = _both(olamd, a, x, s, z, olamd.INT4, (2048, 4096), axis=0)
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16))


def test_noalloc_rejections(olamd, oracle, dev):
    rng = np.random.default_rng(3)
    # a weight whose dequantised copy (32 MiB) exceeds the array: refused on the host
    M, K, N = 32, 4096, 4096
    a = torch.zeros((M, K), dtype=torch.float16, device=dev)
    x = torch.zeros((K, N), dtype=torch.int8, device=dev)
    s = torch.ones((N,), dtype=torch.float16, device=dev)
    with pytest.raises(olamd.Unsupported, match="no-allocation entry point holds"):
        olamd.dequantize_linear_matmul_noalloc(a, x, s, None, axis=1)
    # host payloads are refused (no staging without allocation)
    a_h, x_h, s_h, _ = _int4_case(oracle, rng, 2, 256, 64, 32, False, torch.device("cpu"))
    with pytest.raises(olamd.InvalidArgument, match="device payloads only"):
        olamd.dequantize_linear_matmul_noalloc(a_h.to(dev), x_h, s_h.to(dev), None, axis=0, x_dtype=olamd.INT4,
                                               x_shape=(256, 64))
