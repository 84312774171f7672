"""GroupedMatMul on the GPU (FLOAT16 / BFLOAT16): the reference's backend cases
bit for bit; random MoE-shaped problems against the oracle within the float
path's tolerance |got - ref| <= 1e-2 |ref| + u sum_k |x w| (u = 2^-11 fp16,
2^-8 bf16), on both the MFMA core (K % 32 == 0, N % 16 == 0) and the
per-element kernel; integer-valued inputs, whose fp32 sums are exact in any
order, bit for bit; index validation; HIP graph replays with new routing."""
import numpy as np
import pytest
import torch

from grouped_cases import BFLOAT16, FLOAT16, expand
from test_gpu_float import T, assert_close, bits_tensor, tensor_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _name(dt):
    return "f16" if dt == FLOAT16 else "bf16"


def _enc(oracle, dt, a):
    a = np.asarray(a, np.float32)
    return oracle.f32_to_f16_bits(a) if dt == FLOAT16 else oracle.f32_to_bf16_bits(a)


def _dec(oracle, dt, bits):
    return (oracle.f16_bits_to_f32(bits) if dt == FLOAT16 else oracle.bf16_bits_to_f32(bits)).astype(np.float64)


def test_reference_cases(olamd, oracle, dev):
    done = 0
    for name, dt, x, w, idx, bias, tb, want in expand(oracle):
        if dt not in (FLOAT16, BFLOAT16):
            with pytest.raises(olamd.Unsupported):
                olamd.grouped_matmul(T(x, dev), T(w, dev), T(idx, dev), None if bias is None else T(bias, dev), tb)
            continue
        n = _name(dt)
        y = olamd.grouped_matmul(bits_tensor(x, n, dev), bits_tensor(w, n, dev), T(idx, dev),
                                 None if bias is None else bits_tensor(bias, n, dev), tb)
        assert np.array_equal(tensor_bits(y), want), name
        done += 1
    assert done == 38


@pytest.mark.parametrize("dt", [FLOAT16, BFLOAT16])
@pytest.mark.parametrize("M,S", [(0, 2), (3, 0)])
def test_empty(olamd, dev, dt, M, S):
    n = _name(dt)
    tdt = torch.float16 if dt == FLOAT16 else torch.bfloat16
    y = olamd.grouped_matmul(torch.zeros((M, 64), dtype=tdt, device=dev), torch.zeros((2, 64, 32), dtype=tdt, device=dev),
                             torch.zeros((M, S), dtype=torch.int64, device=dev), None, 0)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (M, S, 32), n


SHAPES = [
    # M, K, N, G, S, transB, bias, index dtype
    (300, 256, 128, 8, 2, 0, False, np.int64),   # core, 3 routed tile-rows per group on average
    (300, 256, 128, 8, 2, 1, True, np.int32),    # core, transposed weights, bias
    (64, 96, 48, 5, 3, 1, False, np.int64),      # core: a trailing half K step, a partial column tile
    (517, 512, 384, 16, 2, 1, True, np.int32),   # many groups, uneven routing
    (1, 64, 64, 4, 1, 0, False, np.int64),       # one token
    (128, 2048, 256, 4, 2, 1, False, np.int64),  # long K
    (40, 50, 20, 3, 2, 0, True, np.int64),       # per-element kernel (K % 32, N % 16)
    (33, 64, 40, 6, 2, 1, False, np.int32),      # per-element kernel (N % 16)
]


@pytest.mark.parametrize("dt", [FLOAT16, BFLOAT16])
@pytest.mark.parametrize("shape", SHAPES, ids=[str(s[:7]) for s in SHAPES])
def test_random_vs_oracle(olamd, oracle, dev, dt, shape):
    M, K, N, G, S, tb, with_bias, idt = shape
    rng = np.random.default_rng(M * 131 + K * 7 + N + G * 3 + S + tb * 11 + dt)
    x = _enc(oracle, dt, rng.standard_normal((M, K)))
    w = _enc(oracle, dt, rng.standard_normal((G, N, K) if tb else (G, K, N)) * 0.5)
    b = _enc(oracle, dt, rng.standard_normal((G, N))) if with_bias else None
    # skewed routing: some groups busy, some empty
    p = rng.random(G) ** 3
    idx = rng.choice(G, size=(M, S), p=p / p.sum()).astype(idt)
    ref = oracle.grouped_matmul(x, w, idx, b, tb, dt)
    n = _name(dt)
    y = olamd.grouped_matmul(bits_tensor(x, n, dev), bits_tensor(w, n, dev), T(idx, dev),
                             None if b is None else bits_tensor(b, n, dev), tb)
    wf = _dec(oracle, dt, w)
    wg = np.transpose(wf, (0, 2, 1))[idx] if tb else wf[idx]             # [M, S, K, N]
    mag = np.einsum("mk,mskn->msn", np.abs(_dec(oracle, dt, x)), np.abs(wg))
    if b is not None:
        mag = mag + np.abs(_dec(oracle, dt, b))[idx]
    assert_close(tensor_bits(y), ref, mag, n, oracle, f"grouped {shape}")


@pytest.mark.parametrize("dt", [FLOAT16, BFLOAT16])
@pytest.mark.parametrize("K,N,tb", [(256, 128, 0), (256, 128, 1), (96, 48, 1), (50, 20, 0)])
def test_integer_values_bit_exact(olamd, oracle, dev, dt, K, N, tb):
    """Small integers: products and fp32 partial sums are exact whatever the
    order, and the results are representable, so GPU and oracle agree bit for
    bit."""
    rng = np.random.default_rng(K + N + tb + dt)
    M, G, S = 300, 5, 2
    lim = 2 if dt == FLOAT16 else 1  # |sum| <= 1024 (fp16) / 256 (bf16): exact
    x = _enc(oracle, dt, rng.integers(-lim, lim + 1, (M, K)))
    w = _enc(oracle, dt, rng.integers(-lim, lim + 1, (G, N, K) if tb else (G, K, N)))
    idx = rng.integers(0, G, (M, S))
    ref = oracle.grouped_matmul(x, w, idx, None, tb, dt)
    n = _name(dt)
    y = olamd.grouped_matmul(bits_tensor(x, n, dev), bits_tensor(w, n, dev), T(idx, dev), None, tb)
    assert np.array_equal(tensor_bits(y), ref)


def test_index_validation(olamd, dev):
    x = torch.ones((4, 64), dtype=torch.float16, device=dev)
    w = torch.ones((3, 64, 32), dtype=torch.float16, device=dev)
    bad = np.array([[0, 1], [2, 3], [1, 1], [0, -1]], np.int64)
    with pytest.raises(olamd.InvalidArgument, match=r"\[0,G\)"):  # host indices
        olamd.grouped_matmul(x, w, bad, None, 0)
    with pytest.raises(olamd.InvalidArgument, match=r"\[0,G\)"):  # device indices, checked
        olamd.grouped_matmul(x, w, T(bad, dev), None, 0)
    y = olamd.grouped_matmul(x, w, T(bad, dev), None, 0, check=False)  # unchecked: NaN rows
    yc = y.float().cpu().numpy().reshape(8, 32)
    invalid = np.array([False, False, False, True, False, False, False, True])
    assert np.isnan(yc[invalid]).all() and np.all(yc[~invalid] == 64.0)


def test_graph_replays_follow_new_routing(olamd, oracle, dev):
    """One captured call replayed with new indices written into the same
    buffer between replays: the routing is recomputed on the device each time
    (no host-side state), every replay equals an eager call."""
    rng = np.random.default_rng(77)
    M, K, N, G, S = 200, 128, 64, 6, 2
    x = bits_tensor(_enc(oracle, FLOAT16, rng.standard_normal((M, K))), "f16", dev)
    w = bits_tensor(_enc(oracle, FLOAT16, rng.standard_normal((G, K, N))), "f16", dev)
    idx = torch.zeros((M, S), dtype=torch.int64, device=dev)
    y = torch.empty((M, S, N), dtype=torch.float16, device=dev)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        olamd.grouped_matmul(x, w, idx, None, 0, out=y, check=False)  # warm-up: workspace sized
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        olamd.grouped_matmul(x, w, idx, None, 0, out=y, check=False)
    for r in range(3):
        idx.copy_(torch.from_numpy(rng.integers(0, G, (M, S))).to(dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = olamd.grouped_matmul(x, w, idx, None, 0)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16)), r
