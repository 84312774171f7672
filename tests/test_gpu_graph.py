"""C-ABI calls captured into HIP graphs: every replay must match the eager
call bit for bit (the kernels are deterministic).  The graphs are replayed
several times with eager calls of the same entry points and synchronisations
between the replays, because the split-K GEMV and the int8 GEMM share the
library's per-device workspace and counters with the eager calls."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _capture(calls):
    """Captures `calls` (prepared C-ABI calls) into one graph on a side stream."""
    side = torch.cuda.Stream()
    bound = [c.on(side) for c in calls]
    with torch.cuda.stream(side):
        for c in bound:  # warm-up: the workspace reaches its size before capture
            c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for c in bound:
            c()
    return g


def _gemv_call(olamd, dev, rng, M, K, N):
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(dev)
    q = rng.integers(0, 256, (K, N // 2), dtype=np.uint8)
    wq = torch.from_numpy(q).to(dev)
    sc = torch.from_numpy(rng.uniform(0.002, 0.02, (K // 32, N)).astype(np.float16)).to(dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    call = olamd.prepare("dequantize_linear_matmul", a, wq, sc, None, 0, 0, y,
                         descs={1: olamd.describe(wq, olamd.INT4, (K, N))})
    return call, y


def test_gemv_graph_replays_match_eager(olamd, dev):
    rng = np.random.default_rng(11)
    # split over K (partials + per-strip counters) in both shapes
    c1, y1 = _gemv_call(olamd, dev, rng, 8, 4096, 2048)
    c2, y2 = _gemv_call(olamd, dev, rng, 3, 2048, 1040)
    c1()
    c2()
    torch.cuda.synchronize()
    ref1, ref2 = y1.clone(), y2.clone()
    g = _capture([c1, c2])
    for rep in range(4):
        y1.zero_()
        y2.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), ref1.view(torch.int16)), f"replay {rep}: first call"
        assert torch.equal(y2.view(torch.int16), ref2.view(torch.int16)), f"replay {rep}: second call"
        # eager calls of the same entry point between the replays
        c2()
        c1()
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), ref1.view(torch.int16)), f"eager after replay {rep}"


def test_qlinear_graph_replays_match_eager(olamd, dev):
    rng = np.random.default_rng(12)
    M, K, N = 512, 1024, 768
    a = torch.from_numpy(rng.integers(0, 256, (M, K), dtype=np.uint8)).to(dev)
    b = torch.from_numpy(rng.integers(-128, 128, (K, N), dtype=np.int8)).to(dev)
    y = torch.empty((M, N), dtype=torch.uint8, device=dev)
    scal = lambda v, dt: np.array(v, dtype=dt)
    call = olamd.prepare("qlinear_matmul", a, scal(0.02, np.float32), scal(131, np.uint8), b,
                         scal(0.004, np.float32), scal(-3, np.int8), scal(0.5, np.float32),
                         scal(120, np.uint8), y)
    call()
    torch.cuda.synchronize()
    ref = y.clone()
    g = _capture([call])
    for rep in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep}"
        call()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"eager after replay {rep}"


def test_quantize_graph_replays_match_eager(olamd, dev):
    """QuantizeLinear and the two-pass DynamicQuantizeLinear (its min / max
    partials live in the shared workspace) captured together."""
    g0 = torch.Generator(device=dev).manual_seed(5)
    x1 = torch.randn((1000, 777), generator=g0, device=dev) * 7
    x2 = torch.randn((3001, 1024), generator=g0, device=dev) - 2
    sc = torch.tensor(0.05, device=dev)
    zp = torch.tensor(-3, dtype=torch.int8, device=dev)
    y1 = torch.empty((1000, 777), dtype=torch.int8, device=dev)
    y2 = torch.empty((3001, 1024), dtype=torch.uint8, device=dev)
    s2 = torch.empty((), device=dev)
    z2 = torch.empty((), dtype=torch.uint8, device=dev)
    c1 = olamd.prepare("quantize_linear", x1, sc, zp, 1, 0, y1)
    c2 = olamd.prepare("dynamic_quantize_linear", x2, y2, s2, z2)
    c1()
    c2()
    torch.cuda.synchronize()
    refs = [t.clone() for t in (y1, y2, s2, z2)]
    g = _capture([c2, c1])
    for rep in range(4):
        for t in (y1, y2, s2, z2):
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for t, r in zip((y1, y2, s2, z2), refs):
            assert torch.equal(t, r), f"replay {rep}"
        c1()
        c2()
        torch.cuda.synchronize()
        for t, r in zip((y1, y2, s2, z2), refs):
            assert torch.equal(t, r), f"eager after replay {rep}"
