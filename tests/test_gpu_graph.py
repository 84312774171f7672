"""C-ABI calls captured into HIP graphs: every replay must match the eager
call bit for bit (the kernels are deterministic).  The graphs are replayed
several times with eager calls of the same entry points and synchronisations
between the replays, because the split-K GEMV and the int8 GEMM share the
library's per-device workspace and counters with the eager calls."""
import zlib

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


def _qlm_scalars(rng, a, b, adt, bdt, ydt, a_s):
    """A draw of QLinearMatMul's six scalars (a_scale given) that keeps the
    outputs off the saturation bounds (fp32 scales, an fp16 b_scale)."""
    ia, ib, iy = np.iinfo(adt), np.iinfo(bdt), np.iinfo(ydt)
    za, zb = int(rng.integers(ia.min, ia.max + 1)), int(rng.integers(ib.min, ib.max + 1))
    b_s = np.float16(rng.uniform(0.001, 0.01))
    acc = np.matmul(a.astype(np.int64) - za, b.astype(np.int64) - zb)
    y_s = np.float32(a_s * np.float32(b_s) * (float(np.abs(acc).max()) + 1.0) / 100.0)
    cs = np.float32(np.float32(a_s * np.float32(b_s)) / y_s)
    zy = int(np.clip((int(iy.min) + int(iy.max)) // 2 - round(float(acc.mean()) * float(cs)), iy.min, iy.max))
    return [np.array(a_s), np.array(za, adt), np.array(b_s), np.array(zb, bdt), np.array(y_s), np.array(zy, ydt)]


# shapes reaching each int8 kernel: the pipelined MFMA core (K % 64 == 0,
# N % 16 == 0), the byte-granular tail kernel (K = 200), the K-tail kernel
# (N % 16 != 0) with a batch, and the int64-exact kernel (K = 45000 with
# unread zero points counts as past the int32-exact bound)
QLM_CAPTURE = [((512, 1024), (1024, 768), np.uint8, np.int8, np.uint8),
               ((300, 200), (200, 136), np.int8, np.int8, np.int8),
               ((3, 50, 128), (3, 128, 40), np.uint8, np.uint8, np.int8),
               ((6, 45000), (45000, 40), np.int8, np.uint8, np.uint8)]


@pytest.mark.parametrize("a_shape,b_shape,adt,bdt,ydt", QLM_CAPTURE, ids=["core", "bytes", "ktail", "int64"])
def test_qlinear_graph_device_scalars(olamd, oracle, dev, a_shape, b_shape, adt, bdt, ydt):
    """QLinearMatMul captured with its scalars in device memory (a_scale on the
    host): the kernels read them at replay time, so rewriting them between
    replays changes the output to the oracle's for the new values, bit for
    bit, with eager calls (which read them on the host) in between."""
    rng = np.random.default_rng(zlib.crc32(repr((a_shape, b_shape)).encode()))
    ia, ib = np.iinfo(adt), np.iinfo(bdt)
    a = rng.integers(ia.min, ia.max + 1, a_shape).astype(adt)
    b = rng.integers(ib.min, ib.max + 1, b_shape).astype(bdt)
    y = torch.empty(np.broadcast_shapes(a_shape[:-2], b_shape[:-2]) + (a_shape[-2], b_shape[-1]), dtype=torch.uint8
                    if ydt == np.uint8 else torch.int8, device=dev)
    a_host = np.float32(rng.uniform(0.005, 0.03))  # a_scale stays on the host
    draws = [_qlm_scalars(rng, a, b, adt, bdt, ydt, a_host) for _ in range(3)]
    sc = [torch.from_numpy(v.reshape(())).to(dev) for v in draws[0]]
    a_host = draws[0][0]
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    call = olamd.prepare("qlinear_matmul", ta, a_host, sc[1], tb, sc[2], sc[3], sc[4], sc[5], y)
    yd = oracle.INT8 if ydt == np.int8 else oracle.UINT8

    def ref(d):
        return oracle.qlinear_matmul(a, np.float32(d[0]), int(d[1]), b, np.float32(d[2]), int(d[3]),
                                     np.float32(d[4]), int(d[5]), y_dtype=yd)

    call()
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), ref(draws[0])), "eager"
    g = _capture([call])
    for rep, d in enumerate(draws + draws[:1]):
        for t, v in zip(sc[1:], d[1:]):
            t.copy_(torch.from_numpy(v.reshape(())))
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = ref(d)
        assert np.array_equal(y.cpu().numpy(), want), f"replay {rep}"
        assert 0.05 < np.mean((want > np.iinfo(ydt).min) & (want < np.iinfo(ydt).max)), "outputs not saturated"
        y.zero_()
        call()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want), f"eager after replay {rep}"


@pytest.mark.parametrize("a_shape,b_shape,adt,bdt", [((512, 1024), (1024, 512), np.uint8, np.int8),
                                                     ((300, 200), (200, 136), np.int8, np.uint8)],
                         ids=["core", "bytes"])
def test_matmul_integer_graph_device_zero_points(olamd, oracle, dev, a_shape, b_shape, adt, bdt):
    """MatMulInteger captured with one-element zero points in device memory:
    rewritten between replays (including to the values that make the row /
    column sums weightless), every replay is the oracle's int32 result."""
    rng = np.random.default_rng(sum(a_shape) + sum(b_shape))
    ia, ib = np.iinfo(adt), np.iinfo(bdt)
    a = rng.integers(ia.min, ia.max + 1, a_shape).astype(adt)
    b = rng.integers(ib.min, ib.max + 1, b_shape).astype(bdt)
    y = torch.empty((a_shape[0], b_shape[1]), dtype=torch.int32, device=dev)
    zs = [(int(rng.integers(ia.min, ia.max + 1)), int(rng.integers(ib.min, ib.max + 1))),
          (128 if adt == np.uint8 else 0, 128 if bdt == np.uint8 else 0),
          (int(ia.max), int(ib.min))]
    za = torch.tensor([zs[0][0]], dtype=torch.uint8 if adt == np.uint8 else torch.int8, device=dev)
    zb = torch.tensor([zs[0][1]], dtype=torch.uint8 if bdt == np.uint8 else torch.int8, device=dev)
    call = olamd.prepare("matmul_integer", torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), za, zb, y)
    call()
    torch.cuda.synchronize()
    g = _capture([call])
    for rep, (va, vb) in enumerate(zs + zs[:1]):
        za.fill_(va)
        zb.fill_(vb)
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = oracle.matmul_integer(a, b, np.array([va], np.int32), np.array([vb], np.int32))
        assert np.array_equal(y.cpu().numpy(), want), f"replay {rep}"
        y.zero_()
        call()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want), f"eager after replay {rep}"


def test_conv_capture_rejects_device_scalars(olamd, dev):
    """The convolutions read their scalars on the host: under capture, a
    device-resident one is refused with UNSUPPORTED before anything is
    launched (the capture stays valid and empty), while host scalars capture
    and replay like the eager call."""
    rng = np.random.default_rng(21)
    x = torch.from_numpy(rng.integers(0, 256, (1, 8, 10, 10), dtype=np.uint8)).to(dev)
    w = torch.from_numpy(rng.integers(-128, 128, (4, 8, 3, 3), dtype=np.int8)).to(dev)
    y = torch.empty((1, 4, 8, 8), dtype=torch.uint8, device=dev)
    host = [np.array(0.02, np.float32), np.array(3, np.uint8), np.array([0.01] * 4, np.float32),
            np.array(0, np.int8), np.array(0.5, np.float32), np.array(128, np.uint8)]
    side = torch.cuda.Stream()
    zp_dev = torch.tensor(3, dtype=torch.uint8, device=dev)
    ws = torch.from_numpy(host[2]).to(dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(olamd.Unsupported, match="captured"):
        with torch.cuda.graph(g, stream=side):
            olamd.qlinear_conv(x, host[0], zp_dev, w, ws, host[3], host[4], host[5], out=y, kernel_shape=[3, 3])
    yi = torch.empty((1, 4, 8, 8), dtype=torch.int32, device=dev)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(olamd.Unsupported, match="captured"):
        with torch.cuda.graph(g2, stream=side):
            olamd.conv_integer(x, w, zp_dev, None, out=yi, kernel_shape=[3, 3])
    # host scalars: captured and replayed
    with torch.cuda.stream(side):
        olamd.qlinear_conv(x, host[0], host[1], w, ws, host[3], host[4], host[5], out=y, kernel_shape=[3, 3])
    torch.cuda.synchronize()
    ref = y.clone()
    g3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g3, stream=side):
        olamd.qlinear_conv(x, host[0], host[1], w, ws, host[3], host[4], host[5], out=y, kernel_shape=[3, 3])
    y.zero_()
    torch.cuda.synchronize()
    g3.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
