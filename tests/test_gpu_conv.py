"""GPU parity of ConvInteger and QLinearConv against the CPU oracle and the
reference's known answers: bit-exact (int32 sums; 8-bit requantized
outputs).

Cases cover the three GPU paths: the implicit GEMM (group 1, C % 128 == 0,
P % 16 == 0: the padded NHWC input read by the int8 MFMA GEMM, no im2col
matrix), im2col + the int8 MFMA GEMM (group 1, or any group with a scalar
weight zero point; the fast GEMM kernel when K is a multiple of 64 and the
output plane of 16) and the direct kernel (grouped convolutions with
per-channel weight zero points, and QLinearConv sums past exact int32).  Attributes: strides, dilations, explicit and automatic
padding, 1-D to 3-D.  At the bench shape [32, 256, 28, 28] the output is
checked against the oracle on exact slices (each output depends only on its
image and channel)."""
import zlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DT = {"uint8": 2, "int8": 3}
NP = {"uint8": np.uint8, "int8": np.int8}
LO = {"uint8": 0, "int8": -128}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_known_answers(olamd, oracle, golden, dev):
    for c in golden["conv_integer"]:
        x = np.array(c["x"], NP[c["x_dtype"]]).reshape(c["x_shape"])
        w = np.array(c["w"], NP[c["w_dtype"]]).reshape(c["w_shape"])
        xz = np.array(c["x_zp"], NP[c["x_dtype"]])
        y = olamd.conv_integer(T(x, dev), T(w, dev), xz, None, kernel_shape=c["kernel_shape"], pads=c["pads"])
        assert list(y.shape) == c["y_shape"] and y.cpu().numpy().reshape(-1).tolist() == c["y"], c["name"]
    for c in golden["qlinear_conv"]:
        x = np.array(c["x"], NP[c["x_dtype"]]).reshape(c["x_shape"])
        w = np.array(c["w"], NP[c["w_dtype"]]).reshape(c["w_shape"])
        y = olamd.qlinear_conv(T(x, dev), np.array(c["x_scale"], np.float32), np.array(c["x_zp"], NP[c["x_dtype"]]),
                               T(w, dev), np.array(c["w_scale"], np.float32), np.array(c["w_zp"], NP[c["w_dtype"]]),
                               np.array(c["y_scale"], np.float32), np.array(c["y_zp"], NP[c["y_dtype"]]),
                               kernel_shape=c["kernel_shape"])
        assert y.cpu().numpy().reshape(-1).astype(int).tolist() == c["y"], c["name"]


CASES = [
    # x shape, w shape, attrs (group included)
    ((2, 3, 9, 8), (4, 3, 3, 3), dict(pads=[1, 1, 1, 1])),
    ((1, 4, 10, 7), (6, 2, 3, 2), dict(group=2, strides=[2, 1], pads=[0, 1, 2, 0])),
    ((2, 4, 11, 11), (4, 1, 3, 3), dict(group=4, dilations=[2, 2], auto_pad="SAME_UPPER")),
    ((1, 2, 8, 9), (3, 2, 2, 3), dict(strides=[2, 2], auto_pad="SAME_LOWER")),
    ((1, 3, 7, 6), (2, 3, 3, 3), dict(auto_pad="VALID", strides=[1, 2])),
    ((3, 5, 17), (4, 5, 4), dict(strides=[3], pads=[2, 1], dilations=[2])),
    ((1, 2, 5, 6, 4), (3, 2, 2, 3, 2), dict(pads=[1, 0, 1, 0, 1, 1])),
    ((2, 6, 6, 6), (6, 3, 1, 1), dict(group=2)),
    ((2, 64, 16, 16), (96, 64, 3, 3), dict(pads=[1, 1, 1, 1])),          # fast GEMM: K = 576, P = 256
    ((1, 128, 14, 14), (64, 128, 1, 1), dict()),                          # 1x1, P = 196
    ((2, 32, 12, 12), (32, 1, 3, 3), dict(group=32, pads=[1, 1, 1, 1])),  # depthwise
    # implicit GEMM (group 1, C % 128 == 0, P % 16 == 0): padded NHWC input
    ((2, 128, 8, 8), (40, 128, 3, 3), dict(pads=[1, 1, 1, 1])),
    ((1, 128, 16, 16), (24, 128, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ((2, 128, 12, 12), (16, 128, 3, 3), dict(dilations=[2, 2], pads=[2, 2, 2, 2])),
    ((1, 128, 8, 20), (8, 128, 1, 5), dict(pads=[0, 2, 0, 2])),
    ((1, 256, 4, 8), (300, 256, 1, 1), dict()),
    ((1, 128, 8, 8), (16, 128, 3, 3), dict(strides=[2, 2], auto_pad="SAME_UPPER")),
    ((2, 128, 48), (16, 128, 3), dict(pads=[1, 1])),
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("dts", [("uint8", "int8"), ("int8", "uint8"), ("uint8", "uint8"), ("int8", "int8")])
def test_conv_vs_oracle(olamd, oracle, dev, case, dts):
    xs, ws, a = CASES[case]
    rng = np.random.default_rng(zlib.crc32(repr((case, dts)).encode()))
    x = rng.integers(LO[dts[0]], LO[dts[0]] + 256, xs).astype(NP[dts[0]])
    w = rng.integers(LO[dts[1]], LO[dts[1]] + 256, ws).astype(NP[dts[1]])
    M = ws[0]
    xz = np.array(rng.integers(LO[dts[0]], LO[dts[0]] + 256), NP[dts[0]])
    wz_vec = rng.integers(LO[dts[1]], LO[dts[1]] + 256, M).astype(NP[dts[1]])
    wz_sc = np.array(wz_vec[0], NP[dts[1]])
    oattrs = dict(group=a.get("group", 1), strides=a.get("strides"), pads=a.get("pads"),
                  dilations=a.get("dilations"), auto_pad=a.get("auto_pad", "NOTSET"))
    xd, wd = T(x, dev), T(w, dev)
    # ConvInteger: no zero points, scalar, per-channel (device)
    for xzp, wzp in ((None, None), (xz, wz_sc), (xz, wz_vec)):
        want = oracle.conv_integer(x, DT[dts[0]], w, DT[dts[1]], None if xzp is None else xzp.reshape(1),
                                   wzp, **oattrs)
        wz_arg = None if wzp is None else (T(wzp, dev) if wzp.ndim else wzp)
        got = olamd.conv_integer(xd, wd, xzp, wz_arg, **a).cpu().numpy()
        assert got.shape == want.shape and np.array_equal(got, want), (case, dts, xzp is None, np.ndim(wzp))
    # QLinearConv: per-channel scale, bias, both output dtypes
    xs_ = np.float32(rng.uniform(0.01, 0.05))
    ws_ = rng.uniform(0.001, 0.01, M).astype(np.float32)
    ys_ = np.float32(rng.uniform(0.5, 4.0))
    bias = rng.integers(-20000, 20000, M).astype(np.int32)
    for y_dt, yz, wzp, use_bias in (("uint8", 120, wz_vec, True), ("int8", -7, wz_sc, False)):
        want = oracle.qlinear_conv(x, DT[dts[0]], xs_, int(xz), w, DT[dts[1]], ws_, wzp, ys_, yz, DT[y_dt],
                                   bias=bias if use_bias else None, **oattrs)
        got = olamd.qlinear_conv(xd, np.array(xs_), xz, wd, T(ws_, dev), T(np.atleast_1d(wzp), dev) if wzp.ndim
                                 else wzp, np.array(ys_), np.array(yz, NP[y_dt]), T(bias, dev) if use_bias else None,
                                 **a).cpu().numpy()
        bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
        assert bad.size == 0, (case, dts, y_dt, bad[:5], got.reshape(-1)[bad[:5]], want.reshape(-1)[bad[:5]])


def test_qlinear_conv_past_exact_int32(olamd, oracle, dev):
    """K = 4096 * 9 input values: sums past 2^31 / (255 * 255) take the
    direct kernel's int64 accumulation, as the reference accumulates."""
    rng = np.random.default_rng(3)
    x = rng.integers(0, 256, (1, 4096, 3, 3)).astype(np.uint8)
    w = np.full((2, 4096, 3, 3), 255, np.uint8)
    w[1] = 0
    args = (np.float32(0.002), 0, np.array([0.001, 0.002], np.float32), np.array([0, 255], np.uint8),
            np.float32(1.0), 3)
    want = oracle.qlinear_conv(x, 2, args[0], args[1], w, 2, args[2], args[3], args[4], args[5], 2)
    got = olamd.qlinear_conv(T(x, dev), np.array(args[0]), np.array(0, np.uint8), T(w, dev), T(args[2], dev),
                             T(args[3], dev), np.array(args[4]), np.array(3, np.uint8)).cpu().numpy()
    assert np.array_equal(got, want)


def test_bench_shape_slices(olamd, oracle, dev):
    """The bench layer: x u8 [32, 256, 28, 28], w s8 [256, 256, 3, 3], pads 1,
    per-channel w_scale and bias, on the implicit-GEMM path; images 0 and 31
    and channels 0-15 and 240-255 against the oracle."""
    rng = np.random.default_rng(11)
    x = rng.integers(0, 256, (32, 256, 28, 28)).astype(np.uint8)
    w = rng.integers(-128, 128, (256, 256, 3, 3)).astype(np.int8)
    ws_ = rng.uniform(0.0005, 0.002, 256).astype(np.float32)
    bias = rng.integers(-30000, 30000, 256).astype(np.int32)
    q = (np.float32(0.02), 128, np.float32(0.8), 120)
    got = olamd.qlinear_conv(T(x, dev), np.array(q[0]), np.array(q[1], np.uint8), T(w, dev), T(ws_, dev),
                             np.array(0, np.int8), np.array(q[2]), np.array(q[3], np.uint8), T(bias, dev),
                             pads=[1, 1, 1, 1]).cpu().numpy()
    got_i = olamd.conv_integer(T(x, dev), T(w, dev), np.array(q[1], np.uint8), None, pads=[1, 1, 1, 1]).cpu().numpy()
    for n in (0, 31):
        for m0 in (0, 240):
            sl = slice(m0, m0 + 16)
            want = oracle.qlinear_conv(x[n:n + 1], 2, q[0], q[1], w[sl], 3, ws_[sl], np.zeros(1, np.int8), q[2], q[3],
                                       2, bias=bias[sl], pads=[1, 1, 1, 1])
            assert np.array_equal(got[n:n + 1, sl], want), (n, m0)
            want_i = oracle.conv_integer(x[n:n + 1], 2, w[sl], 3, np.array([q[1]], np.uint8), None, pads=[1, 1, 1, 1])
            assert np.array_equal(got_i[n:n + 1, sl], want_i), (n, m0)
