"""CPU checks of the oracle's ConvInteger and QLinearConv (oracle/oracle.c,
restating nn/kernel_conv_integer.cc and kq/kernel_qlinearconv.cc): the known
answers the reference's own tests hold, and an independent numpy closed form.
The closed form pads x with its zero point and sums strided slices, where
the restatement loops over taps and skips padded ones, over strides,
dilations, explicit and automatic padding, groups, per-channel zero points
and scales, bias, and 1-D to 3-D inputs."""
import itertools
import zlib

import numpy as np
import pytest

DT = {"uint8": 2, "int8": 3}
NP = {"uint8": np.uint8, "int8": np.int8}


def test_conv_integer_known_answers(oracle, golden):
    for c in golden["conv_integer"]:
        x = np.array(c["x"], NP[c["x_dtype"]]).reshape(c["x_shape"])
        w = np.array(c["w"], NP[c["w_dtype"]]).reshape(c["w_shape"])
        xz = None if c["x_zp"] is None else np.array([c["x_zp"]], NP[c["x_dtype"]])
        y = oracle.conv_integer(x, DT[c["x_dtype"]], w, DT[c["w_dtype"]], xz, None,
                                kernel_shape=c["kernel_shape"], pads=c["pads"])
        assert list(y.shape) == c["y_shape"] and y.reshape(-1).tolist() == c["y"], c["name"]


def test_qlinear_conv_known_answers(oracle, golden):
    for c in golden["qlinear_conv"]:
        x = np.array(c["x"], NP[c["x_dtype"]]).reshape(c["x_shape"])
        w = np.array(c["w"], NP[c["w_dtype"]]).reshape(c["w_shape"])
        y = oracle.qlinear_conv(x, DT[c["x_dtype"]], c["x_scale"], c["x_zp"], w, DT[c["w_dtype"]], c["w_scale"],
                                c["w_zp"], c["y_scale"], c["y_zp"], DT[c["y_dtype"]],
                                kernel_shape=c["kernel_shape"])
        assert list(y.shape) == c["y_shape"] and y.reshape(-1).astype(int).tolist() == c["y"], c["name"]
    c = golden["qlinear_conv_closed_form"]
    x = (np.arange(49) * 4).astype(np.uint8).reshape(c["x_shape"])
    y = oracle.qlinear_conv(x, 2, c["x_scale"], c["x_zp"], np.array(c["w"], np.uint8).reshape(1, 1, 1, 1), 2,
                            c["w_scale"], c["w_zp"], c["y_scale"], c["y_zp"], 2)
    cs = np.float32(np.float32(c["x_scale"]) * np.float32(c["w_scale"][0])) / np.float32(c["y_scale"])
    acc = (x.astype(np.int64) - c["x_zp"]) * (0 - 255)
    want = np.clip(np.rint(acc.astype(np.float32) * cs) + c["y_zp"], 0, 255).astype(np.uint8)
    assert np.array_equal(y, want)


def closed_form_acc(x, xz, w, wz, group, k, s, d, pads_begin, out_sp):
    """int64 accumulator by padding x with its zero point and summing strided
    slices (a formulation independent of the oracle's tap loop)."""
    N, C = x.shape[:2]
    M, cpg = w.shape[:2]
    sr = x.ndim - 2
    big = [(0, 0), (0, 0)] + [(pads_begin[a], (out_sp[a] - 1) * s[a] + (k[a] - 1) * d[a] + 1) for a in range(sr)]
    xp = np.pad(x.astype(np.int64) - xz, big, constant_values=0)
    wz = np.broadcast_to(np.asarray(wz, np.int64).reshape(-1), (M,))
    wc = w.astype(np.int64) - wz.reshape((M,) + (1,) * (w.ndim - 1))
    mpg = M // group
    acc = np.zeros((N, M) + tuple(out_sp), np.int64)
    for kp in itertools.product(*[range(kk) for kk in k]):
        sl = tuple(slice(kp[a] * d[a], kp[a] * d[a] + (out_sp[a] - 1) * s[a] + 1, s[a]) for a in range(sr))
        patch = xp[(slice(None), slice(None)) + sl]  # [N, C, out...]
        for g in range(group):
            wg = wc[g * mpg:(g + 1) * mpg][(slice(None), slice(None)) + tuple(kp)]  # [mpg, cpg]
            acc[:, g * mpg:(g + 1) * mpg] += np.einsum("mc,nc...->nm...", wg, patch[:, g * cpg:(g + 1) * cpg])
    return acc


CASES = [
    # x shape, w shape, group, attrs
    ((2, 3, 9, 8), (4, 3, 3, 3), 1, dict(pads=[1, 1, 1, 1])),
    ((1, 4, 10, 7), (6, 2, 3, 2), 2, dict(strides=[2, 1], pads=[0, 1, 2, 0])),
    ((2, 4, 11, 11), (4, 1, 3, 3), 4, dict(dilations=[2, 2], auto_pad="SAME_UPPER")),
    ((1, 2, 8, 9), (3, 2, 2, 3), 1, dict(strides=[2, 2], auto_pad="SAME_LOWER")),
    ((1, 3, 7, 6), (2, 3, 3, 3), 1, dict(auto_pad="VALID", strides=[1, 2])),
    ((3, 5, 17), (4, 5, 4), 1, dict(strides=[3], pads=[2, 1], dilations=[2])),
    ((1, 2, 5, 6, 4), (3, 2, 2, 3, 2), 1, dict(pads=[1, 0, 1, 0, 1, 1])),
    ((2, 6, 6, 6), (6, 3, 1, 1), 2, dict()),
]


def _attrs(a):
    return dict(strides=a.get("strides"), pads=a.get("pads"), dilations=a.get("dilations"),
                auto_pad=a.get("auto_pad", "NOTSET"))


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("dts", [("uint8", "int8"), ("int8", "uint8"), ("uint8", "uint8"), ("int8", "int8")])
def test_conv_closed_form(oracle, case, dts):
    xs, ws, group, a = CASES[case]
    rng = np.random.default_rng(zlib.crc32(repr((case, dts)).encode()))
    lo = {"uint8": 0, "int8": -128}
    x = rng.integers(lo[dts[0]], lo[dts[0]] + 256, xs).astype(NP[dts[0]])
    w = rng.integers(lo[dts[1]], lo[dts[1]] + 256, ws).astype(NP[dts[1]])
    xz = np.array([rng.integers(lo[dts[0]], lo[dts[0]] + 256)], NP[dts[0]])
    M = ws[0]
    wz = rng.integers(lo[dts[1]], lo[dts[1]] + 256, M).astype(NP[dts[1]])
    k, s, d, pads, out_sp = oracle.conv_geometry(xs, ws, **_attrs(a))
    acc = closed_form_acc(x, int(xz[0]), w, wz, group, k, s, d, pads[:len(k)], out_sp)
    y = oracle.conv_integer(x, DT[dts[0]], w, DT[dts[1]], xz, wz, group=group, **_attrs(a))
    assert np.array_equal(y, acc.astype(np.int64).astype(np.uint32).astype(np.int32) if acc.size else y)
    # QLinearConv: per-channel scale, bias, both output types
    xs_ = np.float32(rng.uniform(0.01, 0.05))
    ws_ = rng.uniform(0.001, 0.01, M).astype(np.float32)
    ys_ = np.float32(rng.uniform(0.5, 4.0))
    bias = rng.integers(-5000, 5000, M).astype(np.int32)
    for y_dt, yz in (("uint8", 120), ("int8", -7)):
        yq = oracle.qlinear_conv(x, DT[dts[0]], xs_, int(xz[0]), w, DT[dts[1]], ws_, wz, ys_, yz, DT[y_dt],
                                 bias=bias, group=group, **_attrs(a))
        cs = (xs_ * ws_) / ys_
        tot = acc + bias.reshape((1, M) + (1,) * len(k))
        f = tot.astype(np.float32) * cs.reshape((1, M) + (1,) * len(k))
        r = np.rint(f) + np.float32(yz)
        want = np.clip(r, *((0, 255) if y_dt == "uint8" else (-128, 127))).astype(NP[y_dt])
        assert np.array_equal(yq, want), (case, dts, y_dt)


def test_geometry_matches_onnx_rules(oracle):
    # SAME_UPPER puts the extra pad at the end, SAME_LOWER at the start
    _, _, _, pu, ou = oracle.conv_geometry((1, 1, 5, 5), (1, 1, 2, 2), auto_pad="SAME_UPPER")
    _, _, _, pl, ol = oracle.conv_geometry((1, 1, 5, 5), (1, 1, 2, 2), auto_pad="SAME_LOWER")
    assert ou == ol == (5, 5) and pu == (0, 0, 1, 1) and pl == (1, 1, 0, 0)
    assert oracle.conv_geometry((1, 1, 7), (1, 1, 3), strides=[2], auto_pad="VALID")[4] == (3,)
