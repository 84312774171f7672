"""MX / NVFP4 weights on the GPU against the oracle (oracle.mx_reconstruct,
pinned by the reference's fixtures in test_oracle_mx.py):
onnxl_amd_dequantize_mx_weights bit for bit in FLOAT, FLOAT16, BFLOAT16 and
DOUBLE on the fixtures and on random weights of every format, from host and
device inputs and from unaligned device views; the first failing group and
element raised with the reference's message, whichever thread finds it."""
import numpy as np
import pytest
import torch

from test_gpu_float import T
from test_gpu_gptq_fp8 import _bits, _ref_bits, _raises
from test_oracle_mx import LEVELS, _write6

pytestmark = pytest.mark.gpu

DTYPES = [1, 10, 16, 11]
E4M3 = 17


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _codes_shape(fmt, rows, cols):
    return (rows, cols) if fmt == "mxfp8" else ((rows, cols // 4 * 3) if fmt == "mxfp6_e2m3" else (rows, cols // 2))


def _run(olamd, fmt, w, s, g, out, dev, host=False, offset=0):
    code = E4M3 if fmt == "mxfp8" else None
    scode = E4M3 if fmt == "nvfp4" else None
    if host:
        return olamd.dequantize_mx_weights(fmt, np.ascontiguousarray(w), np.ascontiguousarray(s), g, code, scode, out)
    if offset:
        # a device view starting `offset` bytes into its allocation
        base = torch.zeros(w.size + 64, dtype=torch.uint8, device=dev)
        wt = base[offset:offset + w.size].view(w.shape)
        wt.copy_(torch.from_numpy(np.ascontiguousarray(w)).to(dev))
        return olamd.dequantize_mx_weights(fmt, wt, T(s, dev), g, code, scode, out)
    return olamd.dequantize_mx_weights(fmt, T(w, dev), T(s, dev), g, code, scode, out)


def _check(olamd, oracle, dev, fmt, rows, cols, w, s, g=0.0, host=False, offset=0):
    for out in DTYPES:
        rc, grp, el, ref = oracle.mx_reconstruct(fmt, rows, cols, w, s, g, out_dtype=out)
        if rc:  # only the output range (a 2^125-scaled row in FLOAT16)
            assert rc == 6
            _raises(olamd, lambda: _run(olamd, fmt, w, s, g, out, dev, host, offset), oracle.mx_error(fmt, rc, grp, el))
            continue
        y = _run(olamd, fmt, w, s, g, out, dev, host, offset)
        assert np.array_equal(np.asarray(_bits(y)).reshape(-1), _ref_bits(ref, out).reshape(-1)), (fmt, out)


def _random(fmt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, _codes_shape(fmt, rows, cols)).astype(np.uint8)
    group = 16 if fmt == "nvfp4" else 32
    if fmt == "mxfp8":
        w[(w & 0x7F) == 0x7F] = 0x3C
    if fmt == "nvfp4":
        s = rng.integers(0x08, 0x78, (rows, cols // group)).astype(np.uint8)  # positive finite E4M3FN
    else:
        s = rng.integers(90, 160, (rows, cols // group)).astype(np.uint8)
        s[0, 0], s[-1, -1] = 0, 127  # 2^-127 (subnormal products) and 1
    return w, s


def test_fixtures(olamd, oracle, dev):
    packed = np.array([0x10, 0x32, 0x54, 0x76, 0x90, 0xba, 0xdc, 0xfe] * 2, np.uint8).reshape(1, 16)
    _check(olamd, oracle, dev, "mxfp4", 1, 32, packed, np.array([[127]], np.uint8))
    rows = np.repeat(np.array([0x66, 0xee, 0x66, 0x66], np.uint8), 16).reshape(2, 32)
    _check(olamd, oracle, dev, "mxfp4", 2, 64, rows, np.array([[125, 128], [126, 129]], np.uint8))
    six = np.concatenate([_write6([c] * 32) for c in (24, 31, 31, 24, 31, 24, 0, 31)]).reshape(4, 48)
    _check(olamd, oracle, dev, "mxfp6_e2m3", 4, 64, six,
           np.array([[125, 126], [126, 127], [127, 128], [0, 252]], np.uint8))
    _check(olamd, oracle, dev, "mxfp6_e2m3", 2, 32, _write6(list(range(64))).reshape(2, 24),
           np.array([[127], [0]], np.uint8))
    nv = np.array([0x10, 0x32, 0x54, 0x76, 0x90, 0xBA, 0xDC, 0xFE] * 2, np.uint8).reshape(1, 16)
    _check(olamd, oracle, dev, "nvfp4", 1, 32, nv, np.array([[0x7E, 0x6E]], np.uint8), 224.0)
    _check(olamd, oracle, dev, "nvfp4", 1, 16, np.full((1, 8), 0x33, np.uint8), np.array([[0x01]], np.uint8), 7.0)
    y = olamd.dequantize_mx_weights("mxfp4", T(packed, dev), T(np.array([[127]], np.uint8), dev))
    assert np.array_equal(y.cpu().numpy().reshape(-1), np.array(LEVELS * 2, np.float32))


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp6_e2m3", "mxfp8", "nvfp4"])
@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 96), (64, 4096), (300, 224)])
def test_random_vs_oracle(olamd, oracle, dev, fmt, rows, cols):
    w, s = _random(fmt, rows, cols, rows * 131 + cols)
    _check(olamd, oracle, dev, fmt, rows, cols, w, s, 0.75 if fmt == "nvfp4" else 0.0)


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp6_e2m3", "mxfp8", "nvfp4"])
def test_host_and_unaligned_inputs(olamd, oracle, dev, fmt):
    w, s = _random(fmt, 5, 64, 7)
    g = 3.0 if fmt == "nvfp4" else 0.0
    _check(olamd, oracle, dev, fmt, 5, 64, w, s, g, host=True)
    _check(olamd, oracle, dev, fmt, 5, 64, w, s, g, offset=2)


def _expect_error(olamd, oracle, dev, fmt, rows, cols, w, s, g=0.0, out=1):
    rc, grp, el, _ = oracle.mx_reconstruct(fmt, rows, cols, w, s, g, out_dtype=out)
    assert rc != 0
    _raises(olamd, lambda: _run(olamd, fmt, w, s, g, out, dev), oracle.mx_error(fmt, rc, grp, el))


def test_first_failure_in_reference_order(olamd, oracle, dev):
    rows, cols = 64, 4096
    w, s = _random("mxfp4", rows, cols, 1)
    s[40, 100] = 255
    s[3, 7] = 254
    w[3, 7 * 16 + 5] = 0x70  # a 6 in group 3 * 128 + 7, at 2^127: an overflow before the NaN scale's group
    _expect_error(olamd, oracle, dev, "mxfp4", rows, cols, w, s)
    s[2, 127] = 255
    _expect_error(olamd, oracle, dev, "mxfp4", rows, cols, w, s)
    w8, s8 = _random("mxfp8", rows, cols, 2)
    w8[10, 33] = 0x7F
    w8[10, 40] = 0x7E
    s8[10, 1] = 254  # group 10 * 128 + 1 at 2^127: its first overflow against element 1's NaN code
    _expect_error(olamd, oracle, dev, "mxfp8", rows, cols, w8, s8)
    s8[9, 127] = 255
    _expect_error(olamd, oracle, dev, "mxfp8", rows, cols, w8, s8)
    w6, s6 = _random("mxfp6_e2m3", rows, cols, 3)
    s6[20, 5] = 254
    _expect_error(olamd, oracle, dev, "mxfp6_e2m3", rows, cols, w6, s6)
    wn, sn = _random("nvfp4", rows, cols, 4)
    sn[30, 200] = 0x00
    _expect_error(olamd, oracle, dev, "nvfp4", rows, cols, wn, sn, 1.0)
    _expect_error(olamd, oracle, dev, "nvfp4", rows, cols, wn, sn, float("inf"))
    _expect_error(olamd, oracle, dev, "nvfp4", rows, cols, wn, sn, 1e-40)
    w4, s4 = _random("mxfp4", 4, 64, 5)
    s4[:] = 160
    _expect_error(olamd, oracle, dev, "mxfp4", 4, 64, w4, s4, out=10)


def test_argument_errors(olamd, dev):
    w = T(np.zeros((2, 16), np.uint8), dev)
    s = T(np.full((2, 1), 127, np.uint8), dev)
    _raises(olamd, lambda: olamd.dequantize_mx_weights("mxfp4", T(np.zeros((2, 8), np.uint8), dev), s),
            "MXFP4 WEIGHT requires positive [rows,cols] with cols divisible by 32.")
    _raises(olamd, lambda: olamd.dequantize_mx_weights("mxfp4", w, T(np.full((2, 2), 127, np.uint8), dev)),
            "Invalid MXFP4 WEIGHT tensor type, shape or storage.")
    _raises(olamd, lambda: olamd.dequantize_mx_weights("mxfp6_e2m3", T(np.zeros((2, 25), np.uint8), dev), s),
            "Invalid MXFP6 E2M3 packed columns.")
    _raises(olamd, lambda: olamd.dequantize_mx_weights("mxfp8", T(np.zeros((2, 32), np.uint8), dev), s),
            "Invalid MX tensor type, shape or storage.")
    _raises(olamd, lambda: olamd.dequantize_mx_weights("nvfp4", w, T(np.full((2, 2), 0x38, np.uint8), dev), 1.0),
            "Invalid NVFP4 WEIGHT tensor type, shape or storage.")
