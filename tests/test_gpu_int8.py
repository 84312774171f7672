"""GPU parity of MatMulInteger and QLinearMatMul (int8 MFMA GEMM) against the
CPU oracle and the reference's known answers: bit-exact.  Shapes cover the
vector and byte-wise load paths, tile tails, batch broadcasting, 1-D operands,
empty inputs and every zero-point form (absent / scalar / per-row /
per-column)."""
import hashlib
import json
import os
import zlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NP = {"uint8": np.uint8, "int8": np.int8}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def T(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def test_matmul_integer_known_answers(olamd, golden, dev):
    for c in golden["matmul_integer"]:
        a = np.array(c["a"], NP[c["a_dtype"]]).reshape(c["a_shape"])
        b = np.array(c["b"], NP[c["b_dtype"]]).reshape(c["b_shape"])
        za = None if c["a_zp"] is None else T(np.array(c["a_zp"]["values"], a.dtype).reshape(c["a_zp"]["shape"]), dev)
        zb = None if c["b_zp"] is None else T(np.array(c["b_zp"]["values"], b.dtype).reshape(c["b_zp"]["shape"]), dev)
        y = olamd.matmul_integer(T(a, dev), T(b, dev), za, zb)
        assert list(y.shape) == c["y_shape"], c["name"]
        assert y.cpu().reshape(-1).tolist() == c["y"], c["name"]


SHAPES = [
    ((64, 256), (256, 128)),        # one tile, vector path
    ((300, 200), (200, 136)),       # tails in M and N; K % 16 != 0 -> byte path
    ((513, 128), (128, 264)),       # M tail, N % 8 == 0
    ((37, 45), (45, 29)),           # everything ragged
    ((2, 96, 64), (2, 64, 80)),     # batched
    ((3, 1, 40, 32), (5, 32, 24)),  # broadcast batch dims
    ((1, 70, 48), (4, 48, 16)),     # A broadcast over B's batch
    ((64,), (64, 40)),              # 1-D A
    ((33, 64), (64,)),              # 1-D B
    ((48,), (48,)),                 # both 1-D -> scalar
    ((0, 32), (32, 16)),            # empty M
    ((8, 0), (0, 16)),              # K = 0 -> zeros
    ((1, 4096), (4096, 8)),         # long K, many K steps
]


def _zps(kind, dt, n, rng):
    info = np.iinfo(dt)
    if kind == "absent":
        return None
    if kind == "scalar":
        return np.array(rng.integers(info.min, info.max + 1), dt)
    if kind == "one":
        return np.array([rng.integers(info.min, info.max + 1)], dt)
    return rng.integers(info.min, info.max + 1, n).astype(dt)  # per-row / per-column


@pytest.mark.parametrize("shapes", SHAPES, ids=[f"{a}x{b}" for a, b in SHAPES])
@pytest.mark.parametrize("dts", [(np.uint8, np.int8), (np.int8, np.int8), (np.uint8, np.uint8),
                                 (np.int8, np.uint8)], ids=["u8s8", "s8s8", "u8u8", "s8u8"])
def test_matmul_integer_vs_oracle(olamd, oracle, dev, shapes, dts):
    a_shape, b_shape = shapes
    rng = np.random.default_rng(zlib.crc32(repr((a_shape, b_shape, str(dts))).encode()))
    ia, ib = np.iinfo(dts[0]), np.iinfo(dts[1])
    a = rng.integers(ia.min, ia.max + 1, a_shape).astype(dts[0])
    b = rng.integers(ib.min, ib.max + 1, b_shape).astype(dts[1])
    M = a_shape[-2] if len(a_shape) > 1 else 1
    N = b_shape[-1] if len(b_shape) > 1 else 1
    for ka, kb in [("absent", "absent"), ("scalar", "one"), ("vec", "vec"), ("vec", "absent"),
                   ("absent", "vec")]:
        za = _zps(ka, dts[0], M, rng)
        zb = _zps(kb, dts[1], N, rng)
        if (ka == "vec" and M == 1) or (kb == "vec" and N == 1):
            continue
        y = olamd.matmul_integer(T(a, dev), T(b, dev), None if za is None else T(za, dev),
                                 None if zb is None else T(zb, dev))
        ref = oracle.matmul_integer(a, b, None if za is None else za.reshape(-1).astype(np.int32),
                                    None if zb is None else zb.reshape(-1).astype(np.int32))
        assert tuple(y.shape) == ref.shape
        assert np.array_equal(y.cpu().numpy(), ref), (ka, kb)


def test_matmul_integer_host_payloads(olamd, oracle, dev):
    """Host (numpy) inputs and output: the library stages them itself."""
    rng = np.random.default_rng(4)
    a = rng.integers(0, 256, (130, 96)).astype(np.uint8)
    b = rng.integers(-128, 128, (96, 72)).astype(np.int8)
    za = rng.integers(0, 256, 130).astype(np.uint8)
    y = np.zeros((130, 72), np.int32)
    olamd.matmul_integer(a, b, za, np.array(3, np.int8), out=y)
    assert np.array_equal(y, oracle.matmul_integer(a, b, za.astype(np.int32), [3]))


def _fixtures():
    path = os.path.join(ROOT, "tests", "golden", "config_fixtures.json")
    with open(path) as f:
        return json.load(f)


def _synth(olamd):
    import importlib
    return importlib.import_module("onnx_light_amd.synth")


def test_config1_plumbing_case(olamd, oracle, dev):
    syn = _synth(olamd)
    x = syn.config_inputs(1)
    y = olamd.matmul_integer(T(x["a"], dev), T(x["b"], dev), T(x["a_zp"], dev), T(x["b_zp"], dev))
    ref = oracle.matmul_integer(x["a"], x["b"], [128], [0])
    got = y.cpu().numpy()
    assert np.array_equal(got, ref)
    fx = _fixtures()["c1"]
    assert hashlib.sha256(got.tobytes()).hexdigest() == fx["sha256"]


def test_config5_batched_attention_scores(olamd, oracle, dev):
    syn = _synth(olamd)
    x = syn.config_inputs(5)
    y = olamd.matmul_integer(T(x["a"], dev), T(x["b"], dev), T(x["a_zp"], dev), T(x["b_zp"], dev))
    got = y.cpu().numpy()
    fx = _fixtures()["c5"]
    assert hashlib.sha256(got.tobytes()).hexdigest() == fx["sha256"]
    # exact integer closed form at full size (float64 sums of |x| < 2^53 are exact)
    a = torch.from_numpy(x["a"]).to(dev).double() - torch.from_numpy(x["a_zp"]).to(dev).double()[None, :, None]
    b = torch.from_numpy(x["b"]).to(dev).double() - torch.from_numpy(x["b_zp"]).to(dev).double()[None, None, :]
    ref = torch.matmul(a, b)
    assert torch.equal(y.double(), ref)


def _qlinear_args(c, dt, dev, f16=False):
    def sc(v):
        return T(np.array(v, np.float16 if f16 else np.float32), dev)
    return (T(np.array(c["a"], dt).reshape(c["a_shape"]), dev), sc(c["a_scale"]), T(np.array(c["a_zp"], dt), dev),
            T(np.array(c["b"], dt).reshape(c["b_shape"]), dev), sc(c["b_scale"]), T(np.array(c["b_zp"], dt), dev),
            sc(c["y_scale"]), T(np.array(c["y_zp"], dt), dev))


def test_qlinear_known_answers(olamd, golden, dev):
    for c in golden["qlinear_matmul"]:
        dt = NP[c["dtype"]]
        y = olamd.qlinear_matmul(*_qlinear_args(c, dt, dev))
        assert y.cpu().reshape(-1).tolist() == c["y"], c["name"]
    # fp16 scales give the same 2-D outputs (cases_qlinearmatmul.cc:172-184)
    for c in golden["qlinear_matmul"][:2]:
        y = olamd.qlinear_matmul(*_qlinear_args(c, NP[c["dtype"]], dev, f16=True))
        assert y.cpu().reshape(-1).tolist() == c["y"], c["name"]


@pytest.mark.parametrize("shapes", [((64, 256), (256, 128)), ((300, 200), (200, 136)),
                                    ((2, 96, 64), (64, 80)), ((3, 17, 40), (3, 40, 24)),
                                    ((1024, 512), (512, 384)),
                                    # whole K steps without zero-point sums (the K-split
                                    # waves): one, three and five steps, tails, batches
                                    ((300, 384), (384, 136)), ((3, 50, 128), (3, 128, 48)),
                                    ((257, 640), (640, 272))])
@pytest.mark.parametrize("dts", [(np.uint8, np.int8, np.uint8), (np.int8, np.int8, np.int8),
                                 (np.uint8, np.uint8, np.int8), (np.int8, np.uint8, np.uint8)],
                         ids=["u8s8-u8", "s8s8-s8", "u8u8-s8", "s8u8-u8"])
def test_qlinear_vs_oracle(olamd, oracle, dev, shapes, dts):
    a_shape, b_shape = shapes
    rng = np.random.default_rng(zlib.crc32(repr((a_shape, b_shape, str(dts))).encode()))
    ia, ib, iy = np.iinfo(dts[0]), np.iinfo(dts[1]), np.iinfo(dts[2])
    a = rng.integers(ia.min, ia.max + 1, a_shape).astype(dts[0])
    b = rng.integers(ib.min, ib.max + 1, b_shape).astype(dts[1])
    K = a_shape[-1]
    for trial in range(3):
        za = int(rng.integers(ia.min, ia.max + 1)) if trial else (128 if dts[0] == np.uint8 else 0)
        zb = int(rng.integers(ib.min, ib.max + 1)) if trial else (128 if dts[1] == np.uint8 else 0)
        a_s, b_s = np.float32(rng.uniform(0.005, 0.03)), np.float32(rng.uniform(0.001, 0.01))
        # y_scale maps max|acc| to ~100 output steps; y_zero_point centres the
        # mean, so the outputs exercise rounding rather than only saturation
        acc = np.matmul(a.astype(np.int64) - za, b.astype(np.int64) - zb)
        y_s = np.float32(a_s * b_s * (float(np.abs(acc).max()) + 1.0) / 100.0)
        cs = np.float32(np.float32(a_s * b_s) / y_s)
        mid = (int(iy.min) + int(iy.max)) // 2
        zy = int(np.clip(mid - round(float(acc.mean()) * float(cs)), iy.min, iy.max))
        args = (T(a, dev), T(np.array(a_s), dev), T(np.array(za, dts[0]), dev), T(b, dev),
                T(np.array(b_s), dev), T(np.array(zb, dts[1]), dev), T(np.array(y_s), dev),
                T(np.array(zy, dts[2]), dev))
        y = olamd.qlinear_matmul(*args).cpu().numpy()
        ref = oracle.qlinear_matmul(a, a_s, za, b, b_s, zb, y_s, zy,
                                    y_dtype=oracle.INT8 if dts[2] == np.int8 else oracle.UINT8)
        assert np.array_equal(y, ref), trial
        # the outputs are not all saturated: the check exercises the rounding
        assert 0.05 < np.mean((ref > iy.min) & (ref < iy.max))


def test_config2_qlinear_full_size(olamd, oracle, dev):
    syn = _synth(olamd)
    x = syn.config_inputs(2)
    args = [T(x[k], dev) for k in ("a", "a_scale", "a_zp", "b", "b_scale", "b_zp", "y_scale", "y_zp")]
    y = olamd.qlinear_matmul(*args)
    got = y.cpu().numpy()
    fx = _fixtures()["c2"]
    assert hashlib.sha256(got.tobytes()).hexdigest() == fx["sha256"]
    # oracle rows at spread positions (bit-exact)
    rows = [0, 1, 255, 256, 1023, 1500, 2047]
    for r in rows:
        ref = oracle.qlinear_matmul(x["a"], x["a_scale"], 128, x["b"], x["b_scale"], 0, x["y_scale"], 128,
                                    rows=(r, r + 1))
        assert np.array_equal(got[r], ref[r]), r
    # full-size closed form: exact int sums in float64, then the fp32 requant
    acc = torch.matmul(args[0].double() - 128.0, args[3].double())
    cs = np.float32(np.float32(x["a_scale"]) * np.float32(x["b_scale"])) / np.float32(x["y_scale"])
    v = torch.round(acc.float() * float(cs)) + 128.0
    ref = v.clamp(0, 255).to(torch.uint8)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("shapes,centred", [(((5, 40000), (40000, 70)), False),
                                            (((2, 3, 33100), (33100, 17)), False),
                                            (((1, 65536), (65536, 16)), False),
                                            (((3, 140000), (140000, 24)), True)])
def test_qlinear_past_int32_exact(olamd, oracle, dev, shapes, centred):
    """K * max|a - za| * max|b - zb| >= 2^31: the reference's int64 sums
    (kq/kernel_qlinearmatmul.cc:187-191) on the int64-accumulating kernel.
    Row 0 against column 0 sums past int32 (every a and b at the far end of
    its range), which a wrapped int32 sum would turn negative; ragged tiles
    and a batch.  With zero points 128 the other sums centre on 0 and y_scale
    spreads them over many output steps, so the rounding is exercised."""
    a_shape, b_shape = shapes
    rng = np.random.default_rng(zlib.crc32(repr(shapes).encode()))
    a = rng.integers(0, 256, a_shape).astype(np.uint8)
    b = rng.integers(0, 256, b_shape).astype(np.uint8)
    far = 0 if centred else 255
    a.reshape(-1, a_shape[-1])[0] = far
    b[:, 0] = far
    za = zb = 128 if centred else 0
    acc = np.matmul(a.astype(np.int64) - za, b.astype(np.int64) - zb)
    assert np.abs(acc).max() >= 2 ** 31
    a_s, b_s = np.float32(0.02), np.float32(0.01)
    spread = float(np.std(acc.reshape(-1, acc.shape[-1])[1:, 1:])) / 8 if centred else float(np.abs(acc).max()) / 200
    y_s = np.float32(a_s * b_s * (spread + 1.0))
    zy = 128 if centred else 20
    args = (T(a, dev), T(np.array(a_s), dev), T(np.array(za, np.uint8), dev), T(b, dev),
            T(np.array(b_s), dev), T(np.array(zb, np.uint8), dev), T(np.array(y_s), dev),
            T(np.array(zy, np.uint8), dev))
    y = olamd.qlinear_matmul(*args).cpu().numpy()
    ref = oracle.qlinear_matmul(a, a_s, za, b, b_s, zb, y_s, zy, y_dtype=oracle.UINT8)
    assert np.array_equal(y, ref)
    assert ref.reshape(-1, ref.shape[-1])[0, 0] == ref.max() > 128  # the sum past int32, the largest output
    if centred:
        assert len(np.unique(ref)) > 10


@pytest.mark.parametrize("a_shape,b_shape", [((6, 45000), (45000, 40)), ((45000,), (45000, 24)),
                                             ((7, 45000), (45000,))])
def test_qlinear_past_int32_signed_and_1d(olamd, oracle, dev, a_shape, b_shape):
    """The int64-accumulating kernel with INT8 a and b, zero points away from
    0 and an INT8 output (the signed clamp and narrowing), and with 1-D
    operands: K * max|a - za| * max|b - zb| = 45000 * 228 * 217 > 2^31, and
    the first row / column pair sums to -45000 * 228 * 217, which a wrapped
    int32 sum would make positive."""
    rng = np.random.default_rng(zlib.crc32(repr((a_shape, b_shape)).encode()))
    a = rng.integers(-128, 128, a_shape).astype(np.int8)
    b = rng.integers(-128, 128, b_shape).astype(np.int8)
    za, zb, zy = 100, -90, -20
    a.reshape(-1, a_shape[-1])[0] = -128
    (b if b.ndim == 1 else b[:, 0])[...] = 127
    a2 = a.reshape(-1, a_shape[-1]).astype(np.int64) - za
    b2 = (b.reshape(-1, 1) if b.ndim == 1 else b).astype(np.int64) - zb
    acc = a2 @ b2
    assert acc[0, 0] == -45000 * 228 * 217 and acc[0, 0] < -2 ** 31
    a_s, b_s = np.float32(0.02), np.float32(0.01)
    y_s = np.float32(a_s * b_s * (float(np.abs(acc).max()) / 100 + 1.0))
    args = (T(a, dev), T(np.array(a_s), dev), T(np.array(za, np.int8), dev), T(b, dev),
            T(np.array(b_s), dev), T(np.array(zb, np.int8), dev), T(np.array(y_s), dev),
            T(np.array(zy, np.int8), dev))
    y = olamd.qlinear_matmul(*args).cpu().numpy()
    ref = oracle.qlinear_matmul(a, a_s, za, b, b_s, zb, y_s, zy, y_dtype=oracle.INT8)
    assert y.dtype == np.int8 and y.shape == ref.shape
    assert np.array_equal(y, ref)
    assert ref.reshape(-1)[0] == ref.min() < -100  # the sum past int32 is the most negative output


def test_qlinear_scalars_host_device_mixed(olamd, oracle, dev):
    """The six scalars read in one pass: device-resident ones copied on the
    call's stream with one synchronisation, host ones read directly; every
    mix (and an fp16 scale) gives the oracle's bytes."""
    rng = np.random.default_rng(11)
    a = rng.integers(0, 256, (33, 96)).astype(np.uint8)
    b = rng.integers(-128, 128, (96, 40)).astype(np.int8)
    vals = [np.array(0.02, np.float32), np.array(131, np.uint8), np.array(0.01, np.float16),
            np.array(-3, np.int8), np.array(0.9, np.float32), np.array(7, np.int8)]
    ref = oracle.qlinear_matmul(a, np.float32(0.02), 131, b, np.float32(np.float16(0.01)), -3, np.float32(0.9), 7,
                                y_dtype=oracle.INT8)
    for mask in (0, 0b101010, 0b010101, 0b111111, 0b100000):
        sc = [T(v, dev) if mask >> i & 1 else v for i, v in enumerate(vals)]
        y = olamd.qlinear_matmul(T(a, dev), sc[0], sc[1], T(b, dev), sc[2], sc[3], sc[4], sc[5]).cpu().numpy()
        assert np.array_equal(y, ref), bin(mask)
