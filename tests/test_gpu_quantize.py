"""GPU parity of QuantizeLinear and DynamicQuantizeLinear (the producers in
front of MatMulInteger / QLinearMatMul) against the CPU oracle and the
reference's known answers.  Both are integer / byte results: bit-exact.

Cases: the known answers of the reference's tests
(tests/golden/reference_known_answers.json); random inputs in every output
type, scale layout (per tensor, per axis, blocked) and x dtype, with and
without a zero point, at ragged sizes that leave vector tails and at
misaligned addresses that take the scalar path; the special values (ties,
NaN, infinities, fp8 overflow and subnormals, zero and subnormal scales);
the BASELINE activation shape [2048, 4096]; and the dynamic quantizer's
two-pass reduction at sizes below, at and above its partial-result limit."""
import os
import zlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DT = {"float": 1, "uint8": 2, "int8": 3, "uint16": 4, "int16": 5, "float16": 10, "float8e4m3fn": 17,
      "uint4": 21, "int4": 22}
NP = {"uint8": np.uint8, "int8": np.int8, "uint16": np.uint16, "int16": np.int16, "float8e4m3fn": np.uint8}
RANGE = {"uint8": (0, 255), "int8": (-128, 127), "uint16": (0, 65535), "int16": (-32768, 32767),
         "uint4": (0, 15), "int4": (-8, 7)}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _dev_tensor(a, dev):
    """numpy storage -> device tensor of the matching torch dtype (uint16
    arrays that hold FLOAT16 bits are handled by the caller)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.uint16)
    return torch.from_numpy(a).to(dev)


def _half(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.float16)


def _xs(oracle, xv, x_dtype, dev):
    """(oracle storage, device tensor) of float32 values in x_dtype."""
    if x_dtype == "float16":
        bits = oracle.f32_to_f16_bits(np.asarray(xv, np.float32))
        return bits, _half(bits, dev)
    a = np.ascontiguousarray(xv, np.float32)
    return a, torch.from_numpy(a).to(dev)


def _zp(oracle, zv, y_dtype, shape):
    if y_dtype in ("uint4", "int4"):
        return oracle.pack_int4(np.asarray(zv).reshape(-1))
    if y_dtype == "float8e4m3fn":
        return oracle.f32_to_f8e4m3fn_bits(np.asarray(zv, np.float32)).reshape(shape)
    return np.asarray(zv, NP[y_dtype]).reshape(shape)


def _storage(y, y_dtype):
    """Device output -> the oracle's raw storage layout."""
    if y_dtype == "float8e4m3fn":
        return y.view(torch.uint8).cpu().numpy()
    if y_dtype == "uint16":
        return y.view(torch.int16).cpu().numpy().view(np.uint16)
    return y.cpu().numpy()


def _run(olamd, oracle, dev, xv, x_dtype, sv, y_dtype, zv=None, axis=1, output_dtype=0, offset=0):
    """Runs the GPU path and the oracle on the same inputs; returns both raw
    storages.  offset > 0 places x (and y) at an address that is not 16-byte
    aligned, which the kernels serve with per-element accesses."""
    x_o, x_t = _xs(oracle, xv, x_dtype, dev)
    s_o, s_t = _xs(oracle, sv, x_dtype, dev)
    zp_o = None if zv is None else _zp(oracle, zv, y_dtype, np.shape(sv))
    zp_t = None if zp_o is None else _dev_tensor(zp_o, dev)
    shape = x_o.shape
    if offset:
        flat = torch.empty(x_t.numel() + offset, dtype=x_t.dtype, device=dev)
        flat[offset:] = x_t.reshape(-1)
        x_t = flat[offset:].view(shape)
    out = None
    if offset:
        n = int(np.prod(shape))
        nbytes = (n + 1) // 2 if y_dtype in ("uint4", "int4") else n
        tdt = {"uint8": torch.uint8, "int8": torch.int8, "uint16": torch.int16, "int16": torch.int16,
               "float8e4m3fn": torch.uint8, "uint4": torch.uint8, "int4": torch.uint8}[y_dtype]
        raw = torch.empty(nbytes + 1, dtype=tdt, device=dev)
        out = raw[1:] if y_dtype in ("uint4", "int4") else raw[1:].view(shape)
    y = olamd.quantize_linear(x_t, s_t, zp_t, axis, output_dtype, y_dtype=DT[y_dtype], out=out)
    torch.cuda.synchronize()
    got = _storage(y, y_dtype)
    # the kernel takes the normalised axis; QuantizeLinear::Run normalises (:928-930)
    oaxis = axis + len(shape) if axis < 0 else axis
    want = oracle.quantize_linear(x_o, DT[x_dtype], s_o, DT[x_dtype], DT[y_dtype], zp_o, oaxis)
    return got.reshape(-1), want.reshape(-1)


def test_known_answers(olamd, oracle, golden, dev):
    for c in golden["quantize_linear"]:
        xv = np.array(c["x"], np.float32).reshape(c["x_shape"])
        sv = np.array(c["scale"], np.float32).reshape(c["scale_shape"])
        x_o, x_t = _xs(oracle, xv, c["x_dtype"], dev)
        s_o, s_t = _xs(oracle, sv, c["scale_dtype"], dev)
        y_dtype = c["y_dtype"]
        zp_t = None
        if c["zp"] is not None:
            zp_t = _dev_tensor(_zp(oracle, c["zp"], y_dtype, c["zp_shape"]), dev)
        odt = DT[c["output_dtype"]] if c.get("output_dtype") else 0
        y = olamd.quantize_linear(x_t, s_t, zp_t, c["axis"], odt, y_dtype=DT[y_dtype])
        got = _storage(y, y_dtype).reshape(-1)
        if y_dtype in ("uint4", "int4"):
            nib = np.stack([got & 15, got >> 4], axis=1).reshape(-1)[:xv.size].astype(np.int64)
            got = np.where(nib >= 8, nib - 16, nib) if y_dtype == "int4" else nib
        assert got.astype(np.int64).tolist() == c["y"], c["name"]


LAYOUTS = [
    # (x shape, axis, scale shape): per tensor, per axis on each dimension,
    # blocked along rows and along columns, ragged element counts
    ((1000,), 1, ()),
    ((7, 37), 1, (37,)),
    ((7, 37), 0, (7,)),
    ((3, 5, 33), -2, (5,)),
    ((3, 5, 33), 2, (33,)),
    ((64, 48), 0, (4, 48)),
    ((12, 96), 1, (12, 6)),
    ((2, 9, 40), 2, (2, 9, 5)),
    ((4111,), 0, ()),
]


@pytest.mark.parametrize("y_dtype", ["uint8", "int8", "uint16", "int16", "uint4", "int4", "float8e4m3fn"])
@pytest.mark.parametrize("x_dtype", ["float", "float16"])
def test_random_vs_oracle(olamd, oracle, dev, y_dtype, x_dtype):
    rng = np.random.default_rng(zlib.crc32(repr((y_dtype, x_dtype)).encode()))
    lo, hi = RANGE.get(y_dtype, (-4, 4))
    for shape, axis, s_shape in LAYOUTS:
        xv = (rng.standard_normal(shape) * rng.choice([2.0, 30.0, 500.0])).astype(np.float32)
        sv = rng.uniform(0.03, 3.0, s_shape).astype(np.float32)
        if y_dtype == "float8e4m3fn":
            zv = rng.choice([0.0, 1.0, -2.0, 0.5, 3.5], s_shape).astype(np.float32)
        else:
            zv = rng.integers(lo // 2 if lo < 0 else 0, hi // 2 + 1, s_shape)
        for with_zp in (True, False):
            if not with_zp and y_dtype not in ("uint8", "int8", "uint16", "int16"):
                continue  # without a zero point the output types are 8- and 16-bit integers
            # without a zero point: output_dtype, or the UINT8 default of a scalar scale
            odt = 0 if with_zp or (s_shape == () and y_dtype == "uint8" and shape[0] % 2) else DT[y_dtype]
            for offset in (0, 1):
                got, want = _run(olamd, oracle, dev, xv, x_dtype, sv, y_dtype, zv if with_zp else None,
                                 axis, odt, offset)
                bad = np.flatnonzero(got != want)
                assert bad.size == 0, (y_dtype, x_dtype, shape, axis, s_shape, with_zp, offset,
                                       bad[:5], got[bad[:5]], want[bad[:5]])


def test_special_values(olamd, oracle, dev):
    """Ties to even before the zero point; NaN -> 0; infinities and
    x / 0 saturate; 0 / 0 -> 0; subnormal inputs and scales; fp8 overflow,
    NaN (with the sign x86-64 gives it), subnormal and rounding ties."""
    tiny = np.float32(1.5e-39)
    xv = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30,
                   tiny, -tiny, 3e-45, 127.5, 128.5, 254.5, 255.5, 65534.5, 7.5, 8.5, -8.5, -7.5,
                   448.0, 464.0, 480.0, 500.0, 1e9, 0.001953125, 0.0029296875, 0.0009765625,
                   0.013671875, 0.0146484375, 1.0625, 1.1875, 3.0e-3, -3.0e-3], np.float32)
    for y_dtype in ("uint8", "int8", "uint16", "int16", "uint4", "int4", "float8e4m3fn"):
        for sv, zv in ((1.0, 0), (1.0, 1), (2.0 ** -130, 0), (0.0, 0), (np.inf, 0), (-1.0, 0)):
            z = zv if y_dtype != "float8e4m3fn" else float(zv)
            got, want = _run(olamd, oracle, dev, xv, "float", np.array(sv, np.float32), y_dtype, z)
            assert np.array_equal(got, want), (y_dtype, sv, zv, np.flatnonzero(got != want)[:5])
    for sv, zv in ((1.0, np.nan), (1.0, -np.nan), (np.nan, 0.0), (-np.nan, 1.0), (0.0, np.nan)):
        got, want = _run(olamd, oracle, dev, xv, "float", np.array(sv, np.float32), "float8e4m3fn", zv)
        assert np.array_equal(got, want), ("float8e4m3fn", sv, zv, np.flatnonzero(got != want)[:5])


# ---- the other output types of the reference: three fp8 variants,
# FLOAT4E2M1, UINT2 / INT2 and the two FLOAT6 types (raw codes throughout) ----
CODES = {"float8e4m3fnuz": 18, "float8e5m2": 19, "float8e5m2fnuz": 20, "float4e2m1": 23, "uint2": 25,
         "int2": 26, "float6e2m3": 27, "float6e3m2": 28}
BITS = {23: 4, 25: 2, 26: 2, 27: 6, 28: 6}
ZP_VALUES = {18: [0.0, 1.0, -2.0, 0.5, 3.5], 19: [0.0, 1.0, -2.0, 0.5, 3.5], 20: [0.0, 1.0, -2.0, 0.5, 3.5],
             23: [0.0, 0.5, -1.0, 1.5], 27: [0.0, 0.25, -1.0, 2.0], 28: [0.0, 0.25, -1.0, 2.0]}


def _zp_raw(oracle, codes, code, s_shape):
    """Zero point codes -> the raw storage QuantizeLinear takes."""
    c = np.asarray(codes).reshape(-1)
    if code in BITS:
        return oracle.pack_bits(c, BITS[code])
    return c.astype(np.uint8).reshape(s_shape)


def _random_zp(oracle, rng, code, s_shape):
    n = int(np.prod(s_shape, dtype=np.int64))
    if code in (25, 26):
        return _zp_raw(oracle, rng.integers(0, 4, n), code, s_shape)
    vals = rng.choice(ZP_VALUES[code], n).astype(np.float32)
    return _zp_raw(oracle, oracle.float_code(vals, code), code, s_shape)


def _run_code(olamd, oracle, dev, xv, x_dtype, sv, code, zp_raw, axis=1, offset=0):
    """GPU and oracle raw outputs of one QuantizeLinear to output type `code`
    (with zp_raw None: no zero point, output_dtype = code)."""
    x_o, x_t = _xs(oracle, xv, x_dtype, dev)
    s_o, s_t = _xs(oracle, sv, x_dtype, dev)
    zp_t = None if zp_raw is None else _dev_tensor(zp_raw, dev)
    shape = x_o.shape
    n = int(np.prod(shape, dtype=np.int64))
    out = None
    if offset:
        flat = torch.empty(x_t.numel() + offset, dtype=x_t.dtype, device=dev)
        flat[offset:] = x_t.reshape(-1)
        x_t = flat[offset:].view(shape)
        nbytes = (n * BITS[code] + 7) // 8 if code in BITS else n
        raw = torch.empty(nbytes + 1, dtype=torch.uint8, device=dev)
        out = raw[1:] if code in BITS else raw[1:].view(shape)
    y = olamd.quantize_linear(x_t, s_t, zp_t, axis, 0 if zp_raw is not None else code, y_dtype=code, out=out)
    torch.cuda.synchronize()
    got = y.view(torch.uint8).cpu().numpy().reshape(-1)
    oaxis = axis + len(shape) if axis < 0 else axis
    want = oracle.quantize_linear(x_o, DT[x_dtype], s_o, DT[x_dtype], code, zp_raw, oaxis).reshape(-1)
    return got, want


@pytest.mark.parametrize("y_name", sorted(CODES))
@pytest.mark.parametrize("x_dtype", ["float", "float16"])
def test_other_outputs_random_vs_oracle(olamd, oracle, dev, y_name, x_dtype):
    """Every scale layout, with a zero point (and without one for the per
    tensor FLOAT4E2M1 / FLOAT6 cases the reference allows), aligned and
    misaligned, at magnitudes inside and far past each type's range."""
    code = CODES[y_name]
    rng = np.random.default_rng(zlib.crc32(repr((y_name, x_dtype)).encode()))
    for shape, axis, s_shape in LAYOUTS:
        xv = (rng.standard_normal(shape) * rng.choice([0.3, 2.0, 30.0, 500.0])).astype(np.float32)
        sv = rng.uniform(0.03, 3.0, s_shape).astype(np.float32)
        zps = [_random_zp(oracle, rng, code, s_shape)]
        if s_shape == () and code in (23, 27, 28):
            zps.append(None)
        for zp in zps:
            for offset in (0, 1):
                got, want = _run_code(olamd, oracle, dev, xv, x_dtype, sv, code, zp, axis, offset)
                bad = np.flatnonzero(got != want)
                assert bad.size == 0, (y_name, x_dtype, shape, axis, s_shape, zp is None, offset,
                                       bad[:5], got[bad[:5]], want[bad[:5]])


@pytest.mark.parametrize("y_name", sorted(CODES))
def test_other_outputs_special_values(olamd, oracle, dev, y_name):
    """Each code's midpoints with its neighbours (ties to even) and the
    points either side, signed zeros, NaN, infinities, overflow, subnormal
    inputs and scales, x / 0, NaN scales and NaN zero points (the fp8
    types' NaN sign as x86-64 gives it)."""
    code = CODES[y_name]
    n = {23: 16, 27: 64, 28: 64, 25: 4, 26: 4}.get(code, 256)
    if code in (25, 26):
        mids = np.arange(-4.5, 4.5, 0.5, dtype=np.float32)
    else:
        raw = np.arange(n, dtype=np.uint8) if code not in BITS else oracle.pack_bits(np.arange(n), BITS[code])
        vals = oracle.dq_decode(raw, code, n).astype(np.float64)
        vals = np.unique(vals[np.isfinite(vals)])
        mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
        mids = np.concatenate([vals.astype(np.float32), mids, np.nextafter(mids, np.float32(np.inf)),
                               np.nextafter(mids, np.float32(-np.inf))])
    tiny = np.float32(1.5e-39)
    xv = np.concatenate([mids, np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30, tiny, -tiny,
                                         3e-45, 1e9, -1e9], np.float32)])
    zero = _zp_raw(oracle, [0], code, ())
    cases = [(1.0, zero), (2.0 ** -130, zero), (0.0, zero), (np.inf, zero), (-1.0, zero), (np.nan, zero),
             (-np.nan, zero), (3.0, _random_zp(oracle, np.random.default_rng(code), code, ()))]
    if code in (23, 27, 28):
        cases += [(1.0, None), (-1.0, None), (0.0, None)]
    nan_codes = {18: [0x80], 19: [0x7E, 0xFE, 0x7F, 0xFD], 20: [0x80]}.get(code, [])
    cases += [(sv, _zp_raw(oracle, [c], code, ())) for c in nan_codes for sv in (1.0, 0.0, np.nan)]
    for sv, zp in cases:
        got, want = _run_code(olamd, oracle, dev, xv, "float", np.array(sv, np.float32), code, zp)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, (y_name, sv, None if zp is None else zp.tolist(), bad[:5], got[bad[:5]],
                               want[bad[:5]])


def test_activation_shape(olamd, oracle, dev):
    """The BASELINE activation [2048, 4096] in both fp32 -> uint8 (scalar
    scale and zero point, the QLinearMatMul producer) and fp16 -> int8 per
    row (axis 0)."""
    rng = np.random.default_rng(7)
    xv = (rng.standard_normal((2048, 4096)) * 4).astype(np.float32)
    got, want = _run(olamd, oracle, dev, xv, "float", np.array(0.031, np.float32), "uint8", 128)
    assert np.array_equal(got, want)
    sv = rng.uniform(0.01, 0.1, (2048,)).astype(np.float32)
    got, want = _run(olamd, oracle, dev, xv, "float16", sv, "int8", np.zeros(2048, np.int64), axis=0)
    assert np.array_equal(got, want)


def test_unsupported_output_rejected(olamd, dev):
    """FLOAT8E8M0 has no QuantizeLinear path in the reference either."""
    x = torch.zeros(8, device=dev)
    s = torch.ones((), device=dev)
    z = torch.zeros(1, dtype=torch.uint8, device=dev)
    with pytest.raises(olamd.InvalidArgument):
        olamd.quantize_linear(x, s, z, y_dtype=24, out=torch.empty(8, dtype=torch.uint8, device=dev))


# ---- DynamicQuantizeLinear ---------------------------------------------------

def _dql(olamd, dev, xv, offset=0):
    x_t = torch.from_numpy(np.ascontiguousarray(xv, np.float32)).to(dev)
    out = None
    if offset:
        flat = torch.empty(x_t.numel() + offset, device=dev)
        flat[offset:] = x_t.reshape(-1)
        x_t = flat[offset:].view(x_t.shape)
        raw = torch.empty(x_t.numel() + 1, dtype=torch.uint8, device=dev)
        out = (raw[1:].view(x_t.shape), torch.empty((), device=dev),
               torch.empty((), dtype=torch.uint8, device=dev))
    y, sc, zp = olamd.dynamic_quantize_linear(x_t, out)
    return y.cpu().numpy(), np.float32(sc.item()), int(zp.item())


def test_dynamic_known_answers(olamd, oracle, golden, dev):
    for c in golden["dynamic_quantize_linear"]:
        xv = np.array(c["x"], np.float32).reshape(c["x_shape"])
        y, sc, zp = _dql(olamd, dev, xv)
        y_o, sc_o, zp_o = oracle.dynamic_quantize_linear(xv)
        assert sc == np.float32(sc_o) and abs(float(sc) - c["scale"]) <= c["scale_tol"], c["name"]
        assert zp == int(zp_o) == c["zp"], c["name"]
        assert y.reshape(-1).tolist() == c["y"], c["name"]


@pytest.mark.parametrize("n", [1, 7, 16, 4095, 4096, 65539, 1 << 20, 2_097_152, 5_000_011, 8_388_608,
                               12_582_912])
def test_dynamic_random_vs_oracle(olamd, oracle, dev, n):
    """Sizes below, at and above 512 x 4096 elements, where every workgroup
    of the min / max pass covers more than one chunk, up to the BASELINE
    activation (2^23) and beyond; ragged sizes and misaligned offsets take
    the per-element paths."""
    rng = np.random.default_rng(n)
    for shift, spread, offset in ((0.0, 1.0, 0), (3.0, 0.5, 1), (-5.0, 0.01, 0), (0.0, 1e-30, 2)):
        xv = (shift + spread * rng.standard_normal(n)).astype(np.float32)
        y, sc, zp = _dql(olamd, dev, xv, offset)
        y_o, sc_o, zp_o = oracle.dynamic_quantize_linear(xv)
        assert sc == np.float32(sc_o) and zp == int(zp_o), (n, shift, spread, sc, sc_o, zp, zp_o)
        bad = np.flatnonzero(y.reshape(-1) != y_o.reshape(-1))
        assert bad.size == 0, (n, shift, spread, offset, bad[:5])


def test_dynamic_constant_and_signed_inputs(olamd, oracle, dev):
    for xv in (np.zeros(1000, np.float32), np.full(999, 3.25, np.float32), np.full(4097, -2.0, np.float32),
               np.array([-0.0, 0.0, -0.0], np.float32), np.array([1e-45, -1e-45], np.float32),
               np.array([3.4e38, -3.4e38, 0.0], np.float32)):
        y, sc, zp = _dql(olamd, dev, xv)
        y_o, sc_o, zp_o = oracle.dynamic_quantize_linear(xv)
        assert sc == np.float32(sc_o) and zp == int(zp_o) and np.array_equal(y, y_o), xv[:3]


def test_dynamic_non_finite_rejected(olamd, golden, dev):
    """The reference raises for NaN / +-inf (kernel_dynamicquantizelinear.cc:
    86-87); the library reports them as y_scale = NaN, which the wrapper
    turns into the same InvalidArgument."""
    for v in golden["dynamic_quantize_linear_rejects"]["values"]:
        for pos in (0, 5000, 99_999):
            xv = np.zeros(100_000, np.float32)
            xv[pos] = float(v)
            x_t = torch.from_numpy(xv).to(dev)
            with pytest.raises(olamd.InvalidArgument, match="x elements must be finite"):
                olamd.dynamic_quantize_linear(x_t)
            _, sc, _ = olamd.dynamic_quantize_linear(x_t, check=False)
            assert torch.isnan(sc).item()
