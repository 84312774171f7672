"""GPU parity of the float paths against the CPU oracle and the reference's
known answers:

- DequantizeLinear and the FLOAT -> FLOAT16 / BFLOAT16 Cast: bit-exact.
- FLOAT16 / BFLOAT16 MatMul and the fused DequantizeLinear -> [Cast] ->
  MatMul: the dequantised weights are rounded exactly as the unfused chain
  rounds them, so only the fp32 summation order differs from the oracle;
  the fp8 matrix-core path instead scales the fp32 sums, skipping each
  weight's bf16 rounding (<= 2^-8 relative), which the magnitude term below
  covers.  The stated tolerance is
      |got - ref| <= 1e-2 * |ref| + u * sum_k |a_mk * w_kn|
  with u the unit roundoff of the output type (2^-11 FLOAT16, 2^-8 BFLOAT16):
  relative 1e-2 as the north star states, plus the magnitude term that a
  pure relative bound cannot provide for outputs that cancel to near zero.
"""
import json
import os
import zlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NP = {"uint8": np.uint8, "int8": np.int8, "uint16": np.uint16, "int16": np.int16}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def T(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def bits_tensor(bits, dt, dev):
    """uint16 bit patterns -> device torch tensor of FLOAT16 / BFLOAT16."""
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev)
    return t.view(torch.bfloat16 if dt == "bf16" else torch.float16)


def tensor_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def decode(bits, dt, oracle):
    return (oracle.bf16_bits_to_f32(bits) if dt == "bf16" else oracle.f16_bits_to_f32(bits)).astype(np.float64)


def assert_close(got_bits, ref_bits, mag, dt, oracle, what):
    got, ref = decode(got_bits, dt, oracle), decode(ref_bits, dt, oracle)
    u = 2.0 ** -8 if dt == "bf16" else 2.0 ** -11
    bound = 1e-2 * np.abs(ref) + u * mag
    err = np.abs(got - ref)
    bad = ~(err <= bound)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; worst err "
                           f"{err[bad].max():.3g} at bound {bound[bad][np.argmax(err[bad])]:.3g}")


# ---------------------------------------------------------------------------
# DequantizeLinear


def _x_raw(c, oracle):
    dt = c["x_dtype"]
    if dt == "float8e4m3fn":
        return oracle.f32_to_f8e4m3fn_bits(c["x_float"]), oracle.FLOAT8E4M3FN
    if dt in ("int4", "uint4"):
        return oracle.pack_int4(c["x"]), oracle.INT4 if dt == "int4" else oracle.UINT4
    code = {"uint8": oracle.UINT8, "int8": oracle.INT8, "uint16": oracle.UINT16, "int16": oracle.INT16}[dt]
    return np.array(c["x"], NP[dt]), code


def _zp_raw(c, oracle, x_code):
    if c["zp"] is None:
        return None
    v = c["zp"]["values"]
    if x_code in (oracle.INT4, oracle.UINT4):
        return oracle.pack_int4(v)
    if x_code == oracle.FLOAT8E4M3FN:
        return oracle.f32_to_f8e4m3fn_bits(v)
    return np.array(v, NP[c["x_dtype"]]).reshape(c["zp"]["shape"])


def test_dequantize_known_answers(olamd, oracle, golden, dev):
    for c in golden["dequantize_linear"]:
        x, code = _x_raw(c, oracle)
        if c["scale_dtype"] == "float16":
            sc = (np.array(c["scale_bits"], np.uint16).view(np.float16) if "scale_bits" in c
                  else np.array(c["scale_float"], np.float16))
        else:
            sc = np.array(c["scale"], np.float32)
        sc = sc.reshape(c["scale_shape"])
        zp = _zp_raw(c, oracle, code)
        y = olamd.dequantize_linear(x, sc, zp, axis=c["axis"], x_dtype=code, x_shape=c["x_shape"])
        y = y.cpu().numpy() if hasattr(y, "cpu") else y
        if "y_bits" in c:
            assert y.view(np.uint16).reshape(-1).tolist() == c["y_bits"], c["name"]
        else:
            assert y.astype(np.float32).reshape(-1).tolist() == [float(v) for v in c["y"]], c["name"]


DQ_CASES = [
    # (x kind, x shape, scale kind, axis, block)
    ("uint8", (37, 20), "tensor", 1, None),
    ("int8", (6, 50, 7), "axis", 1, None),
    ("int16", (40, 33), "axis", 0, None),
    ("uint16", (9, 64), "blocked", 1, 16),
    ("int32", (12, 30), "axis", 1, None),
    ("int4", (64, 48), "blocked", 0, 32),
    ("uint4", (5, 7, 9), "axis", 2, None),
    ("int4", (33,), "tensor", 0, None),
    ("fp8", (128, 24), "axis", 1, None),
    ("fp8", (2, 64, 8), "blocked", 1, 16),
    # every code of the further types (NaN and infinity codes included)
    ("e4m3fnuz", (64, 24), "axis", 1, None),
    ("e5m2", (2, 64, 8), "blocked", 1, 16),
    ("e5m2fnuz", (37, 20), "tensor", 1, None),
    ("fp4", (64, 48), "blocked", 0, 32),
    ("uint2", (5, 7, 12), "axis", 2, None),
    ("int2", (33, 4), "tensor", 0, None),
    ("fp6e2m3", (32, 16), "axis", 0, None),
    ("fp6e3m2", (8, 64), "blocked", 1, 32),
]
# the further DequantizeLinear input types: oracle dtype name, bits per code
SUB_KINDS = {"e4m3fnuz": ("FLOAT8E4M3FNUZ", 8), "e5m2": ("FLOAT8E5M2", 8), "e5m2fnuz": ("FLOAT8E5M2FNUZ", 8),
             "fp4": ("FLOAT4E2M1", 4), "uint2": ("UINT2", 2), "int2": ("INT2", 2), "fp6e2m3": ("FLOAT6E2M3", 6),
             "fp6e3m2": ("FLOAT6E3M2", 6)}


def _codes(oracle, rng, kind, count, shape):
    name, bits = SUB_KINDS[kind]
    q = rng.integers(0, 1 << bits, count)
    raw = q.astype(np.uint8).reshape(shape) if bits == 8 else oracle.pack_bits(q, bits)
    return raw, getattr(oracle, name)


@pytest.mark.parametrize("case", DQ_CASES, ids=[f"{c[0]}-{c[2]}-ax{c[3]}" for c in DQ_CASES])
@pytest.mark.parametrize("s16", [False, True], ids=["f32scale", "f16scale"])
@pytest.mark.parametrize("with_zp", [False, True], ids=["nozp", "zp"])
def test_dequantize_vs_oracle(olamd, oracle, dev, case, s16, with_zp):
    kind, shape, skind, axis, block = case
    rng = np.random.default_rng(zlib.crc32(repr((case, s16, with_zp)).encode()))
    n = int(np.prod(shape))
    if kind in SUB_KINDS:
        x, code = _codes(oracle, rng, kind, n, shape)
    elif kind in ("int4", "uint4"):
        lo, hi = (-8, 8) if kind == "int4" else (0, 16)
        q = rng.integers(lo, hi, n)
        x, code = oracle.pack_int4(q), oracle.INT4 if kind == "int4" else oracle.UINT4
    elif kind == "fp8":
        x, code = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(n).astype(np.float32) * 40), oracle.FLOAT8E4M3FN
    else:
        dt = {"uint8": np.uint8, "int8": np.int8, "int16": np.int16, "uint16": np.uint16, "int32": np.int32}[kind]
        info = np.iinfo(dt)
        lo, hi = max(info.min, -100000), min(info.max, 100000)
        x = rng.integers(lo, hi + 1, n).astype(dt).reshape(shape)
        code = {"uint8": oracle.UINT8, "int8": oracle.INT8, "int16": oracle.INT16, "uint16": oracle.UINT16,
                "int32": oracle.INT32}[kind]
    if skind == "tensor":
        s_shape = ()
    elif skind == "axis":
        s_shape = (shape[axis],)
    else:
        s_shape = tuple(d // block if i == axis else d for i, d in enumerate(shape))
    sc = rng.uniform(0.01, 0.5, s_shape).astype(np.float32)
    if s16:
        sc = sc.astype(np.float16)
    zp = None
    if with_zp:
        m = int(np.prod(s_shape)) if s_shape else 1
        if kind in SUB_KINDS:
            zp = _codes(oracle, rng, kind, m, s_shape)[0]
        elif kind in ("int4", "uint4"):
            lo, hi = (-8, 8) if kind == "int4" else (0, 16)
            zp = oracle.pack_int4(rng.integers(lo, hi, m))
        elif kind == "fp8":  # finite fp8 zero points, signed and fractional
            zp = oracle.f32_to_f8e4m3fn_bits(rng.choice([0.0, 0.5, -1.0, 2.0, -3.5, 448.0], m).astype(np.float32))
            zp = zp.reshape(s_shape)
        else:
            zp = rng.integers(-20 if kind not in ("uint8", "uint16") else 0, 30, m).astype(x.dtype).reshape(s_shape)
    got = olamd.dequantize_linear(T(x, dev), T(sc, dev), None if zp is None else T(zp, dev), axis=axis,
                                  x_dtype=code, x_shape=shape)
    ref = oracle.dequantize_linear(x, code, shape, sc.view(np.uint16) if s16 else sc,
                                   oracle.FLOAT16 if s16 else oracle.FLOAT, zp, axis)
    if s16:
        assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), ref)
    else:
        g = got.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), ref.view(np.uint32))


def test_cast_vs_oracle(olamd, oracle, dev):
    rng = np.random.default_rng(7)
    u = rng.integers(0, 2**32, 1 << 16, dtype=np.uint64).astype(np.uint32)
    u[:8] = [0, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0x7f800001, 0x3f808000, 0x3f818000]
    u[100:1100] = (u[100:1100] & 0xffff0000) | 0x8000          # bf16 ties
    u[2000:3000] = (u[2000:3000] & 0xffffe000) | 0x1000        # fp16 ties
    x = u.view(np.float32)
    tx = T(x, dev)
    yb = tensor_bits(olamd.cast(tx, olamd.BFLOAT16))
    yh = tensor_bits(olamd.cast(tx, olamd.FLOAT16))
    nan = np.isnan(x)
    rb, rh = oracle.f32_to_bf16_bits(x), oracle.f32_to_f16_bits(x)
    assert np.array_equal(yb[~nan], rb[~nan]) and np.array_equal(yh[~nan], rh[~nan])
    # NaN: the reference keeps the sign/payload top bits (bf16) or writes sign|0x7e00 (fp16)
    assert np.array_equal(yb[nan], rb[nan]) and np.array_equal(yh[nan], rh[nan])


# ---------------------------------------------------------------------------
# FLOAT16 / BFLOAT16 MatMul

MM_SHAPES = [
    ((300, 192), (192, 144)),        # MFMA core: tails in M and N
    ((2, 64, 128), (128, 64)),       # MFMA core, batched A
    ((3, 1, 40, 64), (5, 64, 32)),   # broadcast batch dims
    ((37, 45), (45, 29)),            # simple kernel (K % 64, N % 16)
    ((64,), (64, 40)),               # 1-D A
    ((8, 0), (0, 16)),               # K = 0
]


@pytest.mark.parametrize("shapes", MM_SHAPES, ids=[f"{a}x{b}" for a, b in MM_SHAPES])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_matmul_half_vs_oracle(olamd, oracle, dev, shapes, dt):
    a_shape, b_shape = shapes
    rng = np.random.default_rng(zlib.crc32(repr((a_shape, b_shape, dt)).encode()))
    enc = oracle.f32_to_bf16_bits if dt == "bf16" else oracle.f32_to_f16_bits
    a = enc(rng.standard_normal(a_shape).astype(np.float32))
    b = enc(rng.standard_normal(b_shape).astype(np.float32))
    y = olamd.matmul(bits_tensor(a, dt, dev), bits_tensor(b, dt, dev))
    code = oracle.BFLOAT16 if dt == "bf16" else oracle.FLOAT16
    ref = oracle.matmul_half(a, b, code)
    assert tuple(y.shape) == ref.shape
    mag = np.abs(decode(a, dt, oracle)) @ np.abs(decode(b, dt, oracle)) if a.size and b.size else np.zeros(ref.shape)
    assert_close(tensor_bits(y), ref, np.asarray(mag).reshape(ref.shape), dt, oracle, f"{shapes} {dt}")


def test_matmul_half_known_answer(olamd, oracle, golden, dev):
    c = golden["matmul_half"][0]
    for dt, tol in (("f16", c["tol_float16"]), ("bf16", c["tol_bfloat16"])):
        enc = oracle.f32_to_bf16_bits if dt == "bf16" else oracle.f32_to_f16_bits
        a = enc(np.array(c["a"], np.float32).reshape(c["a_shape"]))
        b = enc(np.array(c["b"], np.float32).reshape(c["b_shape"]))
        y = decode(tensor_bits(olamd.matmul(bits_tensor(a, dt, dev), bits_tensor(b, dt, dev))), dt, oracle)
        assert np.abs(y.reshape(-1) - np.array(c["y"])).max() <= tol


# ---------------------------------------------------------------------------
# Fused DequantizeLinear -> [Cast] -> MatMul


def _chain_ref(oracle, a_bits, x, code, K, N, sc, s16, zp, axis, cast, dt, rows=None):
    """Oracle chain of the unfused graph: DequantizeLinear, optional Cast, MatMul."""
    w = oracle.dequantize_linear(x, code, (K, N), sc.view(np.uint16) if s16 else sc,
                                 oracle.FLOAT16 if s16 else oracle.FLOAT, zp, axis)
    if not s16:
        w = oracle.f32_to_bf16_bits(w) if cast == "bf16" else oracle.f32_to_f16_bits(w)
    a = a_bits if rows is None else a_bits[rows]
    y = oracle.matmul_half(a, w, oracle.BFLOAT16 if dt == "bf16" else oracle.FLOAT16, nthreads=os.cpu_count())
    mag = np.abs(decode(a, dt, oracle)) @ np.abs(decode(w, dt, oracle))
    return y, mag


DQM_CASES = [
    # name, weight kind, M, K, N, scale mode ("blocked"/"col"/"tensor"), block, zp, activations dtype
    ("gemv-int4-b32", "int4", 8, 512, 1024, "blocked", 32, False, "f16"),
    ("gemv-int4-b64-zp", "int4", 5, 256, 136, "blocked", 64, True, "f16"),
    ("gemv-uint4-col", "uint4", 1, 1024, 264, "col", None, False, "f16"),
    ("gemv-uint4-b32-zp", "uint4", 16, 2048, 392, "blocked", 32, True, "f16"),
    ("gemv-int4-tensor", "int4", 3, 96, 64, "tensor", None, False, "f16"),
    ("gemv-int4-longk", "int4", 8, 8192, 128, "blocked", 32, False, "f16"),
    # N % 16 == 0: 16 columns per lane, 256-column strips (the last one partial)
    ("gemv-uint4-b32-zp-wide", "uint4", 16, 2048, 400, "blocked", 32, True, "f16"),
    ("gemv-int4-col-zp-wide", "int4", 4, 512, 784, "col", None, True, "f16"),
    ("gemv-int4-tensor-zp-wide", "int4", 2, 160, 48, "tensor", None, True, "f16"),
    ("gemv-uint4-b16-wide", "uint4", 7, 1024, 512, "blocked", 16, False, "f16"),
    ("gemv-int4-b128-wide", "int4", 12, 4096, 2304, "blocked", 128, False, "f16"),
    ("fp8-col", "fp8", 300, 256, 272, "col", None, False, "bf16"),
    ("fp8-tensor", "fp8", 64, 128, 64, "tensor", None, False, "bf16"),
    ("fallback-int8-f16", "int8", 37, 80, 24, "col", None, True, "f16"),
    ("fallback-uint8-bf16", "uint8", 40, 128, 48, "blocked", 32, False, "bf16"),
    ("fallback-int4-prefill", "int4", 300, 128, 96, "blocked", 32, False, "f16"),
    ("fallback-fp8-oddN", "fp8", 20, 64, 30, "col", None, False, "bf16"),
    ("fallback-int4-bf16", "int4", 9, 64, 40, "blocked", 16, False, "bf16"),
]


@pytest.mark.parametrize("case", DQM_CASES, ids=[c[0] for c in DQM_CASES])
def test_dq_matmul_vs_oracle(olamd, oracle, dev, case):
    name, kind, M, K, N, smode, block, with_zp, dt = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    enc = oracle.f32_to_bf16_bits if dt == "bf16" else oracle.f32_to_f16_bits
    a = enc(rng.standard_normal((M, K)).astype(np.float32))
    if kind in ("int4", "uint4"):
        lo, hi = (-8, 8) if kind == "int4" else (0, 16)
        x, code = oracle.pack_int4(rng.integers(lo, hi, K * N)), oracle.INT4 if kind == "int4" else oracle.UINT4
    elif kind == "fp8":
        x, code = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(K * N).astype(np.float32)).reshape(K, N), oracle.FLOAT8E4M3FN
    else:
        dtp = np.int8 if kind == "int8" else np.uint8
        info = np.iinfo(dtp)
        x, code = rng.integers(info.min, info.max + 1, (K, N)).astype(dtp), oracle.INT8 if kind == "int8" else oracle.UINT8
    if smode == "blocked":
        s_shape, axis = (K // block, N), 0
    elif smode == "col":
        s_shape, axis = (N,), 1
    else:
        s_shape, axis = (), 1
    # fp16 scales -> DequantizeLinear emits FLOAT16 (fp16 activations, no Cast);
    # bf16 activations need FLOAT scales and a Cast to BFLOAT16
    s16 = dt == "f16"
    sc = rng.uniform(0.002, 0.02, s_shape).astype(np.float16 if s16 else np.float32)
    zp = None
    if with_zp:
        m = int(np.prod(s_shape)) if s_shape else 1
        if kind in ("int4", "uint4"):
            lo, hi = (-8, 8) if kind == "int4" else (0, 16)
            zp = oracle.pack_int4(rng.integers(lo, hi, m))
        else:
            zp = rng.integers(0, 20, m).astype(x.dtype).reshape(s_shape)
    y = olamd.dequantize_linear_matmul(bits_tensor(a, dt, dev), T(x, dev), T(sc, dev),
                                       None if zp is None else T(zp, dev), axis=axis,
                                       cast_to=0 if s16 else olamd.BFLOAT16, x_dtype=code, x_shape=(K, N))
    ref, mag = _chain_ref(oracle, a, x, code, K, N, sc, s16, zp, axis, "bf16", dt)
    assert_close(tensor_bits(y), ref, mag, dt, oracle, name)


def test_dq_matmul_repeat_calls_reset_counters(olamd, oracle, dev):
    """The split-K GEMV leaves its per-strip counters at zero: two calls in a
    row (the second smaller) must both be right."""
    rng = np.random.default_rng(5)
    for M, K, N in ((8, 4096, 1024), (4, 2048, 256)):
        a = oracle.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
        q = rng.integers(-8, 8, K * N)
        x = oracle.pack_int4(q)
        sc = rng.uniform(0.002, 0.02, (K // 32, N)).astype(np.float16)
        y = olamd.dequantize_linear_matmul(bits_tensor(a, "f16", dev), T(x, dev), T(sc, dev), None, axis=0,
                                           x_dtype=olamd.INT4, x_shape=(K, N))
        ref, mag = _chain_ref(oracle, a, x, oracle.INT4, K, N, sc, True, None, 0, None, "f16")
        assert_close(tensor_bits(y), ref, mag, "f16", oracle, f"repeat {M}x{K}x{N}")


# ---------------------------------------------------------------------------
# Full-size configurations 3 and 4 against the committed oracle fixtures


def _synth():
    import importlib.util
    spec = importlib.util.spec_from_file_location("olamd_synth", os.path.join(ROOT, "onnx-light_amd", "synth.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_config3_full_size(olamd, oracle, dev):
    fx = np.load(os.path.join(ROOT, "tests", "golden", "config_fixtures_float.npz"))
    x = _synth().config_inputs(3)
    K, N = x["w_shape"]
    a = x["a"].view(np.uint16)
    y = olamd.dequantize_linear_matmul(bits_tensor(a, "f16", dev), T(x["w"], dev), T(x["scale"], dev), None,
                                       axis=0, x_dtype=olamd.INT4, x_shape=(K, N))
    got = tensor_bits(y)
    rows = fx["c3_rows"]
    ref = fx["c3_y_bits"]
    w = oracle.dequantize_linear(x["w"], oracle.INT4, (K, N), x["scale"].view(np.uint16), oracle.FLOAT16, None, 0)
    mag = np.abs(decode(a[rows], "f16", oracle)) @ np.abs(decode(w, "f16", oracle))
    assert_close(got[rows], ref, mag, "f16", oracle, "config 3")


def test_config4_full_size(olamd, oracle, dev):
    fx = np.load(os.path.join(ROOT, "tests", "golden", "config_fixtures_float.npz"))
    x = _synth().config_inputs(4)
    K, N = x["w"].shape
    y = olamd.dequantize_linear_matmul(bits_tensor(x["a_bits"], "bf16", dev), T(x["w"], dev), T(x["scale"], dev),
                                       None, axis=1, cast_to=olamd.BFLOAT16, x_dtype=olamd.FLOAT8E4M3FN)
    rows = fx["c4_rows"]
    got = tensor_bits(y)[rows]
    w = oracle.f32_to_bf16_bits(oracle.dequantize_linear(x["w"], oracle.FLOAT8E4M3FN, (K, N), x["scale"],
                                                         oracle.FLOAT, None, 1))
    mag = np.abs(decode(x["a_bits"][rows], "bf16", oracle)) @ np.abs(decode(w, "bf16", oracle))
    assert_close(got, fx["c4_y_bits"], mag, "bf16", oracle, "config 4")
    _fp8_chain_closed_form(y, x["a_bits"], x["w"], x["scale"], dev, "config 4")
    # the bench draws the same inputs on the GPU (torch SplitMix64): bit for bit these
    xt = _synth().config4_torch(dev)
    assert torch.equal(xt["w"].cpu(), torch.from_numpy(x["w"]))
    assert torch.equal(xt["a"].view(torch.int16).cpu(), torch.from_numpy(x["a_bits"].view(np.int16)))
    assert torch.equal(xt["scale"].cpu(), torch.from_numpy(x["scale"]))


def _fp8_chain_closed_form(y, a_bits, w_bits, scale, dev, what):
    """Every output element against a float64 closed form of the chain,
    computed on the device: W = bf16(fp32(decode(x)) * scale[n]), the rounding
    of DequantizeLinear(FLOAT) -> Cast(BFLOAT16), then sum_k a_mk * W_kn in
    float64.  The bound is what the fused path can differ by, nothing more:
    it skips each weight's bf16 rounding (|q s - W| <= u |q s|, u = 2^-8 the
    unit roundoff of bf16's 8 significant bits), sums in fp32 in another
    order (<= 2 K 2^-24 of sum_k |a q s|, allowing a truncating adder) and
    rounds the scaled sum once to bf16 (<= u |y|):
        |got - ref| <= u (1 + 2^-7) |ref| + (u (1 + 2^-7) + 2 K 2^-24) sum_k |a_mk W_kn|.
    It covers every tile of the launch; the oracle rows above pin the weight
    decode and the chain's rounding bit for bit, and test_gpu_exact.py pins
    every k-term of this GEMM on dyadic inputs."""
    w = T(w_bits, dev).view(torch.float8_e4m3fn).to(torch.float32) * T(scale, dev)
    w64 = w.to(torch.bfloat16).to(torch.float64)
    del w
    K = w64.shape[0]
    a64 = bits_tensor(a_bits, "bf16", dev).to(torch.float64)
    ref = a64 @ w64
    mag = a64.abs() @ w64.abs()
    del a64, w64
    err = (y.to(torch.float64) - ref).abs()
    c = 2.0 ** -8 * (1 + 2.0 ** -7)
    bad = ~(err <= c * ref.abs() + (c + 2.0 * K * 2.0 ** -24) * mag)
    n_bad = int(bad.sum())
    assert n_bad == 0, f"{what}: {n_bad} of {bad.numel()} outside tolerance (max err {float(err.max()):.3g})"
    assert bool(torch.isfinite(y.float()).all())


def test_fp8_gemm_column_split(olamd, oracle, dev):
    """A 4096 x 8448 fp8 GEMM has 528 tiles of 256 x 256: the first 8192
    columns run as whole rounds of such tiles and the last 256 columns as a
    second launch in 256 x 128 tiles, with the full matrices' row pitches and
    the offset scales.  Rows checked against the oracle chain, every column."""
    rng = np.random.default_rng(20261202)
    M, K, N = 4096, 64, 8448
    a = oracle.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    x = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(K * N).astype(np.float32)).reshape(K, N)
    sc = rng.uniform(0.005, 0.05, N).astype(np.float32)
    y = olamd.dequantize_linear_matmul(bits_tensor(a, "bf16", dev), T(x, dev), T(sc, dev), None, axis=1,
                                       cast_to=olamd.BFLOAT16, x_dtype=oracle.FLOAT8E4M3FN, x_shape=(K, N))
    rows = np.array([0, 1, 255, 256, 2047, 3840, 4095])
    ref, mag = _chain_ref(oracle, a, x, oracle.FLOAT8E4M3FN, K, N, sc, False, None, 1, "bf16", "bf16", rows=rows)
    assert_close(tensor_bits(y)[rows], ref, mag, "bf16", oracle, "fp8 column split")
    _fp8_chain_closed_form(y, a, x, sc, dev, "fp8 column split")


def test_fp8_gemm_large_odd_k_step(olamd, oracle, dev):
    """512 tiles of 256 x 256 would take the whole-K-step 256 x 256 kernel,
    but K = 96 leaves half a K step: the launcher falls back to 256 x 128
    tiles (every element against the float64 closed form of the chain, rows
    against the oracle)."""
    rng = np.random.default_rng(20261203)
    M, K, N = 4096, 96, 8192
    a = oracle.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    x = oracle.f32_to_f8e4m3fn_bits(rng.standard_normal(K * N).astype(np.float32)).reshape(K, N)
    sc = rng.uniform(0.005, 0.05, N).astype(np.float32)
    y = olamd.dequantize_linear_matmul(bits_tensor(a, "bf16", dev), T(x, dev), T(sc, dev), None, axis=1,
                                       cast_to=olamd.BFLOAT16, x_dtype=oracle.FLOAT8E4M3FN, x_shape=(K, N))
    rows = np.array([0, 255, 2048, 4095])
    ref, mag = _chain_ref(oracle, a, x, oracle.FLOAT8E4M3FN, K, N, sc, False, None, 1, "bf16", "bf16", rows=rows)
    assert_close(tensor_bits(y)[rows], ref, mag, "bf16", oracle, "fp8 K=96")
    _fp8_chain_closed_form(y, a, x, sc, dev, "fp8 K=96")
