"""Dyadic inputs for bit-exact checks of the float GEMM / GEMV paths.

Every activation is a small integer, every dequantised weight a small integer
times a power of two, every scale a power of two.  Then each product
a_mk * w_kn is a whole multiple of one power of two `unit`, and when
sum_k |a_mk * w_kn| < 2^24 * unit every fp32 partial sum is exact, in any
order: the oracle's k-sequential fp32 sum (km/kernel_matmul.cc:136-141) and a
GPU kernel's blocked MFMA / split-K sums both hold the exact sum, and the
single output conversion (round to nearest even) gives the same bits.  Where
the reference chain rounds each weight first (DequantizeLinear -> Cast, the
packed decodes), these weights are representable, so that rounding is exact
too and the fused kernels, which skip or reorder it, must agree bit for bit.

The activations are sparse and the weights kept small, so the exact outputs
stay well inside the output type's exact range: a k-term that a kernel drops
or adds twice moves the output by at least one of its ulps and changes the
rounded bits.  ``drop_one_term`` builds such a wrong answer on the CPU, and
tests/test_exact_inputs.py shows that each generator's check rejects it.
"""
import numpy as np

P_BF16, P_F16 = 8, 11  # significant bits of the output types


def sparse_act(rng, shape, density):
    """Small-integer activations: 0 with probability 1 - density, otherwise
    +-1 (7/8 of the nonzeros) or +-2."""
    mag = np.where(rng.random(shape) < 0.125, 2.0, 1.0)
    sign = np.where(rng.random(shape) < 0.5, -1.0, 1.0)
    return np.where(rng.random(shape) < density, mag * sign, 0.0).astype(np.float32)


def pow2(rng, shape, lo, hi):
    """Powers of two 2^-e, e uniform in [lo, hi]."""
    return np.ldexp(1.0, -rng.integers(lo, hi + 1, shape)).astype(np.float32)


def lsb_exponent(x) -> int:
    """The smallest e such that every element of x is a whole multiple of
    2^e (x finite, not all zero)."""
    x = np.asarray(x, np.float64).reshape(-1)
    x = x[x != 0]
    m, e = np.frexp(x)
    im = np.abs(m * 2.0 ** 53).astype(np.int64)
    tz = np.log2((im & -im).astype(np.float64)).astype(np.int64)  # trailing zero bits
    return int((e - 53 + tz).min())


def check_premise(a64, w64):
    """Asserts that every fp32 partial sum of a @ w is exact (the products
    are multiples of 2^(lsb a + lsb w) and the largest sum of magnitudes stays
    below 2^24 such units); returns that unit's exponent."""
    e = lsb_exponent(a64) + lsb_exponent(w64)
    mag = np.abs(a64) @ np.abs(w64)
    assert mag.max() < 2.0 ** (24 + e), "dyadic premise: fp32 partial sums would round"
    return e


def exact_out_bits(oracle, a64, w64, out):
    """The exact product a @ w (float64: exact under the premise), rounded
    once to the output type ("bf16" / "f16"), as bit patterns."""
    y = np.asarray(a64, np.float64) @ np.asarray(w64, np.float64)
    y32 = y.astype(np.float32)
    assert np.array_equal(y32.astype(np.float64), y), "exact sums must be fp32 values"
    return oracle.f32_to_bf16_bits(y32) if out == "bf16" else oracle.f32_to_f16_bits(y32)


def drop_one_term(a, rng):
    """A copy of the activations with one nonzero term of every row removed
    (a_mk set to 0 for one k per row): the answer of a kernel that loses that
    k-term."""
    a = np.array(a, copy=True)
    flat = a.reshape(-1, a.shape[-1])
    for r in range(flat.shape[0]):
        nz = np.flatnonzero(flat[r])
        if nz.size:
            flat[r, nz[rng.integers(nz.size)]] = 0
    return a


def enc(oracle, x, dt):
    """fp32 values (exactly representable) -> bf16 / fp16 bit patterns."""
    x = np.asarray(x, np.float32)
    bits = oracle.f32_to_bf16_bits(x) if dt == "bf16" else oracle.f32_to_f16_bits(x)
    dec = oracle.bf16_bits_to_f32(bits) if dt == "bf16" else oracle.f16_bits_to_f32(bits)
    assert np.array_equal(dec, x), "dyadic values must be exact in the operand type"
    return bits


# ---- weights ---------------------------------------------------------------

def fp8_codes(oracle, rng, shape):
    """float8e4m3fn weights +-m * 2^e, m in {1, 1.125, .., 1.875}, e in
    {-1, 0} (every mantissa pattern of two exponents), a quarter of them 0:
    returns (codes uint8, values float32)."""
    m = 1.0 + rng.integers(0, 8, shape) / 8.0
    v = m * np.ldexp(1.0, -rng.integers(0, 2, shape)) * np.where(rng.random(shape) < 0.5, -1.0, 1.0)
    v = np.where(rng.random(shape) < 0.25, 0.0, v).astype(np.float32)
    codes = oracle.f32_to_f8e4m3fn_bits(v).reshape(shape)
    assert np.array_equal(oracle.f8e4m3fn_bits_to_f32(codes).reshape(shape), v)
    return codes, v


def int4_codes(rng, shape, signed=True):
    return rng.integers(-8, 8, shape) if signed else rng.integers(0, 16, shape)


def block_scales(rng, shape):
    """Blocked / per-column scales 2^-4 .. 2^-6 (fp16 and bf16 exact)."""
    return pow2(rng, shape, 4, 6)


# ---- GGUF blocks (layouts of onnx_core/runtime/dequantize_packed.cc) -------

def _f16_bytes(oracle, v):
    b = oracle.f32_to_f16_bits(np.asarray(v, np.float32))
    return (b & 255).astype(np.uint8), (b >> 8).astype(np.uint8)


def gguf_blocks(oracle, rng, fmt, N, K):
    """Random GGUF blocks of a [N, K] weight whose values are small integers
    times a power-of-two d (fp16 scales 2^-4 .. 2^-6; q2_k, q4_k and q5_k
    with dmin = d and small sub-block scales and minima; q3_k and q6_k
    sub-block scales +-1..+-3; iq4_xs scales +-1, +-2; q8_0 codes in
    [-16, 16]): the chain's fp32 decode steps and its FLOAT16 rounding are
    then exact."""
    size = oracle.packed_block_bytes(fmt)
    nb = N * K // oracle.packed_block_values(fmt)
    x = rng.integers(0, 256, (nb, size)).astype(np.uint8)
    d = pow2(rng, nb, 4, 6)
    lo, hi = _f16_bytes(oracle, d)
    if fmt == "gguf:q4_0":
        x[:, 0], x[:, 1] = lo, hi
    elif fmt == "gguf:q8_0":
        x[:, 0], x[:, 1] = lo, hi
        x[:, 2:] = rng.integers(-16, 17, (nb, 32)).astype(np.int8).view(np.uint8)
    elif fmt == "gguf:q4_k":
        x[:, 0], x[:, 1], x[:, 2], x[:, 3] = lo, hi, lo, hi
        sc = rng.integers(1, 4, (nb, 8))
        mn = rng.integers(0, 8, (nb, 8))
        # 6-bit scale / minimum of sub-block g: g < 4 in bytes g and g + 4,
        # g >= 4 split over the low nibbles of byte g + 4 and bits 6-7 of
        # bytes g - 4 / g (all below 16 here: those high bits stay 0)
        x[:, 4:8] = sc[:, :4]
        x[:, 8:12] = mn[:, :4]
        x[:, 12:16] = (sc[:, 4:] | (mn[:, 4:] << 4)).astype(np.uint8)
    elif fmt == "gguf:q6_k":
        x[:, 208], x[:, 209] = lo, hi
        s = rng.integers(1, 4, (nb, 16)) * np.where(rng.random((nb, 16)) < 0.5, -1, 1)
        x[:, 192:208] = s.astype(np.int8).view(np.uint8)
    elif fmt == "gguf:q2_k":
        # d = dmin; byte g of the 16: scale 1..3 (low nibble), minimum 0..3
        x[:, 80], x[:, 81], x[:, 82], x[:, 83] = lo, hi, lo, hi
        x[:, :16] = (rng.integers(1, 4, (nb, 16)) | (rng.integers(0, 4, (nb, 16)) << 4)).astype(np.uint8)
    elif fmt == "gguf:q3_k":
        # 6-bit scales s + 32 (s = +-1..+-3) of the 16 sub-blocks: low nibble
        # of sub-block g in byte 96 + g % 8 (bits 4 (g / 8)), its two high bits
        # in byte 104 + g % 4 (bits 2 ((g / 4) % 4))
        x[:, 108], x[:, 109] = lo, hi
        s = rng.integers(1, 4, (nb, 16)) * np.where(rng.random((nb, 16)) < 0.5, -1, 1) + 32
        x[:, 96:108] = 0
        for g in range(16):
            x[:, 96 + g % 8] |= ((s[:, g] & 15) << (4 * (g // 8))).astype(np.uint8)
            x[:, 104 + g % 4] |= ((s[:, g] >> 4) << (2 * ((g // 4) % 4))).astype(np.uint8)
    elif fmt == "gguf:q5_k":
        x[:, 0], x[:, 1], x[:, 2], x[:, 3] = lo, hi, lo, hi  # d = dmin, scales as q4_k's
        sc = rng.integers(1, 3, (nb, 8))
        mn = rng.integers(0, 8, (nb, 8))
        x[:, 4:8] = sc[:, :4]
        x[:, 8:12] = mn[:, :4]
        x[:, 12:16] = (sc[:, 4:] | (mn[:, 4:] << 4)).astype(np.uint8)
    elif fmt == "gguf:iq4_xs":
        # sub-block scales s + 32 (s = +-1, +-2): low nibbles in bytes 4..7,
        # two high bits each in the 16-bit word at byte 2; codes restricted to
        # the codebook values of magnitude 49..127 (a wider spread would leave
        # a dropped small term below an output ulp)
        x[:, 0], x[:, 1] = lo, hi
        s = rng.integers(1, 3, (nb, 8)) * np.where(rng.random((nb, 8)) < 0.5, -1, 1) + 32
        high = np.zeros(nb, np.int64)
        x[:, 4:8] = 0
        for g in range(8):
            x[:, 4 + g // 2] |= ((s[:, g] & 15) << (4 * (g % 2))).astype(np.uint8)
            high |= (s[:, g] >> 4) << (2 * g)
        x[:, 2], x[:, 3] = high & 255, high >> 8
        codes = np.array([0, 1, 2, 3, 4, 12, 13, 14, 15])[rng.integers(0, 9, (nb, 256))]
        x[:, 8:] = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)  # any nibble order: every code is kept
    else:
        raise ValueError(fmt)
    x = x.reshape(-1)
    w = oracle.dequantize_packed(x, fmt, (N, K), 1)  # FLOAT values
    assert np.array_equal(oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(w)), w), "fp16-exact weights"
    return x, w


# ---- whole cases: activations, the weight as the kernel takes it, and the
# chain's dequantised weight W [K, N] (float32 values) ----------------------

# Activation densities: low enough that the exact outputs stay where a
# dropped term is at least one ulp (tests/test_exact_inputs.py measures it).
DENSITY = {"fp8": 0.125, "half": 0.125, "int4": 0.25, "gguf": 0.25}


def fp8_case(oracle, rng, M, K, N):
    """bf16 activations x DequantizeLinear(float8e4m3fn [K, N], per-column
    fp32 scale 2^-3 .. 2^-8, axis 1) -> Cast(BFLOAT16): W = q * s exactly."""
    a = sparse_act(rng, (M, K), DENSITY["fp8"])
    codes, q = fp8_codes(oracle, rng, (K, N))
    scale = pow2(rng, N, 3, 8)
    return dict(a=a, a_bits=enc(oracle, a, "bf16"), x=codes, scale=scale, w=q * scale[None, :], out="bf16")


def half_case(oracle, rng, M, K, N, dt):
    """FLOAT16 / BFLOAT16 MatMul: B = small integers (-8..7) times 2^-2 ..
    2^-4 per element (FLOAT16) or 2^-2 .. 2^-3 (BFLOAT16, whose 8-bit
    outputs need the narrower range and sparser activations)."""
    a = sparse_act(rng, (M, K), DENSITY["half"] / (2 if dt == "bf16" else 1))
    b = (rng.integers(-8, 8, (K, N)) * pow2(rng, (K, N), 2, 3 if dt == "bf16" else 4)).astype(np.float32)
    return dict(a=a, a_bits=enc(oracle, a, dt), b_bits=enc(oracle, b, dt), w=b, out=dt)


def int4_case(oracle, rng, M, K, N, block, signed, with_zp, dt):
    """DequantizeLinear(INT4 / UINT4 [K, N], blocked scales [K / block, N]
    along K, optional zero points) -> MatMul; fp16 scales for FLOAT16
    activations, fp32 scales and a Cast for BFLOAT16 ones (8-bit outputs:
    scales 2^-4 .. 2^-5 and sparser activations)."""
    bf = dt == "bf16"
    a = sparse_act(rng, (M, K), DENSITY["int4"] / (8 if bf else 1))
    q = int4_codes(rng, (K, N), signed)
    s = pow2(rng, (K // block, N), 4, 5) if bf else block_scales(rng, (K // block, N))
    z = int4_codes(rng, (K // block, N), signed) if with_zp else np.zeros((K // block, N), np.int64)
    w = ((q - np.repeat(z, block, axis=0)) * np.repeat(s, block, axis=0)).astype(np.float32)
    return dict(a=a, a_bits=enc(oracle, a, dt), x=oracle.pack_int4(q.reshape(-1)),
                zp=oracle.pack_int4(z.reshape(-1)) if with_zp else None,
                scale=s.astype(np.float16) if dt == "f16" else s, w=w, out=dt)


def ckpt_case(oracle, rng, kind, M, K, N, group, dt):
    """Packed checkpoint weights prepared for the fused node: kind
    "awq" (AWQ gemm, 4 bits), "gptq4" / "gptq8" (GPTQ v2, 4 / 8 bits),
    "nbits2" / "nbits4" / "nbits8" (ORT MatMulNBits with zero points).  W = (q - z) * s
    with power-of-two scales (FLOAT16 for fp16 activations; BFLOAT16 for AWQ /
    GPTQ with bf16 activations); 8-bit codes lie within 24 of their zero
    point.  Returns the case with the checkpoint arrays under "ckpt"."""
    from awq_gptq_cases import awq_pack, gptq_pack
    from nbits_cases import ort_pack
    bits = 8 if kind.endswith("8") else (2 if kind.endswith("2") else 4)
    groups = K // group
    if bits == 8:
        z = rng.integers(120, 137, (groups, N))
        q = np.repeat(z, group, axis=0) + rng.integers(-24, 25, (K, N))
    elif bits == 2:
        z = rng.integers(0, 4, (groups, N))
        q = rng.integers(0, 4, (K, N))
    else:
        z = rng.integers(0, 16, (groups, N))
        q = rng.integers(0, 16, (K, N))
    bf = dt == "bf16"
    s = pow2(rng, (groups, N), 4, 5) if bf else block_scales(rng, (groups, N))
    w = ((q - np.repeat(z, group, axis=0)) * np.repeat(s, group, axis=0)).astype(np.float32)
    a = sparse_act(rng, (M, K), DENSITY["int4"] / (8 if bf else 1) / (4 if bits == 8 else 1))
    if kind == "awq":
        ck = awq_pack("gemm", q, z, s.astype(np.float16), group)
        _, _, vals = oracle.awq_decode("gemm", ck["qweight"], ck["qzeros"], s, K, N, group)
        ck["scales"] = s  # float32 values, exact in FLOAT16 and BFLOAT16
    elif kind.startswith("gptq"):
        qw, qz = gptq_pack(q, z, bits, 4, False)
        g_idx = (np.arange(K) // group).astype(np.int32)
        ck = dict(qweight=qw, qzeros=qz, scales=s, g_idx=g_idx)
        _, _, vals = oracle.gptq_decode("gptq_v2", bits, qw, qz, s, g_idx, K, N, group)
    else:
        B, zpk = ort_pack(q, z, bits, group)
        sb = oracle.f32_to_f16_bits(np.ascontiguousarray(s.T))
        ck = dict(B=B, scale_bits=sb, zp=zpk, bits=bits)
        vals = oracle.ort_nbits_decode(B, np.ascontiguousarray(s.T), zpk, K, N, bits, group).T
    assert np.array_equal(np.ascontiguousarray(np.asarray(vals, np.float32).T), w), "oracle decode = (q - z) s"
    return dict(a=a, a_bits=enc(oracle, a, dt), ckpt=ck, w=w, out=dt)


def gguf_case(oracle, rng, M, K, N, fmt):
    """fp16 activations x DequantizePacked(fmt, [N, K])^T."""
    a = sparse_act(rng, (M, K), DENSITY["gguf"])
    x, w_nk = gguf_blocks(oracle, rng, fmt, N, K)
    return dict(a=a, a_bits=enc(oracle, a, "f16"), x=x, w=np.ascontiguousarray(w_nk.T), out="f16")


def visible_drop_fraction(oracle, case, rng):
    """Removes one nonzero term a_mk from every row m and returns the share of
    the outputs (m, n) that term touched (w_kn != 0) whose rounded value
    changes, with the wrong answer."""
    a = case["a"]
    dropped = drop_one_term(a, rng)
    want = exact_out_bits(oracle, a, case["w"], case["out"])
    wrong = exact_out_bits(oracle, dropped, case["w"], case["out"])
    rows, ks = np.nonzero(dropped != a)
    touched = np.zeros(want.shape, bool)
    touched[rows] = case["w"][ks] != 0
    return float(np.mean(want[touched] != wrong[touched])), wrong
