"""The AWQ and GPTQ restatements of the oracle (oracle.awq_decode,
oracle.gptq_decode) against the reference tests' fixtures, packed words and
expected codes / values (unittests/cc/onnx_core/runtime/test_awq.cc:120-175,
unittests/cc/onnx_core/runtime/test_gptq.cc:126-330), and this suite's own
packers (awq_gptq_cases.awq_pack / gptq_pack) against the same pinned
upstream words, then round trips through the oracle at other shapes."""
import numpy as np
import pytest

from awq_gptq_cases import (awq_expected, awq_fixture, awq_pack, gptq_fixture, gptq_pack, gptq_upstream_v1_zeros,
                            gptq_upstream_words, stream_words)


def _f32(a):
    return np.asarray(a).astype(np.float32)


# ---- AWQ ----------------------------------------------------------------------

def test_awq_fixture_packed_words():
    """test_awq.cc:160-175."""
    gemm = awq_fixture("gemm")
    assert gemm["qweight"].view(np.uint32)[0, 0] == 0x1357ACE0
    assert gemm["qzeros"].view(np.uint32)[0, 0] == 0x75316420
    assert awq_fixture("gemv")["qweight"].view(np.uint32)[0, 0] == 0x52FC9630
    assert awq_fixture("gemv_fast")["qweight"].view(np.uint16)[0, 0] == 0x9180


@pytest.mark.parametrize("variant", ["gemm", "gemv", "gemv_fast", "llm-awq"])
@pytest.mark.parametrize("group_size", [-1, 64, 128])
def test_awq_fixture_codes_and_values(oracle, variant, group_size):
    """test_awq.cc:120-158: every code and every FLOAT value, exactly."""
    fx = awq_fixture(variant, group_size)
    codes, zeros, values = oracle.awq_decode(variant, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), 128, 8,
                                             group_size)
    eff = 128 if group_size == -1 else group_size
    for n in range(8):
        for k in range(128):
            g = k // eff
            assert codes[n, k] == awq_expected(n, k), (variant, n, k)
            assert values[n, k] == (awq_expected(n, k) - (n + g) % 16) * ((g + 1) * 0.25), (variant, n, k)
            if variant in ("gemm", "gemv"):
                assert zeros[n, g] == (n + g) % 16


def test_awq_gemv_fast_value_rounds_product_then_adds(oracle):
    """gemv_fast / llm-awq (awq.cc:238-241): code * scale is rounded to FLOAT
    before the zero term is added.  With scale 1 + 2^-10 and zero term
    -2^13 the sums code * scale - 2^13 need the product's rounding first."""
    fx = awq_fixture("gemv_fast", -1)
    scales = _f32(fx["scales"]).copy()
    terms = _f32(fx["qzeros"]).copy()
    scales[0, 0] = np.float32(1.0009765625)
    terms[0, 0] = np.float32(-8192.0)
    codes, _, values = oracle.awq_decode("gemv_fast", fx["qweight"], terms, scales, 128, 8, -1)
    for k in range(128):
        prod = np.float32(np.float32(int(codes[0, k])) * scales[0, 0])
        assert values[0, k] == np.float32(prod + terms[0, 0])


@pytest.mark.parametrize("group_size", [-1, 64, 128])
def test_awq_packers_reproduce_the_fixture(oracle, group_size):
    """awq_pack of the fixture's codes and zeros gives the fixture's words."""
    eff = 128 if group_size == -1 else group_size
    groups = 128 // eff
    codes = np.array([[awq_expected(n, k) for n in range(8)] for k in range(128)])
    zeros = np.array([[(n + g) % 16 for n in range(8)] for g in range(groups)])
    scales = np.array([[(g + 1) * 0.25] * 8 for g in range(groups)], np.float16)
    gemm = awq_pack("gemm", codes, zeros, scales, group_size)
    fx = awq_fixture("gemm", group_size)
    assert np.array_equal(gemm["qweight"], fx["qweight"]) and np.array_equal(gemm["qzeros"], fx["qzeros"])
    gemv = awq_pack("gemv", codes, zeros, scales, group_size)
    fx = awq_fixture("gemv", group_size)
    assert np.array_equal(gemv["qweight"], fx["qweight"])
    # the fixture's zero padding is 0xfedcba98 nibbles and its scale padding -3: compare the used parts
    c1, z1, v1 = oracle.awq_decode("gemv", gemv["qweight"], gemv["qzeros"], _f32(gemv["scales"]), 128, 8, group_size)
    c2, z2, v2 = oracle.awq_decode("gemv", fx["qweight"], fx["qzeros"], _f32(fx["scales"]), 128, 8, group_size)
    assert np.array_equal(c1, c2) and np.array_equal(z1, z2) and np.array_equal(v1, v2)


@pytest.mark.parametrize("variant,K,N,group", [("gemm", 256, 48, 32), ("gemm", 192, 16, -1), ("gemv", 256, 24, 16),
                                               ("gemv", 1024, 8, 64), ("gemv", 512, 8, 256), ("gemm8", 128, 12, 64)])
def test_awq_round_trip(oracle, variant, K, N, group):
    """Random codes, zeros and scales through awq_pack and the oracle's decode:
    codes, zeros and (code - zero) * scale back exactly (8-bit gemm too)."""
    rng = np.random.default_rng(K + N)
    bits = 8 if variant == "gemm8" else 4
    eff = K if group == -1 else group
    groups = K // eff
    codes = rng.integers(0, 1 << bits, (K, N))
    zeros = rng.integers(0, 1 << bits, (groups, N))
    scales = rng.uniform(0.01, 2.0, (groups, N)).astype(np.float16)
    pk = awq_pack(variant, codes, zeros, scales, group)
    name = "gemm" if variant == "gemm8" else variant
    c, z, v = oracle.awq_decode(name, pk["qweight"], pk["qzeros"], _f32(pk["scales"]), K, N, group, bits=bits)
    assert np.array_equal(c, codes.T) and np.array_equal(z, zeros.T)
    g_of_k = np.arange(K) // eff
    want = ((codes - zeros[g_of_k]).astype(np.float32) * scales.astype(np.float32)[g_of_k]).T
    assert np.array_equal(v, want)


# ---- GPTQ ---------------------------------------------------------------------

GPTQ_CASES = [(f, b) for f in ("gptq", "gptq_v2", "gptq_p") for b in range(2, 9) if f == "gptq_p" or b not in (5, 6, 7)]


@pytest.mark.parametrize("fmt,bits", GPTQ_CASES)
def test_gptq_upstream_fixtures(oracle, fmt, bits):
    """test_gptq.cc:126-178: codes (k * 7 + 3) & maxq, zeros ((n * 5 + 3) %
    maxq) + 1 for v1 and (n * 7 + 3) & maxq otherwise, values exact."""
    fx = gptq_fixture(bits, fmt)
    codes, zeros, values = oracle.gptq_decode(fmt, bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), fx["g_idx"],
                                              32, 32, 16)
    maxq = (1 << bits) - 1
    for n in range(32):
        zero = (n * 5 + 3) % maxq + 1 if fmt == "gptq" else (n * 7 + 3) & maxq
        assert zeros[n, 0] == zero and zeros[n, 1] == zero
        for k in range(32):
            assert codes[n, k] == (k * 7 + 3) & maxq
            assert values[n, k] == (((k * 7 + 3) & maxq) - zero) * (0.5 if k % 2 == 0 else 1.5)


@pytest.mark.parametrize("width", [1, 2, 4, 8])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_gptq_word_widths(oracle, width, bits):
    """test_gptq.cc:187-210 (INT8 / INT16 / INT32), and INT64 words, which
    the format also accepts (gptq.cc:76-83): the same byte stream gives the
    same codes at every width."""
    fx = gptq_fixture(bits, "gptq_v2", width)
    codes, _, _ = oracle.gptq_decode("gptq_v2", bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]), fx["g_idx"],
                                     32, 32, 16)
    assert np.array_equal(codes, np.tile((np.arange(32) * 7 + 3) % (1 << bits), (32, 1)))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_gptq_sparse_crossing(oracle, bits):
    """test_gptq.cc:212-238: only codes 10 and 21 at maxq, including the
    3-bit codes that cross word boundaries."""
    words = {2: [0x00300000, 0x00000C00], 3: [0xC0000000, 0x80000001, 0x00000003], 4: [0, 0x00000F00, 0x00F00000, 0],
             8: [0, 0, 0x00FF0000, 0, 0, 0x0000FF00, 0, 0]}[bits]
    fx = gptq_fixture(bits)
    w = np.array(words, np.uint32).view(np.int32)
    fx["qweight"] = np.repeat(w[:, None], 32, axis=1)
    fx["qzeros"] = np.stack([w, w])
    codes, zeros, _ = oracle.gptq_decode("gptq_v2", bits, fx["qweight"], fx["qzeros"], _f32(fx["scales"]),
                                         fx["g_idx"], 32, 32, 16)
    hot = np.isin(np.arange(32), [10, 21])
    assert np.array_equal(zeros[:, 0], np.where(hot, (1 << bits) - 1, 0))
    assert np.array_equal(codes, np.tile(np.where(hot, (1 << bits) - 1, 0), (32, 1)))


@pytest.mark.parametrize("bits", [3, 5, 6, 7])
def test_gptq_planar_adjacent_blocks(oracle, bits):
    """test_gptq.cc:240-290: two distinct planar 32-code blocks, K = N = 64."""
    second = {3: [0xB1B1B1B1, 0xB1B1B1B1, 0x96969696],
              5: [0x630DA741, 0xEB852FC9, 0x630DA741, 0xEB852FC9, 0xF81F07E0],
              6: [0x630DA741, 0xEB852FC9, 0x630DA741, 0xEB852FC9, 0xAA955400, 0x554003FF],
              7: [0x630DA741, 0xEB852FC9, 0x630DA741, 0xEB852FC9, 0xAA955400, 0x554003FF, 0xFFE00000]}[bits]
    words = np.array(gptq_upstream_words(bits, True) + second, np.uint32).view(np.int32)
    qweight = np.repeat(words[:, None], 64, axis=1)
    qzeros = np.repeat(words[None, :], 4, axis=0)
    scales = np.full((4, 64), 0.5, np.float32)
    g_idx = (np.arange(64) % 4).astype(np.int32)
    codes, zeros, _ = oracle.gptq_decode("gptq_p", bits, qweight, qzeros, scales, g_idx, 64, 64, 16)
    expected = np.array([(i * 7 + 3 if i < 32 else (i - 32) * 3 + 1) % (1 << bits) for i in range(64)])
    assert np.array_equal(zeros[:, 0], expected)
    assert np.array_equal(codes, np.tile(expected, (64, 1)))


def test_gptq_partial_words(oracle):
    """test_gptq.cc:292-312: K = N = 3 in one word, padding nibbles ignored."""
    gptq_decode = oracle.gptq_decode
    qweight = np.array([[0xDEADF210] * 3], np.uint32).view(np.int32)
    qzeros = np.array([[0xABCDF210]], np.uint32).view(np.int32)
    codes, zeros, _ = gptq_decode("gptq_v2", 4, qweight, qzeros, np.ones((1, 3), np.float32),
                                  np.zeros(3, np.int32), 3, 3, 16)
    assert np.array_equal(codes, np.tile([0, 1, 2], (3, 1)))
    assert zeros[2, 0] == 2


# every word width the layout allows: gptq_p, 3-bit and planar layouts use INT32 words (gptq.cc:85-92)
PACKER_CASES = [(f, b, w) for f, b in GPTQ_CASES for w in (1, 2, 4, 8)
                if w == 4 or not (f == "gptq_p" or b in (3, 5, 6, 7))]


@pytest.mark.parametrize("fmt,bits,width", PACKER_CASES)
def test_gptq_packer_reproduces_upstream_words(fmt, bits, width):
    """gptq_pack of the upstream codes gives the pinned upstream words (and v1
    zero words), for every word width the layout allows."""
    planar = bits in (5, 6, 7) or (fmt == "gptq_p" and bits == 3)  # gptq.cc:89
    codes = np.tile(((np.arange(32) * 7 + 3) % (1 << bits))[:, None], (1, 32))
    stored = ((np.arange(32) * 5 + 3) % ((1 << bits) - 1)) if fmt == "gptq" else (np.arange(32) * 7 + 3) % (1 << bits)
    qw, qz = gptq_pack(codes, np.stack([stored, stored]), bits, width, planar)
    words = gptq_upstream_words(bits, planar)
    w = stream_words(words, width)
    z = stream_words(gptq_upstream_v1_zeros(bits) if fmt == "gptq" else words, width)
    assert np.array_equal(qw, np.repeat(w[:, None], 32, axis=1))
    assert np.array_equal(qz, np.stack([z, z]))


@pytest.mark.parametrize("fmt,bits,width,K,N,group", [
    ("gptq_v2", 4, 4, 256, 40, 64), ("gptq", 4, 4, 128, 24, 32), ("gptq", 3, 4, 256, 64, 128),
    ("gptq_v2", 2, 2, 96, 20, 32), ("gptq_p", 5, 4, 128, 32, 64), ("gptq_p", 6, 4, 64, 64, -1),
    ("gptq_p", 7, 4, 96, 32, 32), ("gptq_v2", 8, 8, 64, 10, 16), ("gptq_p", 3, 4, 128, 96, 64),
    ("gptq_v2", 4, 1, 80, 6, 48)])
def test_gptq_round_trip(oracle, fmt, bits, width, K, N, group):
    """Random codes and zeros through gptq_pack and the oracle's decode, with
    the trivial group map and a permuted one (act-order)."""
    rng = np.random.default_rng(K * N + bits)
    planar = bits in (5, 6, 7) or (fmt == "gptq_p" and bits == 3)
    eff = K if group == -1 else group
    groups = -(-K // eff)
    maxq = (1 << bits) - 1
    codes = rng.integers(0, maxq + 1, (K, N))
    zeros = rng.integers(1, maxq + 1, (groups, N)) if fmt == "gptq" else rng.integers(0, maxq + 1, (groups, N))
    stored = zeros - 1 if fmt == "gptq" else zeros
    qw, qz = gptq_pack(codes, stored, bits, width, planar)
    scales = rng.uniform(0.01, 2.0, (groups, N)).astype(np.float16).astype(np.float32)
    for g_idx in (np.arange(K) // eff, rng.permutation(np.arange(K) // eff)):
        g_idx = g_idx.astype(np.int32)
        c, z, v = oracle.gptq_decode(fmt, bits, qw, qz, scales, g_idx, K, N, group)
        assert np.array_equal(c, codes.T) and np.array_equal(z, zeros.T)
        want = ((codes - zeros[g_idx]).astype(np.float32) * scales[g_idx]).T
        assert np.array_equal(v, want)
