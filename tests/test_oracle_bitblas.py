"""The BitBLAS oracle (oracle.c, orc_bitblas_reconstruct) pinned by vectors
the reference's tests hold.

- tests/golden/bitblas_native_v1_digest.json comes from the reference's
  fixture (unittests/python/backend/data/bitblas_native_v1.json, written by
  the upstream row packer): all 13 cases (GPTQ 2/4/8-bit symmetric or not,
  AWQ 2-8 bits, per-channel and grouped) with their packed tensors, and
  SHA-256 digests of their raw codes and expected FLOAT weights.  Every case
  must reproduce bit for bit.
- The fixture of unittests/cc/onnx_core/runtime/test_bitblas.cc: bytes 0xE4
  are the 2-bit codes 0, 1, 2, 3, zeros 0x55 are 1, and symmetric GPTQ codes
  are signed (0.5 * {0, 1, -2, -1}); CheckScales' rejected and accepted FP16
  scale patterns."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bitblas_native_v1_digest.json")


def _arr(t):
    return np.frombuffer(bytes.fromhex(t["hex"]), dtype=np.dtype(t["dtype"]).newbyteorder("<")).reshape(t["shape"])


def bitblas_cases():
    return json.load(open(GOLDEN))


def case_id(c):
    return f"{c['method']}-{c['bits']}bit-sym{int(c['symmetric'])}-k{c['in_features']}-n{c['out_features']}-g{c['group_size']}"


def golden_args(c):
    """(method, k, n, group, bits, symmetric, qweight, scales, qzeros)."""
    t = {k: _arr(v) for k, v in c["tensors"].items()}
    return (c["method"], c["in_features"], c["out_features"], c["group_size"], c["bits"], bool(c["symmetric"]),
            t["qweight"], t["scales"], t["qzeros"])


def signed(method, symmetric):
    return method == "gptq" and symmetric


@pytest.mark.parametrize("c", bitblas_cases(), ids=case_id)
def test_golden_bitblas_cases(oracle, c):
    m, k, n, g, bits, sym, qw, sc, qz = golden_args(c)
    rc, out, codes = oracle.bitblas_reconstruct(k, n, g, bits, signed(m, sym), qw, sc, qz)
    assert rc == 0 and list(out.shape) == c["expected_shape"] == [n, k]
    assert hashlib.sha256(codes.tobytes()).hexdigest() == c["codes_sha256"]
    bits_ = out.reshape(-1).view(np.uint32)
    assert bits_[:64].tolist() == c["expected_head_bits"] and bits_[-64:].tolist() == c["expected_tail_bits"]
    assert hashlib.sha256(out.astype("<f4").tobytes()).hexdigest() == c["expected_sha256"]


def test_golden_rejects_the_wrong_signedness_and_scale_order(oracle):
    """Plausible decoder mistakes change the golden results: reading symmetric
    GPTQ codes as unsigned with a midpoint zero no longer applies, and
    scales read [groups, n] instead of [n, groups]."""
    c = next(c for c in bitblas_cases() if c["method"] == "gptq" and c["bits"] == 4 and c["symmetric"])
    m, k, n, g, bits, sym, qw, sc, qz = golden_args(c)
    zeros = np.full((k // g, n * bits // 8), 0x88, np.uint8).view(np.int8)  # unsigned reading, zero 8
    rc, out, _ = oracle.bitblas_reconstruct(k, n, g, bits, False, qw, sc, zeros)
    assert rc == 0 and hashlib.sha256(out.tobytes()).hexdigest() != c["expected_sha256"]
    c = next(c for c in bitblas_cases() if c["method"] == "gptq" and c["bits"] == 2)
    m, k, n, g, bits, sym, qw, sc, qz = golden_args(c)
    swapped = np.ascontiguousarray(sc.T).reshape(sc.shape)
    rc, out, _ = oracle.bitblas_reconstruct(k, n, g, bits, False, qw, swapped, qz)
    assert rc == 0 and hashlib.sha256(out.tobytes()).hexdigest() != c["expected_sha256"]


def cc_fixture(symmetric):
    """test_bitblas.cc Fixture(): gptq, 32 x 32, 2 bits, one group."""
    qw = np.full((32, 8), 0xE4, np.uint8).view(np.int8)
    sc = np.full((32, 1), 0.5, np.float16)
    qz = np.zeros(0, np.int8) if symmetric else np.full((1, 8), 0x55, np.uint8).view(np.int8)
    return qw, sc, qz


@pytest.mark.parametrize("symmetric", [False, True])
def test_cc_raw_codes_zeros_and_signedness(oracle, symmetric):
    qw, sc, qz = cc_fixture(symmetric)
    rc, out, codes = oracle.bitblas_reconstruct(32, 32, -1, 2, symmetric, qw, sc, qz)
    assert rc == 0
    i = np.arange(1024)
    assert np.array_equal(codes.reshape(-1), i % 4)
    c = i % 4
    want = 0.5 * (np.where(c < 2, c, c - 4) if symmetric else c - 1)
    assert np.array_equal(out.reshape(-1), want.astype(np.float32))


@pytest.mark.parametrize("symmetric", [False, True])
def test_cc_every_fp16_scale_is_checked(oracle, symmetric):
    qw, sc, qz = cc_fixture(symmetric)
    for bits in (0x0000, 0x8000, 0xBC00, 0x7C00, 0xFC00, 0x7E01):
        bad = sc.copy().view(np.uint16)
        bad.reshape(-1)[-1] = bits
        assert oracle.bitblas_reconstruct(32, 32, -1, 2, symmetric, qw, bad.view(np.float16), qz)[0] == 1, hex(bits)
    for bits in (0x0001, 0x7BFF):
        ok = sc.copy().view(np.uint16)
        ok.reshape(-1)[-1] = bits
        assert oracle.bitblas_reconstruct(32, 32, -1, 2, symmetric, qw, ok.view(np.float16), qz)[0] == 0


def test_output_dtype_overflow(oracle):
    """255 * 65504 fits FLOAT and BFLOAT16, not FLOAT16 (WriteFloat)."""
    qw = np.full((16, 32), 0xFF, np.uint8).view(np.int8)  # awq 8-bit codes 255, k 32, n 16
    sc = np.full((16, 1), 65504.0, np.float16)
    qz = np.zeros((1, 16), np.int8)
    assert orc.bitblas_reconstruct(32, 16, -1, 8, False, qw, sc, qz)[0] == 0
    assert orc.bitblas_reconstruct(32, 16, -1, 8, False, qw, sc, qz, out_dtype=orc.BFLOAT16)[0] == 0
    assert orc.bitblas_reconstruct(32, 16, -1, 8, False, qw, sc, qz, out_dtype=orc.FLOAT16)[0] == 4
