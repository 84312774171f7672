"""The QQQ oracle (oracle.c, orc_qqq_*) pinned by vectors the reference's
tests hold.

- tests/golden/qqq_native_v1_digest.json comes from the reference's fixture
  (unittests/python/backend/data/qqq_native_v1.json, written by the upstream
  QQQ packer): every case's packed words and scales, and SHA-256 digests of
  its unpacked codes and its expected FLOAT weights (plus their first and
  last 64 bit patterns).  Every case must reproduce bit for bit.
- The fixtures of unittests/cc/onnx_core/runtime/test_qqq.cc: the packer's
  own permutation (restated below from the test, not from the decoder) with
  its known words at indices 0, 31 and 127, every weight of the closed form
  integer * channel scale, the ties, saturation and signed zeros of the
  group rounding, the fp32 rounding of 48 * (1 + 2^-23), a subnormal channel
  scale and a zero weight under the largest channel scale.
- CheckData's and WriteFloat's errors, each on a minimal input."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qqq_native_v1_digest.json")


def _arr(t):
    return np.frombuffer(bytes.fromhex(t["hex"]), dtype=np.dtype(t["dtype"]).newbyteorder("<")).reshape(t["shape"])


def qqq_cases():
    return json.load(open(GOLDEN))


def golden_tensors(c):
    t = {k: _arr(v) for k, v in c["tensors"].items()}
    return c["in_features"], c["out_features"], c["group_size"], t["B"], t["s_channel"], t["s_group"]


@pytest.mark.parametrize("name", [c["name"] for c in qqq_cases()])
def test_golden_qqq_cases(oracle, name):
    c = next(c for c in qqq_cases() if c["name"] == name)
    k, n, g, B, sc, sg = golden_tensors(c)
    rc, out, codes = oracle.qqq_reconstruct(k, n, g, B, sc, sg)
    assert rc == 0
    assert list(out.shape) == c["expected_shape"] == [n, k]
    assert hashlib.sha256(codes.tobytes()).hexdigest() == c["codes_sha256"]
    bits = out.reshape(-1).view(np.uint32)
    assert bits[:64].tolist() == c["expected_head_bits"] and bits[-64:].tolist() == c["expected_tail_bits"]
    assert hashlib.sha256(out.astype("<f4").tobytes()).hexdigest() == c["expected_sha256"], name


def test_golden_rejects_swapped_nibbles_and_the_other_order(oracle):
    """Plausible decoder mistakes change the grouped case: nibbles read high
    first, or the per-channel interleave used for a grouped weight."""
    c = next(c for c in qqq_cases() if c["name"] == "k256-n128-g128-extremeTrue")
    k, n, g, B, sc, sg = golden_tensors(c)
    w = B.view(np.uint8)
    swapped = ((w & 15) << 4 | (w >> 4)).astype(np.uint8)
    rc, out, _ = oracle.qqq_reconstruct(k, n, g, swapped, sc, sg)
    assert rc == 0 and hashlib.sha256(out.tobytes()).hexdigest() != c["expected_sha256"]
    # k == 128 with group 128 is the per-channel order: the same words read that way differ
    assert orc.qqq_position(256, 128, 128, 5, 3) != orc.qqq_position(256, 128, -1, 5, 3)


# ---- test_qqq.cc fixtures -------------------------------------------------------

def _expected_code(n, k):
    return (n * 7 + k * 3 + k // 16 + k // 64) % 16


def _channel_scale(n):
    return np.float32(n % 31 + 1) / np.float32(32)


def _group_scale(g, n):
    return np.float32((g + n) % 17) / np.float32(2)


def _pack_perm(grouped):
    """The upstream pack()'s permutation as test_qqq.cc Fixture() builds it."""
    perm = []
    for i in range(32):
        first = [16 * row + i // 4 + 8 * block for block in (0, 1) for row in range(4 * (i % 4), 4 * (i % 4) + 4)]
        for j in range(4):
            perm += [p + 256 * j for p in first]
    inter = [0, 2, 4, 6, 1, 3, 5, 7] if grouped else [4, 0, 5, 1, 6, 2, 7, 3]
    return [perm[s + inter[lane]] for s in range(0, 1024, 8) for lane in range(8)]


def pack_codes(codes, k, n, grouped):
    """Codes [n, k] -> the int32 words B [k / 16, 2n] (the test's packer)."""
    tiled = np.zeros(k * n, np.uint8)
    off = 0
    for kb in range(k // 16):
        for nb in range(n // 16):
            tiled[off:off + 256] = codes[nb * 16:nb * 16 + 16, kb * 16:kb * 16 + 16].T.reshape(-1)
            off += 256
    perm = np.array(_pack_perm(grouped))
    words = np.zeros(k * n // 8, np.uint32)
    for block in range(0, k * n, 1024):
        src = tiled[block + perm].astype(np.uint32)
        idx = (block + np.arange(1024)) // 8
        np.bitwise_or.at(words, idx, src << (4 * (np.arange(1024) % 8)).astype(np.uint32))
    return words.view(np.int32).reshape(k // 16, 2 * n)


def fixture(k, n, group):
    grouped = group == 128 and k != 128
    codes = np.array([[_expected_code(c, r) for r in range(k)] for c in range(n)], np.uint8)
    B = pack_codes(codes, k, n, grouped)
    single = [2 * i + j for i in range(4) for j in (0, 1, 8, 9, 16, 17, 24, 25)]
    channel = np.array([_channel_scale((i // 32) * 32 + single[i % 32]) for i in range(n)], np.float32)
    sg = np.zeros(0, np.float16)
    if grouped:
        sp = [i + 8 * j for i in range(8) for j in range(8)]
        src = [(i // 64) * 64 + sp[i % 64] for i in range(k // 128 * n)]
        sg = np.array([_group_scale(s // n, s % n) for s in src], np.float32).astype(np.float16)
        sg = sg.reshape(k // 128, n)
    return codes, B, channel.reshape(1, n), sg


@pytest.mark.parametrize("k,n,group", [(64, 64, -1), (128, 320, 128), (256, 128, 128), (384, 64, -1), (384, 320, 128)])
def test_cc_source_permutations_and_reconstruct(oracle, k, n, group):
    grouped = group == 128 and k != 128
    codes, B, sc, sg = fixture(k, n, group)
    w = B.reshape(-1).view(np.uint32)
    assert (int(w[0]), int(w[31]), int(w[127])) == (
        (0x1b93e860, 0xc64e931b, 0x60e83db5) if grouped else (0x916e3b08, 0x4c19e6b3, 0xe6b3805d))
    rc, out, got_codes = oracle.qqq_reconstruct(k, n, group, B, sc, sg)
    assert rc == 0 and np.array_equal(got_codes, codes)
    for col in range(n):
        c = codes[col].astype(np.float32)
        if grouped:
            gs = np.array([_group_scale(r // 128, col) for r in range(k)], np.float32)
            integer = np.clip(np.rint((c - np.float32(8)) * gs), -128, 127)
        else:
            integer = np.where(c >= 8, c - 16, c) * np.float32(16)
        assert np.array_equal(out[col].view(np.uint32), (integer * _channel_scale(col)).astype(np.float32).view(np.uint32))


def test_cc_ties_saturation_and_float_rounding(oracle):
    one_plus = np.array([0x3f800001], np.uint32).view(np.float32)[0]
    codes = np.tile(np.arange(256) % 16, (64, 1)).astype(np.uint8)
    B = pack_codes(codes, 256, 64, True)
    channel = np.full((1, 64), one_plus, np.float32)
    for scale in (0.0, -0.0, 2.0 ** -24, 0.5, 1.5, 32.0, 65504.0):
        sg = np.full((2, 64), scale, np.float16)
        rc, out, _ = oracle.qqq_reconstruct(256, 64, 128, B, channel, sg)
        assert rc == 0
        row = out.reshape(-1)
        if scale == 0.5:  # (code - 8) / 2: ties to even, signed zeros
            assert row[9] == 0 and row[11] == 2 * one_plus and row[7] == 0 and row[5] == -2 * one_plus
            assert np.signbit(row[7]) and not np.signbit(row[9])
        if scale == 1.5:
            assert int(row[10:11].view(np.uint32)[0]) == 0x40400002
        if scale == 32.0:
            assert row[0] == -128 * one_plus and row[15] == 127 * one_plus
        if scale == 0.0:  # (code - 8) * +-0: the zeros keep the product's sign
            neg = bool(np.signbit(np.float32(scale)))
            assert bool(np.signbit(row[9])) == neg and bool(np.signbit(row[7])) != neg
    codes = np.full((64, 64), 3, np.uint8)
    B = pack_codes(codes, 64, 64, False)
    sg0 = np.zeros(0, np.float16)
    rc, out, _ = oracle.qqq_reconstruct(64, 64, -1, B, channel, sg0)
    assert rc == 0 and int(out.reshape(-1)[:1].view(np.uint32)[0]) == 0x42400002
    tiny = np.full((1, 64), np.finfo(np.float32).smallest_subnormal, np.float32)
    rc, out, _ = oracle.qqq_reconstruct(64, 64, -1, B, tiny, sg0)
    assert rc == 0 and int(out.reshape(-1)[:1].view(np.uint32)[0]) == 48
    codes8 = np.full((64, 256), 8, np.uint8)
    _, _, _, sg = fixture(256, 64, 128)
    huge = np.full((1, 64), np.finfo(np.float32).max, np.float32)
    rc, out, _ = oracle.qqq_reconstruct(256, 64, 128, pack_codes(codes8, 256, 64, True), huge, sg)
    assert rc == 0 and out.reshape(-1)[0] == 0


def test_checks_and_errors(oracle):
    codes, B, sc, sg = fixture(256, 64, 128)
    assert oracle.qqq_reconstruct(256, 64, 128, B, sc, sg)[0] == 0
    bad = sc.copy()
    bad[0, 5] = -1.0
    assert oracle.qqq_reconstruct(256, 64, 128, B, bad, sg)[0] == 1
    bad[0, 5] = np.nan
    assert oracle.qqq_reconstruct(256, 64, 128, B, bad, sg)[0] == 1
    badg = sg.copy()
    badg[1, 3] = np.inf
    assert oracle.qqq_reconstruct(256, 64, 128, B, sc, badg)[0] == 2
    badg[1, 3] = -0.5
    assert oracle.qqq_reconstruct(256, 64, 128, B, bad, badg)[0] == 1  # channel first
    assert oracle.qqq_reconstruct(256, 64, 128, B, sc, badg)[0] == 2
    big = np.full((1, 64), 3e37, np.float32)  # |integer| up to 128: overflows FLOAT
    assert oracle.qqq_reconstruct(256, 64, 128, B, big, sg)[0] == 3
    mid = np.full((1, 64), 1e4, np.float32)  # fine in FLOAT and BFLOAT16, past FLOAT16
    assert oracle.qqq_reconstruct(256, 64, 128, B, mid, sg)[0] == 0
    assert oracle.qqq_reconstruct(256, 64, 128, B, mid, sg, out_dtype=orc.BFLOAT16)[0] == 0
    assert oracle.qqq_reconstruct(256, 64, 128, B, mid, sg, out_dtype=orc.FLOAT16)[0] == 4
    rc, out, _ = oracle.qqq_reconstruct(256, 64, 128, B, sc, sg, out_dtype=orc.DOUBLE)
    assert rc == 0 and np.array_equal(out, oracle.qqq_reconstruct(256, 64, 128, B, sc, sg)[1].astype(np.float64))
