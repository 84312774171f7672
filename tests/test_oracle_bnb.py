"""The bitsandbytes oracle (oracle.c, orc_bnb_*) pinned by vectors the
reference's tests hold.

- tests/golden/bitsandbytes_native_v1.json is the reference's fixture
  (unittests/python/backend/data/bitsandbytes_native_v1.json), written by
  bitsandbytes 0.50.2 itself (generate_bitsandbytes_native.py): packed codes,
  absmax / nested state, quant maps and bitsandbytes' own dequantize_4bit and
  int8 results.  Every case must reproduce bit for bit, and its quant map
  must equal the oracle's table (the canonical-table rule).
- The fixtures of unittests/cc/onnx_core/runtime/test_bitsandbytes.cc:
  nibble order, partial last block, nested scales with offset 2.0, signed
  int8 codes with row scales, the little-endian 1.0 in every output dtype.
- The error paths of CheckParameters and the reconstruction's finiteness
  checks, each on a minimal input."""
import json
import os

import numpy as np
import pytest

import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bitsandbytes_native_v1.json")


def _arr(t):
    return np.frombuffer(bytes.fromhex(t["hex"]), dtype=np.dtype(t["dtype"]).newbyteorder("<")).reshape(t["shape"])


def _cases():
    return json.load(open(GOLDEN))


def golden_case(c):
    """A golden record as oracle arguments: (fmt, rows, cols, block, kwargs, expected float32)."""
    t = {k: _arr(v) for k, v in c["tensors"].items()}
    expected = _arr(c["expected"]).astype(np.float32)
    rows, cols = expected.shape
    if "weight_scb" in t:
        return "int8", rows, cols, 0, dict(codes=t["weight"], absmax=t["weight_scb"]), expected
    state = json.loads(bytes(t["weight_quant_state"]).decode())
    assert state["shape"] == [rows, cols]
    kw = dict(codes=t["weight"], absmax=t["weight_absmax"], quant_map=t["weight_quant_map"])
    if "weight_nested_absmax" in t:
        kw.update(nested_absmax=t["weight_nested_absmax"], nested_map=t["weight_nested_quant_map"],
                  offset=float(state["nested_offset"]))
    return state["quant_type"], rows, cols, state["blocksize"], kw, expected


@pytest.mark.parametrize("name", [c["name"] for c in _cases()])
def test_golden_bitsandbytes_cases(oracle, name):
    c = next(c for c in _cases() if c["name"] == name)
    fmt, rows, cols, block, kw, expected = golden_case(c)
    qm = kw.pop("quant_map", None)
    assert oracle.bnb_check(fmt, rows, cols, block, kw["absmax"], qm, kw.get("nested_absmax"),
                            kw.get("nested_map"), kw.get("offset", 0.0)) == 0
    if qm is not None:  # the library's own table is the oracle's
        assert np.array_equal(qm.view(np.uint32), oracle.bnb_table(fmt).view(np.uint32))
    rc, got = oracle.bnb_reconstruct(fmt, rows, cols, block, **kw)
    assert rc == 0
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), name


def test_golden_rejects_a_swapped_nibble_order(oracle):
    """A plausible decoder mistake (low nibble first) changes the nf4 case."""
    fmt, rows, cols, block, kw, expected = golden_case(_cases()[0])
    kw.pop("quant_map")
    w = kw["codes"].reshape(-1)
    kw["codes"] = ((w & 15) << 4 | (w >> 4)).astype(np.uint8)
    rc, got = oracle.bnb_reconstruct(fmt, rows, cols, block, **kw)
    assert rc == 0 and not np.array_equal(got, expected)


def _cc_fixture(nested, offset=2.0):
    """test_bitsandbytes.cc Fixture(): nf4, block 32, shape [3, 11], 17 bytes
    whose logical codes run 0..15 (the last byte's padding nibble unused)."""
    codes = np.array([((2 * i % 16) << 4) | ((2 * i + 1) % 16) for i in range(17)], np.uint8)
    codes[-1] = 0x0D
    if nested:
        nmap = np.zeros(256, np.float32)
        nmap[0], nmap[-1] = -1, 1
        return codes, dict(absmax=np.array([0, 255], np.uint8), nested_absmax=np.array([0.5], np.float32),
                           nested_map=nmap, offset=offset)
    return codes, dict(absmax=np.array([2.0, 0.0], np.float32))


@pytest.mark.parametrize("nested", [False, True])
def test_cc_native_nibbles_partial_blocks_and_nested_state(oracle, nested):
    codes, kw = _cc_fixture(nested)
    table = oracle.bnb_table("nf4")
    rc, got = oracle.bnb_reconstruct("nf4", 3, 11, 32, codes, **kw)
    assert rc == 0
    i = np.arange(33)
    want = table[i % 16] * np.where(i < 32, 1.5 if nested else 2.0, 2.5 if nested else 0.0).astype(np.float32)
    assert np.array_equal(got.reshape(-1), want.astype(np.float32))


@pytest.mark.parametrize("text,offset", [("0.5", 0.5), ("2.0", 2.0), ("3.4028234663852886e38", 3.4028234663852886e38)])
def test_cc_nested_offset_values(oracle, text, offset):
    codes, kw = _cc_fixture(True, offset)
    rc, got = oracle.bnb_reconstruct("nf4", 3, 11, 32, codes, **kw)
    assert rc == 0
    assert got.reshape(-1)[0] == np.float32(-(np.float32(offset) - np.float32(0.5)))
    assert got.reshape(-1)[32] == np.float32(-(np.float32(offset) + np.float32(0.5)))


def test_cc_int8_signed_codes_and_row_scales(oracle):
    w = np.array([128, 129, 255, 0, 1, 127], np.uint8)
    rc, got = oracle.bnb_reconstruct("int8", 2, 3, 0, w, np.array([127.0, 254.0], np.float32))
    assert rc == 0 and got.reshape(-1).tolist() == [-128, -127, -1, 0, 2, 254]


@pytest.mark.parametrize("dtype,bits", [(orc.FLOAT, 0x3F800000), (orc.FLOAT16, 0x3C00), (orc.BFLOAT16, 0x3F80)])
def test_cc_little_endian_one_in_every_dtype(oracle, dtype, bits):
    rc, got = oracle.bnb_reconstruct("int8", 1, 1, 0, np.array([1], np.uint8), np.array([127.0], np.float32),
                                     out_dtype=dtype)
    assert rc == 0
    assert int(got.view(np.uint32 if dtype == orc.FLOAT else np.uint16).reshape(-1)[0]) == bits


def test_fp4_table_is_bitsandbytes_over_12(oracle):
    """fp4: get_4bit_type("fp4") normalized by 12, native index order."""
    want = np.array([0, 1 / 192, 2 / 3, 1, 1 / 3, 0.5, 1 / 6, 0.25], np.float64)
    assert np.array_equal(oracle.bnb_table("fp4"), np.concatenate([want, -want]).astype(np.float32))


def test_checks_and_errors(oracle):
    t = oracle.bnb_table("nf4")
    ok = np.array([1.0, 2.0], np.float32)
    assert oracle.bnb_check("nf4", 2, 32, 32, ok, t) == 0
    assert oracle.bnb_check("nf4", 2, 32, 32, np.array([1.0, -1.0], np.float32), t) == 3
    assert oracle.bnb_check("nf4", 2, 32, 32, np.array([1.0, np.inf], np.float32), t) == 3
    bad = t.copy()
    bad[3] = np.nextafter(bad[3], np.float32(0))
    assert oracle.bnb_check("nf4", 2, 32, 32, ok, bad) == 4
    assert oracle.bnb_check("fp4", 2, 32, 32, ok, t) == 4  # the other format's table
    nan_map = t.copy()
    nan_map[0] = np.nan
    assert oracle.bnb_check("nf4", 2, 32, 32, ok, nan_map) == 3
    assert oracle.bnb_check("int8", 2, 3, 0, np.array([1.0, -2.0], np.float32)) == 3
    # nested: a scale that overflows fp32 is the reconstruction error, in the check already
    codes = np.zeros(32, np.uint8)
    nmap = np.ones(256, np.float32)
    big = dict(nested_absmax=np.array([3e38], np.float32), nested_map=nmap * 2, offset=0.0)
    assert oracle.bnb_check("nf4", 2, 32, 32, np.zeros(2, np.uint8), t, big["nested_absmax"], big["nested_map"]) == 2
    assert oracle.bnb_reconstruct("nf4", 2, 32, 32, codes, np.zeros(2, np.uint8), **big)[0] == 2
    # FLOAT16 overflow of a finite fp32 value (code -1 is nf4 entry 0), fine in FLOAT
    one = np.array([1e5], np.float32)
    assert oracle.bnb_reconstruct("nf4", 1, 32, 32, codes[:16], one)[0] == 0
    assert oracle.bnb_reconstruct("nf4", 1, 32, 32, codes[:16], one, out_dtype=orc.FLOAT16)[0] == 2
    assert oracle.bnb_reconstruct("nf4", 1, 32, 32, codes[:16], one, out_dtype=orc.BFLOAT16)[0] == 0
