"""The EXL3 oracle (oracle.c, orc_exl3_reconstruct) pinned two ways:

- the reference test's all-zero trellis (unittests/cc/onnx_core/runtime/
  test_exl3.cc:16-31, 76-105): suh = -0.5, svh = 2 and state zero decoding
  to 0.76806640625 (3INST), 1.84375 (MCG) and -3.453125 (MUL1), GPTQModel's
  binary16 values, give element [0, 0] = -128 * decoded (within the test's
  1e-4: two fp32 roundings of 1 / sqrt 128) and exact zeros elsewhere, at
  every rate 1..8;
- an independent restatement of the upstream format built here from its
  definition (the reference's Python test describes the same construction,
  unittests/python/backend/test_exl3.py:12-101): symbols written as
  big-endian bit strings, packed as little-endian 32-bit words, each state
  the 16-bit window of the cyclic string ending at the symbol, the codebooks
  in numpy binary16 arithmetic, the fragment placement, and the butterflies
  as whole-array float32 operations.  Every rate and codebook at 128 x 256,
  and every one of the 65,536 states at 128 x 1024, bit for bit.
A mistake in the word order inside a tile, the window offset, the fragment
placement, a butterfly's order or the normalisation fails one of these."""
import numpy as np
import pytest

ZERO_STATE = {0: 0.76806640625, 1: 1.84375, 2: -3.453125}


def pack_stream(symbols, bits):
    stream = "".join(f"{s:0{bits}b}" for s in symbols)
    words = [int(stream[i:i + 32], 2) for i in range(0, len(stream), 32)]
    return np.array(words, "<u4").view(np.int16), stream


def states_of(stream, bits):
    cyclic = stream[-16:] + stream
    return [int(cyclic[(i + 1) * bits:(i + 1) * bits + 16], 2) for i in range(256)]


def codebook(states, book):
    st = np.array(states, np.uint64)
    if book < 2:
        raw = (st * 89226354 + 64248484 if book == 0 else st * 0xCBAC1FED) & 0xFFFFFFFF
        raw = 0x3B603B60 ^ (raw & 0x8FFF8FFF)
        lo = (raw & 0xFFFF).astype(np.uint16).view(np.float16)
        hi = (raw >> 16).astype(np.uint16).view(np.float16)
        return (lo + hi).astype(np.float32)
    raw = (st * 0x83DCD12D) & 0xFFFFFFFF
    total = sum((raw >> sh) & 255 for sh in (0, 8, 16, 24))
    acc = (total + 0x6400).astype(np.uint16).view(np.float16).astype(np.float64)
    factor, bias = np.array([0x1EEE, 0xC931], np.uint16).view(np.float16).astype(np.float64)
    return (acc * factor + bias).astype(np.float16).astype(np.float32)  # one rounding: exact fma in float64


def butterflies(m, axis):
    v = np.moveaxis(m, axis, -1).astype(np.float32).copy()
    for w in (1, 2, 4, 8, 16, 32, 64):
        blocks = v.reshape(*v.shape[:-1], -1, 2 * w)
        a, b = blocks[..., :w].copy(), blocks[..., w:].copy()
        blocks[..., :w] = a + b
        blocks[..., w:] = a - b
    v *= np.float32(0.08838834764831845)
    return np.moveaxis(v, -1, axis)


def fixture(bits, book, rows=128, cols=256, exhaustive=False):
    words, values = [], []
    for tile in range(rows * cols // 256):
        if exhaustive:
            syms = [s for low in range((tile % 2) * 128, (tile % 2 + 1) * 128) for s in (tile // 2, low)]
        else:
            syms = [((i * 29 + tile * 11) ^ (i >> 3)) % (1 << bits) for i in range(256)]
        w, stream = pack_stream(syms, bits)
        words.append(w)
        values.append(codebook(states_of(stream, bits), book))
    m = np.empty((rows, cols), np.float32)
    for tile, vals in enumerate(values):
        for p in range(256):
            lane, item = p // 8, p % 8
            r = tile // (cols // 16) * 16 + (lane % 4) * 2 + (item & 1) + (8 if item & 2 else 0)
            c = tile % (cols // 16) * 16 + lane // 4 + (8 if item & 4 else 0)
            m[r, c] = vals[p]
    trellis = np.concatenate(words).reshape(rows // 16, cols // 16, 16 * bits)
    suh = np.resize(np.array([-0.375, 0.625, 1.25, -2.5, 0.3], np.float16), rows)
    svh = np.resize(np.array([1.875, -1.1, 0.45], np.float16), cols)
    expected = butterflies(m, 0) * suh.astype(np.float32)[:, None]
    expected = butterflies(expected, 1) * svh.astype(np.float32)
    return trellis, suh, svh, expected


@pytest.mark.parametrize("book", [0, 1, 2])
@pytest.mark.parametrize("bits", range(1, 9))
def test_zero_trellis(oracle, bits, book):
    trellis = np.zeros((8, 8, 16 * bits), np.int16)
    rc, v = oracle.exl3_reconstruct(trellis, np.full(128, -0.5, np.float16), np.full(128, 2, np.float16), book)
    assert rc == 0
    assert abs(v[0, 0] - np.float32(-128 * ZERO_STATE[book])) < 1e-4  # the test's EXPECT_NEAR
    assert np.count_nonzero(v) == 1


@pytest.mark.parametrize("book", [0, 1, 2])
@pytest.mark.parametrize("bits", range(1, 9))
def test_independent_restatement(oracle, bits, book):
    trellis, suh, svh, expected = fixture(bits, book)
    rc, v = oracle.exl3_reconstruct(trellis, suh, svh, book)
    assert rc == 0
    assert np.array_equal(v.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("book", [0, 1, 2])
def test_every_state(oracle, book):
    trellis, suh, svh, expected = fixture(8, book, cols=1024, exhaustive=True)
    rc, v = oracle.exl3_reconstruct(trellis, suh, svh, book)
    assert rc == 0
    assert np.array_equal(v.view(np.uint32), expected.view(np.uint32))


def test_output_range(oracle):
    trellis, suh, svh, _ = fixture(3, 0)
    big = np.full(128, 60000, np.float16)
    rc, _ = oracle.exl3_reconstruct(trellis, big, np.full(256, 60000, np.float16), 0, out_dtype=10)
    assert rc == 4
