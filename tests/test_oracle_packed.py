"""CPU checks of the oracle's DequantizePacked for the 32-value GGUF formats
(oracle/oracle.c, restating onnx_core/runtime/dequantize_packed.cc:173-235):
the FNV-1a hashes of the reference test's corpus, which that test takes from
independent GGML-C oracles, and hand-checked values of each layout."""
import numpy as np
import pytest

FORMATS = ["gguf:q4_0", "gguf:q4_1", "gguf:q5_0", "gguf:q5_1", "gguf:q8_0", "gguf:q8_1", "gguf:iq4_nl"]
AFFINE = {"gguf:q4_1", "gguf:q5_1"}


def corpus(oracle, fmt, scales):
    """64 blocks: byte j of block i is (73j + 29i + 17(j // 7) + 11(i // 3)) mod 256,
    then the fp16 scale (and, for the affine formats, the fp16 minimum of the
    next scale) over the first bytes."""
    size = oracle.packed_block_bytes(fmt)
    i = np.arange(64)[:, None]
    j = np.arange(size)[None, :]
    blocks = ((j * 73 + i * 29 + (j // 7) * 17 + (i // 3) * 11) & 255).astype(np.uint8)
    d = oracle.f32_to_f16_bits(np.array([scales[k % 8] for k in range(64)], np.float32))
    blocks[:, 0], blocks[:, 1] = d & 255, d >> 8
    if fmt in AFFINE:
        m = oracle.f32_to_f16_bits(np.array([scales[(k + 1) % 8] for k in range(64)], np.float32))
        blocks[:, 2], blocks[:, 3] = m & 255, m >> 8
    return blocks.reshape(-1)


def fnv1a64(values: np.ndarray) -> str:
    h = 14695981039346656037
    for byte in np.ascontiguousarray(values, np.float32).reshape(-1).view(np.uint8).tolist():
        h = ((h ^ byte) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


@pytest.mark.parametrize("fmt", FORMATS)
def test_ggml_oracle_hashes(oracle, golden, fmt):
    g = golden["dequantize_packed_gguf"]
    x = corpus(oracle, fmt, g["corpus_scales"])
    y = oracle.dequantize_packed(x, fmt, (2, 32 * 32))
    assert fnv1a64(y) == g["fnv1a64"][fmt]


def test_layouts_by_hand(oracle):
    # q4_0: d = 2, low nibbles are elements 0..15, high nibbles 16..31, minus 8
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x40]  # fp16 2.0
    blk[2] = 0xF3            # element 0 -> 3 - 8, element 16 -> 15 - 8
    y = oracle.dequantize_packed(blk, "gguf:q4_0", (32,))
    assert y[0] == -10.0 and y[16] == 14.0 and y[1] == -16.0
    # q5_1: element 5 takes bit 5 of qh as its fifth bit, then d * q + m
    blk = np.zeros(24, np.uint8)
    blk[0:2] = [0x00, 0x3C]  # d = 1
    blk[2:4] = [0x00, 0xBC]  # m = -1
    blk[4:8] = [0x20, 0, 0, 0]
    blk[8 + 5] = 0x01
    y = oracle.dequantize_packed(blk, "gguf:q5_1", (32,))
    assert y[5] == 16 + 1 - 1 and y[0] == -1.0
    # q8_1: codes start after d and s
    blk = np.zeros(36, np.uint8)
    blk[0:2] = [0x00, 0x38]  # d = 0.5
    blk[4] = 0x80            # -128
    assert oracle.dequantize_packed(blk, "gguf:q8_1", (32,))[0] == -64.0
    # iq4_nl: the non-linear table
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2] = 0x0F
    y = oracle.dequantize_packed(blk, "gguf:iq4_nl", (32,))
    assert y[0] == 113.0 and y[16] == -127.0
