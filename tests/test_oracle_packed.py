"""CPU checks of the oracle's DequantizePacked for the 32-value GGUF formats
(oracle/oracle.c, restating onnx_core/runtime/dequantize_packed.cc:173-235):
the FNV-1a hashes of the reference test's corpus, which that test takes from
independent GGML-C oracles, and hand-checked values of each layout."""
import numpy as np
import pytest

FORMATS = ["gguf:q4_0", "gguf:q4_1", "gguf:q5_0", "gguf:q5_1", "gguf:q8_0", "gguf:q8_1", "gguf:iq4_nl",
           "gguf:q4_k", "gguf:q6_k", "gguf:q2_k", "gguf:q3_k", "gguf:q5_k", "gguf:q8_k", "gguf:iq4_xs",
           "gguf:tq1_0", "gguf:tq2_0", "gguf:mxfp4", "gguf:nvfp4", "gguf:q1_0", "gguf:q2_0"]
# the codebook profiles (lattice grids of ggml-common.h)
IQ_FORMATS = ["gguf:iq2_xxs", "gguf:iq2_xs", "gguf:iq2_s", "gguf:iq3_xxs", "gguf:iq3_s", "gguf:iq1_s",
              "gguf:iq1_m"]
ALL_FORMATS = FORMATS + IQ_FORMATS
AFFINE = {"gguf:q4_1", "gguf:q5_1", "gguf:q2_k", "gguf:q4_k", "gguf:q5_k"}  # a second fp16 (minimum) after d
# byte offset of the fp16 scale d; None: no fp16 d (q8_k's is fp32, the fp4
# formats carry scale bytes)
D_OFFSET = {"gguf:q2_k": 80, "gguf:q3_k": 108, "gguf:q6_k": 208, "gguf:tq1_0": 52, "gguf:tq2_0": 64,
            "gguf:q8_k": None, "gguf:mxfp4": None, "gguf:nvfp4": None, "gguf:iq1_m": None}
VALUES = {"gguf:nvfp4": 64, "gguf:q2_0": 64, "gguf:q1_0": 128}


def block_values(fmt):
    if fmt in VALUES:
        return VALUES[fmt]
    small = ("gguf:q4_0", "gguf:q4_1", "gguf:q5_0", "gguf:q5_1", "gguf:q8_0", "gguf:q8_1", "gguf:iq4_nl",
             "gguf:mxfp4")
    return 32 if fmt in small else 256


def d_offset(fmt):
    return D_OFFSET.get(fmt, 0)


def corpus(oracle, fmt, scales):
    """The reference test's 64-block corpus (test_dequantize_packed.cc:41-73):
    byte j of block i is (73j + 29i + 17(j // 7) + 11(i // 3)) mod 256, then
    the fp16 scale d at its offset and, for the formats with a minimum, the
    fp16 of the next scale right after it; q8_k takes the fp32 scale / 3 in
    its first 4 bytes, mxfp4 the scale byte (17 i) mod 256, iq1_m the fp16
    scale's four nibbles in the top nibbles of its 16-bit scale words at 48."""
    size = oracle.packed_block_bytes(fmt)
    i = np.arange(64)[:, None]
    j = np.arange(size)[None, :]
    blocks = ((j * 73 + i * 29 + (j // 7) * 17 + (i // 3) * 11) & 255).astype(np.uint8)
    at = d_offset(fmt)
    if at is not None:
        d = oracle.f32_to_f16_bits(np.array([scales[k % 8] for k in range(64)], np.float32))
        blocks[:, at], blocks[:, at + 1] = d & 255, d >> 8
        if fmt in AFFINE:
            m = oracle.f32_to_f16_bits(np.array([scales[(k + 1) % 8] for k in range(64)], np.float32))
            blocks[:, at + 2], blocks[:, at + 3] = m & 255, m >> 8
    elif fmt == "gguf:q8_k":
        bits = np.array([np.float32(scales[k % 8] / 3) for k in range(64)], np.float32).view(np.uint32)
        for b in range(4):
            blocks[:, b] = (bits >> (8 * b)) & 255
    elif fmt == "gguf:mxfp4":
        blocks[:, 0] = (np.arange(64) * 17) & 255
    elif fmt == "gguf:iq1_m":
        d = oracle.f32_to_f16_bits(np.array([scales[k % 8] for k in range(64)], np.float32)).astype(np.int64)
        for j in range(4):
            word = blocks[:, 48 + 2 * j].astype(np.int64) | (blocks[:, 49 + 2 * j].astype(np.int64) << 8)
            word = (word & 0x0FFF) | (((d >> (4 * j)) & 15) << 12)
            blocks[:, 48 + 2 * j], blocks[:, 49 + 2 * j] = word & 255, word >> 8
    return blocks.reshape(-1)


def fnv1a64(values: np.ndarray) -> str:
    h = 14695981039346656037
    for byte in np.ascontiguousarray(values, np.float32).reshape(-1).view(np.uint8).tolist():
        h = ((h ^ byte) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


@pytest.mark.parametrize("fmt", ALL_FORMATS)
def test_ggml_oracle_hashes(oracle, golden, fmt):
    g = golden["dequantize_packed_gguf"]
    x = corpus(oracle, fmt, g["corpus_scales"])
    y = oracle.dequantize_packed(x, fmt, (2, 32 * block_values(fmt)))
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


def test_k_quant_layouts_by_hand(oracle):
    # q4_k: d = 1, dmin = 0.5; sub-block 0 scale 3 / minimum 2 (bytes 4, 8);
    # sub-block 5 scale (byte 13 & 15) | ((byte 5 >> 6) << 4) = 4 | 16,
    # minimum (byte 13 >> 4) | ((byte 9 >> 6) << 4) = 0; byte 5 is also
    # sub-block 1's scale (& 63 = 0)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x38]
    blk[4] = 3
    blk[8] = 2
    blk[16] = 0xA7          # element 0 -> 7 (low nibble), element 32 -> 10 (high nibble)
    blk[5] = 0x40
    blk[13] = 0x04
    y = oracle.dequantize_packed(blk, "gguf:q4_k", (256,))
    assert y[0] == 3 * 7 - 0.5 * 2
    assert y[32] == 0.0  # sub-block 1: scale 0, minimum 0
    # element 168 = sub-block 5, byte (168 // 64) * 32 + 168 % 32 = 72, high nibble
    blk[16 + 72] = 0x90
    y = oracle.dequantize_packed(blk, "gguf:q4_k", (256,))
    assert y[168] == (4 | 16) * 9
    # q6_k: d = 2 at byte 208, scale -3 for values 0..15; value 0 = (0x5 | (2 << 4)) - 32 = 5
    blk = np.zeros(210, np.uint8)
    blk[208:210] = [0x00, 0x40]
    blk[192] = 0xFD
    blk[0] = 0x05
    blk[128] = 0x02
    y = oracle.dequantize_packed(blk, "gguf:q6_k", (256,))
    assert y[0] == 2 * -3 * (0x25 - 32)
    assert y[1] == 2 * -3 * -32


def test_codebook_layouts_by_hand(oracle):
    """Single octets of each codebook profile built by hand from the grids'
    first rows (ggml-common.h: iq2xxs_grid[1] = 0x080808080808082b,
    iq3xxs_grid[5] = 0x04040c3e, iq1s_grid[1] = 0xffffffffffffff01)."""
    one = [0x00, 0x3C]  # fp16 1.0
    # iq2_xxs: octet 0 index 1, w = scale nibble 2 (<< 28), lane 0 signs 0b0000001
    # (odd count: the parity bit 7 is set too): scale (1 * 2.5) * 0.25 = 0.625
    blk = np.zeros(66, np.uint8)
    blk[0:2] = one
    blk[2] = 1
    w = (2 << 28) | 0b0000001
    blk[6:10] = [w & 255, (w >> 8) & 255, (w >> 16) & 255, w >> 24]
    y = oracle.dequantize_packed(blk, "gguf:iq2_xxs", (256,))
    assert list(y[:8]) == [-0.625 * 43, 0.625 * 8, 0.625 * 8, 0.625 * 8, 0.625 * 8, 0.625 * 8, 0.625 * 8,
                           -0.625 * 8]
    # iq3_xxs: octet 0 indices 5 (row 0x04040c3e: 62, 12, 4, 4) and 0; scale
    # nibble 0: (1 * 0.5) * 0.5 = 0.25; no signs
    blk = np.zeros(98, np.uint8)
    blk[0:2] = one
    blk[2] = 5
    y = oracle.dequantize_packed(blk, "gguf:iq3_xxs", (256,))
    assert list(y[:8]) == [0.25 * 62, 0.25 * 12, 0.25 * 4, 0.25 * 4, 1.0, 1.0, 1.0, 1.0]
    # iq1_s: octet 0 index 1 (lanes +1, -1 x 7), word at 34 = 0x8000 | (1 << 12):
    # scale 1 * 3, delta -0.125
    blk = np.zeros(50, np.uint8)
    blk[0:2] = one
    blk[2] = 1
    blk[34:36] = [0x00, 0x90]
    y = oracle.dequantize_packed(blk, "gguf:iq1_s", (256,))
    assert list(y[:8]) == [3 * 0.875] + [3 * -1.125] * 7
    # iq1_m: d from the words' top nibbles (0x3C00 = 1.0: nibbles 0, 0, 12, 3),
    # octet 0 index 1, scale field 0 of word 0 = 2 -> 5, nibble of byte 32 = 8:
    # delta -0.125
    blk = np.zeros(56, np.uint8)
    blk[0] = 1
    blk[32] = 8
    words = [2, 0, 0xC000, 0x3000]
    for j, wv in enumerate(words):
        blk[48 + 2 * j], blk[49 + 2 * j] = wv & 255, wv >> 8
    y = oracle.dequantize_packed(blk, "gguf:iq1_m", (256,))
    assert list(y[:8]) == [5 * 0.875] + [5 * -1.125] * 7
