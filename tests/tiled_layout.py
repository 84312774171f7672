"""numpy restatement of the tiled 4-bit weight layout, shared by the tests."""
import numpy as np


def tile_int4(x_packed, K, N, signed):
    """numpy restatement of the tiled layout (onnx-light_amd/csrc/kernels.hpp):
    16-column tiles, 128-row groups of 64 lanes x 4 dwords; lane 16g + i,
    dword c = column 16t + i, rows 128q + 32c + 8g + (0..7); row j of the 8 at
    bit 4*(j//2) (j even) or 16 + 4*(j//2) (j odd); offset-binary values."""
    flat = np.asarray(x_packed, dtype=np.uint8).reshape(-1)
    nib = np.empty(flat.size * 2, dtype=np.uint8)
    nib[0::2] = flat & 15
    nib[1::2] = flat >> 4
    vals = nib[:K * N].reshape(K, N).astype(np.uint32)
    if signed:
        vals ^= 8
    nt, ng = (N + 15) // 16, (K + 127) // 128
    pad = np.full((ng * 128, nt * 16), 8 if signed else 0, dtype=np.uint32)
    pad[:K, :N] = vals
    # [t][q][g][i][c][j] <- row 128q + 32c + 8g + j, column 16t + i
    v = pad.reshape(ng, 4, 4, 8, nt, 16)           # q, c, g, j, t, i
    v = v.transpose(4, 0, 2, 5, 1, 3)              # t, q, g, i, c, j
    shifts = np.array([0, 16, 4, 20, 8, 24, 12, 28], dtype=np.uint32)
    words = np.bitwise_or.reduce(v << shifts, axis=-1).astype(np.uint32)
    return words.reshape(-1)
