"""ORT MatMulNBits packing for tests: codes [K, N] and zero points [groups, N]
into the B [N, groups, block * bits / 8] and packed UINT8 zero-point
[N, ceil(groups * bits / 8)] arrays the ORT format stores: column n's block g
is one blob, row g * block + j at bit (j % (8 / bits)) * bits of byte
j / (8 / bits), padding bits zero (onnx_core/runtime/quantization.cc:
1790-1880)."""
import numpy as np


def ort_pack(codes, zp, bits, block):
    codes = np.asarray(codes, np.int64)
    K, N = codes.shape
    per = 8 // bits
    groups = (K + block - 1) // block
    blob = block * bits // 8
    B = np.zeros((N, groups, blob), np.uint8)
    for r in range(K):
        g, j = divmod(r, block)
        B[:, g, j // per] |= (codes[r, :] << ((j % per) * bits)).astype(np.uint8)
    zpk = None
    if zp is not None:
        zp = np.asarray(zp, np.int64)
        zpk = np.zeros((N, (groups + per - 1) // per), np.uint8)
        for g in range(groups):
            zpk[:, g // per] |= (zp[g, :] << ((g % per) * bits)).astype(np.uint8)
    return B, zpk
