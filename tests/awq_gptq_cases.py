"""AWQ and GPTQ checkpoints for tests.

- The fixtures of the reference's own tests, rebuilt here from their
  construction rules and pinned words
  (unittests/cc/onnx_core/runtime/test_awq.cc:18-118,
  unittests/cc/onnx_core/runtime/test_gptq.cc:18-124): ``awq_fixture`` and
  ``gptq_fixture``, ``gptq_upstream_words`` / ``gptq_upstream_v1_zeros`` (the
  words the reference pins as outputs of the upstream GPTQModel packers).
- Packers for arbitrary shapes (``awq_pack``, ``gptq_pack``), written from
  the layout rules of onnx_core/runtime/awq.cc:185-247 and gptq.cc:166-205;
  the CPU tests check them against the pinned upstream words before the GPU
  tests use them.
"""
import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)    # column n of a word's slot j (pack_awq_columns)
AWQ_INVERSE = (0, 4, 1, 5, 2, 6, 3, 7)  # nibble of column n % 8


def f16(values):
    return np.asarray(values, np.float32).astype(np.float16)


# ---- the reference tests' fixtures ------------------------------------------

def awq_expected(n, k):
    return (n * 7 + k * 3 + k // 16 + k // 64) % 16


def awq_fixture(variant, group_size=64):
    """test_awq.cc:36-118: K = 128, N = 8; codes awq_expected(n, k), zeros
    (n + g) % 16, scales (g + 1) / 4.  Returns dict(qweight, qzeros, scales)
    with numpy arrays of the checkpoint dtypes (scales float16)."""
    K, N = 128, 8
    group = 128 if group_size == -1 else group_size
    groups = 128 // group
    multiplier = 1 if group >= 128 else 128 // group
    padded = multiplier * 8
    if variant == "gemm":
        words = np.zeros(128, np.uint32)
        zeros = np.zeros(groups, np.uint32)
        for k in range(128):
            for j in range(8):
                words[k] |= np.uint32(awq_expected(AWQ_ORDER[j], k) << (4 * j))
        for g in range(groups):
            for j in range(8):
                zeros[g] |= np.uint32(((AWQ_ORDER[j] + g) % 16) << (4 * j))
        scales = np.array([[(g + 1) * 0.25] * 8 for g in range(groups)], np.float32)
        return dict(qweight=words.view(np.int32).reshape(128, 1), qzeros=zeros.view(np.int32).reshape(groups, 1),
                    scales=f16(scales))
    if variant == "gemv":
        words = np.zeros(8 * 16, np.uint32)
        zeros = np.full(8 * padded // 8, 0xFEDCBA98, np.uint32)
        for n in range(8):
            for k in range(128):
                words[n * 16 + k // 8] |= np.uint32(awq_expected(n, k) << (4 * (k % 8)))
            for g in range(groups):
                i = n * (padded // 8) + g // 8
                zeros[i] = (int(zeros[i]) & ~(15 << (4 * (g % 8))) & 0xFFFFFFFF) | (((n + g) % 16) << (4 * (g % 8)))
        scales = np.full((8, padded), -3, np.float32)
        for n in range(8):
            for g in range(groups):
                scales[n, g] = (g + 1) * 0.25
        return dict(qweight=words.view(np.int32).reshape(8, 16),
                    qzeros=zeros.view(np.int32).reshape(8, padded // 8), scales=f16(scales))
    # gemv_fast / llm-awq: the source's forward reshape / permute chain
    permuted = np.zeros(8 * 128, np.uint8)
    for n in range(8):
        for block in range(4):
            first = [0] * 32
            for a in range(4):
                for b in range(4):
                    for c in range(2):
                        first[(a * 4 + b) * 2 + c] = awq_expected(n, block * 32 + (b * 4 + a) * 2 + c)
            for a in range(4):
                for b in range(2):
                    for c in range(4):
                        permuted[n * 128 + block * 32 + a * 8 + b * 4 + c] = first[a * 8 + c * 2 + b]
    words = np.zeros(2 * 128, np.uint32)
    for nb in range(2):
        for kb in range(2):
            for j in range(64):
                for lane in range(4):
                    flat = j * 4 + lane
                    words[nb * 128 + kb * 64 + j] |= np.uint32(
                        int(permuted[(nb * 4 + flat // 64) * 128 + kb * 64 + flat % 64]) << (4 * lane))
    scales = np.full((padded, 8), -3, np.float32)
    zero_terms = np.full((padded, 8), 7, np.float32)
    for g in range(groups):
        for n in range(8):
            scales[g, n] = (g + 1) * 0.25
            zero_terms[g, n] = -float((n + g) % 16) * scales[g, n]
    return dict(qweight=(words & 0xFFFF).astype(np.uint16).view(np.int16).reshape(2, 128), qzeros=f16(zero_terms),
                scales=f16(scales))


def gptq_upstream_words(bits, planar):
    """test_gptq.cc:18-40: upstream packings of codes (arange(32) * 7 + 3) % 2^bits."""
    table = {
        2: [0x1b1b1b1b, 0x1b1b1b1b],
        4: [0x4d6f81a3, 0xc5e7092b, 0x4d6f81a3, 0xc5e7092b],
        5: [0x4d6f81a3, 0xc5e7092b, 0x4d6f81a3, 0xc5e7092b, 0xc663399c],
        6: [0x4d6f81a3, 0xc5e7092b, 0x4d6f81a3, 0xc5e7092b, 0xa543e950, 0x503e940f],
        7: [0x4d6f81a3, 0xc5e7092b, 0x4d6f81a3, 0xc5e7092b, 0xa543e950, 0x503e940f, 0xf803fe00],
        8: [0x18110a03, 0x342d261f, 0x5049423b, 0x6c655e57, 0x88817a73, 0xa49d968f, 0xc0b9b2ab, 0xdcd5cec7],
    }
    if bits == 3:
        return [0x1b1b1b1b, 0x1b1b1b1b, 0xf0f0f0f0] if planar else [0x53977053, 0x70539770, 0x97705397]
    return table[bits]


def gptq_upstream_v1_zeros(bits):
    """test_gptq.cc:42-56: upstream v1 packings of zero fields (arange(32) * 5 + 3) % (2^bits - 1)."""
    return {2: [0x18618618, 0x86186186], 3: [0x3174298b, 0xd0a62e85, 0x98ba14c5],
            4: [0x83d83d83, 0x3d83d83d, 0xd83d83d8, 0x83d83d83]}.get(
        bits, [0x120d0803, 0x26211c17, 0x3a35302b, 0x4e49443f, 0x625d5853, 0x76716c67, 0x8a85807b, 0x9e99948f])


WORD_DTYPES = {1: np.int8, 2: np.int16, 4: np.int32, 8: np.int64}


def stream_words(words, width):
    """The little-endian byte stream of 32-bit `words` read back as words of
    `width` bytes (test_gptq.cc:58-75, NativeWord)."""
    raw = np.asarray(words, np.uint32).astype("<u4").tobytes()
    return np.frombuffer(raw, WORD_DTYPES[width]).copy()


def gptq_fixture(bits=4, fmt="gptq_v2", width=4):
    """test_gptq.cc:86-124: K = N = 32, group 16; every column holds the
    stream of gptq_upstream_words, both zero rows the same stream (the v1
    zero stream for "gptq"); scales 0.5 (group 0) and 1.5 (group 1) FLOAT16;
    g_idx[k] = k % 2."""
    planar = bits in (5, 6, 7) or fmt == "gptq_p"
    w = stream_words(gptq_upstream_words(bits, planar), width)
    z = stream_words(gptq_upstream_v1_zeros(bits) if fmt == "gptq" else gptq_upstream_words(bits, planar), width)
    qweight = np.repeat(w[:, None], 32, axis=1)
    qzeros = np.stack([z, z])
    scales = f16(np.array([[0.5] * 32, [1.5] * 32], np.float32))
    g_idx = (np.arange(32) % 2).astype(np.int32)
    return dict(qweight=qweight, qzeros=qzeros, scales=scales, g_idx=g_idx)


# ---- packers for arbitrary shapes ---------------------------------------------

def awq_pack(variant, codes, zeros, scales, group):
    """Pack codes [K, N] and zero points [groups, N] (integers) with scales
    [groups, N] (float16 or bfloat16 bits) into an AWQ checkpoint: variant
    "gemm" (4 bits), "gemm8" (the 8-bit gemm layout) or "gemv".  gemv pads
    the group axis as awq.cc:97-100 does, with zero words 0 and scales 1.0
    in the padding."""
    codes = np.asarray(codes, np.int64)
    zeros = np.asarray(zeros, np.int64)
    K, N = codes.shape
    groups = zeros.shape[0]
    if variant == "gemm":
        qw = np.zeros((K, N // 8), np.uint32)
        qz = np.zeros((groups, N // 8), np.uint32)
        for n in range(N):
            qw[:, n // 8] |= (codes[:, n] << (4 * AWQ_INVERSE[n % 8])).astype(np.uint32)
            qz[:, n // 8] |= (zeros[:, n] << (4 * AWQ_INVERSE[n % 8])).astype(np.uint32)
        return dict(qweight=qw.view(np.int32), qzeros=qz.view(np.int32), scales=np.asarray(scales))
    if variant == "gemm8":
        return dict(qweight=codes.astype(np.uint8).reshape(K, N // 4, 4).view("<u4")[..., 0].view(np.int32),
                    qzeros=zeros.astype(np.uint8).reshape(groups, N // 4, 4).view("<u4")[..., 0].view(np.int32),
                    scales=np.asarray(scales))
    assert variant == "gemv"
    eff = K // groups
    multiplier = 1 if eff >= 128 else 128 // eff
    words = -(-groups // 8)
    padded = -(-words // multiplier) * multiplier * 8
    qw = np.zeros((N, K // 8), np.uint32)
    for k in range(K):
        qw[:, k // 8] |= (codes[k, :] << (4 * (k % 8))).astype(np.uint32)
    qz = np.zeros((N, padded // 8), np.uint32)
    for g in range(groups):
        qz[:, g // 8] |= (zeros[g, :] << (4 * (g % 8))).astype(np.uint32)
    sc = np.ones((N, padded), np.float16)
    sc[:, :groups] = np.asarray(scales).T
    return dict(qweight=qw.view(np.int32), qzeros=qz.view(np.int32), scales=sc)


def _pieces(bits, word_bits, planar, index):
    """(word, shift, width, offset) pieces of logical code `index` (gptq.cc:168-189)."""
    if not planar:
        bit = index * bits
        shift = bit % word_bits
        low = min(bits, word_bits - shift)
        out = [(bit // word_bits, shift, low, 0)]
        if low != bits:
            out.append((bit // word_bits + 1, 0, bits - low, low))
        return out
    out, offset, word = [], 0, (index // 32) * bits
    for plane in (4, 2, 1):
        if bits & plane:
            factor = 32 // plane
            out.append((word + (index % 32) // factor, ((index % 32) % factor) * plane, plane, offset))
            offset += plane
            word += plane
    return out


def gptq_pack(codes, stored_zeros, bits, width=4, planar=False):
    """Pack codes [K, N] and stored zero fields [groups, N] (the value minus 1
    for format "gptq") into qweight [ceil(K bits / word bits), N] and qzeros
    [groups, ceil(N bits / word bits)] words of `width` bytes."""
    codes = np.asarray(codes, np.uint64)
    zs = np.asarray(stored_zeros, np.uint64)
    K, N = codes.shape
    groups = zs.shape[0]
    wb = 8 * width
    rows = -(-K * bits // wb)
    zcols = -(-N * bits // wb)
    qw = np.zeros((rows, N), np.uint64)
    qz = np.zeros((groups, zcols), np.uint64)
    for k in range(K):
        for word, shift, nb, off in _pieces(bits, wb, planar, k):
            qw[word, :] |= ((codes[k, :] >> np.uint64(off)) & np.uint64((1 << nb) - 1)) << np.uint64(shift)
    for n in range(N):
        for word, shift, nb, off in _pieces(bits, wb, planar, n):
            qz[:, word] |= ((zs[:, n] >> np.uint64(off)) & np.uint64((1 << nb) - 1)) << np.uint64(shift)
    dt = WORD_DTYPES[width]
    return qw.astype(np.dtype(dt).str.replace("i", "u")).view(dt), qz.astype(np.dtype(dt).str.replace("i", "u")).view(dt)
