"""GPU parity of DequantizePacked for the 32-value GGUF formats against the
oracle: bit-exact in all four output dtypes (FLOAT, FLOAT16, BFLOAT16,
DOUBLE).  The reference test's corpus is checked against its GGML-C hashes
through the GPU too; random blocks include NaN, infinite, subnormal and
maximal fp16 scales; outputs at unaligned addresses take the per-element
stores."""
import numpy as np
import pytest
import torch

from test_oracle_packed import FORMATS, corpus, fnv1a64

pytestmark = pytest.mark.gpu
OUT = {"float": (1, torch.float32), "float16": (10, torch.float16), "bfloat16": (16, torch.bfloat16),
       "double": (11, torch.float64)}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _bits(t, out):
    c = t.cpu()
    if out in ("float16", "bfloat16"):
        return c.view(torch.int16).numpy().view(np.uint16)
    return c.numpy()


@pytest.mark.parametrize("fmt", FORMATS)
def test_corpus_hashes_on_gpu(olamd, oracle, golden, dev, fmt):
    g = golden["dequantize_packed_gguf"]
    x = corpus(oracle, fmt, g["corpus_scales"])
    y = olamd.dequantize_packed(torch.from_numpy(x).to(dev), fmt, (2, 1024))
    assert fnv1a64(y.cpu().numpy()) == g["fnv1a64"][fmt]


@pytest.mark.parametrize("out", list(OUT))
@pytest.mark.parametrize("fmt", FORMATS)
def test_random_blocks_vs_oracle(olamd, oracle, dev, fmt, out):
    rng = np.random.default_rng(len(fmt) * 7 + len(out) + FORMATS.index(fmt) * 101)
    size = oracle.packed_block_bytes(fmt)
    for shape in [(32,), (3, 5, 64), (7, 4096), (1, 96)]:
        nb = int(np.prod(shape)) // 32
        x = rng.integers(0, 256, (nb, size)).astype(np.uint8)
        # scales: random fp16 bit patterns, with NaN, inf, subnormal and 65504 among them
        special = np.array([0x7E00, 0xFC00, 0x0001, 0x7BFF, 0x8000, 0x3C00], np.uint16)
        d = rng.integers(0, 65536, nb).astype(np.uint16)
        d[: min(nb, len(special))] = special[: min(nb, len(special))]
        x[:, 0], x[:, 1] = d & 255, d >> 8
        x = x.reshape(-1)
        want = oracle.dequantize_packed(x, fmt, shape, OUT[out][0])
        for offset in (0, 1):
            if offset:
                raw = torch.empty(int(np.prod(shape)) + 1, dtype=OUT[out][1], device=dev)
                y = raw[1:].view(shape)
            else:
                y = None
            got = olamd.dequantize_packed(torch.from_numpy(x).to(dev), fmt, shape, OUT[out][0], out=y)
            g = _bits(got, out)
            if out in ("float", "double"):
                same = np.array_equal(g.view(np.uint32 if out == "float" else np.uint64),
                                      want.view(np.uint32 if out == "float" else np.uint64))
            else:
                same = np.array_equal(g, want)
            assert same, (fmt, out, shape, offset)


def test_empty_shape(olamd, dev):
    y = olamd.dequantize_packed(torch.zeros(0, dtype=torch.uint8, device=dev), "gguf:q4_0", (0, 32))
    assert tuple(y.shape) == (0, 32)
