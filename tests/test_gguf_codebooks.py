"""The GGUF IQ codebooks in onnx-light_amd/csrc/gguf_codebooks.h (shared by
the device decode and the oracle):

- every entry against the reference's own text of the grids
  (onnx_light/onnx_core/runtime/dequantize_packed_codebooks.inc, re-read and
  re-encoded by onnx-light_amd/gen_gguf_codebooks.py), when the reference
  tree is present;
- always: the grids' value sets and distinct rows, and first rows as ggml
  publishes them (src/ggml-common.h).  The decode through them is pinned by
  the reference test's GGML-C hashes (test_oracle_packed.py, GPU in
  test_gpu_packed.py).
"""
import importlib.util
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "onnx-light_amd", "csrc", "gguf_codebooks.h")
REFERENCE = "/root/reference"


def _header():
    text = open(HEADER).read()
    out = {}
    for name, body in re.findall(r"(kGguf\w+)\[\d+\]\s*=\s*\{([^}]*)\}", text):
        out[name] = [int(v, 16) for v in re.findall(r"0x[0-9a-f]+", body)]
    return out


def _gen():
    spec = importlib.util.spec_from_file_location("gen_gguf_codebooks",
                                                  os.path.join(ROOT, "onnx-light_amd", "gen_gguf_codebooks.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _lanes(word, n):
    return [((word >> (8 * j)) & 255) - (256 if (word >> (8 * j)) & 128 else 0) for j in range(n)]


VALUES = {"kGgufIq2xxs": {8, 25, 43}, "kGgufIq2xs": {8, 25, 43}, "kGgufIq2s": {8, 25, 43},
          "kGgufIq3xxs": {4, 12, 20, 28, 36, 44, 52, 62}, "kGgufIq3s": {1, 3, 5, 7, 9, 11, 13, 15},
          "kGgufIq1s": {-1, 0, 1}}
SIZES = {"kGgufIq2xxs": 256, "kGgufIq2xs": 512, "kGgufIq2s": 1024, "kGgufIq3xxs": 256, "kGgufIq3s": 512,
         "kGgufIq1s": 2048}


def test_value_sets_and_distinct_rows():
    h = _header()
    for name, size in SIZES.items():
        rows = h[name]
        lanes = 4 if "Iq3" in name else 8
        assert len(rows) == size, name
        assert len(set(rows)) == size, f"{name}: repeated rows"
        assert set(v for r in rows for v in _lanes(r, lanes)) <= VALUES[name], name


def test_published_first_rows():
    h = _header()
    assert h["kGgufIq2xxs"][:4] == [0x0808080808080808, 0x080808080808082b, 0x0808080808081919, 0x0808080808082b08]
    assert h["kGgufIq3xxs"][:4] == [0x04040404, 0x04040414, 0x04040424, 0x04040c0c]
    assert h["kGgufIq1s"][:2] == [0xffffffffffffffff, 0xffffffffffffff01]


@pytest.mark.skipif(not os.path.isdir(os.path.join(REFERENCE, "onnx_light")), reason="reference tree absent")
def test_header_matches_reference_text():
    gen = _gen()
    want = gen.grids_from_reference(REFERENCE)
    assert _header() == want
    with open(HEADER) as f:
        assert f.read() == gen.render(want), "header is the generator's output"
