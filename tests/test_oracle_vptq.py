"""The VPTQ oracle (oracle.c, orc_vptq_reconstruct) pinned by the reference's
golden fixture tests/golden/vptq_native_v1.json (copied from
unittests/python/backend/data/, written by the pinned upstream
VPTQLinear.dequantize: plain, residual, outlier, grouped by size and by
count, norm along either dim, permuted, in FLOAT, FLOAT16 and BFLOAT16
codebooks, with indices crossing INT32 words).  Every case reproduces bit
for bit; planted decoder mistakes (the residual not rounded to the codebook
dtype, the permutation ignored) are rejected; CheckData's errors."""
import json
import os

import numpy as np
import pytest

import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vptq_native_v1.json")
DTYPE_CODES = {"float32": 1, "float16": 10, "bfloat16": 16}


def _arr(t):
    raw = bytes.fromhex(t["raw_hex"])
    if t["dtype"] == "bfloat16":
        return np.frombuffer(raw, "<u2").reshape(t["shape"]).copy()
    return np.frombuffer(raw, np.dtype(t["dtype"]).newbyteorder("<")).reshape(t["shape"]).copy()


def vptq_cases():
    return json.load(open(GOLDEN))["fixtures"]


def golden(f):
    """(config, tensors, expected FLOAT values [n, k])."""
    tensors = {k: _arr(v) for k, v in f["tensors"].items()}
    dtype = DTYPE_CODES[f["tensors"]["centroids.weight"]["dtype"]]
    e = _arr(f["expected"])
    expected = (e.astype(np.uint32) << 16).view(np.float32) if dtype == 16 else e.astype(np.float32)
    return orc.vptq_config(f["parameters"], dtype), tensors, expected


@pytest.mark.parametrize("f", vptq_cases(), ids=lambda f: f["name"])
def test_golden_vptq_cases(oracle, f):
    cfg, tensors, expected = golden(f)
    rc, out = oracle.vptq_reconstruct(cfg, tensors)
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32)), f["name"]


def test_golden_rejects_planted_mistakes(oracle):
    f = next(f for f in vptq_cases() if f["name"] == "combined_float16_norm0_perm_tails")
    cfg, tensors, expected = golden(f)
    t = dict(tensors)
    t["perm"] = np.arange(cfg.k, dtype=np.int32)  # the permutation ignored
    rc, out = oracle.vptq_reconstruct(cfg, t)
    assert rc == 0 and not np.array_equal(out, expected)
    f = next(f for f in vptq_cases() if f["name"] == "residual_float32")
    cfg, tensors, expected = golden(f)
    t = dict(tensors)
    t["res_centroids.weight"] = np.zeros_like(tensors["res_centroids.weight"])  # the residual dropped
    rc, out = oracle.vptq_reconstruct(cfg, t)
    assert rc == 0 and not np.array_equal(out, expected)


def test_checks_and_errors(oracle):
    f = next(f for f in vptq_cases() if f["name"] == "combined_float16_norm0_perm_tails")
    cfg, tensors, _ = golden(f)
    t = dict(tensors)
    t["indices"] = np.full_like(tensors["indices"], -1)  # every field all ones: main 7, residual 3
    assert oracle.vptq_reconstruct(cfg, t)[0] == 0       # 8 and 4 entries
    cfg.num_centroids[1] = 7                              # same 3-bit field, entry 7 now past the codebook
    assert oracle.vptq_reconstruct(cfg, t)[0] == 1
    cfg, tensors, _ = golden(f)
    t = dict(tensors)
    oi = tensors["outlier_indices"].copy()
    oi.reshape(-1)[2] = 5  # 5 outlier centroids
    t["outlier_indices"] = oi
    assert oracle.vptq_reconstruct(cfg, t)[0] == 2
    t = dict(tensors)
    p = tensors["perm"].copy()
    p[3] = p[4]
    t["perm"] = p
    assert oracle.vptq_reconstruct(cfg, t)[0] == 3
    f = next(f for f in vptq_cases() if f["name"] == "base_float32_cross_word_sign")
    cfg, tensors, _ = golden(f)
    t = dict(tensors)
    c = tensors["centroids.weight"].copy()
    c.reshape(-1)[:] = 1e5  # fits FLOAT and BFLOAT16, not FLOAT16
    t["centroids.weight"] = c
    assert oracle.vptq_reconstruct(cfg, t)[0] == 0
    assert oracle.vptq_reconstruct(cfg, t, out_dtype=orc.FLOAT16)[0] == 4
    c.reshape(-1)[:] = np.nan
    assert oracle.vptq_reconstruct(cfg, t)[0] == 5
