"""The reference's GroupedMatMul backend cases (tests/golden/
grouped_matmul_cases.json), expanded over the dtypes, index types, transB
values and bias modes the reference's case builder loops over."""
import json
import os

import numpy as np

FLOAT, FLOAT16, DOUBLE, BFLOAT16 = 1, 10, 11, 16
HERE = os.path.dirname(os.path.abspath(__file__))


def encode(values, dtype, oracle):
    v = np.asarray(values, np.float64)
    if dtype == FLOAT:
        return v.astype(np.float32)
    if dtype == DOUBLE:
        return v
    if dtype == FLOAT16:
        return oracle.f32_to_f16_bits(v.astype(np.float32))
    return oracle.f32_to_bf16_bits(v.astype(np.float32))


def expand(oracle):
    """[(name, dtype, x, w, idx, bias, transB, expected)], arrays in the
    dtype's storage (uint16 bits for FLOAT16 / BFLOAT16)."""
    src = json.load(open(os.path.join(HERE, "golden", "grouped_matmul_cases.json")))
    out = []

    def t(spec, dtype):
        shape, vals = spec
        return encode(vals, dtype, oracle).reshape(shape)

    def add(name, c, dtype, wkey="weights", tb=None, bias=None, okey="output", idx_dt=np.int64):
        idx = np.asarray(c["indices"][1], idx_dt).reshape(c["indices"][0])
        out.append((name, dtype, t(c["input"], dtype), t(c[wkey], dtype), idx,
                    None if bias is None else t(bias, dtype), c.get("transB", 0) if tb is None else tb,
                    t(c[okey], dtype)))

    for key in ("basic", "permutation", "with_bias", "unused_group", "single_group"):
        c = src[key]
        for dt in c["dtypes"]:
            for idx_dt in (np.int64, np.int32):
                add(f"{key}_{dt}_{np.dtype(idx_dt).name}", c, dt, bias=c["bias"], idx_dt=idx_dt)
    c = src["transB_bias_modes"]
    for dt in c["dtypes"]:
        for idx_dt in (np.int64, np.int32):
            for tb in c["transB_values"]:
                for with_bias in (False, True):
                    add(f"transB_{tb}_{dt}_{np.dtype(idx_dt).name}_bias_{int(with_bias)}", c, dt,
                        "weights_transB" if tb else "weights_transB0", tb, c["bias"] if with_bias else None,
                        "output_bias" if with_bias else "output", idx_dt)
    e = src["empty"]
    for m, s in e["tokens_selections"]:
        for with_bias in (False, True):
            for tb in (0, 1):
                w_shape = (e["G"], e["N"], e["K"]) if tb else (e["G"], e["K"], e["N"])
                out.append((f"empty_{m}x{s}_bias_{int(with_bias)}_transB_{tb}", FLOAT,
                            np.zeros((m, e["K"]), np.float32), np.zeros(w_shape, np.float32),
                            np.zeros((m, s), np.int64),
                            np.zeros((e["G"], e["N"]), np.float32) if with_bias else None, tb,
                            np.zeros((m, s, e["N"]), np.float32)))
    return out
