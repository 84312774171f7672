"""Writes tests/golden/<name>_digest.json from the reference's golden files
for the QQQ and BitBLAS encodings (unittests/python/backend/data/
qqq_native_v1.json and bitblas_native_v1.json, written by the upstream
packers at the revision they name): every case's metadata and input tensors
kept whole, its codes and expected FLOAT weights [out_features,
in_features] kept as SHA-256 digests of their little-endian bytes plus the
first and last 64 values, so the files stay small while still pinning every
output bit.  Run where the reference sits at /root/reference (or pass its
data directory)."""
import hashlib
import json
import os
import sys

import numpy as np

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/unittests/python/backend/data"
HERE = os.path.dirname(os.path.abspath(__file__))
NAMES = ("qqq_native_v1", "bitblas_native_v1")


def arr(t):
    return np.frombuffer(bytes.fromhex(t["hex"]), dtype=np.dtype(t["dtype"]).newbyteorder("<")).reshape(t["shape"])


def digest(case):
    codes, expected = arr(case["codes"]), arr(case["expected"])
    ev = expected.astype("<f4").reshape(-1).view(np.uint32)
    out = {k: v for k, v in case.items() if k not in ("codes", "expected", "source_sha256", "torch_version")}
    out.update({
        "codes_sha256": hashlib.sha256(codes.astype(np.uint8).tobytes()).hexdigest(),
        "expected_shape": list(expected.shape),
        "expected_sha256": hashlib.sha256(expected.astype("<f4").tobytes()).hexdigest(),
        "expected_head_bits": [int(v) for v in ev[:64]],
        "expected_tail_bits": [int(v) for v in ev[-64:]],
    })
    return out


def main():
    for name in NAMES:
        cases = json.load(open(os.path.join(SRC, name + ".json")))
        json.dump([digest(c) for c in cases], open(os.path.join(HERE, name + "_digest.json"), "w"), indent=0)


if __name__ == "__main__":
    main()
