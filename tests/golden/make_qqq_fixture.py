"""Writes tests/golden/qqq_native_v1_digest.json from the reference's QQQ
fixture (unittests/python/backend/data/qqq_native_v1.json, written by the
upstream QQQ packer at the revision it names): every case's inputs (the
packed words B, s_channel, s_group) kept whole, its codes and expected FLOAT
weights [out_features, in_features] kept as SHA-256 digests of their
little-endian bytes plus the first and last 64 values, so the file stays
small while still pinning every output bit.  Run in a checkout that has the
reference at /root/reference (or pass its data path)."""
import hashlib
import json
import os
import sys

import numpy as np

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/unittests/python/backend/data/qqq_native_v1.json"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qqq_native_v1_digest.json")


def arr(t):
    return np.frombuffer(bytes.fromhex(t["hex"]), dtype=np.dtype(t["dtype"]).newbyteorder("<")).reshape(t["shape"])


def main():
    out = []
    for c in json.load(open(SRC)):
        codes, expected = arr(c["codes"]), arr(c["expected"])
        ev = expected.reshape(-1).view(np.uint32)
        out.append({
            "name": c["name"], "in_features": c["in_features"], "out_features": c["out_features"],
            "group_size": c["group_size"], "upstream_revision": c["upstream_revision"],
            "tensors": c["tensors"],
            "codes_sha256": hashlib.sha256(codes.astype(np.uint8).tobytes()).hexdigest(),
            "expected_shape": list(expected.shape),
            "expected_sha256": hashlib.sha256(expected.astype("<f4").tobytes()).hexdigest(),
            "expected_head_bits": [int(v) for v in ev[:64]],
            "expected_tail_bits": [int(v) for v in ev[-64:]],
        })
    json.dump(out, open(DST, "w"), indent=0)


if __name__ == "__main__":
    main()
