"""Writes pool_digests.json: for each case of pool_cases.CASES, the SHA-256
of its inputs (source pool, destination pool before the transfer, slot
lists) and of its results (the packed transfer rows and the destination pool
after unpack), computed by numpy indexing of the layout views
(pool_cases.numpy_pack_unpack).

    python tests/golden/make_pool_digests.py
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import pool_cases  # noqa: E402


def sha(a) -> str:
    return hashlib.sha256(a.tobytes()).hexdigest()


def main():
    out = {"_comment": "SHA-256 digests of the pool_cases.CASES transfers; written by make_pool_digests.py "
                       "from numpy views of the page-major layout (kv_cache.rs:653-700)."}
    for c in pool_cases.CASES:
        rows, dst = pool_cases.numpy_pack_unpack(c)
        out[c.name] = {
            "src_pool": sha(c.src_pool()), "dst_pool_before": sha(c.dst_pool()),
            "src_slots": sha(c.src_slots()), "dst_slots": sha(c.dst_slots()),
            "rows": sha(rows), "dst_pool_after": sha(dst),
        }
    with open(os.path.join(HERE, "pool_digests.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
