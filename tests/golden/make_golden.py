"""Writes tests/golden/attn_golden.npz: per case the input hash and the fp64 oracle's O and LSE (stored as
float32). Run from the repository root: python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
sys.path.insert(0, HERE)
import cases  # noqa: E402


def main():
    out = {}
    for mk in cases.CASES:
        c = mk()
        o, lse = cases.oracle_of(c)
        out[c["name"] + ".hash"] = np.array(c["hash"])
        out[c["name"] + ".o"] = o.astype(np.float32)
        out[c["name"] + ".lse"] = lse.astype(np.float32)
    path = os.path.join(HERE, "attn_golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
