"""Writes tests/golden/tiny_seed1.npz: the inputs of the tiny Weaver workload
(8 q / 8 kv heads, head_dim 64, hot 256 tokens, cold 1024 codes per kv head,
512-atom shared dictionary, scale 1 with q ~ N(0,1)/8) and of a small
per-kv-head-dictionary variant (4 q / 2 kv heads), with the fp64 oracle's
outputs.

Inputs are stored, not regenerated, so the fixture does not depend on the
random generator of any library version.  Run from the repository root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from aether_nexus_amd import workloads as W  # noqa: E402
from oracle import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "tiny_seed1.npz"


def main():
    blobs = {}
    for tag, geom in (("shared", W.tiny()), ("perhead", W.tiny(q_heads=4, kv_heads=2, dict_heads=2))):
        a = W.host_arrays(W.generate(geom, seed=1))
        for k in ("q", "hot_k", "cold", "refs", "dictionary"):
            blobs[f"{tag}_{k}"] = a[k]
        blobs[f"{tag}_out_f64"] = oracle.decode_f64(geom, a)
    np.savez_compressed(OUT, **blobs)
    print(OUT, OUT.stat().st_size)


if __name__ == "__main__":
    main()
