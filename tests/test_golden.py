"""Committed golden vectors (CPU only): the oracle reproduces the stored
fp64 outputs of the tiny workload from the stored inputs."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from aether_nexus_amd import workloads as W
from oracle import oracle

FIX = Path(__file__).resolve().parent / "golden" / "tiny_seed1.npz"
GEOMS = {"shared": W.tiny(), "perhead": W.tiny(q_heads=4, kv_heads=2, dict_heads=2)}


def load(tag):
    z = np.load(FIX)
    a = {k: z[f"{tag}_{k}"] for k in ("q", "hot_k", "cold", "refs", "dictionary")}
    return a, z[f"{tag}_out_f64"]


@pytest.mark.parametrize("tag", sorted(GEOMS))
def test_oracle_reproduces_golden(tag):
    a, out = load(tag)
    np.testing.assert_array_equal(oracle.decode_f64(GEOMS[tag], a), out)
    r32 = oracle.decode_ref32(GEOMS[tag], a).astype(np.float64)
    assert np.abs(r32 - out).max() < 2e-3
