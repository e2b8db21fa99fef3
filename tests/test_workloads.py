"""Seeded workload generators and the algorithmic-bytes accounting (CPU only)."""
from __future__ import annotations

import numpy as np
import torch

from aether_nexus_amd import workloads as W
from aether_nexus_amd.types import unpack_codes


def test_generation_is_deterministic_and_shaped():
    g = W.tiny(batch=2, queries=3, copies=2)
    a = W.generate(g, seed=5)
    b = W.generate(g, seed=5)
    c = W.generate(g, seed=6)
    for k in ("q", "hot_k", "cold", "refs", "dictionary"):
        assert torch.equal(getattr(a, k), getattr(b, k))
    assert not torch.equal(a.q, c.q)
    assert a.q.shape == (1, 2, 3, 8, 64)
    assert a.hot_k.shape == (1, g.hot_blocks, 16, 8, 64)
    assert a.cold.shape == (1, g.cold_blocks, 16, 8, 8)
    assert a.refs.shape == (2, 1, 2, g.refs_stride)


def test_refs_cover_each_block_once():
    g = W.tiny(batch=3, copies=2, layers=2)
    a = W.generate(g, seed=1)
    refs = a.refs.numpy().view(np.uint32)
    for l in range(2):
        hot = np.sort(refs[:, l, :, : g.hot_count].reshape(-1))
        cold = np.sort(refs[:, l, :, g.hot_count:].reshape(-1))
        np.testing.assert_array_equal(hot, np.arange(g.hot_blocks))
        np.testing.assert_array_equal(cold, np.arange(g.cold_blocks))


def test_dictionary_rows_unit_norm_and_codes_in_range():
    g = W.tiny()
    a = W.host_arrays(W.generate(g, seed=2))
    D = a["dictionary"].view(np.float16).astype(np.float64).reshape(-1, g.head_dim)
    np.testing.assert_allclose(np.linalg.norm(D, axis=1), 1.0, atol=2e-3)
    idx, coef = unpack_codes(a["cold"])
    assert idx.max() < g.dict_size
    assert 0.4 < coef.astype(np.float64).std() < 0.6  # N(0, 0.5)


def test_zipf_indices_are_heavy_tailed():
    """Zipf(1.1) over 4096 atoms: the top atom takes ~1/H = 16% of the slots."""
    gen = torch.Generator().manual_seed(0)
    codes = W.make_codes(gen, (20000,), 4096, 0.5, 1.1, "cpu")
    idx, _ = unpack_codes(codes.numpy().view(np.uint16))
    counts = np.bincount(idx.reshape(-1).astype(np.int64), minlength=4096)
    top = np.sort(counts)[::-1] / counts.sum()
    h = (np.arange(1, 4097, dtype=np.float64) ** -1.1).sum()
    assert abs(top[0] - 1 / h) < 0.01
    assert top[:16].sum() > 0.4


def test_algorithmic_bytes_match_the_published_table():
    """Bytes per step of the benchmark shapes (reference layout, K == V)."""
    assert W.tiny().algorithmic_bytes()["total"] == 461_120
    assert W.hot_only().algorithmic_bytes()["total"] == 8_406_016
    assert W.hot_cold().algorithmic_bytes()["total"] == 9_462_272
    assert W.batched().algorithmic_bytes()["total"] == 1_212_170_240
    assert W.spec_verify().algorithmic_bytes()["total"] == 3_292_659_712
    assert W.sweep(64).algorithmic_bytes()["total"] == 539_525_120
