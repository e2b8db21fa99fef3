"""Seeded random geometries through aw_decode_device against the fp64 oracle:
kv heads 1-8, GQA groups 1-7, 1-4 query tokens (causal or not), head_dim 64
or 128, dictionaries of 16-1024 atoms shared or per kv head (those of at most
128 KiB per head with a multiple of 32 atoms take the cold kernel's value
partials, the others its bins), 0-9 hot and 0-39 cold blocks per sequence,
ragged per-sequence counts, separate V, bit 31 on refs, uniform or Zipf atom
indices, either cold pool order, 1-2 layers.  Each case draws its geometry
from its own seed, so a failure names a reproducible shape."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aether_nexus_amd import workloads as W
from oracle import oracle

from tests.helpers import assert_close

pytestmark = pytest.mark.gpu


def draw(seed: int):
    rng = np.random.default_rng(1000 + seed)
    kv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 7]))
    queries = int(rng.integers(1, min(4, 64 // g) + 1))
    hot, cold = int(rng.integers(0, 10)), int(rng.integers(0, 40))
    geom = W.Geometry(layers=int(rng.integers(1, 3)), batch=int(rng.integers(1, 6)), queries=queries,
                      q_heads=kv * g, kv_heads=kv, head_dim=int(rng.choice([64, 128])),
                      dict_size=int(rng.choice([16, 48, 96, 256, 512, 1008, 1024])),
                      dict_heads=1 if rng.random() < 0.5 else kv,
                      hot_count=hot, cold_count=cold, scale=float(rng.uniform(0.05, 0.5)),
                      causal=bool(rng.random() < 0.5), separate_v=bool(hot and rng.random() < 0.3),
                      zipf=1.1 if rng.random() < 0.3 else None, tag_bit31=bool(rng.random() < 0.5))
    ragged = rng.random() < 0.5
    hb = bool(cold and rng.random() < 0.5)
    return geom, ragged, hb, rng


@pytest.mark.parametrize("seed", range(48))
def test_random_geometry_matches_oracle(engine, stream, seed):
    geom, ragged, hb, rng = draw(seed)
    wl = W.generate(geom, seed=seed)
    if ragged:
        shape = (geom.layers, geom.batch)
        wl.seq_hot = torch.from_numpy(rng.integers(0, geom.hot_count + 1, shape).astype(np.int32))
        wl.seq_cold = torch.from_numpy(rng.integers(0, geom.cold_count + 1, shape).astype(np.int32))
    print(f"random case {seed}: {geom} ragged={ragged} head_blocked={hb}", flush=True)
    dev = wl.to("cuda:0")
    out = torch.full(dev.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
    desc = W.device_desc(dev, out, cold_head_blocked=W.head_blocked(dev.cold) if hb else None)
    engine.decode_device(desc, stream=stream)
    engine.check_device_errors(stream)
    assert_close(out.cpu().numpy(), oracle.decode_f64(geom, W.host_arrays(wl)), f"random case {seed}")
