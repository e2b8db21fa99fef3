"""Geometries that take the row-tile finish (one cold split per row and at least
1024 rows): 16 rows per work-group over an atom range, the bins and D^T in the
MFMA lane order, one range (merged in place) or several (merge_kernel).  Each
case names its shape; rows are compared with the fp64 oracle on a spread sample
that includes the first and last rows and every 16-row tile boundary class.

Shapes: shared and per-kv-head dictionaries, head_dim 128 and 64, GQA 4, 2 and 3
(3: row chunks of 2, rows per group not a multiple of 16), 1 and 2 layers,
ragged cold counts with empty sequences (rows without bins), both cold pool
orders, 1 and 2 atom ranges."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aether_nexus_amd import workloads as W
from oracle import oracle

from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

CASES = {
    # name: (geometry, ragged cold counts, head-blocked cold order)
    "b64_shared_2ranges": (W.Geometry(batch=64, hot_count=4, cold_count=48, dict_size=4096, scale=0.09), False, True),
    "b64_per_head": (W.Geometry(batch=64, hot_count=3, cold_count=40, dict_size=512, dict_heads=8, scale=0.1), False, False),
    "b128_one_range": (W.Geometry(batch=128, hot_count=2, cold_count=32, dict_size=1024, scale=0.1), False, True),
    "b64_d64": (W.Geometry(batch=64, head_dim=64, hot_count=2, cold_count=40, dict_size=1024, scale=0.15), False, False),
    "b128_gqa2_ragged": (W.Geometry(batch=128, q_heads=16, hot_count=2, cold_count=32, dict_size=2048, scale=0.1),
                         True, True),
    "b50_gqa3_chunks": (W.Geometry(batch=50, q_heads=24, hot_count=3, cold_count=36, dict_size=1024, scale=0.1),
                        False, False),
    "l2_b32": (W.Geometry(layers=2, batch=32, hot_count=2, cold_count=32, dict_size=2048, scale=0.1), True, False),
}


@pytest.fixture(autouse=True)
def _bins(engine):
    """These shapes are the finish kernel's: the cold kernel writes bins for it,
    also where its dictionary is small enough for value partials."""
    from aether_nexus_amd.types import AW_COLD_OUT_AUTO, AW_COLD_OUT_BINS
    engine.set_cold_output(AW_COLD_OUT_BINS)
    yield
    engine.set_cold_output(AW_COLD_OUT_AUTO)


def sample_rows(geom, n=160, seed=0):
    total = geom.layers * geom.batch * geom.queries * geom.q_heads
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(total, size=min(n, total), replace=False).tolist())
    rows |= {0, total - 1, total // 2}
    rows |= set(range(0, total, max(1, total // 64)))
    return np.array(sorted(rows), dtype=np.uint64)


@pytest.mark.parametrize("name", list(CASES))
def test_row_tile_finish_matches_oracle(engine, stream, name):
    geom, ragged, hb = CASES[name]
    seed = 11 + list(CASES).index(name)
    wl = W.generate(geom, seed=seed)
    if ragged:
        rng = np.random.default_rng(seed)
        sc = rng.integers(0, geom.cold_count + 1, (geom.layers, geom.batch)).astype(np.int32)
        sc[:, ::7] = 0  # sequences without cold tokens: their rows have no bins
        wl.seq_cold = torch.from_numpy(sc)
    print(f"row-tile finish case {name}: {geom} ragged={ragged} head_blocked={hb}", flush=True)
    dev = wl.to("cuda:0")
    out = torch.full(dev.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
    desc = W.device_desc(dev, out, cold_head_blocked=W.head_blocked(dev.cold) if hb else None)
    engine.decode_device(desc, stream=stream)
    engine.check_device_errors(stream)
    got = out.cpu().numpy().reshape(-1, geom.head_dim).astype(np.float64)
    rows = sample_rows(geom, seed=seed)
    assert np.all(np.isfinite(got)), f"{name}: non-finite output"
    ref = oracle.decode_f64(geom, W.host_arrays(wl), rows=rows, threads=16)
    assert_close(got[rows.astype(np.int64)], ref.reshape(rows.size, geom.head_dim), f"row-tile finish {name}")
