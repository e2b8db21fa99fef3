"""Value partials from the cold kernel (AW_COLD_OUT_VALUES) against the fp64
oracle and against the bins + finish path on the same inputs.

For dictionary heads of at most 128 KiB the cold kernel multiplies its own
bins by the dictionary, sum_a bin[a][r] * D[a] in fp32, and hands each split's
(m, l, O) to the merge beside the hot splits; no finish runs.  Both forms are
exact rewrites of the cold sum of weaver_kernel.metal:172-222, so each is held
to the attention bar against the fp64 brute force, and the two are compared
with each other.

Shapes: shared and per-kv-head dictionaries, one sequence with many cold
splits (row chunks of 1), R = 16 and 32 rows per kv head (chunks of 4), no hot
pool, head_dim 64, a dictionary size that is not a power of two, bit-31 refs,
two layers, ragged sequences with empty cold and hot parts, and the peaked
softmax with an fp32 q_latent."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aether_nexus_amd import workloads as W
from aether_nexus_amd.types import (AW_COLD_OUT_AUTO, AW_COLD_OUT_BINS, AW_COLD_OUT_VALUES, AW_PROJECT_AUTO,
                                    AW_PROJECT_VALU)
from aether_nexus_amd.weaver import plan
from oracle import oracle

from tests.helpers import assert_close, errors, run_gpu

pytestmark = pytest.mark.gpu

CASES = {
    "tiny_shared": W.tiny(),
    "tiny_per_head_b2_q2_causal": W.tiny(batch=2, queries=2, causal=True, dict_heads=8),
    "one_seq_512x8": W.hot_cold(hot_count=8, cold_count=256, dict_size=512, dict_heads=8),
    "one_seq_512x8_verify4": W.hot_cold(queries=4, causal=True, hot_count=8, cold_count=256, dict_size=512,
                                        dict_heads=8),
    "b8_shared_512": W.hot_cold(batch=8, hot_count=4, cold_count=64, dict_size=512),
    "b2_q8_r32": W.hot_cold(batch=2, queries=8, causal=True, hot_count=4, cold_count=64, dict_size=512,
                            dict_heads=8),
    "cold_only": W.hot_cold(hot_count=0, cold_count=64, dict_size=512, dict_heads=8),
    "d64_1024": W.hot_cold(batch=2, head_dim=64, hot_count=2, cold_count=40, dict_size=1024),
    "atoms_480": W.hot_cold(batch=2, hot_count=2, cold_count=40, dict_size=480, dict_heads=8),
    "bit31": W.tiny(dict_heads=8, tag_bit31=True),
    "l2_b4": W.Geometry(layers=2, batch=4, hot_count=2, cold_count=48, dict_size=512, dict_heads=8, scale=0.1),
}


def _mode(engine, mode):
    class _M:
        def __enter__(self):
            engine.set_cold_output(mode)

        def __exit__(self, *exc):
            engine.set_cold_output(AW_COLD_OUT_AUTO)
    return _M()


def _desc_plan(geom, q_latent_f32=False):
    wl = W.generate(geom, seed=0)
    out = torch.empty(wl.out_shape(), dtype=torch.float16)
    return plan(W.device_desc(wl, out, q_latent_f32=q_latent_f32))


@pytest.mark.parametrize("name", list(CASES))
def test_values_and_bins_match_oracle(engine, stream, name):
    geom = CASES[name]
    seed = 300 + list(CASES).index(name)
    assert _desc_plan(geom).cold_output == AW_COLD_OUT_VALUES, "the planner takes value partials here"
    wl = W.generate(geom, seed=seed)
    print(f"cold values case {name}: {geom}", flush=True)
    ref = oracle.decode_f64(geom, W.host_arrays(wl))
    with _mode(engine, AW_COLD_OUT_VALUES):
        got_v = run_gpu(engine, wl, stream)
    with _mode(engine, AW_COLD_OUT_BINS):
        got_b = run_gpu(engine, wl, stream)
    assert_close(got_v, ref, f"{name} values")
    assert_close(got_b, ref, f"{name} bins")
    ma, rl = errors(got_v, got_b)
    print(f"{name}: values against bins max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= 2e-3 and rl <= 1e-3


def test_values_ragged_sequences(engine, stream):
    """Sequences with no cold tokens (their cold splits are empty: m = -inf,
    l = 0 and no O written), no hot tokens, or neither."""
    geom = W.hot_cold(batch=4, hot_count=6, cold_count=40, dict_size=512, dict_heads=8)
    wl = W.generate(geom, seed=310)
    wl.seq_hot = torch.tensor([[6, 0, 0, 3]], dtype=torch.int32)
    wl.seq_cold = torch.tensor([[0, 40, 0, 7]], dtype=torch.int32)
    ref = oracle.decode_f64(geom, W.host_arrays(wl))
    with _mode(engine, AW_COLD_OUT_VALUES):
        got = run_gpu(engine, wl, stream)
    assert np.all(got.reshape(4, -1)[2] == 0.0), "a sequence with nothing visible gives zeros"
    assert_close(got, ref, "values, ragged")


def test_values_repeat_calls_bit_identical(engine, stream):
    """Static token order and ordered sums: the same bits on every call."""
    geom = W.hot_cold(batch=2, hot_count=8, cold_count=256, dict_size=512, dict_heads=8)
    wl = W.generate(geom, seed=311)
    with _mode(engine, AW_COLD_OUT_VALUES):
        a = run_gpu(engine, wl, stream)
        b = run_gpu(engine, wl, stream)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("hot_count", [0, 8], ids=["cold_only", "hot_cold"])
def test_values_peaked_softmax(engine, stream, hot_count):
    """The peaked softmax (coefficient std 6, q std 2) over 512-atom per-kv-head
    dictionaries with an fp32 q_latent: outputs reach [4, 8), where the f16
    output's half-ulp is 1.95e-3, so the 2e-3 bar applies beyond it."""
    geom = W.hot_cold(batch=2, hot_count=hot_count, cold_count=256, dict_size=512, dict_heads=8, coef_std=6.0,
                      q_std=2.0)
    wl = W.generate(geom, seed=312)
    ref = oracle.decode_f64(geom, W.host_arrays(wl))
    with _mode(engine, AW_COLD_OUT_VALUES):
        got = run_gpu(engine, wl, stream, q_latent_f32=True).astype(np.float64)
    half_ulp = np.spacing(np.abs(got).astype(np.float16)).astype(np.float64) / 2
    excess = np.abs(got - ref) - half_ulp
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    print(f"values, peaked, hot {hot_count}: max-abs {np.abs(got - ref).max():.2e}, beyond f16 rounding "
          f"{excess.max():.2e}, rel-L2 {rel:.2e}, max |out| {np.abs(ref).max():.2f}", flush=True)
    assert np.all(np.isfinite(got)) and excess.max() <= 2e-3 and rel <= 1e-3


@pytest.mark.parametrize("queries", [1, 4], ids=["decode", "verify_4"])
def test_values_tiered_requests(engine, stream, queries):
    """The tiered cache's requests: hot 2048 + cold 32768 tokens over 512-atom
    per-kv-head dictionaries, fp32 q_latent, separate V, causal, one query or
    four (R = 16 rows per kv head, row chunks of 4)."""
    geom = W.hot_cold(queries=queries, dict_size=512, dict_heads=8, separate_v=True, causal=True)
    assert _desc_plan(geom, q_latent_f32=True).cold_output == AW_COLD_OUT_VALUES
    wl = W.generate(geom, seed=320 + queries)
    ref = oracle.decode_f64(geom, W.host_arrays(wl))
    got = run_gpu(engine, wl, stream, q_latent_f32=True)
    assert_close(got, ref, f"values, tiered request, {queries} queries")


@pytest.mark.parametrize("path", ["mfma_kernel", "valu_kernel", "callers"])
def test_values_q_latent_sources(engine, stream, path):
    """Value partials with q_latent from the projection's MFMA tiles (the
    planner's choice), its VALU kernel (AW_PROJECT_VALU set), or handed over by
    the caller (the reference's buffer, f16; the projection then only writes
    D^T)."""
    geom = W.hot_cold(batch=2, queries=2, causal=True, hot_count=4, cold_count=64, dict_size=512, dict_heads=8)
    wl = W.generate(geom, seed=330)
    a = W.host_arrays(wl)
    if path == "callers":
        ql = oracle.qlatent_f64(geom, a).astype(np.float16)
        a["q_latent"] = ql.view(np.uint16)
        wl.q_latent = torch.from_numpy(ql.view(np.int16).copy()).view(torch.float16)
    ref = oracle.decode_f64(geom, a)
    engine.set_projection(AW_PROJECT_VALU if path == "valu_kernel" else AW_PROJECT_AUTO)
    try:
        with _mode(engine, AW_COLD_OUT_VALUES):
            got = run_gpu(engine, wl, stream)
    finally:
        engine.set_projection(AW_PROJECT_AUTO)
    assert_close(got, ref, f"values, q_latent from the {path}")
