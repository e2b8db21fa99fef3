"""Pins of the CPU oracle (oracle/weaver_oracle.c), CPU only.

The reference has no runnable CPU path and no numeric tests (its only Weaver
test checks "some output is non-zero", nexus-core/src/weaver.rs:413), so the
oracle is pinned here by:
  * known answers derived from the reference's own test and bench inputs
    (weaver.rs:369-396, bench.rs:113-133);
  * closed forms: one visible token, equal scores, zero codes, empty pools;
  * invariants a plausible indexing mistake breaks: cold codes equal their
    decompressed rows attended as hot tokens, block-table permutations,
    masked ref bits, causal masking, score scale, per-head vs shared
    dictionaries, GQA head sharing;
  * agreement of its two independent restatements (fp32 kernel-order vs fp64
    dense brute force).
"""
from __future__ import annotations

import math
from dataclasses import replace

import numpy as np
import pytest

from aether_nexus_amd import workloads as W
from aether_nexus_amd.types import pack_codes
from oracle import oracle

BLOCK = 16


def f16(x):
    return np.asarray(x, dtype=np.float16).view(np.uint16)


def base_arrays(geom, seed=0):
    return W.host_arrays(W.generate(geom, seed=seed))


def assert_rel(got, ref, tol):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300)
    assert err <= tol, f"rel err {err:.3e} > {tol}"


# ------------------------------------------------------------ known answers

def test_reference_test_inputs_give_one():
    """weaver.rs:369-396: all-ones q, q_latent, hot pool and dictionary, zero codes,
    refs [0,1,2], 32/8/128, 512 atoms per kv head.  32 hot tokens score 128,
    16 cold tokens score 0: every output is 1.0 (e^-128 underflows in fp32)."""
    g = W.Geometry(q_heads=32, kv_heads=8, head_dim=128, dict_size=512, dict_heads=8, hot_count=2,
                   cold_count=1, scale=1.0)
    one = np.float16(1.0).view(np.uint16)
    arrs = {
        "q": np.full(32 * 128, one, np.uint16),
        "q_latent": np.full(32 * 512, one, np.uint16),
        "hot_k": np.full(2 * 16 * 8 * 128, one, np.uint16),
        "cold": np.zeros((3 * 16 * 8, 8), np.uint16),  # refs name cold block 2
        "refs": np.arange(3, dtype=np.uint32),
        "dictionary": np.full(8 * 512 * 128, one, np.uint16),
    }
    d64 = oracle.decode_f64(_Pools(g, hot_blocks=2, cold_blocks=3), arrs).reshape(-1)
    r32 = oracle.decode_ref32(_Pools(g, hot_blocks=2, cold_blocks=3), arrs).reshape(-1)
    assert np.all(d64 == 1.0)
    assert np.all(r32.view(np.uint16) == 0x3C00)


def test_reference_bench_inputs_closed_form():
    """bench.rs:113-133: 0.01 everywhere, 64 hot + 16 cold blocks, zero codes,
    refs 0..80.  1024 hot tokens of score 128*f16(0.01)^2, 256 cold tokens of
    score 0 and value 0: out = 1024 e^s v / (1024 e^s + 256) = 0.0080222 -> 0x201B."""
    g = W.Geometry(q_heads=32, kv_heads=8, head_dim=128, dict_size=512, dict_heads=8, hot_count=64,
                   cold_count=16, scale=1.0)
    v = np.float16(0.01)
    vb = v.view(np.uint16)
    arrs = {
        "q": np.full(32 * 128, vb, np.uint16),
        "q_latent": np.full(32 * 512, vb, np.uint16),
        "hot_k": np.full(64 * 16 * 8 * 128, vb, np.uint16),
        "cold": np.zeros((80 * 16 * 8, 8), np.uint16),
        "refs": np.arange(80, dtype=np.uint32),
        "dictionary": np.full(8 * 512 * 128, vb, np.uint16),
    }
    p = _Pools(g, hot_blocks=64, cold_blocks=80)
    out = oracle.decode_f64(p, arrs).reshape(-1)
    vf = float(v)
    s = 128 * vf * vf
    expect = 1024 * math.exp(s) * vf / (1024 * math.exp(s) + 256)
    assert abs(expect - 0.0080222) < 1e-6
    np.testing.assert_allclose(out, expect, rtol=1e-12)
    assert np.all(np.float16(out).view(np.uint16) == 0x201B)
    r32 = oracle.decode_ref32(p, arrs).reshape(-1).view(np.uint16)
    assert set(np.unique(r32)).issubset({0x201B, 0x201C})


class _Pools:
    """Geometry with explicit pool capacities (for hand-built arrays)."""

    def __init__(self, geom, hot_blocks, cold_blocks):
        self._g = geom
        self.hot_blocks = hot_blocks
        self.cold_blocks = cold_blocks

    def __getattr__(self, k):
        return getattr(self._g, k)


# ------------------------------------------------------------ closed forms

def test_empty_pools_give_zero():
    """hot_count = cold_count = 0: nothing visible, output 0 (metal:227-239)."""
    g = W.tiny(hot_count=0, cold_count=0)
    a = base_arrays(g)
    assert np.all(oracle.decode_f64(g, a) == 0.0)
    assert np.all(oracle.decode_ref32(g, a).view(np.uint16) == 0)


def test_equal_scores_give_mean_of_values():
    """q = 0: every score is 0, the output is the plain mean of the value rows."""
    g = W.tiny(cold_count=0, hot_count=4, kv_heads=2, q_heads=4)
    a = base_arrays(g, seed=3)
    a["q"] = np.zeros_like(a["q"])
    out = oracle.decode_f64(g, a)
    hot = a["hot_k"].view(np.float16).astype(np.float64).reshape(g.hot_blocks, 16, g.kv_heads, g.head_dim)
    refs = a["refs"].reshape(-1)[: g.hot_count]
    rows = hot[refs & 0x7FFFFFFF]  # [blocks, 16, Hkv, d]
    mean = rows.reshape(-1, g.kv_heads, g.head_dim).mean(axis=0)  # [Hkv, d]
    for h in range(g.q_heads):
        np.testing.assert_allclose(out[0, 0, 0, h], mean[h // g.gqa], rtol=1e-12, atol=1e-15)


def test_single_visible_token_gives_its_value():
    """Causal drafts: with Q = 16 queries over one hot block, query 0 sees only
    token 0 (ops.metal:549 rule), so its output is exactly V_0."""
    g = W.tiny(hot_count=1, cold_count=0, queries=16, causal=True, q_heads=2, kv_heads=1)
    a = base_arrays(g, seed=4)
    out = oracle.decode_f64(g, a)
    hot = a["hot_k"].view(np.float16).astype(np.float64).reshape(g.hot_blocks, 16, g.kv_heads, g.head_dim)
    blk = a["refs"].reshape(-1)[0] & 0x7FFFFFFF
    for h in range(2):
        np.testing.assert_array_equal(out[0, 0, 0, h], hot[blk, 0, 0])


def test_zero_codes_closed_form():
    """Zero codes score 0 and carry value 0: with n_c cold tokens,
    out = sum_hot e^s V / (sum_hot e^s + n_c)."""
    g = W.tiny(hot_count=2, cold_count=3)
    a = base_arrays(g, seed=5)
    a["cold"] = np.zeros_like(a["cold"])
    with_cold = oracle.decode_f64(g, a)
    g0 = replace(g, cold_count=0)
    a0 = dict(a)
    a0["refs"] = np.ascontiguousarray(a["refs"][..., : g.hot_count])
    hot_only = oracle.decode_f64(_Pools(g0, g.hot_blocks, 0), a0)
    # recover the hot-only softmax denominators to apply the closed form
    qf = a["q"].view(np.float16).astype(np.float64).reshape(g.q_heads, g.head_dim)
    hot = a["hot_k"].view(np.float16).astype(np.float64).reshape(g.hot_blocks, 16, g.kv_heads, g.head_dim)
    refs = a["refs"].reshape(-1)[: g.hot_count] & 0x7FFFFFFF
    for h in range(g.q_heads):
        k = hot[refs, :, h // g.gqa].reshape(-1, g.head_dim)
        s = g.scale * k @ qf[h]
        m = s.max()
        den = np.exp(s - m).sum()
        n_c = g.cold_count * 16
        expect = hot_only[0, 0, 0, h] * den / (den + n_c * math.exp(-m))
        np.testing.assert_allclose(with_cold[0, 0, 0, h], expect, rtol=1e-10, atol=1e-14)


# ------------------------------------------------------------ invariants

def _decompress_to_hot(g, a):
    """Dense rows sum_k c_k D[idx_k] of every referenced cold token, laid out as
    a hot pool (K == V) with identity refs."""
    D = a["dictionary"].view(np.float16).astype(np.float64).reshape(g.dict_heads, g.dict_size, g.head_dim)
    codes = a["cold"].reshape(g.cold_blocks, 16, g.kv_heads, 8)
    refs = a["refs"].reshape(-1)[g.hot_count: g.hot_count + g.cold_count] & 0x7FFFFFFF
    idx = codes[refs][..., :4].astype(np.int64)
    coef = codes[refs][..., 4:].copy().view(np.float16).astype(np.float64)
    rows = np.zeros((g.cold_count, 16, g.kv_heads, g.head_dim))
    for kv in range(g.kv_heads):
        Dh = D[0 if g.dict_heads == 1 else kv]
        rows[:, :, kv] = np.einsum("btk,btkd->btd", coef[:, :, kv], Dh[idx[:, :, kv]])
    return rows


def test_cold_equals_decompressed_hot():
    """The cold pass on codes equals ordinary attention over the decompressed
    rows sum_k c_k D[idx_k] (the identity (q.D^T).c = q.(D^T c)).  The rows are
    rounded to f16 to become a hot pool, so the comparison tolerates that."""
    g = W.tiny(hot_count=0, cold_count=8, dict_heads=8, coef_std=0.25)
    a = base_arrays(g, seed=6)
    cold_out = oracle.decode_f64(g, a)
    rows = _decompress_to_hot(g, a)
    gh = replace(g, hot_count=g.cold_count, cold_count=0)
    ah = {"q": a["q"], "hot_k": f16(rows).reshape(-1), "refs": np.arange(g.cold_count, dtype=np.uint32)}
    hot_out = oracle.decode_f64(_Pools(gh, g.cold_count, 0), ah)
    np.testing.assert_allclose(cold_out, hot_out, rtol=0, atol=2e-3 * max(1.0, np.abs(rows).max()))
    assert_rel(cold_out, hot_out, 2e-3)
    # and a planted indexing mistake (atoms of the wrong kv head) is caught
    a_bad = dict(a)
    D = a["dictionary"].reshape(g.dict_heads, -1)
    a_bad["dictionary"] = np.ascontiguousarray(np.roll(D, 1, axis=0)).reshape(-1)
    assert np.abs(oracle.decode_f64(g, a_bad) - cold_out).max() > 1e-2


def test_block_table_permutation_invariance_and_bit31():
    """Moving blocks in the pools and the refs together changes nothing; bit 31
    of a ref is ignored (weaver_kernel.metal:145,174)."""
    g = W.tiny()
    a = base_arrays(g, seed=7)
    out = oracle.decode_f64(g, a)
    rng = np.random.default_rng(0)
    ph = rng.permutation(g.hot_blocks)
    pc = rng.permutation(g.cold_blocks)
    b = dict(a)
    hot = a["hot_k"].reshape(g.hot_blocks, -1)
    cold = a["cold"].reshape(g.cold_blocks, -1)
    inv_h = np.argsort(ph)
    inv_c = np.argsort(pc)
    b["hot_k"] = np.ascontiguousarray(hot[ph]).reshape(-1)  # new block i holds old block ph[i]
    b["cold"] = np.ascontiguousarray(cold[pc]).reshape(a["cold"].shape)
    refs = a["refs"].copy().reshape(-1)
    refs[: g.hot_count] = inv_h[refs[: g.hot_count]]
    refs[g.hot_count:] = inv_c[refs[g.hot_count:]]
    refs[::3] |= np.uint32(1 << 31)
    b["refs"] = refs
    np.testing.assert_array_equal(oracle.decode_f64(g, b), out)
    np.testing.assert_array_equal(oracle.decode_ref32(g, b), oracle.decode_ref32(g, a))


def test_scale_equals_scaled_query():
    """scale 2 with q equals scale 1 with 2q (exact in f16)."""
    g = W.tiny(scale=2.0)
    a = base_arrays(g, seed=8)
    b = dict(a)
    b["q"] = f16(a["q"].view(np.float16).astype(np.float32) * 2)
    np.testing.assert_allclose(oracle.decode_f64(g, a), oracle.decode_f64(replace(g, scale=1.0), b),
                               rtol=1e-12, atol=1e-15)


def test_causal_masked_tokens_do_not_matter():
    """Query j sees hot tokens p < n - Q + 1 + j: changing the last hot token
    changes only the last query's output."""
    g = W.tiny(queries=4, causal=True, hot_count=2, cold_count=2)
    a = base_arrays(g, seed=9)
    out = oracle.decode_f64(g, a)
    b = dict(a)
    hot = a["hot_k"].reshape(g.hot_blocks, 16, -1).copy()
    last_blk = a["refs"].reshape(-1)[g.hot_count - 1] & 0x7FFFFFFF
    hot[last_blk, 15] = f16(np.full(hot.shape[-1], 3.0))
    b["hot_k"] = hot.reshape(-1)
    out2 = oracle.decode_f64(g, b)
    np.testing.assert_array_equal(out2[:, :, :3], out[:, :, :3])
    assert np.abs(out2[:, :, 3] - out[:, :, 3]).max() > 1e-3


def test_shared_dictionary_equals_identical_per_head():
    g = W.tiny(dict_heads=1)
    a = base_arrays(g, seed=10)
    gp = replace(g, dict_heads=g.kv_heads)
    b = dict(a)
    b["dictionary"] = np.ascontiguousarray(np.repeat(a["dictionary"], g.kv_heads, axis=1))
    np.testing.assert_array_equal(oracle.decode_f64(g, a), oracle.decode_f64(gp, b))


def test_gqa_heads_share_kv():
    """q heads of one kv group with the same query row get the same output."""
    g = W.tiny(q_heads=8, kv_heads=2)
    a = base_arrays(g, seed=11)
    q = a["q"].reshape(g.q_heads, g.head_dim).copy()
    q[1] = q[0]
    q[5] = q[4]
    a["q"] = q.reshape(-1)
    out = oracle.decode_f64(g, a)[0, 0, 0]
    np.testing.assert_array_equal(out[1], out[0])
    np.testing.assert_array_equal(out[5], out[4])
    assert np.abs(out[4] - out[0]).max() > 1e-4  # different kv heads differ


def test_q_latent_identity():
    """Passing q_latent = q.D^T in f16 reproduces the computed-q_latent result
    within the f16 rounding of q_latent."""
    g = W.tiny(dict_heads=8)
    a = base_arrays(g, seed=12)
    base = oracle.decode_f64(g, a)
    b = dict(a)
    b["q_latent"] = f16(oracle.qlatent_f64(g, a)).reshape(-1)
    assert_rel(oracle.decode_f64(g, b), base, 2e-3)
    # direct check of the projection against numpy
    D = a["dictionary"].view(np.float16).astype(np.float64).reshape(g.kv_heads, g.dict_size, g.head_dim)
    q = a["q"].view(np.float16).astype(np.float64).reshape(g.q_heads, g.head_dim)
    ql = oracle.qlatent_f64(g, a).reshape(g.q_heads, g.dict_size)
    np.testing.assert_allclose(ql, np.einsum("hd,had->ha", q, D[np.arange(g.q_heads) // g.gqa]), rtol=1e-12)


def test_f16_q_latent_envelope_on_a_peaked_softmax():
    """Why device-computed q_latent stays fp32: with coefficient std 6 and q std
    2 the reference's f16 q_latent buffer alone moves the fp64 decode past the
    2e-3 tolerance (f16 rounding shifts each score by up to 2^-11 of
    sum_k |c_k q_latent[idx_k]|, and a peaked softmax amplifies it), while an fp32
    q_latent stays well inside it."""
    geom = W.hot_cold(hot_count=0, cold_count=256, coef_std=6.0, q_std=2.0)
    a = base_arrays(geom, seed=11)
    exact = oracle.decode_f64(geom, a)
    ql = oracle.qlatent_f64(geom, a)
    b = dict(a)
    b["q_latent"] = f16(ql).reshape(-1)
    err16 = np.abs(oracle.decode_f64(geom, b) - exact).max()
    assert err16 > 2e-3, err16
    # fp32 rounding of q_latent: scores move by 2^-24 relative, 2^13 times less.
    q32 = ql.astype(np.float32).astype(np.float64)
    scale = geom.scale * (np.abs(q32).max() * 4 * 6.0 * 4)  # generous bound on |score| (coefficients within 4 std)
    assert scale * 2.0 ** -24 < 1e-5


def test_ref32_restatement_matches_f64():
    """The fp32 kernel-order restatement and the fp64 brute force agree to the
    accuracy of fp32 accumulation and f16 rounding of q_latent and outputs."""
    for geom, seed in [(W.tiny(), 1), (W.tiny(dict_heads=8, queries=3, causal=True), 2),
                       (W.hot_cold(hot_count=8, cold_count=32, dict_size=512), 3)]:
        a = base_arrays(geom, seed=seed)
        r32 = oracle.decode_ref32(geom, a).astype(np.float64)
        r64 = oracle.decode_f64(geom, a)
        assert np.abs(r32 - r64).max() < 2e-3
        assert_rel(r32, r64, 1e-3)


def test_row_subsets_match_full_decode():
    g = W.tiny(batch=2, queries=2)
    a = base_arrays(g, seed=13)
    full = oracle.decode_f64(g, a).reshape(-1, g.head_dim)
    rows = np.array([0, 5, 17, full.shape[0] - 1], dtype=np.uint64)
    np.testing.assert_array_equal(oracle.decode_f64(g, a, rows=rows), full[rows])
    full32 = oracle.decode_ref32(g, a).reshape(-1, g.head_dim)
    np.testing.assert_array_equal(oracle.decode_ref32_rows(g, a, rows), full32[rows])


def test_out_of_range_inputs_are_rejected():
    g = W.tiny()
    a = base_arrays(g, seed=14)
    b = dict(a)
    refs = a["refs"].copy().reshape(-1)
    refs[0] = g.hot_blocks  # past the hot pool
    b["refs"] = refs
    with pytest.raises(oracle.OracleError):
        oracle.decode_f64(g, b)
    c = dict(a)
    cold = a["cold"].copy()
    cold[..., 0] = g.dict_size  # atom index past the dictionary
    c["cold"] = cold
    with pytest.raises(oracle.OracleError):
        oracle.decode_f64(g, c)


def test_pack_codes_feeds_the_oracle():
    """Codes built with pack_codes are read by the oracle as the reference reads
    SparseCode (indices then f16 coefficients)."""
    g = W.tiny(hot_count=0, cold_count=1, q_heads=1, kv_heads=1, dict_size=512)
    a = base_arrays(g, seed=15)
    idx = np.tile(np.array([3, 3, 3, 3]), (16, 1))
    coef = np.tile(np.array([1.0, 0.0, 0.0, 0.0]), (16, 1))
    a["cold"] = pack_codes(idx, coef).reshape(g.cold_blocks, 16, 1, 8)
    out = oracle.decode_f64(g, a)[0, 0, 0, 0]
    D = a["dictionary"].view(np.float16).astype(np.float64).reshape(g.dict_size, g.head_dim)
    np.testing.assert_allclose(out, D[3], rtol=1e-12)  # 16 identical tokens: their value


# ---------------------------------------------------------------- encoder oracle
# Pins of or_encode_blocks / or_block_entropy (distiller.rs:126-159, 171-246).

def _rand_pool(rng, blocks, hkv, hd, scale=1.0):
    return (rng.standard_normal((blocks, 16, hkv, hd)) * scale).astype(np.float16).view(np.uint16)


def _unit_dict(rng, dh, a, hd):
    d = rng.standard_normal((dh, a, hd))
    return (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float16).view(np.uint16)


def test_encoder_zero_dictionary_reference_test():
    """distiller.rs:286-310: with a zeroed dictionary every score is 0; the
    stable order picks atoms 0, 1, 2, 3 (the reference test checks the first code)."""
    rng = np.random.default_rng(3)
    hot = _rand_pool(rng, 2, 8, 64)
    d = np.zeros((8, 512, 64), np.uint16)
    cold = oracle.encode_blocks(hot, d, [0, 1])
    assert (cold[..., :4] == np.array([0, 1, 2, 3], np.uint16)).all()
    assert ((cold[..., 4:] & 0x7FFF) == 0).all()  # coefficients are +-0


def test_encoder_one_hot_dictionary():
    """D[a] = e_a for a < head_dim, zero rows after: the score of atom a is the
    token's component a, so the code holds the four largest components (their
    f16 bits as coefficients) -- found here by a sort of the components."""
    rng = np.random.default_rng(4)
    hd, a = 64, 128
    hot = _rand_pool(rng, 1, 4, hd)
    d = np.zeros((1, a, hd), np.float16)
    d[0, np.arange(hd), np.arange(hd)] = 1.0
    cold = oracle.encode_blocks(hot, d.view(np.uint16), [0])
    x = hot.view(np.float16).astype(np.float64)
    for t in range(16):
        for g in range(4):
            comp = x[0, t, g]
            scores = np.concatenate([comp, np.zeros(a - hd)])
            order = sorted(range(a), key=lambda i: (-scores[i], i))[:4]
            assert list(cold[0, t, g, :4]) == order
            want = np.array([np.float16(scores[i]) for i in order]).view(np.uint16)
            got = cold[0, t, g, 4:]
            # exact: each score is one product x*1 plus zeros
            assert (np.where(want == 0x8000, 0, want) == np.where(got == 0x8000, 0, got)).all()


def test_encoder_matches_f64_projection():
    """Independent formulation: numpy f64 dot products.  Where the 4th and 5th
    largest scores differ by more than the f32 summation error bound the four
    indices match, and every coefficient is within one f16 ulp of f16(f64 score)."""
    rng = np.random.default_rng(5)
    hkv, hd, a = 2, 64, 256
    hot = _rand_pool(rng, 3, hkv, hd)
    d = _unit_dict(rng, hkv, a, hd)
    cold = oracle.encode_blocks(hot, d, [2, 0])
    x = hot.view(np.float16).astype(np.float64)
    D = d.view(np.float16).astype(np.float64)
    checked = 0
    for blk in (2, 0):
        for t in range(16):
            for g in range(hkv):
                s = D[g] @ x[blk, t, g]
                order = np.lexsort((np.arange(a), -s))
                bound = 2 * hd * 2.0 ** -24 * (np.abs(D[g]) @ np.abs(x[blk, t, g])).max()
                if s[order[3]] - s[order[4]] > bound:
                    assert list(cold[blk, t, g, :4]) == list(order[:4])
                    checked += 1
                got = cold[blk, t, g, 4:].view(np.float16).astype(np.float64)
                want = np.array([np.float16(s[i]) for i in cold[blk, t, g, :4]], dtype=np.float64)
                ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
                assert (np.abs(got - want) <= ulp).all()
    assert checked > 60  # of 64 token-heads


def test_encoder_planted_mistake_is_caught():
    """The f64 check above must fail for a plausible mistake: the other kv head's
    dictionary (a swapped head index)."""
    rng = np.random.default_rng(6)
    hkv, hd, a = 2, 64, 128
    hot = _rand_pool(rng, 1, hkv, hd)
    d = _unit_dict(rng, hkv, a, hd)
    cold = oracle.encode_blocks(hot, d[::-1].copy(), [0])  # heads swapped
    x = hot.view(np.float16).astype(np.float64)
    D = d.view(np.float16).astype(np.float64)
    mismatches = sum(list(cold[0, t, g, :4]) != list(np.lexsort((np.arange(a), -(D[g] @ x[0, t, g])))[:4])
                     for t in range(16) for g in range(hkv))
    assert mismatches > 16


def test_encoder_layouts_and_destinations():
    """Codes of hot block src[i] land in cold block dst[i] (default: the same
    index, distiller.rs:177), head-blocked order is the same codes transposed, and
    blocks not named are left as they were."""
    rng = np.random.default_rng(7)
    hot = _rand_pool(rng, 4, 4, 64)
    d = _unit_dict(rng, 4, 128, 64)
    base = oracle.encode_blocks(hot, d, [0, 1, 2, 3])
    pre = rng.integers(0, 65535, (6, 16, 4, 8), dtype=np.uint16)
    out = oracle.encode_blocks(hot, d, [3, 1], dst=[5, 0], cold=pre.copy())
    assert (out[5] == base[3]).all() and (out[0] == base[1]).all()
    assert (out[[1, 2, 3, 4]] == pre[[1, 2, 3, 4]]).all()
    hb = oracle.encode_blocks(hot, d, [0, 1, 2, 3], head_blocked=True)
    assert (hb == base.transpose(0, 2, 1, 3)).all()


def test_entropy_reference_tests_and_numpy():
    """distiller.rs:261-283: an all-zero block gives 0 and a block of 1.0 gives a
    variance below 1e-3 (exactly 0).  Random blocks agree with numpy's f64
    variance to 1e-12 relative before the final f32 rounding."""
    assert oracle.block_entropy(np.zeros(512, np.uint16)) == 0.0
    assert oracle.block_entropy(np.full(512, np.float16(1.0).view(np.uint16))) == 0.0
    assert oracle.block_entropy(np.array([0x8000, 0], np.uint16)) == 0.0  # -0 counts as zero
    rng = np.random.default_rng(8)
    for scale in (1.0, 0.01, 100.0):
        v = (rng.standard_normal(16 * 8 * 128) * scale).astype(np.float16)
        got = oracle.block_entropy(v.view(np.uint16))
        want = np.float32(np.var(v.astype(np.float64)))
        assert abs(float(got) - float(want)) <= 2 * np.spacing(want)
