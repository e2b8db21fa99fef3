"""CPU checks of the contiguous-cache attention oracle and of the inference-loop
host logic (aether_nexus_amd.inference): the oracle against torch's SDPA, closed
forms and the C decode oracle; the speculative-verify rule on hand-worked cases;
the KV cache bookkeeping of forward_batch / push_loom / pop_loom."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from aether_nexus_amd import inference as I
from oracle import attention_oracle as AO
from oracle import oracle


def rand_case(rng, nq, kv_len, hq, hkv, d, cap=None):
    cap = cap or -(-max(kv_len, 1) // 16) * 16
    q = rng.standard_normal((nq, hq, d)).astype(np.float16)
    k = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    v = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    return q, k, v


@pytest.mark.parametrize("nq,kv_len,hq,hkv,d", [(1, 1, 4, 4, 64), (1, 37, 8, 2, 64), (4, 21, 32, 8, 128),
                                                (16, 70, 14, 2, 64), (3, 3, 6, 3, 32)])
def test_oracle_matches_torch_sdpa(nq, kv_len, hq, hkv, d):
    """torch's scaled_dot_product_attention (float64, CPU) with the causal tail as
    an explicit mask and GQA by repeating kv heads."""
    rng = np.random.default_rng(nq * 1000 + kv_len)
    q, k, v = rand_case(rng, nq, kv_len, hq, hkv, d)
    got = AO.multihead_attention_f64(q, k, v, kv_len, nq)
    g = hq // hkv
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)[None]  # [1, hq, nq, d]
    kt = torch.from_numpy(k[:kv_len].astype(np.float64)).permute(1, 0, 2).repeat_interleave(g, 0)[None]
    vt = torch.from_numpy(v[:kv_len].astype(np.float64)).permute(1, 0, 2).repeat_interleave(g, 0)[None]
    pos = torch.arange(kv_len)[None, :]
    lim = kv_len - nq + 1 + torch.arange(nq)[:, None]
    want = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=pos < lim)
    np.testing.assert_allclose(got, want[0].permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_oracle_closed_forms():
    rng = np.random.default_rng(3)
    # One visible position: the output is that position's V row, for every head of its group.
    q, k, v = rand_case(rng, 1, 1, 8, 2, 64)
    out = AO.multihead_attention_f64(q, k, v, 1, 1)
    for h in range(8):
        np.testing.assert_allclose(out[0, h], v[0, h // 4].astype(np.float64), rtol=0, atol=1e-15)
    # Identical keys: uniform weights, the mean of the visible V rows (query i sees kv_len - nq + 1 + i).
    q, k, v = rand_case(rng, 3, 20, 4, 1, 32)
    k[:] = k[0]
    out = AO.multihead_attention_f64(q, k, v, 20, 3)
    for i in range(3):
        np.testing.assert_allclose(out[i, 2], v[:18 + i, 0].astype(np.float64).mean(axis=0), rtol=1e-12)
    # A query that sees nothing (kv_len = num_queries - 1) gets zeros; the next one sees position 0.
    q, k, v = rand_case(rng, 4, 3, 4, 4, 16)
    out = AO.multihead_attention_f64(q, k, v, 3, 4)
    assert not out[0].any()
    np.testing.assert_allclose(out[1, 3], v[0, 3].astype(np.float64), atol=1e-15)


def test_oracle_matches_c_decode_oracle():
    """The same cache read as a hot pool of 16-token blocks with an identity block
    table, causal, scale 1/sqrt(d), through the C oracle's fp64 decode."""
    rng = np.random.default_rng(4)
    nq, kv_len, hq, hkv, d = 3, 48, 8, 2, 64
    q, k, v = rand_case(rng, nq, kv_len, hq, hkv, d, cap=64)
    geom = SimpleNamespace(layers=1, batch=1, queries=nq, q_heads=hq, kv_heads=hkv, head_dim=d, dict_size=16,
                           dict_heads=1, hot_count=kv_len // 16, cold_count=0, refs_stride=kv_len // 16,
                           causal=True, scale=1.0 / np.sqrt(d), hot_blocks=4, cold_blocks=0)
    arrs = {"q": q.view(np.uint16), "hot_k": k.view(np.uint16), "hot_v": v.view(np.uint16),
            "refs": np.arange(kv_len // 16, dtype=np.uint32)}
    want = oracle.decode_f64(geom, arrs).reshape(nq, hq, d)
    np.testing.assert_allclose(AO.multihead_attention_f64(q, k, v, kv_len, nq), want, rtol=1e-9, atol=1e-12)


# --------------------------------------------------------- speculative verify

def one_hot_rows(argmaxes, vocab=12):
    rows = np.zeros((len(argmaxes), vocab), np.float32)
    for i, a in enumerate(argmaxes):
        rows[i, a] = 1.0
    return rows


@pytest.mark.parametrize("accept", [I.accept_drafts, AO.accept_drafts])
def test_accept_drafts_hand_worked(accept):
    """agent.rs:355-394 on hand-worked rows (row i: the target's logits after input i)."""
    drafts = [5, 7, 9]
    assert accept(drafts, one_hot_rows([5, 7, 9, 2])) == [5, 7, 9, 2]  # all kept + bonus
    assert accept(drafts, one_hot_rows([5, 3, 9, 2])) == [5, 3]        # second replaced, rest dropped
    assert accept(drafts, one_hot_rows([1, 7, 9, 2])) == [1]           # first replaced
    assert accept([], one_hot_rows([4])) == [4]                        # no drafts: one plain step
    tie = np.zeros((1, 6), np.float32)
    tie[0, [2, 4]] = 3.0
    assert accept([], tie) == [2]                                      # ties: the first index


def test_accept_drafts_allowed_tokens_and_rollback():
    rows = one_hot_rows([5, 7, 9, 2])
    rows[:, 8] = 0.5
    # Only {8, 9} allowed: row 0 samples 8 (5 is masked), so draft 5 is replaced by 8.
    assert I.accept_drafts([5, 7, 9], rows, allowed_tokens=[8, 9]) == [8]
    # The position after the verify forward (p0 + drafts + 1) rolls back to p0 + len(new).
    p0 = 100
    for new in ([5, 7, 9, 2], [5, 3], [1]):
        assert I.rollback_position(p0 + 4, 3, len(new)) == p0 + len(new)
        assert AO.rollback_position(p0 + 4, 3, len(new)) == p0 + len(new)
    rng = np.random.default_rng(5)
    for _ in range(50):
        # Drafts that match the target's argmax on a random prefix, random after it.
        n = int(rng.integers(0, 5))
        rows = rng.standard_normal((n + 1, 9)).astype(np.float32)
        keep = int(rng.integers(0, n + 1))
        drafts = [int(np.argmax(r)) for r in rows[:keep]] + [int(x) for x in rng.integers(0, 9, n - keep)]
        got = I.accept_drafts(drafts, rows)
        assert got == AO.accept_drafts(drafts, rows)
        assert len(got) >= keep + 1 and got[:keep] == drafts[:keep]


# ---------------------------------------------------------------- KV cache

def test_kv_cache_bookkeeping():
    c = I.KvCache(layers=2, kv_heads=2, head_dim=8, max_seq_len=40, device="cpu")
    assert c.capacity == 48 and c.position == 0
    k = torch.arange(3 * 2 * 8, dtype=torch.float16).reshape(3, 2, 8)
    c.append(1, k, -k)
    assert torch.equal(c.k[1][:3], k) and torch.equal(c.v[1][:3], -k) and not c.k[0].any()
    c.advance(3)
    saved = c.push_loom()
    assert saved == 3
    c.append(0, k, k)
    assert torch.equal(c.k[0][3:6], k)
    c.advance(3)
    c.pop_loom(saved)
    assert c.position == 3
    with pytest.raises(I.KvCacheError, match="Batch size 0"):
        c.advance(0)
    with pytest.raises(I.KvCacheError, match="Batch size 17"):
        c.check_batch(17)
    c.pop_loom(30)
    with pytest.raises(I.KvCacheError, match="KV cache exhausted"):
        c.check_batch(11)
    c.check_batch(10)
    with pytest.raises(I.KvCacheError):
        c.append(0, k[:, :1], k[:, :1])
    with pytest.raises(I.KvCacheError):
        c.pop_loom(41)
    c.reset()
    assert c.position == 0
