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


class _RecordingEngine:
    """Stands in for WeaverEngine on the CPU: records the requests it is handed."""

    def __init__(self):
        self.encodes, self.decodes = [], []

    def encode_device(self, desc, stream=None):
        self.encodes.append((desc.n_blocks, desc.hot_blocks, desc.flags))

    def decode_device(self, desc, stream=None):
        self.decodes.append({f: getattr(desc, f) for f in ("queries", "hot_count", "cold_count", "refs_stride",
                                                            "hot_tokens", "flags", "hot_blocks", "cold_blocks")})


def test_weaver_kv_cache_tiers():
    """WeaverKvCache's host logic: the prompt's old blocks go straight to the
    cold tier, the hot ring keeps the window, distill moves whole blocks by age,
    the block table lists hot ring slots oldest first then cold blocks, and
    rollback stays inside the hot tier."""
    from aether_nexus_amd.types import AW_F_CAUSAL, AW_F_COLD_HEAD_BLOCKED, AW_F_QLATENT_F32
    layers, hkv, d, win = 2, 2, 8, 32
    dicts = torch.zeros((layers, 1, 64, d), dtype=torch.float16)
    c = I.WeaverKvCache(layers, hkv, d, dicts, hot_window=win, max_seq_len=400, max_batch=4, device="cpu")
    assert c.hot_capacity == -(-(win + 15 + 4) // 16) and c.cold_capacity == 25
    eng = _RecordingEngine()
    n = 100
    ks = [torch.arange(n * hkv * d, dtype=torch.float32).reshape(n, hkv, d).to(torch.float16) + l for l in range(2)]
    vs = [-x for x in ks]
    c.extend(eng, ks, vs)
    # (100 - 32) // 16 = 4 blocks encoded from the prompt rows; 36 tokens stay hot.
    assert (c.position, c.cold_blocks, c.hot_tokens()) == (100, 4, 36)
    assert eng.encodes == [(4, 4, AW_F_COLD_HEAD_BLOCKED)] * layers
    assert torch.equal(c.k[1][0], ks[1][64:80]) and torch.equal(c.v[0][2, :4], vs[0][96:100])
    # A verify step of 4 tokens: queries see both tiers, the new tokens last in the hot tier.
    q = torch.zeros((4, 4, d), dtype=torch.float16)
    for layer in range(layers):
        c.append(layer, ks[layer][:4], vs[layer][:4])
        c.attend(eng, layer, q, torch.empty_like(q))
    got = eng.decodes[-1]
    # q_latent stays fp32 by default (AW_F_QLATENT_F32).
    assert got == {"queries": 4, "hot_count": 3, "cold_count": 4, "refs_stride": 7, "hot_tokens": 40,
                   "flags": AW_F_CAUSAL | AW_F_COLD_HEAD_BLOCKED | AW_F_QLATENT_F32, "hot_blocks": c.hot_capacity,
                   "cold_blocks": c.cold_capacity}
    assert c.refs(3)[:7].tolist() == [0, 1, 2, 0, 1, 2, 3]
    saved = c.push_loom()
    c.advance(4)
    c.pop_loom(saved + 1)  # one draft kept
    assert c.position == 101
    # Distill by age: 101 - 64 = 37 hot tokens, nothing leaves (a block leaves at 48);
    # 12 more make 49 -> the oldest hot block leaves.
    assert c.distill(eng) == 0
    for _ in range(3):
        for layer in range(layers):
            c.append(layer, ks[layer][:4], vs[layer][:4])
        c.advance(4)
    assert c.distill(eng) == 1 and (c.cold_blocks, c.hot_first, c.hot_tokens()) == (5, 1, 33)
    assert eng.encodes[-1] == (1, c.hot_capacity, AW_F_COLD_HEAD_BLOCKED)
    assert c.refs(2)[:7].tolist() == [1, 2, 0, 1, 2, 3, 4]
    with pytest.raises(I.KvCacheError, match="hot tier"):
        c.pop_loom(79)  # inside the cold tier now
    with pytest.raises(I.KvCacheError, match="Batch size 5"):
        c.check_batch(5)
    with pytest.raises(I.KvCacheError):
        I.WeaverKvCache(layers, hkv, d, dicts[:1], hot_window=win, device="cpu")
    c.reset()
    assert (c.position, c.cold_blocks, c.hot_first) == (0, 0, 0)
    # The reference's f16 q_latent on request; a background distill needs the GPU.
    c16 = I.WeaverKvCache(layers, hkv, d, dicts, hot_window=win, max_seq_len=400, max_batch=4, device="cpu",
                          q_latent_f32=False)
    c16.extend(eng, ks, vs)
    c16.append(0, ks[0][:1], vs[0][:1])
    c16.attend(eng, 0, q[:1], torch.empty_like(q[:1]))
    assert eng.decodes[-1]["flags"] == AW_F_CAUSAL | AW_F_COLD_HEAD_BLOCKED
    assert c16.distilling == 0 and not c16.commit()
    with pytest.raises(I.KvCacheError, match="GPU"):
        c16.distill(eng, side_stream=1)
