"""CPU restatement of the reference's contiguous-cache attention and of the
speculative-verify acceptance rule.

TEST INFRASTRUCTURE ONLY: imported by tests/ to check the product's
aw_multihead_attention_device (include/aether_weaver.h) and
aether_nexus_amd.inference, never by the product package.  numpy in float64.

Pins (tests/test_oracle.py):
  * multihead_attention_f64: torch's CPU scaled_dot_product_attention in
    float64 with an explicit causal-tail mask (a library routine, not this
    code); the closed forms of one visible position (out = that V row) and of
    identical keys (out = mean of the visible V rows); the C decode oracle
    (weaver_oracle.c) on the same cache read as a hot pool of 16-token blocks.
  * accept_drafts: hand-worked cases of agent.rs:355-398 (all drafts kept plus
    a bonus token, first mismatch replaced and the rest dropped, the position
    the cache rolls back to).
"""
from __future__ import annotations

import numpy as np


def multihead_attention_f64(q, k_cache, v_cache, kv_len: int, num_queries: int) -> np.ndarray:
    """multihead_attention (ops.metal:528-616) in float64.

    q [num_queries][q_heads][head_dim], caches [tokens][kv_heads][head_dim]
    (float16 or float arrays).  Query i sees cache positions
    p < kv_len - num_queries + 1 + i (ops.metal:549); kv head g = h / (q_heads /
    kv_heads) (:551-552); scores x 1/sqrt(head_dim) (:557); softmax with the max
    subtracted (:575-601); out = sum_p w_p V_p (:604-614).  A query that sees no
    position gets zeros (the reference's loops then run zero times)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k_cache, dtype=np.float64)
    v = np.asarray(v_cache, dtype=np.float64)
    nq, hq, d = q.shape
    hkv = k.shape[1]
    g_size = hq // hkv
    out = np.zeros((nq, hq, d), dtype=np.float64)
    scale = 1.0 / np.sqrt(d)
    for i in range(nq):
        valid = kv_len - num_queries + 1 + i
        if valid <= 0:
            continue
        for g in range(hkv):
            kg = k[:valid, g, :]
            vg = v[:valid, g, :]
            qs = q[i, g * g_size:(g + 1) * g_size, :]
            s = (qs @ kg.T) * scale
            s -= s.max(axis=1, keepdims=True)
            w = np.exp(s)
            w /= w.sum(axis=1, keepdims=True)
            out[i, g * g_size:(g + 1) * g_size, :] = w @ vg
    return out


def argmax_first(logits) -> int:
    """Greedy sample_token (inference.rs:677-693 with temperature < 0.01 and no
    recent tokens): the first index of the largest logit (strict >)."""
    best, best_i = -np.inf, 0
    for i, x in enumerate(np.asarray(logits, dtype=np.float32)):
        if x > best:
            best, best_i = x, i
    return best_i


def accept_drafts(draft_tokens, logits, sample=argmax_first):
    """agent.rs:355-394: row i of `logits` follows input i of
    [last_token] + drafts.  Drafts are kept while each equals the target's
    sample at its row; the first mismatch contributes the target's token and
    ends the step; when every draft is kept, the row after the last draft adds
    a bonus token."""
    new = []
    for i, d in enumerate(draft_tokens):
        t = sample(logits[i])
        if t == d:
            new.append(int(d))
        else:
            new.append(int(t))
            return new
    new.append(int(sample(logits[len(draft_tokens)])))
    return new


def rollback_position(position: int, n_drafts: int, n_new: int) -> int:
    """agent.rs:396-398: correct_pos = push_loom() - (drafts + 1) + new_tokens.len()."""
    return position - (n_drafts + 1) + n_new
