"""The Weaver as the decode attention of the reference's inference loop.

``KvCache`` holds the per-layer K and V caches of ``InferenceEngine``
(nexus-core/src/inference.rs:161-166, MAX_SEQ_LEN tokens each, :219,255-266) on
the device and the position bookkeeping of ``forward_batch`` (:456-483, :631)
and ``push_loom`` / ``pop_loom`` (:437-446):

* ``append(layer, k, v)`` writes the new tokens' rows at the current position
  (the ``copy_buffer`` calls of :547-550);
* ``attend(engine, layer, q, out)`` is ``Ops::multihead_attention`` over the
  cache (:552-562), run by ``aw_multihead_attention_device``: causal GQA
  attention of the new tokens, the last of ``position + num_tokens`` cache
  positions;
* ``advance(num_tokens)`` moves the position once every layer has been written
  (:631); ``push_loom`` returns it and ``pop_loom`` restores a saved one, which
  is how the agent discards rejected drafts (agent.rs:396-399).

``accept_drafts`` and ``rollback_position`` are the speculative-verify rule of
the agent loop (agent.rs:337-399): the target model runs [last_token] + drafts
as one multi-query step (``attend`` with num_tokens = drafts + 1), and the
drafts are kept while they match the target's samples.
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence

import numpy as np
import torch

MAX_SEQ_LEN = 4096  # InferenceEngine::MAX_SEQ_LEN (inference.rs:219)
MAX_BATCH = 16  # InferenceEngine::MAX_BATCH (inference.rs:221): tokens per forward_batch
BLOCK_TOKENS = 16  # the cache is read in 16-token blocks


class KvCacheError(RuntimeError):
    """A request forward_batch rejects (inference.rs:462-475)."""


class KvCache:
    """Per-layer K and V caches [tokens][kv_heads][head_dim] (f16) on one device.

    The capacity is ``max_seq_len`` rounded up to whole 16-token blocks, which the
    attention reads; positions past the sequence are never used."""

    def __init__(self, layers: int, kv_heads: int, head_dim: int, max_seq_len: int = MAX_SEQ_LEN,
                 max_batch: int = MAX_BATCH, device="cuda:0"):
        if layers < 1 or kv_heads < 1 or head_dim < 1 or max_seq_len < 1 or max_batch < 1:
            raise KvCacheError("layers, kv_heads, head_dim, max_seq_len and max_batch must be >= 1")
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim
        self.max_seq_len, self.max_batch = max_seq_len, max_batch
        self.capacity = -(-max_seq_len // BLOCK_TOKENS) * BLOCK_TOKENS
        shape = (self.capacity, kv_heads, head_dim)
        self.k = [torch.zeros(shape, dtype=torch.float16, device=device) for _ in range(layers)]
        self.v = [torch.zeros(shape, dtype=torch.float16, device=device) for _ in range(layers)]
        self.position = 0

    def check_batch(self, num_tokens: int) -> None:
        """forward_batch's guards (inference.rs:462-475)."""
        if num_tokens == 0 or num_tokens > self.max_batch:
            raise KvCacheError(f"Batch size {num_tokens} unsupported (max {self.max_batch})")
        if self.position + num_tokens > self.max_seq_len:
            raise KvCacheError(f"KV cache exhausted: position {self.position} + {num_tokens} >= MAX_SEQ_LEN "
                               f"{self.max_seq_len}.")

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write the new tokens' K and V rows [num_tokens][kv_heads][head_dim] at
        the current position of `layer` (inference.rs:547-550)."""
        n = k.shape[0]
        self.check_batch(n)
        if tuple(k.shape) != (n, self.kv_heads, self.head_dim) or tuple(v.shape) != tuple(k.shape):
            raise KvCacheError(f"k and v must be [{n}][{self.kv_heads}][{self.head_dim}]")
        self.k[layer][self.position:self.position + n].copy_(k)
        self.v[layer][self.position:self.position + n].copy_(v)

    def attend(self, engine, layer: int, q: torch.Tensor, out: torch.Tensor, stream: Optional[int] = None) -> None:
        """Ops::multihead_attention over layer `layer` (inference.rs:552-562): q and
        out [num_tokens][q_heads][head_dim]; the new tokens are cache positions
        position .. position + num_tokens - 1 (append them first)."""
        n, q_heads, head_dim = q.shape
        self.check_batch(n)
        if head_dim != self.head_dim or q_heads % self.kv_heads:
            raise KvCacheError("q must be [num_tokens][q_heads][head_dim] with q_heads a multiple of kv_heads")
        engine.multihead_attention(q, self.k[layer], self.v[layer], out, self.position + n, head_dim, q_heads,
                                   self.kv_heads, n, cache_tokens=self.capacity, stream=stream)

    def advance(self, num_tokens: int) -> None:
        """The position after a forward pass of num_tokens tokens (inference.rs:631)."""
        self.check_batch(num_tokens)
        self.position += num_tokens

    def reset(self) -> None:
        """inference.rs:637-639: the next token starts a new sequence."""
        self.position = 0

    def push_loom(self) -> int:
        """inference.rs:437-439."""
        return self.position

    def pop_loom(self, saved_position: int) -> None:
        """inference.rs:443-446: tokens after saved_position are overwritten later."""
        if not 0 <= saved_position <= self.max_seq_len:
            raise KvCacheError(f"position {saved_position} outside the cache")
        self.position = saved_position


def greedy_sample(logits) -> int:
    """sample_token at temperature < 0.01 without recent tokens (inference.rs:677-693):
    the first index of the largest logit."""
    return int(np.argmax(np.asarray(logits, dtype=np.float32)))


def accept_drafts(draft_tokens: Sequence[int], logits, sample: Callable = greedy_sample,
                  allowed_tokens: Optional[Sequence[int]] = None) -> list:
    """The verify rule of agent.rs:355-394.  ``logits`` [len(drafts) + 1][vocab]:
    row i is the target's output after input i of [last_token] + drafts.  Drafts
    are kept while each equals the target's sample at its row; the first
    mismatch contributes the target's token instead and ends the step; when
    every draft is kept, the last row adds a bonus token.  ``allowed_tokens``
    masks every other token to -inf before sampling (agent.rs:362-368)."""
    rows = np.asarray(logits, dtype=np.float32)
    if rows.ndim != 2 or rows.shape[0] < len(draft_tokens) + 1:
        raise ValueError("logits must hold one row per draft plus one")
    if allowed_tokens is not None:
        mask = np.full(rows.shape[1], -np.inf, dtype=np.float32)
        mask[np.asarray(allowed_tokens, dtype=np.int64)] = 0.0
        rows = rows + mask
    new = []
    for i, d in enumerate(draft_tokens):
        t = int(sample(rows[i]))
        new.append(t)
        if t != d:
            return new
    new.append(int(sample(rows[len(draft_tokens)])))
    return new


def rollback_position(position: int, n_drafts: int, n_new: int) -> int:
    """The position both engines return to after a verify step (agent.rs:396-399):
    the cache keeps last_token and the accepted drafts; the newest token is the
    next step's input."""
    return position - (n_drafts + 1) + n_new
