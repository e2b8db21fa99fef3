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

``WeaverKvCache`` is the same cache with the Weaver's two tiers
(weaver_kernel.metal:118-240): the newest ``hot_window`` tokens stay exact f16 K
and V rows in 16-token blocks, and whole blocks older than that are distilled
into SparseCodes of a per-layer dictionary (``Distiller::distill_block``,
distiller.rs:171-246, run by ``aw_encode_device``), so that ``attend`` is one
hot+cold ``aw_decode_device`` per layer with q_latent = q . D^T computed on the
device.  A SparseCode is the Weaver's one row per token and kv head, used as
both key and value (the reference's pools hold one KV tensor,
weaver_kernel.metal:162-166,206-219): the cold tier encodes the K rows, and a
cold token's value is that same reconstruction.
"""
from __future__ import annotations

import contextlib
import math
from typing import Callable, Optional, Sequence

import numpy as np
import torch

from .weaver import make_desc, make_encode_desc

MAX_SEQ_LEN = 4096  # InferenceEngine::MAX_SEQ_LEN (inference.rs:219)
MAX_BATCH = 16  # InferenceEngine::MAX_BATCH (inference.rs:221): tokens per forward_batch
BLOCK_TOKENS = 16  # the cache is read in 16-token blocks


def _torch_stream(handle: Optional[int]):
    """torch's Stream object for a hipStream_t handle: torch's current stream for
    None or its handle, the null stream for 0 (torch.cuda.ExternalStream(0) makes
    a stream of its own instead), else an external stream wrapping the handle."""
    cur = torch.cuda.current_stream()
    if handle is None or handle == cur.cuda_stream:
        return cur
    if handle == 0:
        return torch.cuda.default_stream()
    return torch.cuda.ExternalStream(handle)


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


class WeaverKvCache:
    """One sequence's per-layer KV cache in the Weaver's two tiers, on one device.

    Tokens [0, cold_tokens) are cold: whole 16-token blocks of SparseCodes
    ``[cold_capacity][kv_heads][16]`` (head-blocked device order) per layer.
    Tokens [cold_tokens, position) are hot: exact f16 K and V rows in a ring of
    16-token blocks ``[hot_capacity][16][kv_heads][head_dim]`` per layer.  One
    block table serves every layer: hot refs (oldest block first) then cold refs.

    ``distill(engine)`` moves the oldest whole hot blocks beyond ``hot_window``
    tokens into the cold tier (the Distiller pass, distiller.rs:60-120, with the
    blocks chosen by age instead of the entropy proxy).  ``pop_loom`` may roll
    back into the hot tier only: distilled tokens are final.

    ``dictionaries``: f16 ``[layers][dict_heads][dict_size][head_dim]`` on the
    device, dict_heads 1 (shared) or kv_heads (the reference's per-kv-head
    dictionary, fabric.rs:159-166).

    ``q_latent_f32`` (default): q . D^T stays fp32 on the device instead of being
    rounded to f16 like the reference's q_latent buffer (weaver_kernel.metal:111).
    f16 rounding moves a cold score by up to 2^-11 of sum_k |c_k q_latent[idx_k]|,
    which a peaked softmax amplifies past the output tolerance.

    Streams: every method takes the HIP stream its device work goes on (None:
    torch's current stream).  The cache orders each call after its previous work
    on any other stream, so the ring writes, the block table and the encodes of a
    distill never overtake one another whatever streams the caller mixes.

    Background distill (the REM pass beside the decode, distiller.rs:60-88, whose
    blocks are distilled one lock at a time so that inference interleaves):
    ``distill(engine, side_stream=s)`` encodes the blocks on stream ``s`` into
    cold blocks no decode reads yet, and leaves them in the hot tier meanwhile;
    decodes keep running on the caller's stream.  ``commit()`` switches the tiers
    once the encodes are done (the caller's stream then waits for them on the
    device, the host never blocks); ``attend``, ``append``, ``advance`` and the
    next ``distill`` commit on their own when the encodes have finished (or, for
    ``append`` and ``distill``, when they need the room)."""

    def __init__(self, layers: int, kv_heads: int, head_dim: int, dictionaries: torch.Tensor,
                 hot_window: int = 2048, max_seq_len: int = 65536, max_batch: int = MAX_BATCH, device="cuda:0",
                 q_latent_f32: bool = True):
        if layers < 1 or kv_heads < 1 or head_dim < 1 or max_batch < 1 or hot_window < BLOCK_TOKENS:
            raise KvCacheError("layers, kv_heads, head_dim, max_batch >= 1 and hot_window >= 16 required")
        if dictionaries.dim() != 4 or dictionaries.shape[0] != layers or dictionaries.shape[3] != head_dim or \
                dictionaries.shape[1] not in (1, kv_heads) or dictionaries.dtype != torch.float16:
            raise KvCacheError("dictionaries must be f16 [layers][1 or kv_heads][dict_size][head_dim]")
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim
        self.dict_heads, self.dict_size = int(dictionaries.shape[1]), int(dictionaries.shape[2])
        self.dictionaries = dictionaries.contiguous()
        self.hot_window, self.max_seq_len, self.max_batch = hot_window, max_seq_len, max_batch
        self.device = device
        # After distill the hot tier holds at most hot_window + 15 tokens (whole
        # blocks leave); a forward batch comes on top.
        self.hot_capacity = -(-(hot_window + BLOCK_TOKENS - 1 + max_batch) // BLOCK_TOKENS)
        self.cold_capacity = max(1, -(-max_seq_len // BLOCK_TOKENS))
        hshape = (self.hot_capacity, BLOCK_TOKENS, kv_heads, head_dim)
        self.k = [torch.zeros(hshape, dtype=torch.float16, device=device) for _ in range(layers)]
        self.v = [torch.zeros(hshape, dtype=torch.float16, device=device) for _ in range(layers)]
        cshape = (self.cold_capacity, kv_heads, BLOCK_TOKENS, 8)  # 8 int16 words = one 16-byte code
        self.cold = [torch.zeros(cshape, dtype=torch.int16, device=device) for _ in range(layers)]
        self.position = 0
        self.cold_blocks = 0   # cold tokens = 16 * cold_blocks
        self.hot_first = 0     # ring slot of the oldest hot block
        self._refs = torch.zeros(self.hot_capacity + self.cold_capacity, dtype=torch.int32, device=device)
        self._refs_key = None
        self.q_latent_f32 = q_latent_f32
        self._cuda = torch.device(device).type == "cuda"
        self._last = None      # stream of the cache's latest device work
        self._pending = None   # background distill: (blocks, done event, index tensors)

    # -- streams
    def _enter(self, stream: Optional[int]):
        """The stream for this call's device work (the caller's handle, or torch's
        current stream), ordered after the cache's latest work on another stream.
        None for a cache in host memory (the host-logic tests)."""
        if not self._cuda:
            return None
        s = _torch_stream(stream)
        if self._last is not None and self._last.cuda_stream != s.cuda_stream:
            with torch.cuda.stream(s):
                capturing = torch.cuda.is_current_stream_capturing()
            # A captured graph cannot wait on work outside it: the caller orders a
            # capture after the cache's eager work (a synchronize before capturing).
            if not capturing:
                s.wait_stream(self._last)
        self._last = s
        return s

    @staticmethod
    def _on(s):
        """Torch work inside runs on stream `s` (none: as it is)."""
        return torch.cuda.stream(s) if s is not None else contextlib.nullcontext()

    @staticmethod
    def _handle(s, stream: Optional[int]) -> Optional[int]:
        return s.cuda_stream if s is not None else stream

    def _capturing(self) -> bool:
        return self._cuda and torch.cuda.is_current_stream_capturing()

    # -- bookkeeping
    @property
    def cold_tokens(self) -> int:
        return self.cold_blocks * BLOCK_TOKENS

    def hot_tokens(self, end: Optional[int] = None) -> int:
        return (self.position if end is None else end) - self.cold_tokens

    def check_batch(self, num_tokens: int) -> None:
        """forward_batch's guards (inference.rs:462-475)."""
        if num_tokens == 0 or num_tokens > self.max_batch:
            raise KvCacheError(f"Batch size {num_tokens} unsupported (max {self.max_batch})")
        if self.position + num_tokens > self.max_seq_len:
            raise KvCacheError(f"KV cache exhausted: position {self.position} + {num_tokens} >= MAX_SEQ_LEN "
                               f"{self.max_seq_len}.")
        if self.hot_tokens() + num_tokens > self.hot_capacity * BLOCK_TOKENS:
            raise KvCacheError("hot tier full: distill before appending more tokens")

    def _slot(self, hot_token: int) -> tuple[int, int]:
        return (self.hot_first + hot_token // BLOCK_TOKENS) % self.hot_capacity, hot_token % BLOCK_TOKENS

    def _write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        t, n = self.hot_tokens(), k.shape[0]
        i = 0
        while i < n:  # block by block (the ring may wrap)
            slot, off = self._slot(t + i)
            m = min(BLOCK_TOKENS - off, n - i)
            self.k[layer][slot, off:off + m].copy_(k[i:i + m])
            self.v[layer][slot, off:off + m].copy_(v[i:i + m])
            i += m

    def refs(self, hot_blocks: int) -> torch.Tensor:
        """The block table: hot ring slots oldest first, then cold blocks 0 ..
        (rebuilt only when the tiers change), written on torch's current stream
        (``attend`` makes that the decode's stream)."""
        key = (self.hot_first, hot_blocks, self.cold_blocks)
        if key != self._refs_key:
            hot = (self.hot_first + np.arange(hot_blocks)) % self.hot_capacity
            table = np.concatenate([hot, np.arange(self.cold_blocks)]).astype(np.int32)
            self._refs[:table.size].copy_(torch.from_numpy(table))
            self._refs_key = key
        return self._refs

    # -- the decode loop's calls
    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, stream: Optional[int] = None) -> None:
        """Write the new tokens' K and V rows [num_tokens][kv_heads][head_dim] at the
        current position of `layer` (inference.rs:547-550), into the hot tier."""
        n = k.shape[0]
        s = self._enter(stream)
        self.commit(wait=self._pending is not None and
                    self.hot_tokens() + n > self.hot_capacity * BLOCK_TOKENS)
        self.check_batch(n)
        if tuple(k.shape) != (n, self.kv_heads, self.head_dim) or tuple(v.shape) != tuple(k.shape):
            raise KvCacheError(f"k and v must be [{n}][{self.kv_heads}][{self.head_dim}]")
        with self._on(s):
            self._write(layer, k, v)

    def attend(self, engine, layer: int, q: torch.Tensor, out: torch.Tensor, stream: Optional[int] = None) -> None:
        """Causal GQA attention of the new tokens (cache positions position ..
        position + num_tokens - 1, appended first) over both tiers of `layer`:
        one aw_decode_device with scale 1/sqrt(head_dim) (ops.metal:557) and
        q_latent computed on the device; query i sees every cold token and hot
        tokens up to its own position (ops.metal:549)."""
        n, q_heads, head_dim = q.shape
        s = self._enter(stream)
        if not self._capturing():
            self.commit()
        self.check_batch(n)
        if head_dim != self.head_dim or q_heads % self.kv_heads or tuple(out.shape) != tuple(q.shape):
            raise KvCacheError("q and out must be [num_tokens][q_heads][head_dim], q_heads a multiple of kv_heads")
        hot_tok = self.hot_tokens(self.position + n)
        hot_blocks = -(-hot_tok // BLOCK_TOKENS)
        with self._on(s):
            refs = self.refs(hot_blocks)
        desc = make_desc(layers=1, batch=1, queries=n, q_heads=q_heads, kv_heads=self.kv_heads, head_dim=head_dim,
                         dict_size=self.dict_size, dict_heads=self.dict_heads, hot_count=hot_blocks,
                         cold_count=self.cold_blocks, refs_stride=max(hot_blocks + self.cold_blocks, 1),
                         hot_blocks=self.hot_capacity, cold_blocks=self.cold_capacity, q=q, out=out,
                         hot_k=self.k[layer], hot_v=self.v[layer], cold=self.cold[layer] if self.cold_blocks else None,
                         refs=refs, dictionary=self.dictionaries[layer] if self.cold_blocks else None,
                         scale=1.0 / math.sqrt(head_dim), causal=True, cold_head_blocked=True,
                         hot_tokens=hot_tok, q_latent_f32=self.q_latent_f32)
        engine.decode_device(desc, stream=self._handle(s, stream))

    def advance(self, num_tokens: int) -> None:
        """The position after a forward pass of num_tokens tokens (inference.rs:631)."""
        self.check_batch(num_tokens)
        self.position += num_tokens
        if not self._capturing():
            self.commit()

    def distill(self, engine, stream: Optional[int] = None, side_stream: Optional[int] = None) -> int:
        """Encode the oldest whole hot blocks beyond the hot window into the cold
        tier of every layer (aw_encode_device: top-4 atoms of the layer's
        dictionary by dot product, coefficient f16(dot), distiller.rs:171-246),
        and drop them from the hot ring.  Returns the number of blocks moved.

        With ``side_stream`` the encodes run there, after the work queued so far
        on ``stream``, and the blocks stay hot until ``commit``: decodes issued
        meanwhile read them in the hot tier and never read the cold blocks being
        written."""
        if side_stream is not None and not self._cuda:
            raise KvCacheError("a background distill needs a cache on the GPU")
        s = self._enter(stream)
        self.commit(wait=True)  # one pass in flight at a time
        over = self.hot_tokens() - self.hot_window
        n = over // BLOCK_TOKENS if over > 0 else 0
        if n == 0:
            return 0
        if self.cold_blocks + n > self.cold_capacity:
            raise KvCacheError("cold tier full")
        # The block lists are made on the device (no host copy, which would wait for
        # a busy side stream), on the caller's stream.
        with self._on(s):
            src = torch.remainder(torch.arange(n, dtype=torch.int32, device=self.device) + self.hot_first,
                                  self.hot_capacity).to(torch.int32)
            dst = torch.arange(self.cold_blocks, self.cold_blocks + n, dtype=torch.int32, device=self.device)
        enc = s if side_stream is None else _torch_stream(side_stream)
        if side_stream is not None:
            enc.wait_stream(s)  # the encodes read the hot rows written so far, and the block lists
        for layer in range(self.layers):
            desc = make_encode_desc(kv_heads=self.kv_heads, head_dim=self.head_dim, dict_size=self.dict_size,
                                    dict_heads=self.dict_heads, hot_blocks=self.hot_capacity,
                                    cold_blocks=self.cold_capacity, hot=self.k[layer],
                                    dictionary=self.dictionaries[layer], src_blocks=src, dst_blocks=dst,
                                    cold=self.cold[layer], cold_head_blocked=True)
            engine.encode_device(desc, stream=self._handle(enc, stream))
        if side_stream is None:
            self.cold_blocks += n
            self.hot_first = (self.hot_first + n) % self.hot_capacity
            return n
        done = torch.cuda.Event()
        done.record(enc)
        self._pending = (n, done, src, dst)
        return n

    @property
    def distilling(self) -> int:
        """Blocks of a background distill not committed yet."""
        return self._pending[0] if self._pending else 0

    def commit(self, wait: bool = False) -> bool:
        """Switch the tiers of a finished background distill: its blocks leave the
        hot ring and become cold blocks.  Without ``wait`` only when its encodes
        have completed; with ``wait`` at once, the cache's stream then waiting for
        them on the device.  Returns whether the tiers changed."""
        if self._pending is None:
            return False
        n, done, _, _ = self._pending
        if not wait and not done.query():
            return False
        if self._last is not None:
            self._last.wait_event(done)  # later ring writes and decodes follow the encodes
        self._pending = None
        self.cold_blocks += n
        self.hot_first = (self.hot_first + n) % self.hot_capacity
        return True

    def extend(self, engine, ks, vs, stream: Optional[int] = None) -> None:
        """Load a prompt of many tokens (per-layer [n][kv_heads][head_dim] rows) at
        the current position, distilling as the hot tier fills.  Into an empty hot
        tier, the whole blocks that would leave the window at once are encoded
        straight from the prompt rows (read as a [n/16][16][kv_heads][head_dim]
        pool), without passing through the hot ring."""
        n = ks[0].shape[0]
        i = 0
        s = self._enter(stream)
        self.commit(wait=True)
        if self.hot_tokens() == 0 and n > self.hot_window:
            nb = (n - self.hot_window) // BLOCK_TOKENS
            if self.cold_blocks + nb > self.cold_capacity or self.position + n > self.max_seq_len:
                raise KvCacheError("prompt longer than the cache")
            src = torch.arange(nb, dtype=torch.int32, device=self.device)
            dst = torch.arange(self.cold_blocks, self.cold_blocks + nb, dtype=torch.int32, device=self.device)
            for layer in range(self.layers):
                rows = ks[layer][:nb * BLOCK_TOKENS]
                if not rows.is_contiguous():  # read in place by the asynchronous encoder
                    raise KvCacheError("prompt rows must be contiguous [n][kv_heads][head_dim]")
                desc = make_encode_desc(kv_heads=self.kv_heads, head_dim=self.head_dim, dict_size=self.dict_size,
                                        dict_heads=self.dict_heads, hot_blocks=nb, cold_blocks=self.cold_capacity,
                                        hot=rows, dictionary=self.dictionaries[layer], src_blocks=src,
                                        dst_blocks=dst, cold=self.cold[layer], cold_head_blocked=True)
                engine.encode_device(desc, stream=self._handle(s, stream))
            self.cold_blocks += nb
            self.position += nb * BLOCK_TOKENS
            i = nb * BLOCK_TOKENS
        while i < n:
            if self.position + 1 > self.max_seq_len:
                raise KvCacheError("prompt longer than the cache")
            room = self.hot_capacity * BLOCK_TOKENS - self.hot_tokens()
            m = min(room, n - i)
            if m <= 0:
                raise KvCacheError("hot window too small to make room")
            with self._on(s):
                for layer in range(self.layers):
                    self._write(layer, ks[layer][i:i + m], vs[layer][i:i + m])
            self.position += m
            i += m
            self.distill(engine, self._handle(s, stream))

    def reset(self) -> None:
        """inference.rs:637-639: the next token starts a new sequence."""
        self.commit(wait=True)  # later writes follow a background distill's encodes
        self.position = self.cold_blocks = self.hot_first = 0
        self._refs_key = None

    def push_loom(self) -> int:
        """inference.rs:437-439."""
        return self.position

    def pop_loom(self, saved_position: int) -> None:
        """inference.rs:443-446, within the hot tier (distilled tokens, and those of
        a background distill in flight, are final)."""
        lo = self.cold_tokens + self.distilling * BLOCK_TOKENS
        if not lo <= saved_position <= self.position:
            raise KvCacheError(f"position {saved_position} outside the hot tier [{lo}, {self.position}]")
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
