"""Host-side mirror of the reference ``WeaverEngine`` (nexus-core/src/weaver.rs).

``WeaverEngine(lib_path)`` replaces ``WeaverEngine::new(metallib_path)``
(weaver.rs:85-132): the path names the gfx950 library instead of a metallib.
``decode(...)`` keeps the argument order and meaning of ``WeaverEngine::decode``
(weaver.rs:139-148) and returns ``DecodeOutput(data)`` with ``q_heads*head_dim``
f16 values; failures raise ``WeaverError`` (the reference's ``Err(String)``).
``device_name()`` / ``max_threads_per_threadgroup()`` mirror weaver.rs:314-321.

``decode_device(...)`` is the batched, device-resident extension: torch device
tensors (or raw device pointers) in, asynchronous on a HIP stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Optional

import numpy as np

from . import _lib
from .types import (AW_F_CAUSAL, AW_F_COLD_HEAD_BLOCKED, AW_F_ENCODE_FULL_SCAN, AW_F_SEQ_HOT_TOKENS, AW_F_QLATENT_F32,
                    SPARSE_CODE_DTYPE, STAGES, STRUCT_SIZES, DecodeDesc, EncodeDesc, PlanInfo, WeaverParams)


class WeaverError(RuntimeError):
    """A failed engine call; carries the status code and the engine's message."""

    def __init__(self, message: str, status: int = 0):
        super().__init__(message)
        self.status = status


@dataclass
class DecodeOutput:
    """``DecodeOutput`` (weaver.rs:59-62): ``q_heads * head_dim`` f16 values."""

    data: np.ndarray


def _status_text(lib, status: int) -> str:
    return lib.aw_status_string(status).decode()


def plan(desc: DecodeDesc, lib_path=None) -> PlanInfo:
    """Validate a request's geometry and return how it is split (no GPU needed)."""
    lib = _lib.load(lib_path)
    info = PlanInfo()
    msg = ctypes.create_string_buffer(256)
    rc = lib.aw_decode_plan(ctypes.byref(desc), ctypes.byref(info), msg, 256)
    if rc:
        raise WeaverError(f"{_status_text(lib, rc)}: {msg.value.decode()}", rc)
    return info


def validate_params(params: WeaverParams, n_q_exact: int, n_q_latent: int, n_hot_pool: int,
                    cold_pool: Optional[np.ndarray], loom_refs: Optional[np.ndarray], n_dictionary: int,
                    n_out: int, lib_path=None) -> None:
    """Host validation of a reference-style call (no GPU needed); raises WeaverError."""
    lib = _lib.load(lib_path)
    msg = ctypes.create_string_buffer(256)
    cold_ptr, n_cold = _codes_ptr(cold_pool)
    refs = None if loom_refs is None else np.ascontiguousarray(loom_refs, dtype=np.uint32)
    rc = lib.aw_validate_params(ctypes.byref(params), n_q_exact, n_q_latent, n_hot_pool, cold_ptr, n_cold,
                                None if refs is None else refs.ctypes.data, 0 if refs is None else refs.size,
                                n_dictionary, n_out, msg, 256)
    if rc:
        raise WeaverError(f"{_status_text(lib, rc)}: {msg.value.decode()}", rc)


def _f16_bits(a: Any) -> np.ndarray:
    """A contiguous uint16 view of f16 data (np.float16 or raw uint16 bits)."""
    arr = np.asarray(a)
    if arr.dtype == np.float16:
        return np.ascontiguousarray(arr).view(np.uint16).reshape(-1)
    if arr.dtype == np.uint16:
        return np.ascontiguousarray(arr).reshape(-1)
    raise TypeError(f"expected float16 or uint16 bits, got {arr.dtype}")


def _aligned16(words: np.ndarray) -> np.ndarray:
    if words.ctypes.data % 16 == 0:
        return words
    buf = np.empty(words.nbytes + 16, dtype=np.uint8)
    off = (-buf.ctypes.data) % 16
    out = buf[off:off + words.nbytes].view(words.dtype).reshape(words.shape)
    out[...] = words
    return out


def _codes_ptr(codes: Optional[np.ndarray]):
    """(pointer, number of codes) of a SparseCode array given as the structured
    dtype or as uint16 words [..., 8]; the pointer is 16-byte aligned."""
    if codes is None:
        return None, 0
    arr = np.asarray(codes)
    if arr.dtype == SPARSE_CODE_DTYPE:
        words = np.ascontiguousarray(arr).view(np.uint16).reshape(-1, 8)
    elif arr.dtype == np.uint16 and arr.shape[-1] == 8:
        words = np.ascontiguousarray(arr).reshape(-1, 8)
    else:
        raise TypeError("cold pool must be SPARSE_CODE_DTYPE or uint16 words [..., 8]")
    words = _aligned16(words)
    _codes_ptr.keepalive = words  # keep the aligned copy alive for the call
    return words.ctypes.data, words.shape[0]


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()  # torch tensor on the device


def _stream(stream: Optional[int]) -> Optional[int]:
    """The hipStream_t to run on: the given handle, else torch's current stream
    (so the work is ordered after the torch work that produced the inputs),
    else HIP's null stream."""
    if stream is not None:
        return stream
    import sys
    torch = sys.modules.get("torch")
    if torch is not None and torch.cuda.is_initialized():
        return torch.cuda.current_stream().cuda_stream or None
    return None


class WeaverEngine:
    """gfx950 Weaver decode engine (reference: weaver.rs:31-56)."""

    def __init__(self, lib_path=None, device: int = 0):
        self._lib = _lib.load(lib_path)
        sizes = (ctypes.c_size_t * 4)()
        self._lib.aw_abi_struct_sizes(sizes)
        if tuple(sizes) != STRUCT_SIZES:
            raise WeaverError(f"ABI mismatch: library struct sizes {tuple(sizes)} != {STRUCT_SIZES}")
        handle = ctypes.c_void_p()
        rc = self._lib.aw_engine_create(device, ctypes.byref(handle))
        if rc:
            raise WeaverError(f"aw_engine_create(device={device}) failed: {_status_text(self._lib, rc)}", rc)
        self._h = handle
        self.device = device

    # -- lifetime
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.aw_engine_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, rc: int, what: str) -> None:
        if rc:
            msg = self._lib.aw_engine_last_error(self._h).decode()
            raise WeaverError(f"{what}: {_status_text(self._lib, rc)}: {msg}", rc)

    # -- reference API
    def device_name(self) -> str:
        return self._lib.aw_engine_device_name(self._h).decode()

    def max_threads_per_threadgroup(self) -> int:
        return int(self._lib.aw_engine_max_threads_per_threadgroup(self._h))

    def decode(self, q_exact, q_latent, hot_pool, cold_pool, loom_refs, dictionary,
               params: WeaverParams) -> DecodeOutput:
        """``WeaverEngine::decode`` (weaver.rs:139-237): one token, reference math,
        synchronous.  ``q_latent`` may be ``None``/empty (then computed as q . D^T)."""
        q = _f16_bits(q_exact)
        ql = _f16_bits(q_latent) if q_latent is not None and np.asarray(q_latent).size else None
        hot = _f16_bits(hot_pool) if hot_pool is not None and np.asarray(hot_pool).size else None
        dic = _f16_bits(dictionary) if dictionary is not None and np.asarray(dictionary).size else None
        refs = np.ascontiguousarray(loom_refs, dtype=np.uint32).reshape(-1) if loom_refs is not None else None
        cold_ptr, n_cold = _codes_ptr(cold_pool if cold_pool is not None and np.asarray(cold_pool).size else None)
        n_out = params.q_heads * params.head_dim
        out = np.empty(n_out, dtype=np.uint16)

        def p(a):
            return None if a is None else a.ctypes.data

        def n(a):
            return 0 if a is None else a.size

        rc = self._lib.aw_decode(self._h, p(q), n(q), p(ql), n(ql), p(hot), n(hot), cold_ptr, n_cold,
                                 p(refs), n(refs), p(dic), n(dic), ctypes.byref(params), out.ctypes.data, n_out)
        self._check(rc, "decode")
        return DecodeOutput(data=out.view(np.float16))

    # -- device API
    def decode_device(self, desc: DecodeDesc, stream: Optional[int] = None) -> None:
        """Enqueue one batched decode described by ``desc`` (device pointers)."""
        rc = self._lib.aw_decode_device(self._h, ctypes.byref(desc), _stream(stream))
        self._check(rc, "decode_device")

    def read_stream(self, buf, nbytes: int, waves_per_cu: int, sink, stream: Optional[int] = None) -> None:
        """Enqueue a read-only stream over ``nbytes`` of ``buf`` (attainable HBM read rate)."""
        rc = self._lib.aw_debug_read_stream(self._h, _ptr(buf), nbytes, waves_per_cu, _ptr(sink), _stream(stream))
        self._check(rc, "read_stream")

    def project(self, desc: DecodeDesc, q_latent, stream: Optional[int] = None) -> None:
        """Run the request's q_latent = q . D^T projection alone into ``q_latent``
        (device, [L][B][Q][Hq][A], f16 or fp32 with AW_F_QLATENT_F32)."""
        rc = self._lib.aw_debug_project(self._h, ctypes.byref(desc), _ptr(q_latent), _stream(stream))
        self._check(rc, "project")

    def read_pools(self, desc: DecodeDesc, sink, stream: Optional[int] = None) -> None:
        """Enqueue a read of every hot row and cold code of ``desc`` through its block
        table, nothing computed (the attainable rate of the decode's pool reads)."""
        rc = self._lib.aw_debug_read_pools(self._h, ctypes.byref(desc), _ptr(sink), _stream(stream))
        self._check(rc, "read_pools")

    def decode_device_noalloc(self, desc: DecodeDesc, stream: Optional[int] = None) -> None:
        """``decode_device`` with its scratch in the library's fixed per-GPU array
        (AW_NOALLOC_SCRATCH_BYTES): allocates nothing; larger requests raise."""
        rc = self._lib.aw_decode_device_noalloc(self._h, ctypes.byref(desc), _stream(stream))
        self._check(rc, "decode_device_noalloc")

    def multihead_attention(self, q, k_cache, v_cache, output, kv_len: int, head_dim: int, q_heads: int,
                            kv_heads: int, num_queries: int, cache_tokens: Optional[int] = None,
                            stream: Optional[int] = None) -> None:
        """``Ops::multihead_attention`` (ops.rs:433-462, ops.metal:528-616) on the
        device: causal GQA attention of ``num_queries`` new tokens, the last of
        the ``kv_len`` cache positions, over contiguous [tokens][kv_heads][head_dim]
        K and V caches, scale 1/sqrt(head_dim).  ``cache_tokens`` (the caches'
        capacity in tokens) defaults to the K cache tensor's length."""
        if cache_tokens is None:
            if not hasattr(k_cache, "numel"):
                raise WeaverError("cache_tokens is required for raw pointers", -1)
            cache_tokens = k_cache.numel() // (kv_heads * head_dim)
        rc = self._lib.aw_multihead_attention_device(self._h, _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(output),
                                                     kv_len, head_dim, q_heads, kv_heads, num_queries, cache_tokens,
                                                     _stream(stream))
        self._check(rc, "multihead_attention")

    def encode_device(self, desc: EncodeDesc, stream: Optional[int] = None) -> None:
        """Enqueue one SparseCode encoder request (``Distiller::distill_block``,
        distiller.rs:171-246, over a batch of blocks; device pointers)."""
        rc = self._lib.aw_encode_device(self._h, ctypes.byref(desc), _stream(stream))
        self._check(rc, "encode_device")

    def block_entropy_device(self, hot, hot_blocks: int, kv_heads: int, head_dim: int, blocks, n_blocks: int,
                             entropy, stream: Optional[int] = None) -> None:
        """Variance proxy of hot blocks on the device (evaluate_entropy's loop,
        distiller.rs:97-120); ``blocks`` None scans blocks 0 .. n_blocks-1."""
        rc = self._lib.aw_block_entropy_device(self._h, _ptr(hot), hot_blocks, kv_heads, head_dim, _ptr(blocks),
                                               n_blocks, _ptr(entropy), _stream(stream))
        self._check(rc, "block_entropy_device")

    def encode(self, hot_pool, dictionary, blocks, cold_pool, kv_heads: int, head_dim: int, dict_size: int,
               dict_heads: int, entropy: bool = False):
        """Host-slice encoder (copy in, encode, copy out, wait): hot block b of
        ``blocks`` -> cold block b (distiller.rs:177).  ``cold_pool`` (uint16
        words or SparseCode records) is updated in place; returns the blocks'
        entropy proxies (distiller.rs:126-159) when asked."""
        hot = _f16_bits(hot_pool)
        dic = _f16_bits(dictionary)
        blk = np.ascontiguousarray(blocks, dtype=np.uint32).reshape(-1)
        if not isinstance(cold_pool, np.ndarray) or not cold_pool.flags.c_contiguous:
            raise TypeError("cold_pool must be a C-contiguous numpy array (updated in place)")
        if cold_pool.dtype == SPARSE_CODE_DTYPE:
            target = cold_pool.view(np.uint16).reshape(-1, 8)
        elif cold_pool.dtype == np.uint16 and cold_pool.shape[-1] == 8:
            target = cold_pool.reshape(-1, 8)
        else:
            raise TypeError("cold pool must be SPARSE_CODE_DTYPE or uint16 words [..., 8]")
        words = _aligned16(np.array(target, dtype=np.uint16, order="C"))
        ent = np.zeros(blk.size, dtype=np.float32) if entropy else None
        rc = self._lib.aw_encode(self._h, hot.ctypes.data, hot.size, dic.ctypes.data, dic.size, kv_heads, head_dim,
                                 dict_size, dict_heads, blk.ctypes.data, blk.size, words.ctypes.data, words.shape[0],
                                 None if ent is None else ent.ctypes.data)
        self._check(rc, "encode")
        np.copyto(target, words)
        return ent

    def check_device_errors(self, stream: Optional[int] = None) -> None:
        self._check(self._lib.aw_engine_check_device_errors(self._h, _stream(stream)), "device check")

    def gather_codes(self, codes, n_codes: int, dictionary, dict_size: int, head_dim: int, idx, coef, atoms,
                     stream: Optional[int] = None) -> None:
        """Bit-exact SparseCode decode + atom gather on the device (device pointers/tensors)."""
        rc = self._lib.aw_debug_gather_codes(self._h, _ptr(codes), n_codes, _ptr(dictionary), dict_size, head_dim,
                                             _ptr(idx), _ptr(coef), _ptr(atoms), _stream(stream))
        self._check(rc, "gather_codes")

    def set_profiling(self, mode) -> None:
        """0/False: off; 1/True: event-time each kernel in the concurrent
        pipeline; 2: event-time each kernel with the stages serialized."""
        self._check(self._lib.aw_engine_set_profiling(self._h, int(mode)), "set_profiling")

    def set_projection(self, mode) -> None:
        """Kernel of q_latent = q . D^T: 0 the planner's choice (MFMA), 1 MFMA
        tiles, 2 the VALU kernel (AW_PROJECT_*)."""
        self._check(self._lib.aw_engine_set_projection(self._h, int(mode)), "set_projection")

    def set_cold_output(self, mode) -> None:
        """What the cold kernel hands on (AW_COLD_OUT_*): 0 the planner's choice,
        1 per-atom bins for the finish kernel, 2 value partials for the merge
        (dictionary heads of at most 128 KiB; bins elsewhere)."""
        self._check(self._lib.aw_engine_set_cold_output(self._h, int(mode)), "set_cold_output")

    def reset_stage_stats(self) -> None:
        self._check(self._lib.aw_engine_reset_stage_stats(self._h), "reset_stage_stats")

    def stage_stats(self) -> dict:
        """{stage: (total_ms, launches)} from the HIP events of profiled launches."""
        out = {}
        for i, name in enumerate(STAGES):
            ms = ctypes.c_double()
            n = ctypes.c_uint64()
            self._check(self._lib.aw_engine_stage_stats(self._h, i, ctypes.byref(ms), ctypes.byref(n)),
                        "stage_stats")
            out[name] = (ms.value, n.value)
        return out


def make_desc(*, layers: int, batch: int, queries: int, q_heads: int, kv_heads: int, head_dim: int,
              dict_size: int, dict_heads: int, hot_count: int, cold_count: int, refs_stride: int,
              hot_blocks: int, cold_blocks: int, q, out, hot_k=None, hot_v=None, cold=None, refs=None,
              dictionary=None, q_latent=None, seq_hot=None, seq_cold=None, scale: float = 1.0,
              causal: bool = False, cold_head_blocked: bool = False, hot_tokens: int = 0,
              seq_hot_tokens: bool = False, q_latent_f32: bool = False) -> DecodeDesc:
    """Build an ``aw_decode_desc`` from device tensors (or raw device pointers).
    ``cold_head_blocked``: the cold pool is [L][blocks][kv_heads][16] instead of
    the reference's [L][blocks][16][kv_heads].  ``hot_tokens``: hot tokens per
    sequence when not whole blocks (0 = hot_count * 16); ``seq_hot_tokens``:
    ``seq_hot`` counts tokens instead of blocks; ``q_latent_f32``: a q_latent
    computed on the device stays fp32 (AW_F_QLATENT_F32)."""
    d = DecodeDesc()
    d.layers, d.batch, d.queries = layers, batch, queries
    d.q_heads, d.kv_heads, d.head_dim = q_heads, kv_heads, head_dim
    d.dict_size, d.dict_heads = dict_size, dict_heads
    d.hot_count, d.cold_count, d.refs_stride = hot_count, cold_count, refs_stride
    d.flags = ((AW_F_CAUSAL if causal else 0) | (AW_F_COLD_HEAD_BLOCKED if cold_head_blocked else 0) |
               (AW_F_SEQ_HOT_TOKENS if seq_hot_tokens else 0) | (AW_F_QLATENT_F32 if q_latent_f32 else 0))
    d.scale = scale
    d.hot_tokens = hot_tokens
    d.hot_blocks, d.cold_blocks = hot_blocks, cold_blocks
    d.q, d.q_latent, d.hot_k, d.hot_v = _ptr(q), _ptr(q_latent), _ptr(hot_k), _ptr(hot_v)
    d.cold, d.refs, d.seq_hot, d.seq_cold = _ptr(cold), _ptr(refs), _ptr(seq_hot), _ptr(seq_cold)
    d.dict, d.out = _ptr(dictionary), _ptr(out)
    # The descriptor holds raw addresses: keep the tensors behind them alive as
    # long as it is (a temporary such as a reordered pool would otherwise go back
    # to torch's cache, and torch.cuda.graph's empty_cache would unmap it).
    d._keep = (q, out, hot_k, hot_v, cold, refs, dictionary, q_latent, seq_hot, seq_cold)
    return d


def make_encode_desc(*, kv_heads: int, head_dim: int, dict_size: int, dict_heads: int, hot_blocks: int,
                     cold_blocks: int, hot, dictionary, src_blocks, cold, dst_blocks=None, entropy=None,
                     cold_head_blocked: bool = False, full_scan: bool = False) -> EncodeDesc:
    """Build an ``aw_encode_desc`` from device tensors (or raw device pointers).
    ``full_scan`` scores every atom exactly instead of prefiltering on MFMA (same codes)."""
    d = EncodeDesc()
    d.kv_heads, d.head_dim, d.dict_size, d.dict_heads = kv_heads, head_dim, dict_size, dict_heads
    n = src_blocks.numel() if hasattr(src_blocks, "numel") else int(np.asarray(src_blocks).size)
    d.n_blocks = n
    d.flags = (AW_F_COLD_HEAD_BLOCKED if cold_head_blocked else 0) | (AW_F_ENCODE_FULL_SCAN if full_scan else 0)
    d.hot_blocks, d.cold_blocks = hot_blocks, cold_blocks
    d.hot, d.dict, d.src_blocks = _ptr(hot), _ptr(dictionary), _ptr(src_blocks)
    d.dst_blocks, d.cold, d.entropy = _ptr(dst_blocks), _ptr(cold), _ptr(entropy)
    d._keep = (hot, dictionary, src_blocks, dst_blocks, cold, entropy)  # as in make_desc
    return d
