"""The dense transformer ops on the gfx950 library (include/aether_ops.h).

``OpsEngine`` mirrors the reference's ``Ops`` (nexus-core/src/ops.rs:21-462):
the same method names, argument order and meaning, over device tensors (or
raw device pointers) instead of Metal buffers.  Every call is asynchronous on a
HIP stream, torch's current stream by default: the reference's batch mode
(``begin_batch`` / ``end_batch``, ops.rs:88-101, one command buffer per
forward pass) is the stream itself, and ``end_batch`` waits for it.  With
tensors the wrapper also checks their dtype, device and element counts before
anything is enqueued (the C ABI takes raw pointers).
"""
from __future__ import annotations

from typing import Optional

from .weaver import WeaverEngine, WeaverError, _ptr, _stream

AW_E_INVALID_ARG = -1


def _check_tensor(t, need: int, what: str, dtypes) -> None:
    """Element count, dtype and device of a tensor argument (raw ints pass)."""
    if t is None or isinstance(t, int):
        return
    import torch
    if not isinstance(t, torch.Tensor):
        raise WeaverError(f"{what}: expected a device tensor or a device pointer", AW_E_INVALID_ARG)
    if t.device.type != "cuda":
        raise WeaverError(f"{what}: tensor is on {t.device}, not the GPU", AW_E_INVALID_ARG)
    if t.dtype not in dtypes:
        raise WeaverError(f"{what}: dtype {t.dtype} (want {' or '.join(map(str, dtypes))})", AW_E_INVALID_ARG)
    if not t.is_contiguous():
        raise WeaverError(f"{what}: tensor is not contiguous", AW_E_INVALID_ARG)
    if t.numel() < need:
        raise WeaverError(f"{what}: {t.numel()} elements, the call reads or writes {need}", AW_E_INVALID_ARG)


def _f16(t, need, what):
    import torch
    _check_tensor(t, need, what, (torch.float16, torch.int16))  # f16 values or their bit patterns


def _f32(t, need, what):
    import torch
    _check_tensor(t, need, what, (torch.float32,))


def _u32(t, need, what):
    import torch
    _check_tensor(t, need, what, (torch.int32,))


class OpsEngine:
    """``Ops`` (ops.rs:21-462) on MI355X.  Shares a ``WeaverEngine`` (device,
    device error word, last-error text) or creates its own."""

    def __init__(self, engine: Optional[WeaverEngine] = None, lib_path=None, device: int = 0):
        self._own = engine is None
        self.engine = engine if engine is not None else WeaverEngine(lib_path=lib_path, device=device)
        self._lib = self.engine._lib

    def close(self) -> None:
        if self._own:
            self.engine.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _call(self, name: str, *args) -> None:
        rc = getattr(self._lib, name)(self.engine._h, *args)
        self.engine._check(rc, name[len("aw_ops_"):] if name.startswith("aw_ops_") else name)

    # -- batch mode (ops.rs:88-101)
    def begin_batch(self) -> None:
        """Nothing to open: calls are already queued on the stream without waiting."""

    def end_batch(self, stream: Optional[int] = None) -> None:
        """Wait until everything queued on the stream has finished (ops.rs:95-101)."""
        import torch
        s = _stream(stream)
        if s is None:
            torch.cuda.synchronize()
        elif s == 0:  # the null stream (torch.cuda.ExternalStream(0) would make a stream of its own)
            torch.cuda.default_stream().synchronize()
        else:
            torch.cuda.ExternalStream(s).synchronize()

    def check_device_errors(self, stream: Optional[int] = None) -> None:
        """Raise if a kernel saw out-of-range input (an embed token id >= vocab_size)."""
        self.engine.check_device_errors(stream)

    # -- the ops
    def copy_buffer(self, src, dst, count: int, src_off: int, dst_off: int, stream: Optional[int] = None) -> None:
        """ops.rs:166-180: dst[dst_off + i] = src[src_off + i], i < count (f16 elements)."""
        _f16(src, src_off + count, "copy_buffer src")
        _f16(dst, dst_off + count, "copy_buffer dst")
        self._call("aw_ops_copy_buffer", _ptr(src), _ptr(dst), count, src_off, dst_off, _stream(stream))

    def embed_lookup(self, token_ids, embed_table, output, hidden_size: int, seq_len: int,
                     vocab_size: Optional[int] = None, stream: Optional[int] = None) -> None:
        """ops.rs:183-206: output[t] = embed_table[token_ids[t]]; ``vocab_size``
        defaults to the table tensor's rows."""
        if vocab_size is None:
            if not hasattr(embed_table, "numel"):
                raise WeaverError("embed_lookup: vocab_size is required for a raw table pointer", AW_E_INVALID_ARG)
            vocab_size = embed_table.numel() // max(hidden_size, 1)
        _u32(token_ids, seq_len, "embed_lookup token_ids")
        _f16(embed_table, vocab_size * hidden_size, "embed_lookup embed_table")
        _f16(output, seq_len * hidden_size, "embed_lookup output")
        self._call("aw_ops_embed_lookup", _ptr(token_ids), _ptr(embed_table), _ptr(output), hidden_size, seq_len,
                   vocab_size, _stream(stream))

    def rms_norm(self, input, weight, output, hidden_size: int, num_tokens: int, eps: float,
                 stream: Optional[int] = None) -> None:
        """ops.rs:209-231: output = input * rsqrt(mean(input^2) + eps) * weight, per token."""
        _f16(input, hidden_size * num_tokens, "rms_norm input")
        _f16(weight, hidden_size, "rms_norm weight")
        _f16(output, hidden_size * num_tokens, "rms_norm output")
        self._call("aw_ops_rms_norm", _ptr(input), _ptr(weight), _ptr(output), hidden_size, num_tokens, eps,
                   _stream(stream))

    def rope(self, q, k, num_tokens: int, q_heads: int, kv_heads: int, head_dim: int, start_position: int,
             theta: float, stream: Optional[int] = None) -> None:
        """ops.rs:234-263: rotary embedding of q and k in place."""
        _f16(q, num_tokens * q_heads * head_dim, "rope q")
        _f16(k, num_tokens * kv_heads * head_dim, "rope k")
        self._call("aw_ops_rope", _ptr(q), _ptr(k), num_tokens, q_heads, kv_heads, head_dim, start_position, theta,
                   _stream(stream))

    def matmul(self, a, b, output, m: int, n: int, k: int, stream: Optional[int] = None) -> None:
        """ops.rs:266-296: output [m][n] = a [m][k] . b [n][k]^T, f16 out."""
        _f16(a, m * k, "matmul a")
        _f16(b, n * k, "matmul b")
        _f16(output, m * n, "matmul output")
        self._call("aw_ops_matmul", _ptr(a), _ptr(b), _ptr(output), m, n, k, _stream(stream))

    def silu_gate(self, gate, up, output, size: int, stream: Optional[int] = None) -> None:
        """ops.rs:299-312: output = SiLU(gate) * up."""
        for t, w in ((gate, "gate"), (up, "up"), (output, "output")):
            _f16(t, size, f"silu_gate {w}")
        self._call("aw_ops_silu_gate", _ptr(gate), _ptr(up), _ptr(output), size, _stream(stream))

    def add_residual(self, x, residual, size: int, stream: Optional[int] = None) -> None:
        """ops.rs:315-327: x += residual."""
        _f16(x, size, "add_residual x")
        _f16(residual, size, "add_residual residual")
        self._call("aw_ops_add_residual", _ptr(x), _ptr(residual), size, _stream(stream))

    def add_bias(self, x, bias, hidden_size: int, num_tokens: int, stream: Optional[int] = None) -> None:
        """ops.rs:330-343: x[t][d] += bias[d]."""
        _f16(x, hidden_size * num_tokens, "add_bias x")
        _f16(bias, hidden_size, "add_bias bias")
        self._call("aw_ops_add_bias", _ptr(x), _ptr(bias), hidden_size, num_tokens, _stream(stream))

    def scale_f16(self, x, count: int, scale: float, stream: Optional[int] = None) -> None:
        """ops.rs:350-363: x *= scale."""
        _f16(x, count, "scale_f16 x")
        self._call("aw_ops_scale_f16", _ptr(x), count, scale, _stream(stream))

    def matmul_scaled(self, a, b, output, m: int, n: int, k: int, scale: float,
                      stream: Optional[int] = None) -> None:
        """ops.rs:366-406: output [m][n] = (a . b^T) * scale, f32 out."""
        _f16(a, m * k, "matmul_scaled a")
        _f16(b, n * k, "matmul_scaled b")
        _f32(output, m * n, "matmul_scaled output")
        self._call("aw_ops_matmul_scaled", _ptr(a), _ptr(b), _ptr(output), m, n, k, scale, _stream(stream))

    def causal_attention(self, q, k, v, output, kv_len: int, head_dim: int, cache_tokens: Optional[int] = None,
                         stream: Optional[int] = None) -> None:
        """ops.rs:409-430: single-head softmax(q.K^T/sqrt(d)) V over kv_len rows.
        ``cache_tokens`` (rows k and v hold, >= kv_len rounded up to 16) defaults
        to the k tensor's rows."""
        if cache_tokens is None:
            if not hasattr(k, "numel"):
                raise WeaverError("causal_attention: cache_tokens is required for raw pointers", AW_E_INVALID_ARG)
            cache_tokens = k.numel() // head_dim
        _f16(q, head_dim, "causal_attention q")
        for t, w in ((k, "k"), (v, "v")):
            _f16(t, cache_tokens * head_dim, f"causal_attention {w}")
        _f16(output, head_dim, "causal_attention output")
        self._call("aw_ops_causal_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(output), kv_len, head_dim,
                   cache_tokens, _stream(stream))

    # -- fused forms (no reference counterpart): the same output bits as the separate calls
    def matmul_add_residual(self, a, b, x, m: int, n: int, k: int, residual_multiplier: float = 1.0,
                            stream: Optional[int] = None) -> None:
        """matmul, scale_f16 by ``residual_multiplier``, add_residual into x, in one launch
        (forward_batch's o_proj and down_proj steps, inference.rs:564-572,592-600)."""
        _f16(a, m * k, "matmul_add_residual a")
        _f16(b, n * k, "matmul_add_residual b")
        _f16(x, m * n, "matmul_add_residual x")
        self._call("aw_ops_matmul_add_residual", _ptr(a), _ptr(b), _ptr(x), m, n, k, residual_multiplier,
                   _stream(stream))

    def matmul_silu_gate(self, a, b_gate, b_up, output, m: int, n: int, k: int, stream: Optional[int] = None) -> None:
        """The gate and up matmuls and silu_gate in one launch (inference.rs:586-591); m <= 64."""
        _f16(a, m * k, "matmul_silu_gate a")
        _f16(b_gate, n * k, "matmul_silu_gate b_gate")
        _f16(b_up, n * k, "matmul_silu_gate b_up")
        _f16(output, m * n, "matmul_silu_gate output")
        self._call("aw_ops_matmul_silu_gate", _ptr(a), _ptr(b_gate), _ptr(b_up), _ptr(output), m, n, k,
                   _stream(stream))

    def matmul_qkv(self, a, b_q, b_k, b_v, q, k_out, v_out, m: int, n_q: int, n_kv: int, k: int,
                   stream: Optional[int] = None) -> None:
        """The q, k and v matmuls in one launch (inference.rs:518-523)."""
        _f16(a, m * k, "matmul_qkv a")
        for t, n, w in ((b_q, n_q, "b_q"), (b_k, n_kv, "b_k"), (b_v, n_kv, "b_v")):
            _f16(t, n * k, f"matmul_qkv {w}")
        for t, n, w in ((q, n_q, "q"), (k_out, n_kv, "k_out"), (v_out, n_kv, "v_out")):
            _f16(t, m * n, f"matmul_qkv {w}")
        self._call("aw_ops_matmul_qkv", _ptr(a), _ptr(b_q), _ptr(b_k), _ptr(b_v), _ptr(q), _ptr(k_out), _ptr(v_out),
                   m, n_q, n_kv, k, _stream(stream))

    def multihead_attention(self, q, k_cache, v_cache, output, kv_len: int, head_dim: int, q_heads: int,
                            kv_heads: int, num_queries: int, cache_tokens: Optional[int] = None,
                            stream: Optional[int] = None) -> None:
        """ops.rs:433-462 (aw_multihead_attention_device)."""
        self.engine.multihead_attention(q, k_cache, v_cache, output, kv_len, head_dim, q_heads, kv_heads,
                                        num_queries, cache_tokens=cache_tokens, stream=stream)
