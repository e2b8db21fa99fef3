"""CPU restatement of the reference's dense transformer ops (nexus-core/src/ops.metal:16-635).

TEST INFRASTRUCTURE ONLY: imported by tests/ to check the product's aw_ops_*
entry points (include/aether_ops.h) and by bench.py's CPU baseline leg, never
by the product package.  numpy.

Two kinds of functions:
  * the fp32 restatements (`*_f32`) evaluate the reference's expressions one
    numpy float32 operation at a time (IEEE single, round to nearest, no fused
    multiply-add) and round to f16 where the kernel stores f16.  Element-wise
    ops (copy, add_residual, add_bias, scale_f16) are then bit-exact
    specifications; where the kernel sums in a different order (rms_norm's sum
    of squares, the products' dot products) or calls a transcendental (silu's
    exp, rope's cos and sin) the GPU is compared within the tolerances the
    tests state.
  * the float64 forms (`*_f64`) compute the same mathematics exactly enough to
    bound those tolerances.

Pins (tests/test_ops_oracle.py): every function against an independent form —
numpy's matmul for the products, a complex multiplication by e^{i*angle} for
rope, np.linalg.norm for rms_norm, scipy.special.expit for silu, numpy
indexing for embed_lookup and copy — plus closed forms (the identity matrix,
angle 0, constant rows, silu(0) = 0), chosen so that the plausible mistakes
(rotating interleaved pairs instead of half-split ones, dividing by H - 1,
a transposed weight matrix) fail them.
"""
from __future__ import annotations

import numpy as np

F16 = np.float16
F32 = np.float32


def _h(x) -> np.ndarray:
    """f16 values (from float16 arrays or their uint16/int16 bit patterns) as float32."""
    a = np.asarray(x)
    if a.dtype in (np.uint16, np.int16):
        a = a.view(np.float16)
    return a.astype(F32)


def copy_buffer(src, dst, count: int, src_off: int, dst_off: int) -> np.ndarray:
    """ops.metal:16-26: dst[dst_off + i] = src[src_off + i], i < count."""
    out = np.array(dst, copy=True)
    out[dst_off:dst_off + count] = np.asarray(src)[src_off:src_off + count]
    return out


def embed_lookup(token_ids, table, hidden_size: int, vocab_size: int) -> np.ndarray:
    """ops.metal:33-49: rows of the table by token id.  An id >= vocab_size
    gives a zero row here (aw_ops_embed_lookup's rule; the reference reads past
    its table)."""
    ids = np.asarray(token_ids, dtype=np.int64)
    tab = np.asarray(table).reshape(vocab_size, hidden_size)
    out = np.zeros((ids.size, hidden_size), dtype=tab.dtype)
    ok = ids < vocab_size
    out[ok] = tab[ids[ok]]
    return out


def rms_norm_f32(x, weight, eps: float) -> np.ndarray:
    """ops.metal:59-99 per row of x [T][H]: s = sum x^2 in float32, inv = 1 /
    sqrt(s / H + eps), out = f16((x * inv) * w)."""
    xs = _h(x)
    w = _h(weight)
    h = xs.shape[-1]
    s = np.sum(xs * xs, axis=-1, dtype=F32)
    inv = F32(1.0) / np.sqrt(s / F32(h) + F32(eps))
    return ((xs * inv[..., None]) * w).astype(F16)


def rms_norm_f64(x, weight, eps: float) -> np.ndarray:
    xs = _h(x).astype(np.float64)
    w = _h(weight).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xs * xs, axis=-1) + eps)
    return xs * inv[..., None] * w


def rope_freqs(head_dim: int, theta: float) -> np.ndarray:
    """freq_p = 1 / theta^(2p / head_dim) (ops.metal:131), in double, rounded to float32."""
    p = np.arange(head_dim // 2, dtype=np.float64)
    return (1.0 / np.power(np.float64(F32(theta)), 2.0 * p / head_dim)).astype(F32)


def rope_f32(x, start_position: int, theta: float) -> np.ndarray:
    """ops.metal:107-155 on x [T][heads][head_dim] (q or k): the pair (x[p],
    x[p + d/2]) rotates by angle = f32(start + t) * freq_p; cos and sin of the
    float32 angle taken in double and rounded to float32; the rotation in
    float32, one rounding per operation; f16 out."""
    xs = _h(x)
    t_n, _, d = xs.shape
    half = d // 2
    freq = rope_freqs(d, theta)
    pos = (np.uint32(start_position) + np.arange(t_n, dtype=np.uint32)).astype(F32)
    ang = pos[:, None] * freq[None, :]                      # [T][d/2] float32
    c = np.cos(ang.astype(np.float64)).astype(F32)[:, None, :]
    s = np.sin(ang.astype(np.float64)).astype(F32)[:, None, :]
    x0, x1 = xs[..., :half], xs[..., half:]
    out = np.empty_like(xs)
    out[..., :half] = x0 * c - x1 * s
    out[..., half:] = x0 * s + x1 * c
    return out.astype(F16)


def matmul_f64(a, b) -> np.ndarray:
    """matmul_f16 / vecmat_f16 (ops.metal:170-271) before rounding: a [M][K] . b [N][K]^T in float64."""
    return _h(a).astype(np.float64) @ _h(b).astype(np.float64).T


def matmul_abs_f64(a, b) -> np.ndarray:
    """sum_k |a_mk| |b_nk|: the scale of each dot product's rounding error."""
    return np.abs(_h(a).astype(np.float64)) @ np.abs(_h(b).astype(np.float64)).T


def silu_gate_f32(gate, up) -> np.ndarray:
    """ops.metal:325-338: f16((g / (1 + exp(-g))) * u) in float32."""
    g = _h(gate)
    u = _h(up)
    with np.errstate(over="ignore"):
        silu = g / (F32(1.0) + np.exp(-g))
    return (silu * u).astype(F16)


def silu_gate_f64(gate, up) -> np.ndarray:
    g = _h(gate).astype(np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * _h(up).astype(np.float64)


def add_residual(x, residual) -> np.ndarray:
    """ops.metal:345-353: f16(x + r) in float32 (exact before the rounding)."""
    return (_h(x) + _h(residual)).astype(F16)


def add_bias(x, bias, hidden_size: int) -> np.ndarray:
    """ops.metal:360-371: f16(x[t][d] + bias[d])."""
    xs = _h(x).reshape(-1, hidden_size)
    return (xs + _h(bias)[None, :hidden_size]).astype(F16)


def scale_f16(x, scale: float) -> np.ndarray:
    """ops.metal:627-635: f16(x * scale) in float32."""
    return (_h(x) * F32(scale)).astype(F16)
