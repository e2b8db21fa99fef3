"""Pins of the dense-ops oracle (oracle/ops_oracle.py) on the CPU.

The reference ships no tests for its ops kernels (nexus-core/src/ops.metal),
so each oracle function is checked against an independent form of the same
mathematics or against closed forms, chosen so that the plausible mistakes
fail: interleaved instead of half-split RoPE pairs, a mean over H - 1, the
weights not transposed, silu without the gate product."""
from __future__ import annotations

import numpy as np
import pytest
from scipy.special import expit

from oracle import ops_oracle as O


def f16(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def ulp16(x):
    return np.spacing(np.abs(np.asarray(x, dtype=np.float16))).astype(np.float64)


def test_matmul_is_a_times_b_transposed():
    """C = A . B^T with B stored [N][K] (ops.metal:163-167): a hand-worked 2x3
    case, the identity and a permutation (exact), and B not transposed fails."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float16)
    b = np.array([[1, 0, 0], [0, 1, 1], [1, 1, 1], [2, 0, -1]], np.float16)
    assert np.array_equal(O.matmul_f64(a, b), [[1, 5, 6, -1], [4, 11, 15, 2]])
    rng = np.random.default_rng(0)
    x = f16(rng, 5, 16)
    assert np.array_equal(O.matmul_f64(x, np.eye(16, dtype=np.float16)), x.astype(np.float64))
    perm = rng.permutation(16)
    p = np.eye(16, dtype=np.float16)[perm]
    assert np.array_equal(O.matmul_f64(x, p), x.astype(np.float64)[:, perm])
    w = f16(rng, 16, 16)
    assert not np.allclose(O.matmul_f64(x, w), x.astype(np.float64) @ w.astype(np.float64))
    # matmul_abs_f64 bounds |C|
    assert np.all(np.abs(O.matmul_f64(x, w)) <= O.matmul_abs_f64(x, w) + 1e-12)


def test_rope_is_a_rotation_of_half_split_pairs():
    """(x[p] + i x[p + d/2]) * e^{i pos theta^(-2p/d)} in complex128, within one
    f16 ulp plus the float32 angle's rounding; position 0 is the identity; the
    interleaved pairing (x[2p], x[2p+1]) fails the same check."""
    rng = np.random.default_rng(1)
    t, h, d, start, theta = 5, 3, 64, 1000, 10000.0
    x = f16(rng, t, h, d)
    got = O.rope_f32(x, start, theta).astype(np.float64)
    xs = x.astype(np.float64)
    pos = start + np.arange(t)
    ang = pos[:, None, None] * theta ** (-2.0 * np.arange(d // 2) / d)[None, None, :]
    z = (xs[..., :d // 2] + 1j * xs[..., d // 2:]) * np.exp(1j * ang)
    want = np.concatenate([z.real, z.imag], axis=-1)
    # float32 angle: |pos * freq| < 1100 rad, rounding <= 2^-24 * 1100 ~ 7e-5 rad, times |x| <= ~5
    tol = ulp16(want) + 5e-4
    assert np.all(np.abs(got - want) <= tol)
    assert np.array_equal(O.rope_f32(x[:1], 0, theta).view(np.uint16), x[:1].view(np.uint16))  # position 0
    inter = xs.copy()
    zi = (xs[..., 0::2] + 1j * xs[..., 1::2]) * np.exp(1j * ang)
    inter[..., 0::2], inter[..., 1::2] = zi.real, zi.imag
    assert np.abs(got - inter).max() > 0.1
    # the pair's norm is kept
    n0 = xs[..., :d // 2] ** 2 + xs[..., d // 2:] ** 2
    n1 = got[..., :d // 2] ** 2 + got[..., d // 2:] ** 2
    assert np.allclose(n0, n1, rtol=4e-3, atol=1e-3)


def test_rope_freqs_closed_form():
    f = O.rope_freqs(8, 10000.0)
    assert f.dtype == np.float32 and f[0] == 1.0
    assert np.allclose(f, [1.0, 0.1, 0.01, 0.001], rtol=1e-7)


def test_rms_norm_against_the_vector_norm():
    """x / (||x|| / sqrt(H)) * w with eps -> 0 (np.linalg.norm), a constant row
    (closed form c / sqrt(c^2 + eps)), and a mean over H - 1 fails."""
    rng = np.random.default_rng(2)
    x = f16(rng, 4, 96)
    w = f16(rng, 96)
    got = O.rms_norm_f32(x, w, 1e-12).astype(np.float64)
    xs = x.astype(np.float64)
    want = xs / (np.linalg.norm(xs, axis=1, keepdims=True) / np.sqrt(96)) * w.astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp16(want) * 0.5 + 1e-6 * np.abs(want) + 1e-7)
    assert np.allclose(O.rms_norm_f64(x, w, 1e-12), want, rtol=1e-12)
    wrong = xs / np.sqrt(np.sum(xs * xs, axis=1, keepdims=True) / 95) * w.astype(np.float64)
    assert np.abs(got - wrong).max() > 4 * ulp16(want).max()
    c = np.full((1, 8), 3.0, np.float16)
    one = np.ones(8, np.float16)
    eps = 0.25
    assert np.allclose(O.rms_norm_f32(c, one, eps).astype(np.float64), 3.0 / np.sqrt(9.0 + eps), atol=1e-3)


def test_silu_gate_against_expit():
    rng = np.random.default_rng(3)
    g = f16(rng, 4096, scale=4.0)
    u = f16(rng, 4096)
    got = O.silu_gate_f32(g, u).astype(np.float64)
    want = g.astype(np.float64) * expit(g.astype(np.float64)) * u.astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp16(want) + 1e-7)
    assert np.allclose(O.silu_gate_f64(g, u), want, rtol=1e-12, atol=1e-300)
    assert np.all(O.silu_gate_f32(np.zeros(4, np.float16), u[:4]) == 0)
    # without the gate product (silu(g) alone) the check fails
    assert np.abs(got - g.astype(np.float64) * expit(g.astype(np.float64))).max() > 0.5
    # large |g|: silu(g) -> g for g >> 0, -> 0 for g << 0 (float32 exp overflows to inf, giving -0)
    big = np.array([30.0, -30.0, -100.0], np.float16)
    assert np.array_equal(O.silu_gate_f32(big, np.ones(3, np.float16)).astype(np.float64), [30.0, 0.0, 0.0])


def test_embed_lookup_and_copy_index_the_right_rows():
    rng = np.random.default_rng(4)
    table = f16(rng, 10, 8)
    ids = np.array([3, 0, 9, 12, 3], np.uint32)
    out = O.embed_lookup(ids, table, 8, 10)
    assert np.array_equal(out[[0, 1, 2, 4]], table[[3, 0, 9, 3]])
    assert np.all(out[3] == 0)  # id 12 >= vocab 10
    src = np.arange(20, dtype=np.uint16)
    dst = np.zeros(20, np.uint16)
    got = O.copy_buffer(src, dst, 5, 3, 10)
    assert list(got[10:15]) == [3, 4, 5, 6, 7] and got[:10].sum() == 0 and got[15:].sum() == 0


@pytest.mark.parametrize("op", ["add_residual", "add_bias", "scale_f16"])
def test_elementwise_closed_forms(op):
    rng = np.random.default_rng(5)
    x = f16(rng, 6, 16)
    if op == "add_residual":
        assert np.all(O.add_residual(x, -x) == 0)
        assert np.array_equal(O.add_residual(x, np.zeros_like(x)).view(np.uint16), x.view(np.uint16))
        r = f16(rng, 6, 16)
        assert np.array_equal(O.add_residual(x, r).view(np.uint16), O.add_residual(r, x).view(np.uint16))
    elif op == "add_bias":
        b = f16(rng, 16)
        assert np.array_equal(O.add_bias(np.zeros_like(x), b, 16).view(np.uint16), np.tile(b, (6, 1)).view(np.uint16))
        assert np.array_equal(O.add_bias(x, np.zeros(16, np.float16), 16).view(np.uint16), x.view(np.uint16))
    else:
        assert np.array_equal(O.scale_f16(x, 2.0).astype(np.float64), 2.0 * x.astype(np.float64))
        assert np.array_equal(O.scale_f16(x, 1.0).view(np.uint16), x.view(np.uint16))
