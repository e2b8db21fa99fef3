"""GPU parity of the dense transformer ops (include/aether_ops.h) against the
CPU oracle (oracle/ops_oracle.py), through the C ABI on cuda:0.

Tolerances: the element-wise ops whose result is one exactly-rounded fp32
operation (copy, add_residual, add_bias, scale_f16, embed_lookup) are
bit-exact.  rms_norm, silu_gate and rope are within one f16 ulp of the fp32
restatement (the kernel sums squares in another order, and takes exp, cos and
sin from the device library).  The products differ from the float64 result
by at most K * 2^-24 * sum_k |a_k b_k| (the worst-case fp32 accumulation error
in any order) plus one f16 ulp, and their rel-L2 error is below 1e-3."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import attention_oracle as AO
from oracle import ops_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(engine):
    from aether_nexus_amd.ops import OpsEngine
    return OpsEngine(engine)


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return torch.from_numpy(a.view(np.int16).copy()).cuda().view(torch.float16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32).copy()).cuda()
    return torch.from_numpy(a.copy()).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def f16(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def ulp16(x):
    return np.spacing(np.abs(np.asarray(x, dtype=np.float64).astype(np.float16))).astype(np.float64)


def bits(x):
    return np.asarray(x).view(np.uint16)


def within_one_ulp(got, want, what):
    g = np.asarray(got, np.float16).astype(np.float64)
    w = np.asarray(want, np.float16).astype(np.float64)
    d = np.abs(g - w)
    exact = float(np.mean(bits(np.asarray(got, np.float16)) == bits(np.asarray(want, np.float16))))
    print(f"{what}: max |diff| {d.max():.3e}, bit-exact {exact:.4f}", flush=True)
    assert np.all(d <= np.maximum(ulp16(w), 2.0 ** -24)), what
    return exact


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 65541])
def test_copy_add_scale_bit_exact(ops, n):
    rng = np.random.default_rng(n)
    src = f16(rng, n + 16)
    dst = f16(rng, n + 16)
    print(f"elementwise n={n}", flush=True)
    for so, do in ((0, 0), (3, 5), (8, 0)):  # (3, 5): not 16-byte aligned, element-wise path
        d = dev(dst)
        ops.copy_buffer(dev(src), d, n, so, do)
        assert np.array_equal(bits(host(d)), bits(O.copy_buffer(src, dst, n, so, do))), (so, do)
    x, r = dev(src[:n]), dev(dst[:n])
    ops.add_residual(x, r, n)
    assert np.array_equal(bits(host(x)), bits(O.add_residual(src[:n], dst[:n])))
    x = dev(src[:n])
    ops.scale_f16(x, n, 0.3712)
    assert np.array_equal(bits(host(x)), bits(O.scale_f16(src[:n], 0.3712)))
    # unaligned views (odd element offset) take the element-wise kernels
    xs, rs = dev(src), dev(dst)
    ops.add_residual(xs[1:], rs[1:], n)
    want = src.copy()
    want[1:n + 1] = O.add_residual(src[1:n + 1], dst[1:n + 1])
    assert np.array_equal(bits(host(xs)), bits(want))


@pytest.mark.parametrize("hidden,tokens", [(4096, 3), (13, 5), (8, 1)])
def test_add_bias_bit_exact(ops, hidden, tokens):
    rng = np.random.default_rng(hidden)
    x = f16(rng, tokens, hidden)
    b = f16(rng, hidden)
    t = dev(x)
    ops.add_bias(t, dev(b), hidden, tokens)
    assert np.array_equal(bits(host(t)), bits(O.add_bias(x, b, hidden)))


@pytest.mark.parametrize("n", [5, 4096, 14336 * 4 + 3])
def test_silu_gate(ops, n):
    rng = np.random.default_rng(n)
    g = f16(rng, n, scale=4.0)
    u = f16(rng, n)
    out = dev(np.zeros(n, np.float16))
    ops.silu_gate(dev(g), dev(u), out, n)
    got = host(out)
    assert within_one_ulp(got, O.silu_gate_f32(g, u), f"silu_gate n={n}") > 0.99
    assert np.all(np.abs(got.astype(np.float64) - O.silu_gate_f64(g, u)) <= ulp16(O.silu_gate_f64(g, u)) + 1e-7)


def test_embed_lookup(ops, engine):
    from aether_nexus_amd.types import AW_E_OOB
    from aether_nexus_amd.weaver import WeaverError
    rng = np.random.default_rng(7)
    for hidden in (4096, 100):
        table = f16(rng, 50, hidden)
        ids = rng.integers(0, 50, 9).astype(np.uint32)
        out = dev(np.zeros((9, hidden), np.float16))
        ops.embed_lookup(dev(ids), dev(table), out, hidden, 9)
        ops.check_device_errors()
        assert np.array_equal(bits(host(out)), bits(O.embed_lookup(ids, table, hidden, 50)))
    ids[4] = 50  # one past the table: a zero row and the device error
    out = dev(np.full((9, 100), 7.0, np.float16))
    ops.embed_lookup(dev(ids), dev(table), out, 100, 9)
    with pytest.raises(WeaverError) as e:
        ops.check_device_errors()
    assert e.value.status == AW_E_OOB and "token id" in str(e.value)
    got = host(out)
    assert np.all(got[4] == 0) and np.array_equal(bits(got), bits(O.embed_lookup(ids, table, 100, 50)))
    engine.check_device_errors()  # the word was cleared by the report


@pytest.mark.parametrize("hidden,tokens", [(4096, 16), (2048, 1), (100, 7), (8, 2)])
def test_rms_norm(ops, hidden, tokens):
    rng = np.random.default_rng(hidden + tokens)
    x = f16(rng, tokens, hidden, scale=3.0)
    w = f16(rng, hidden)
    out = dev(np.zeros((tokens, hidden), np.float16))
    ops.rms_norm(dev(x), dev(w), out, hidden, tokens, 1e-5)
    want = O.rms_norm_f32(x, w, 1e-5)
    within_one_ulp(host(out), want, f"rms_norm H={hidden} T={tokens}")
    t = dev(x)  # in place
    ops.rms_norm(t, dev(w), t, hidden, tokens, 1e-5)
    within_one_ulp(host(t), want, "rms_norm in place")


@pytest.mark.parametrize("hidden", [4096, 2056])
def test_rms_norm_aligned_and_unaligned_rows_same_bits(ops, hidden):
    """A row read through 16-byte loads (aligned pointers) and one-half loads
    (pointers 2 bytes off) is summed in the same order: the same output bits."""
    import torch
    rng = np.random.default_rng(hidden)
    tokens = 3
    x = f16(rng, tokens, hidden, scale=3.0)
    w = f16(rng, hidden)
    out = dev(np.zeros((tokens, hidden), np.float16))
    ops.rms_norm(dev(x), dev(w), out, hidden, tokens, 1e-5)
    # The same data at an odd half offset of larger buffers: the element-wise path.
    xb = torch.zeros(tokens * hidden + 1, dtype=torch.float16, device="cuda:0")
    wb = torch.zeros(hidden + 1, dtype=torch.float16, device="cuda:0")
    ob = torch.zeros(tokens * hidden + 1, dtype=torch.float16, device="cuda:0")
    xb[1:] = dev(x).reshape(-1)
    wb[1:] = dev(w)
    ops.rms_norm(xb[1:], wb[1:], ob[1:], hidden, tokens, 1e-5)
    assert xb[1:].data_ptr() % 16 != 0
    assert np.array_equal(bits(host(ob[1:]).reshape(tokens, hidden)), bits(host(out)))


@pytest.mark.parametrize("tokens,hq,hkv,hd,start", [(1, 32, 8, 128, 4095), (16, 32, 8, 128, 100), (3, 4, 0, 64, 0),
                                                     (5, 2, 2, 6, 7)])
def test_rope(ops, tokens, hq, hkv, hd, start):
    rng = np.random.default_rng(tokens * 100 + hd)
    q = f16(rng, tokens, hq, hd)
    k = f16(rng, tokens, max(hkv, 1), hd)
    tq, tk = dev(q), dev(k)
    ops.rope(tq, tk if hkv else None, tokens, hq, hkv, hd, start, 500000.0)
    ex = within_one_ulp(host(tq).reshape(q.shape), O.rope_f32(q, start, 500000.0), f"rope q T={tokens} d={hd}")
    assert ex > 0.99
    if hkv:
        within_one_ulp(host(tk).reshape(k.shape), O.rope_f32(k, start, 500000.0), "rope k")
    else:
        assert np.array_equal(bits(host(tk)), bits(k))  # no k heads: untouched


# M <= 16, 32, 64 take the skinny kernel with 1, 2, 4 row tiles (16 waves up to 4 weight tiles per CU, 8
# beyond: N = 20000 and 49155), larger M the tiled one; K % 8 != 0 the element-wise loads.
# 256 x 128 tiles where they fill the CUs: 1000 x 8200 x 520 (ragged M, N and a partial
# last k-step); 300 x 33000 x 517 (K % 8 != 0) stays on the 128 x 128 tiles.
SHAPES = [(1, 1, 1), (1, 5, 7), (1, 1000, 4096), (3, 33, 64), (16, 1024, 4096), (17, 100, 200), (20, 20000, 64),
          (64, 256, 520), (65, 130, 96), (200, 300, 520), (256, 1024, 4096), (130, 77, 13), (1000, 8200, 520),
          (300, 33000, 517)]


def check_product(got, a, b, k, what, scale=1.0, f16_out=True):
    ref = O.matmul_f64(a, b) * scale
    bound = O.matmul_abs_f64(a, b) * abs(scale) * k * 2.0 ** -24
    g = np.asarray(got, np.float64)
    d = np.abs(g - ref)
    # one f16 ulp of the result (half for the rounding, half for a binade crossed by the fp32 error)
    tol = bound + (ulp16(ref) if f16_out else np.abs(ref) * 2.0 ** -24) + 1e-30
    rel = np.linalg.norm(g - ref) / max(np.linalg.norm(ref), 1e-30)
    print(f"{what}: max |diff| {d.max():.3e}, rel-L2 {rel:.2e}, worst diff/tol {np.max(d / tol):.3f}", flush=True)
    assert np.all(d <= tol) and rel < 1e-3, what


@pytest.mark.parametrize("m,n,k", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_matmul(ops, m, n, k):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = f16(rng, m, k)
    b = f16(rng, n, k, scale=0.05)
    out = dev(np.full((m, n), np.nan, np.float16))
    ops.matmul(dev(a), dev(b), out, m, n, k)
    check_product(host(out).astype(np.float64), a, b, k, f"matmul {m}x{n}x{k}")


# The benchmarked Llama-3.1-8B products (inference.rs:518-600): gate/up at the
# prefill-sized M = 2048 (tiled), down_proj (K = 14336) at M = 1, 16 and 2048.
LLAMA_SHAPES = [(2048, 14336, 4096), (1, 4096, 14336), (16, 4096, 14336), (2048, 4096, 14336)]


@pytest.mark.parametrize("m,n,k", LLAMA_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in LLAMA_SHAPES])
def test_matmul_llama_shapes(ops, m, n, k):
    """Every output column, and every row up to 16 (128 spread rows of the
    M = 2048 products), within the fp32 accumulation bound of the float64 product."""
    rng = np.random.default_rng(m + n + k)
    a = f16(rng, m, k)
    b = f16(rng, n, k, scale=k ** -0.5)
    out = dev(np.full((m, n), np.nan, np.float16))
    print(f"matmul {m}x{n}x{k}", flush=True)
    ops.matmul(dev(a), dev(b), out, m, n, k)
    got = host(out).astype(np.float64)
    rows = np.arange(m) if m <= 16 else np.unique(np.concatenate([np.arange(16), rng.integers(0, m, 112), [m - 1]]))
    assert np.all(np.isfinite(got))
    check_product(got[rows], a[rows], b, k, f"matmul {m}x{n}x{k} ({rows.size} rows)")


@pytest.mark.parametrize("m", [1, 16])
def test_lm_head_scaled_llama(ops, m):
    """The f32 lm_head of Llama-3.1-8B (128256 x 4096, matmul_scaled) at M = 1 and 16."""
    import torch
    rng = np.random.default_rng(128256 + m)
    n, k = 128256, 4096
    a = f16(rng, m, k)
    b = f16(rng, n, k, scale=k ** -0.5)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    print(f"lm_head {m}x{n}x{k}", flush=True)
    ops.matmul_scaled(dev(a), dev(b), out, m, n, k, 1.0)
    check_product(host(out), a, b, k, f"lm_head {m}x{n}x{k}", f16_out=False)


@pytest.mark.parametrize("m,n,k", [(1, 49155, 2048), (4, 1000, 4096), (100, 250, 64)])
def test_matmul_scaled(ops, m, n, k):
    import torch
    rng = np.random.default_rng(n)
    a = f16(rng, m, k)
    b = f16(rng, n, k, scale=0.05)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    ops.matmul_scaled(dev(a), dev(b), out, m, n, k, 1.0 / 6.0)
    check_product(host(out), a, b, k, f"matmul_scaled {m}x{n}x{k}", scale=1.0 / 6.0, f16_out=False)


@pytest.mark.parametrize("m", [1, 5, 16, 17, 33, 64, 65])
def test_fused_products_match_the_separate_calls(ops, m):
    """matmul_add_residual, matmul_silu_gate and matmul_qkv give the bits of the
    calls they fuse (inference.rs:518-600), at every skinny tile count and in the
    tiled range (m = 65: the residual form; the fused gate is refused there)."""
    import torch
    from aether_nexus_amd.types import AW_E_UNSUPPORTED
    from aether_nexus_amd.weaver import WeaverError
    rng = np.random.default_rng(100 + m)
    n, nkv, k = 96, 40, 264
    a = dev(f16(rng, m, k))

    def z(*shape):
        return torch.zeros(shape, dtype=torch.float16, device="cuda:0")
    for mult in (1.0, 0.5):
        b = dev(f16(rng, n, k, scale=0.1))
        x0 = f16(rng, m, n)
        x1, x2, p = dev(x0), dev(x0), z(m, n)
        ops.matmul(a, b, p, m, n, k)
        if mult != 1.0:
            ops.scale_f16(p, m * n, mult)
        ops.add_residual(x1, p, m * n)
        ops.matmul_add_residual(a, b, x2, m, n, k, mult)
        assert torch.equal(x1.view(torch.int16), x2.view(torch.int16)), ("residual", mult)
    bg, bu = dev(f16(rng, n, k, scale=0.1)), dev(f16(rng, n, k, scale=0.1))
    if m <= 64:
        g, u, f1, f2 = z(m, n), z(m, n), z(m, n), z(m, n)
        ops.matmul(a, bg, g, m, n, k)
        ops.matmul(a, bu, u, m, n, k)
        ops.silu_gate(g, u, f1, m * n)
        ops.matmul_silu_gate(a, bg, bu, f2, m, n, k)
        assert torch.equal(f1.view(torch.int16), f2.view(torch.int16)), "silu gate"
    else:
        with pytest.raises(WeaverError) as e:
            ops.matmul_silu_gate(a, bg, bu, z(m, n), m, n, k)
        assert e.value.status == AW_E_UNSUPPORTED
    bq, bk, bv = dev(f16(rng, n, k, scale=0.1)), dev(f16(rng, nkv, k, scale=0.1)), dev(f16(rng, nkv, k, scale=0.1))
    sep = [z(m, n), z(m, nkv), z(m, nkv)]
    for w, o, nn in zip((bq, bk, bv), sep, (n, nkv, nkv)):
        ops.matmul(a, w, o, m, nn, k)
    fused = [z(m, n), z(m, nkv), z(m, nkv)]
    ops.matmul_qkv(a, bq, bk, bv, *fused, m, n, nkv, k)
    for s_, f_ in zip(sep, fused):
        assert torch.equal(s_.view(torch.int16), f_.view(torch.int16)), "qkv"


@pytest.mark.parametrize("k", [520, 517])
def test_wide_and_tiled_products_same_bits(ops, k):
    """Products with many 256 x 128 tiles take gemm_wide_kernel (K % 8 == 0),
    smaller ones the 128 x 128 tiles; both sum the same k-steps of 32 in the same
    order, so the columns a small product shares with a large one have the same
    bits, for the f16 store, the residual form and the scaled fp32 store (K = 520:
    a partial last k-step; K = 517: both on the 128 x 128 tiles)."""
    import torch
    rng = np.random.default_rng(k)
    m, n, ns = 1000, 8200, 96  # 33 x 8 = 264 wide tiles; 96 columns: 8 tiles of 128 x 128
    a = dev(f16(rng, m, k))
    b = f16(rng, n, k, scale=0.05)
    bb, bs = dev(b), dev(b[:ns])
    big, small = torch.zeros((m, n), dtype=torch.float16, device="cuda:0"), torch.zeros((m, ns), dtype=torch.float16, device="cuda:0")
    ops.matmul(a, bb, big, m, n, k)
    ops.matmul(a, bs, small, m, ns, k)
    assert torch.equal(big[:, :ns].contiguous().view(torch.int16), small.view(torch.int16)), "store"
    x0 = f16(rng, m, n)
    xb, xs = dev(x0), dev(np.ascontiguousarray(x0[:, :ns]))
    ops.matmul_add_residual(a, bb, xb, m, n, k, 0.5)
    ops.matmul_add_residual(a, bs, xs, m, ns, k, 0.5)
    assert torch.equal(xb[:, :ns].contiguous().view(torch.int16), xs.view(torch.int16)), "residual"
    fb = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
    fs = torch.zeros((m, ns), dtype=torch.float32, device="cuda:0")
    ops.matmul_scaled(a, bb, fb, m, n, k, 0.25)
    ops.matmul_scaled(a, bs, fs, m, ns, k, 0.25)
    assert torch.equal(fb[:, :ns].contiguous().view(torch.int32), fs.view(torch.int32)), "scaled"


def test_product_bits_do_not_depend_on_the_wave_count(ops):
    """A product takes 16 waves per weight tile when the tiles are few and 8 when
    they are many; the same rows give the same bits either way (the K partial
    sums are added in one fixed order)."""
    import torch
    rng = np.random.default_rng(5)
    k = 1000
    for m in (1, 30):
        a = dev(f16(rng, m, k))
        big = f16(rng, 20000, k, scale=0.05)  # 1250 weight tiles: 8 waves
        small_out = torch.zeros((m, 96), dtype=torch.float16, device="cuda:0")
        big_out = torch.zeros((m, 20000), dtype=torch.float16, device="cuda:0")
        ops.matmul(a, dev(big[:96]), small_out, m, 96, k)  # 6 tiles: 16 waves
        ops.matmul(a, dev(big), big_out, m, 20000, k)
        assert torch.equal(small_out.view(torch.int16), big_out[:, :96].contiguous().view(torch.int16)), m


def test_causal_attention(ops):
    rng = np.random.default_rng(11)
    for kv_len, hd in ((100, 128), (16, 64), (1, 128)):
        cache = (kv_len + 15) // 16 * 16
        q = f16(rng, hd)
        k = f16(rng, cache, hd)
        v = f16(rng, cache, hd)
        out = dev(np.zeros(hd, np.float16))
        ops.causal_attention(dev(q), dev(k), dev(v), out, kv_len, hd)
        ref = AO.multihead_attention_f64(q.reshape(1, 1, hd), k.reshape(cache, 1, hd), v.reshape(cache, 1, hd),
                                         kv_len, 1).reshape(hd)
        got = host(out).astype(np.float64)
        print(f"causal_attention kv_len={kv_len} d={hd}: max |diff| {np.abs(got - ref).max():.2e}", flush=True)
        assert np.abs(got - ref).max() <= 2e-3


def test_ops_reject_bad_arguments(ops):
    import torch
    from aether_nexus_amd.types import AW_E_INVALID_ARG
    from aether_nexus_amd.weaver import WeaverError
    x = torch.zeros(2, 4, 6, dtype=torch.float16, device="cuda:0")
    with pytest.raises(WeaverError) as e:
        ops.rope(x, None, 2, 4, 0, 5, 0, 10000.0)  # odd head_dim
    assert e.value.status == AW_E_INVALID_ARG
    # the host-side count check: 48 elements cannot hold a 7 x 8 operand
    with pytest.raises(WeaverError) as e:
        ops.matmul(x, x, x, 7, 1, 8)
    assert e.value.status == AW_E_INVALID_ARG and "elements" in str(e.value)
    with pytest.raises(WeaverError):
        ops.rms_norm(x.cpu(), x, x, 6, 1, 1e-5)  # a host tensor
    with pytest.raises(WeaverError) as e:
        ops.embed_lookup(torch.zeros(2, dtype=torch.int32, device="cuda:0"), x, x, 6, 2, vocab_size=0)
    assert e.value.status == AW_E_INVALID_ARG


def _layer_f64(x, p, hq, hkv, hd, pos, eps, theta):
    """One decoder layer of forward_batch (inference.rs:505-600) in float64 on
    the CPU, f16 weights, no intermediate rounding: the reference's order of
    norm, projections, rope, cache append, attention, output projection,
    residual, norm, gated MLP and residual."""
    xs = x.astype(np.float64)
    t = xs.shape[0]

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps) * w.astype(np.float64)

    def mm(v, w):
        return v @ w.astype(np.float64).T

    def rope(v, heads):
        v = v.reshape(t, heads, hd)
        ang = (pos + np.arange(t))[:, None, None] * theta ** (-2.0 * np.arange(hd // 2) / hd)[None, None, :]
        z = (v[..., :hd // 2] + 1j * v[..., hd // 2:]) * np.exp(1j * ang)
        return np.concatenate([z.real, z.imag], axis=-1)

    h = rms(xs, p["ln1"])
    q = rope(mm(h, p["wq"]), hq)
    k = rope(mm(h, p["wk"]), hkv)
    v = mm(h, p["wv"]).reshape(t, hkv, hd)
    kc = np.concatenate([p["k_cache"][:pos].astype(np.float64), k])
    vc = np.concatenate([p["v_cache"][:pos].astype(np.float64), v])
    att = AO.multihead_attention_f64(q, kc, vc, pos + t, t).reshape(t, hq * hd)
    xs = xs + mm(att, p["wo"])
    h = rms(xs, p["ln2"])
    g, u = mm(h, p["wg"]), mm(h, p["wu"])
    return xs + mm(g / (1.0 + np.exp(-g)) * u, p["wd"])


def test_decoder_layer_chain(ops):
    """The ops of one forward_batch layer (inference.rs:505-600) chained on one
    stream — rms_norm, q/k/v matmul, rope, copy into the KV cache,
    multihead_attention, o_proj, add_residual, rms_norm, gate/up matmul,
    silu_gate, down matmul, add_residual — against the same layer in float64
    on the CPU: rel-L2 within 1e-2 (f16 storage of every intermediate)."""
    import torch
    rng = np.random.default_rng(21)
    hidden, hq, hkv, hd, inter, t, pos, eps, theta = 256, 4, 2, 64, 512, 4, 28, 1e-5, 10000.0
    cache = 64
    s = 1.0 / np.sqrt(hidden)
    p = {"ln1": f16(rng, hidden, scale=0.2) + np.float16(1), "ln2": f16(rng, hidden, scale=0.2) + np.float16(1),
         "wq": f16(rng, hq * hd, hidden, scale=s), "wk": f16(rng, hkv * hd, hidden, scale=s),
         "wv": f16(rng, hkv * hd, hidden, scale=s), "wo": f16(rng, hidden, hq * hd, scale=s),
         "wg": f16(rng, inter, hidden, scale=s), "wu": f16(rng, inter, hidden, scale=s),
         "wd": f16(rng, hidden, inter, scale=1.0 / np.sqrt(inter)),
         "k_cache": f16(rng, cache, hkv, hd), "v_cache": f16(rng, cache, hkv, hd)}
    x = f16(rng, t, hidden)
    d = {k: dev(v) for k, v in p.items()}
    kv = hkv * hd
    hid, norm = dev(x), dev(np.zeros((t, hidden), np.float16))
    wq, wk, wv = (dev(np.zeros((t, n), np.float16)) for n in (hq * hd, kv, kv))
    att, proj = dev(np.zeros((t, hq * hd), np.float16)), dev(np.zeros((t, hidden), np.float16))
    g, u, f = (dev(np.zeros((t, inter), np.float16)) for _ in range(3))
    down = dev(np.zeros((t, hidden), np.float16))
    ops.rms_norm(hid, d["ln1"], norm, hidden, t, eps)
    ops.matmul(norm, d["wq"], wq, t, hq * hd, hidden)
    ops.matmul(norm, d["wk"], wk, t, kv, hidden)
    ops.matmul(norm, d["wv"], wv, t, kv, hidden)
    ops.rope(wq, wk, t, hq, hkv, hd, pos, theta)
    ops.copy_buffer(wk, d["k_cache"], kv * t, 0, pos * kv)
    ops.copy_buffer(wv, d["v_cache"], kv * t, 0, pos * kv)
    ops.multihead_attention(wq, d["k_cache"], d["v_cache"], att, pos + t, hd, hq, hkv, t)
    ops.matmul(att, d["wo"], proj, t, hidden, hq * hd)
    ops.add_residual(hid, proj, hidden * t)
    ops.rms_norm(hid, d["ln2"], norm, hidden, t, eps)
    ops.matmul(norm, d["wg"], g, t, inter, hidden)
    ops.matmul(norm, d["wu"], u, t, inter, hidden)
    ops.silu_gate(g, u, f, inter * t)
    ops.matmul(f, d["wd"], down, t, hidden, inter)
    ops.add_residual(hid, down, hidden * t)
    ops.end_batch()
    got = host(hid).astype(np.float64)
    want = _layer_f64(x, p, hq, hkv, hd, pos, eps, theta)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    print(f"decoder layer chain: rel-L2 {rel:.2e}, max |diff| {np.abs(got - want).max():.2e}", flush=True)
    assert rel < 1e-2
    assert torch.isfinite(torch.from_numpy(got)).all()
