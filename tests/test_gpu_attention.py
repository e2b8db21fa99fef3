"""The Weaver as the inference loop's attention on cuda:0:
aw_multihead_attention_device (Ops::multihead_attention, ops.metal:528-616)
against the f64 oracle, token-granular hot pools in a batched decode
(AW_F_SEQ_HOT_TOKENS), and a speculative-verify step through KvCache
(multi-query verify equals one query at a time; rejected drafts rolled back)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aether_nexus_amd import inference as I
from aether_nexus_amd.types import AW_E_INVALID_ARG
from aether_nexus_amd.weaver import WeaverError, make_desc
from oracle import attention_oracle as AO

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-3, 1e-3


def assert_close(got, ref, what=""):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref).max() if ref.size else 0.0
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= MAX_ABS and rel <= REL_L2, (what, err, rel)


def cache_case(seed, nq, kv_len, hq, hkv, d, cap):
    """Random f16 q and caches; cache rows past kv_len hold NaN (stale memory the
    attention must neither score nor read as values)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((nq, hq, d)).astype(np.float16)
    k = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    v = rng.standard_normal((cap, hkv, d)).astype(np.float16)
    k[kv_len:] = np.nan
    v[kv_len:] = np.nan
    return q, k, v


@pytest.mark.parametrize("nq,kv_len,hq,hkv,d", [
    (1, 0, 8, 2, 64),        # an empty cache: zeros
    (1, 1, 32, 8, 128),      # one cached token
    (1, 17, 32, 8, 128),     # one token into the second block
    (4, 100, 32, 8, 128),    # verify of 3 drafts, partial last block
    (16, 4096, 32, 8, 128),  # MAX_BATCH new tokens at MAX_SEQ_LEN
    (3, 5000, 32, 8, 128),   # past the reference's 4096-score limit
    (4, 131072, 32, 8, 128), # 8192 blocks: the reference Fabric's whole hot region (types.rs:500)
    (16, 37, 14, 2, 64),     # G = 7: queries in two groups of <= 9
    (16, 15, 8, 8, 64),      # query 0 sees nothing (zeros), query 1 sees position 0
])
def test_multihead_attention_matches_oracle(engine, stream, nq, kv_len, hq, hkv, d):
    cap = -(-kv_len // 16) * 16 + 16
    q, k, v = cache_case(nq * 7919 + kv_len, nq, kv_len, hq, hkv, d, cap)
    qt, kt, vt = (torch.from_numpy(x.view(np.int16)).cuda() for x in (q, k, v))
    out = torch.full((nq, hq, d), float("nan"), dtype=torch.float16, device="cuda:0")
    print(f"attention: nq {nq} kv_len {kv_len} heads {hq}/{hkv} d {d}", flush=True)
    engine.multihead_attention(qt, kt, vt, out, kv_len, d, hq, hkv, nq, cache_tokens=cap, stream=stream)
    engine.check_device_errors(stream)
    ref = AO.multihead_attention_f64(q, k[:kv_len], v[:kv_len], kv_len, nq)
    assert_close(out.float().cpu().numpy(), ref, (nq, kv_len))


def test_multihead_attention_rejects_bad_requests(engine, stream):
    q = torch.zeros((4, 8, 64), dtype=torch.float16, device="cuda:0")
    kc = torch.zeros((32, 2, 64), dtype=torch.float16, device="cuda:0")
    out = torch.empty_like(q)
    with pytest.raises(WeaverError) as e:  # the new tokens are not all in the cache
        engine.multihead_attention(q, kc, kc, out, 2, 64, 8, 2, 4, stream=stream)
    assert e.value.status == AW_E_INVALID_ARG
    with pytest.raises(WeaverError) as e:  # kv_len 33 reads block 2 (tokens 32..47) of a 32-token cache
        engine.multihead_attention(q, kc, kc, out, 33, 64, 8, 2, 4, stream=stream)
    assert e.value.status == AW_E_INVALID_ARG and "cache" in str(e.value)


def test_decode_seq_hot_tokens(engine, stream):
    """Batched causal decode with per-sequence hot TOKEN counts (AW_F_SEQ_HOT_TOKENS)
    over scattered blocks (bit 31 set on some refs), each sequence against the
    oracle on its blocks gathered into a contiguous cache; with hot_tokens capping
    every sequence too."""
    rng = np.random.default_rng(31)
    B, Q, hq, hkv, d, hc = 3, 2, 8, 2, 64, 4
    n_tok = np.array([5, 33, 64], np.uint32)
    pool_blocks = 16
    k = rng.standard_normal((pool_blocks, 16, hkv, d)).astype(np.float16)
    v = rng.standard_normal((pool_blocks, 16, hkv, d)).astype(np.float16)
    refs = rng.permutation(pool_blocks)[:B * hc].astype(np.uint32).reshape(B, hc)
    for b in range(B):  # stale rows past each sequence's end
        for t in range(int(n_tok[b]), hc * 16):
            k[refs[b, t // 16], t % 16] = np.nan
            v[refs[b, t // 16], t % 16] = np.nan
    tagged = refs.copy()
    tagged[:, 1::2] |= np.uint32(1 << 31)
    q = rng.standard_normal((B, Q, hq, d)).astype(np.float16)
    kt, vt, qt = (torch.from_numpy(x.view(np.int16)).cuda() for x in (k, v, q))
    rt = torch.from_numpy(tagged.view(np.int32)).cuda()
    st = torch.from_numpy(n_tok.view(np.int32)).cuda()
    scale = 1.0 / np.sqrt(d)
    for cap in (0, 40):
        out = torch.full((B, Q, hq, d), float("nan"), dtype=torch.float16, device="cuda:0")
        desc = make_desc(layers=1, batch=B, queries=Q, q_heads=hq, kv_heads=hkv, head_dim=d, dict_size=16,
                         dict_heads=1, hot_count=hc, cold_count=0, refs_stride=hc, hot_blocks=pool_blocks,
                         cold_blocks=0, q=qt, out=out, hot_k=kt, hot_v=vt, refs=rt, seq_hot=st, scale=scale,
                         causal=True, hot_tokens=cap, seq_hot_tokens=True)
        print(f"attention: decode with seq_hot tokens {n_tok.tolist()} cap {cap}", flush=True)
        engine.decode_device(desc, stream=stream)
        engine.check_device_errors(stream)
        got = out.float().cpu().numpy()
        for b in range(B):
            n = int(min(n_tok[b], cap or n_tok[b]))
            kc = k[refs[b]].reshape(hc * 16, hkv, d)
            vc = v[refs[b]].reshape(hc * 16, hkv, d)
            ref = AO.multihead_attention_f64(q[b], kc[:n], vc[:n], n, Q)  # its scale is 1/sqrt(d) too
            assert_close(got[b], ref, (b, n, cap))


def test_speculative_verify_step(engine, stream):
    """KvCache over 2 layers (Llama-3.1-8B heads): a 40-token prompt, then a verify
    step of last_token + 3 drafts in one multi-query call.  Each of its rows
    equals a one-query call over the cache cut at that token; the accept rule then
    rolls the position back to the kept tokens."""
    rng = np.random.default_rng(41)
    hq, hkv, d, layers = 32, 8, 128, 2
    cache = I.KvCache(layers, hkv, d, max_seq_len=256)
    dev = "cuda:0"

    def rows(n):
        return torch.from_numpy(rng.standard_normal((n, hkv, d)).astype(np.float16)).to(dev)

    for chunk in (16, 16, 8):  # prompt in forward_batch-sized pieces
        for layer in range(layers):
            cache.append(layer, rows(chunk), rows(chunk))
        cache.advance(chunk)
    p0 = cache.push_loom()
    assert p0 == 40
    nv = 4
    q = torch.from_numpy(rng.standard_normal((nv, hq, d)).astype(np.float16)).to(dev)
    for layer in range(layers):
        cache.append(layer, rows(nv), rows(nv))
    outs = []
    for layer in range(layers):
        out = torch.empty((nv, hq, d), dtype=torch.float16, device=dev)
        cache.attend(engine, layer, q, out, stream=stream)
        outs.append(out)
    engine.check_device_errors(stream)
    for layer in range(layers):
        kc = cache.k[layer][:p0 + nv].cpu().numpy()
        vc = cache.v[layer][:p0 + nv].cpu().numpy()
        ref = AO.multihead_attention_f64(q.cpu().numpy(), kc, vc, p0 + nv, nv)
        assert_close(outs[layer].float().cpu().numpy(), ref, ("verify", layer))
        for i in range(nv):  # one query at a time: token p0 + i is the newest
            one = torch.empty((1, hq, d), dtype=torch.float16, device=dev)
            engine.multihead_attention(q[i:i + 1], cache.k[layer], cache.v[layer], one, p0 + i + 1, d, hq, hkv, 1,
                                       cache_tokens=cache.capacity, stream=stream)
            assert_close(one[0].float().cpu().numpy(), outs[layer][i].double().cpu().numpy(), ("step", i))
    cache.advance(nv)
    logits = np.zeros((nv, 10), np.float32)
    logits[[0, 1, 2, 3], [6, 2, 9, 1]] = 1.0
    new = I.accept_drafts([6, 3, 4], logits)
    assert new == [6, 2]
    cache.pop_loom(I.rollback_position(cache.push_loom(), 3, len(new)))
    assert cache.position == p0 + 2


@pytest.mark.parametrize("seed", range(16))
def test_multihead_attention_random_shapes(engine, stream, seed):
    """Seeded random shapes: 1-16 new tokens, 0-3000 cached positions, GQA groups
    1-8, head_dim 64 or 128, the cache's capacity 0-40 tokens past the last
    block read; NaN in every row past kv_len."""
    rng = np.random.default_rng(500 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 4, 7, 8]))
    d = int(rng.choice([64, 128]))
    nq = int(rng.integers(1, 17))
    kv_len = int(rng.integers(nq - 1, 3001))
    cap = -(-kv_len // 16) * 16 + int(rng.integers(0, 41))
    q, k, v = cache_case(9000 + seed, nq, kv_len, hq, hkv, d, max(cap, 1))
    qt, kt, vt = (torch.from_numpy(x.view(np.int16)).cuda() for x in (q, k, v))
    out = torch.full((nq, hq, d), float("nan"), dtype=torch.float16, device="cuda:0")
    print(f"attention random {seed}: nq {nq} kv_len {kv_len} cap {cap} heads {hq}/{hkv} d {d}", flush=True)
    engine.multihead_attention(qt, kt, vt, out, kv_len, d, hq, hkv, nq, cache_tokens=cap, stream=stream)
    engine.check_device_errors(stream)
    ref = AO.multihead_attention_f64(q, k[:kv_len], v[:kv_len], kv_len, nq)
    assert_close(out.float().cpu().numpy(), ref, (seed, nq, kv_len))


def decompress_cold(cold_hb, dictionary):
    """Cold rows in f64 from the head-blocked pool [blocks][kv_heads][16][8 words]
    and dictionaries [dict_heads][A][d]: row (block*16 + t, g) = sum_k c_k D_g[idx_k]."""
    w = cold_hb.cpu().numpy().view(np.uint16)
    nb, hkv = w.shape[0], w.shape[1]
    idx = w[..., :4].astype(np.int64)                                  # [nb][hkv][16][4]
    coef = w[..., 4:].copy().view(np.float16).astype(np.float64)       # [nb][hkv][16][4]
    dic = dictionary.cpu().numpy().astype(np.float64)                   # [dh][A][d]
    rows = np.zeros((nb, 16, hkv, dic.shape[-1]))
    for g in range(hkv):
        dg = dic[g if dic.shape[0] > 1 else 0]
        rows[:, :, g, :] = np.einsum("btk,btkd->btd", coef[:, g], dg[idx[:, g]])
    return rows.reshape(nb * 16, hkv, -1)


def hot_rows(cache, layer, n_hot):
    """The hot tier's K and V rows in token order, from the block ring."""
    ks, vs = [], []
    for i in range(-(-n_hot // 16)):
        slot = (cache.hot_first + i) % cache.hot_capacity
        ks.append(cache.k[layer][slot])
        vs.append(cache.v[layer][slot])
    k = torch.cat(ks)[:n_hot].float().cpu().numpy()
    v = torch.cat(vs)[:n_hot].float().cpu().numpy()
    return k, v


def test_weaver_kv_cache_verify_step(engine, stream):
    """WeaverKvCache at Llama-3.1-8B heads over 2 layers with the reference's
    512-atom per-kv-head dictionaries: a 34816-token prompt leaves 2048 hot and
    32768 cold tokens (distilled by aw_encode_device); a verify step of
    last_token + 3 drafts then runs one hot+cold aw_decode_device per layer.  Each
    layer's rows match the fp64 brute force over [decompressed cold rows; hot K/V
    rows] (decode_f64's math on the same pools: a cold token is sum_k c_k D[idx_k]
    as key and value), every row equals a one-query step, and a kept draft rolls
    the position back."""
    hq, hkv, d, layers, A, n = 32, 8, 128, 2, 512, 34816
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(44)
    dd = torch.randn((layers, hkv, A, d), generator=gen, device="cuda:0", dtype=torch.float64)
    dicts = (dd / dd.norm(dim=-1, keepdim=True)).to(torch.float16)
    cache = I.WeaverKvCache(layers, hkv, d, dicts, hot_window=2048, max_seq_len=40000)
    ks = [torch.randn((n, hkv, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    vs = [torch.randn((n, hkv, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    print("weaver cache: prompt of 34816 tokens", flush=True)
    cache.extend(engine, ks, vs, stream=stream)
    engine.check_device_errors(stream)
    assert (cache.cold_tokens, cache.hot_tokens()) == (32768, 2048)
    p0, nv = cache.position, 4
    q = torch.randn((nv, hq, d), generator=gen, device="cuda:0").to(torch.float16)
    new_k = [torch.randn((nv, hkv, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    new_v = [torch.randn((nv, hkv, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    outs = []
    for layer in range(layers):
        cache.append(layer, new_k[layer], new_v[layer])
        out = torch.full((nv, hq, d), float("nan"), dtype=torch.float16, device="cuda:0")
        cache.attend(engine, layer, q, out, stream=stream)
        outs.append(out)
    engine.check_device_errors(stream)
    qn = q.float().cpu().numpy()
    for layer in range(layers):
        cold = decompress_cold(cache.cold[layer][:cache.cold_blocks], dicts[layer])
        hk, hv = hot_rows(cache, layer, 2048 + nv)
        ref = AO.multihead_attention_f64(qn, np.concatenate([cold, hk]), np.concatenate([cold, hv]), p0 + nv, nv)
        assert_close(outs[layer].float().cpu().numpy(), ref, ("tiered verify", layer))
    cache.advance(nv)
    for i in range(nv):  # one query at a time: token p0 + i is the newest
        cache.pop_loom(p0)
        if i:
            cache.advance(i)
        for layer in range(layers):
            one = torch.empty((1, hq, d), dtype=torch.float16, device="cuda:0")
            cache.attend(engine, layer, q[i:i + 1], one, stream=stream)
            assert_close(one[0].float().cpu().numpy(), outs[layer][i].double().cpu().numpy(), ("tiered step", i))
    cache.pop_loom(p0)
    cache.advance(nv)
    logits = np.zeros((nv, 10), np.float32)
    logits[[0, 1, 2, 3], [6, 2, 9, 1]] = 1.0
    new = I.accept_drafts([6, 3, 4], logits)
    cache.pop_loom(I.rollback_position(cache.push_loom(), 3, len(new)))
    assert cache.position == p0 + 2 and cache.cold_tokens == 32768
    del ks, vs
    torch.cuda.empty_cache()



def _tiered_cache(engine, stream, gen, layers, n, q_latent_f32=True, max_seq_len=None):
    """A WeaverKvCache at Llama-3.1-8B heads with 512-atom per-kv-head unit-norm
    dictionaries, loaded with an n-token prompt (2048 stay hot) on `stream`."""
    hkv, d, A = 8, 128, 512
    dd = torch.randn((layers, hkv, A, d), generator=gen, device="cuda:0", dtype=torch.float64)
    dicts = (dd / dd.norm(dim=-1, keepdim=True)).to(torch.float16)
    cache = I.WeaverKvCache(layers, hkv, d, dicts, hot_window=2048, max_seq_len=max_seq_len or n + 256,
                            q_latent_f32=q_latent_f32)
    ks = [torch.randn((n, hkv, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    vs = [torch.randn((n, hkv, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    torch.cuda.synchronize()  # the inputs, made on torch's current stream, before `stream` reads them
    cache.extend(engine, ks, vs, stream=stream)
    engine.check_device_errors(stream)
    torch.cuda.synchronize()
    return cache, dicts


def test_weaver_kv_cache_peaked_verify_fp32_q_latent(engine, stream):
    """A verify step (last token + 3 drafts) over WeaverKvCache on a peaked
    softmax: cold codes with coefficient std 6 (written straight into the cold
    tier) and q std 2, 32768 cold + 2048 hot tokens.  With q_latent kept fp32
    (the cache's default) every output is within 2e-3 of the fp64 brute force
    beyond its own f16 rounding (outputs reach several units, where that rounding
    alone approaches 2e-3) and rel-L2 within 1e-3; the reference's f16 q_latent
    (q_latent_f32=False) is measured beside it and misses by more."""
    hq, hkv, d, A, nv, nb = 32, 8, 128, 512, 4, 2048
    results = {}
    for f32 in (True, False):
        gen = torch.Generator(device="cuda:0")
        gen.manual_seed(52)
        cache, dicts = _tiered_cache(engine, stream, gen, 1, 2048, q_latent_f32=f32, max_seq_len=40000)
        # 2048 cold blocks of random codes (indices uniform, coefficients ~ N(0, 36))
        # become the oldest tokens, in front of the 2048 hot ones.
        idx = torch.randint(0, A, (nb, hkv, 16, 4), generator=gen, device="cuda:0", dtype=torch.int32)
        coef = (torch.randn((nb, hkv, 16, 4), generator=gen, device="cuda:0") * 6.0).to(torch.float16)
        cache.cold[0][:nb] = torch.cat([idx.to(torch.int16), coef.view(torch.int16)], dim=-1)
        cache.cold_blocks = nb
        cache.position += nb * 16
        q = (torch.randn((nv, hq, d), generator=gen, device="cuda:0") * 2.0).to(torch.float16)
        rows = torch.randn((nv, hkv, d), generator=gen, device="cuda:0").to(torch.float16)
        cache.append(0, rows, rows, stream=stream)
        out = torch.full((nv, hq, d), float("nan"), dtype=torch.float16, device="cuda:0")
        print(f"tiered peaked verify, q_latent {'fp32' if f32 else 'f16'}", flush=True)
        cache.attend(engine, 0, q, out, stream=stream)
        engine.check_device_errors(stream)
        p = cache.position
        coldr = decompress_cold(cache.cold[0][:nb], dicts[0])
        hk, hv = hot_rows(cache, 0, cache.hot_tokens(p + nv))
        ref = AO.multihead_attention_f64(q.float().cpu().numpy(), np.concatenate([coldr, hk]),
                                         np.concatenate([coldr, hv]), p + nv, nv)
        got = out.float().cpu().numpy().astype(np.float64)
        half_ulp = np.spacing(np.abs(got).astype(np.float16)).astype(np.float64) / 2
        excess = np.abs(got - ref) - half_ulp
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        results[f32] = (np.abs(got - ref).max(), excess.max(), rel)
        print(f"  max |out| {np.abs(ref).max():.2f}, max-abs {results[f32][0]:.2e}, beyond f16 rounding "
              f"{results[f32][1]:.2e}, rel-L2 {rel:.2e}", flush=True)
        del cache
    assert results[True][1] <= 2e-3 and results[True][2] <= 1e-3
    assert results[True][0] < results[False][0]


def test_weaver_kv_cache_side_stream(engine):
    """Every call of WeaverKvCache on a stream other than torch's current one
    (prompt with ring writes, a distill after each forward that frees a ring slot,
    appends that reuse it, attends), with no synchronisation in between: the
    outputs are the bits of the same calls on the current stream."""
    hq, d, layers, n, steps = 32, 128, 2, 2048 + 16 * 40, 40
    outs = {}
    for mode in ("current", "side"):
        gen = torch.Generator(device="cuda:0")
        gen.manual_seed(61)
        side = torch.cuda.Stream()
        sh = side.cuda_stream if mode == "side" else torch.cuda.current_stream().cuda_stream
        cache, _ = _tiered_cache(engine, sh, gen, layers, n, max_seq_len=n + 16 * (steps + 1))
        qs = [torch.randn((16, hq, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(steps)]
        rows = [torch.randn((16, 8, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(steps)]
        got = [torch.empty((16, hq, d), dtype=torch.float16, device="cuda:0") for _ in range(steps * layers)]
        torch.cuda.synchronize()
        print(f"tiered cache on the {mode} stream: {steps} forwards of 16 tokens", flush=True)
        for i in range(steps):  # a block leaves the window after each forward
            for layer in range(layers):
                cache.append(layer, rows[i], rows[i], stream=sh)
                cache.attend(engine, layer, qs[i], got[i * layers + layer], stream=sh)
            cache.advance(16)
            cache.distill(engine, stream=sh)
        torch.cuda.synchronize()
        engine.check_device_errors(sh)
        assert cache.cold_tokens == 16 * 80
        outs[mode] = torch.stack(got).view(torch.int16)
        del cache
    assert torch.equal(outs["side"], outs["current"])


def test_weaver_kv_cache_background_distill(engine, stream):
    """The Distiller's pass beside the decode: a block leaving the hot window is
    encoded on a side stream (queued behind other work there, so it is still in
    flight) while verify steps run on the main stream.  Every output is the bits
    of a cache where no pass ran (the block still hot) or of one distilled
    synchronously (the block cold), never anything else; while the pass is in
    flight it is the former, and after the commit the latter."""
    hq, d, layers, nv = 32, 128, 2, 4
    side = torch.cuda.Stream()
    caches = []
    for _ in range(3):  # a: background pass; b0: never distilled; b1: distilled synchronously
        gen = torch.Generator(device="cuda:0")
        gen.manual_seed(71)
        caches.append(_tiered_cache(engine, stream, gen, layers, 34816)[0])
    a, b0, b1 = caches
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(72)
    rows = [torch.randn((16, 8, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(layers)]
    qs = [torch.randn((nv, hq, d), generator=gen, device="cuda:0").to(torch.float16) for _ in range(6)]
    for c in caches:  # 16 more tokens: one block beyond the window
        for layer in range(layers):
            c.append(layer, rows[layer], rows[layer], stream=stream)
        c.advance(16)
    assert b1.distill(engine, stream=stream) == 1
    torch.cuda.synchronize()
    # Keep the side stream busy so that the pass is still queued when the decodes run.
    x = torch.randn((4096, 4096), generator=gen, device="cuda:0")
    x = torch.tanh(x @ x * 1e-3)  # the product's library set-up, before the timed queue
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        for _ in range(40):
            x = torch.tanh(x @ x * 1e-3)
    print("background distill: one block per layer queued on a busy side stream", flush=True)
    assert a.distill(engine, stream=stream, side_stream=side.cuda_stream) == 1
    assert a.distilling == 1 and a.cold_tokens == 32768

    def step(c, q):
        outs = []
        for layer in range(layers):
            c.append(layer, rows[layer][:nv], rows[layer][:nv], stream=stream)
            out = torch.empty((nv, hq, d), dtype=torch.float16, device="cuda:0")
            c.attend(engine, layer, q, out, stream=stream)
            outs.append(out)
        p = c.push_loom()
        c.advance(nv)
        c.pop_loom(p)  # a rejected verify step
        return [o.view(torch.int16) for o in outs]

    in_flight = 0
    for i, q in enumerate(qs):
        if i == 3:
            a.commit(wait=True)
        pending = a.distilling
        oa, o0, o1 = step(a, q), step(b0, q), step(b1, q)
        for layer in range(layers):
            same0, same1 = torch.equal(oa[layer], o0[layer]), torch.equal(oa[layer], o1[layer])
            assert same0 or same1, f"step {i} layer {layer}: output of neither state"
            if not pending:
                assert same1, f"step {i}: committed, yet not the distilled cache's output"
        in_flight += pending > 0 and a.distilling > 0
    torch.cuda.synchronize()
    engine.check_device_errors(stream)
    print(f"background distill: {in_flight} steps ran with the pass in flight", flush=True)
    assert in_flight >= 1 and a.distilling == 0 and a.cold_tokens == 32768 + 16
    assert (a.cold_tokens, a.hot_first) == (b1.cold_tokens, b1.hot_first)
