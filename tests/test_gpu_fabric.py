"""The `.aether` Fabric's pools resident in HBM (include/aether_fabric.h) on
cuda:0: upload and write-back are byte exact, the Weaver decodes straight from
the fabric's device pools (checked against the CPU oracle), and one Distiller
REM cycle (entropy -> candidates -> encode -> write-back -> checkpoint,
distiller.rs:60-120) matches the oracle bit for bit."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from aether_nexus_amd import fabric as F
from aether_nexus_amd.types import AW_E_OOB
from aether_nexus_amd.weaver import WeaverError, make_desc
from oracle import fabric_oracle as FO
from oracle import oracle

pytestmark = pytest.mark.gpu

# kv_heads 2, head_dim 64, 64 atoms per kv head: an 8192-block hot pool of 32 MiB
# (two staging chunks), a 16 MiB cold pool.
SMALL = dict(layers=1, q_heads=4, kv_heads=2, head_dim=64, hidden_size=256, intermediate_size=512, vocab_size=1000,
             block_size=16, sparsity_k=4, dict_size=64)


def booted(tmp_path, name="f.aether"):
    path = tmp_path / name
    F.create_genesis(path, F.model_dims("llama8b", **SMALL))
    return path, F.Fabric(path, F.model_dims("llama8b", **SMALL))


def fill_pools(fab, rng, low=(), zero=(), const=()):
    """Hot rows ~ N(0, 1) (blocks in `low` x 0.1, `zero` all zero, `const` all 0.5);
    unit-norm atoms; codes with atom indices < dict_size and f16 coefficients ~ N(0, 0.5)."""
    hot = rng.standard_normal(fab.hot_pool_blocks().shape, dtype=np.float32)
    hot[list(low)] *= 0.1
    hot[list(zero)] = 0.0
    hot[list(const)] = 0.5
    fab.hot_pool_blocks(writable=True)[...] = hot.astype(np.float16).view(np.uint16)
    dd = rng.standard_normal(fab.dictionary_atoms().shape)
    fab.dictionary_atoms(writable=True)[...] = (dd / np.linalg.norm(dd, axis=-1, keepdims=True)).astype(
        np.float16).view(np.uint16)
    codes = fab.cold_pool_blocks(writable=True)
    codes["indices"] = rng.integers(0, fab.dims.dict_size, codes["indices"].shape)
    codes["coeffs"] = (rng.standard_normal(codes["coeffs"].shape) * 0.5).astype(np.float16)


@pytest.mark.parametrize("hb", [False, True], ids=["file_order", "cold_head_blocked"])
def test_attach_pull_push_roundtrip(tmp_path, hb):
    """Upload, then write-back into a zeroed mapping, gives the original bytes; a
    partial push / pull at odd offsets across two staging chunks too (also with
    the device cold pool kept head-blocked, where copies move whole blocks)."""
    _, fab = booted(tmp_path)
    rng = np.random.default_rng(11)
    orig = {}
    for r in ("hot", "cold", "dict"):
        v = fab.region_mut(r)
        v[...] = rng.integers(0, 256, v.size, dtype=np.uint8)
        orig[r] = v.copy()
    fab.force_checkpoint()
    print(f"fabric: attach hot/cold/dict (cold head-blocked {hb})", flush=True)
    fab.attach_device(0, cold_head_blocked=hb)
    assert fab.cold_head_blocked == hb
    for r in orig:
        ptr, n = fab.device_region(r)
        assert ptr % 256 == 0 and n == orig[r].size
        fab.region_mut(r)[...] = 0
        fab.pull(r)
        assert np.array_equal(fab._view(r, False), orig[r]), r
    hot = fab.region_mut("hot")
    a, n = 12345, hot.size - 12345 - 777
    new = rng.integers(0, 256, n, dtype=np.uint8)
    hot[a:a + n] = new
    fab.push("hot", a, n)
    hot[...] = 0
    fab.pull("hot", a, n)
    assert np.array_equal(hot[a:a + n], new)
    assert not hot[:a].any() and not hot[a + n:].any()
    # The same on the cold pool: ranges that start and end inside a block.
    cold = fab.region_mut("cold")
    a, n = 2048 * 3 + 40, cold.size - 2048 * 7 - 1000
    new = rng.integers(0, 256, n, dtype=np.uint8)
    cold[a:a + n] = new
    fab.push("cold", a, n)
    cold[...] = 0
    fab.pull("cold", a, n)
    assert np.array_equal(cold[a:a + n], new)
    assert not cold[:a].any() and not cold[a + n:].any()
    cold[...] = 0
    fab.pull("cold", 17, 3)  # three bytes of block 0
    assert np.array_equal(cold[17:20], orig["cold"][17:20]) and not cold[:17].any() and not cold[20:].any()
    del cold
    fab.detach_device()
    with pytest.raises(F.FabricError):
        fab.device_region("hot")
    del hot
    fab.close()


def test_decode_from_fabric_pools(tmp_path, engine, stream):
    """aw_decode_desc pointing at the fabric's device pools (hot [8192][16][2][64],
    codes [32768][16][2], one dictionary per kv head) against the f64 oracle on the
    mapped host pools; refs pick scattered blocks, bit 31 set on some.  Then the
    cold pool attached head-blocked: the same output bits."""
    _, fab = booted(tmp_path)
    rng = np.random.default_rng(12)
    fill_pools(fab, rng)
    fab.attach_device(0)
    H, C = 24, 40
    refs = np.concatenate([rng.choice(8192, H, replace=False), rng.choice(32768, C, replace=False)]).astype(np.uint32)
    refs[1::3] |= np.uint32(1 << 31)
    q = (rng.standard_normal((1, 1, 1, 4, 64))).astype(np.float16)
    q_t = torch.from_numpy(q.view(np.int16)).cuda()
    refs_t = torch.from_numpy(refs.view(np.int32)).cuda()
    out_t = torch.empty(4 * 64, dtype=torch.float16, device="cuda:0")
    geom = SimpleNamespace(layers=1, batch=1, queries=1, q_heads=4, kv_heads=2, head_dim=64, dict_size=64,
                           dict_heads=2, hot_count=H, cold_count=C, refs_stride=H + C, causal=False, scale=0.125,
                           hot_blocks=8192, cold_blocks=32768)
    desc = make_desc(layers=1, batch=1, queries=1, q_heads=4, kv_heads=2, head_dim=64, dict_size=64, dict_heads=2,
                     hot_count=H, cold_count=C, refs_stride=H + C, hot_blocks=8192, cold_blocks=32768, q=q_t,
                     out=out_t, hot_k=fab.device_region("hot")[0], cold=fab.device_region("cold")[0], refs=refs_t,
                     dictionary=fab.device_region("dict")[0], scale=0.125)
    print("fabric: decode from the device pools", flush=True)
    engine.decode_device(desc, stream=stream)
    engine.check_device_errors(stream)
    got = out_t.float().cpu().numpy().astype(np.float64)
    arrs = {"q": q.view(np.uint16), "hot_k": fab.hot_pool_blocks()[None], "refs": refs,
            "cold": fab.cold_pool().view(np.uint16).reshape(1, 32768, 16, 2, 8),
            "dictionary": fab.dictionary_atoms()[None]}
    ref = oracle.decode_f64(geom, arrs).reshape(-1)
    err = np.abs(got - ref).max()
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 2e-3 and rel <= 1e-3, (err, rel)
    first = out_t.clone()
    # The fabric's own descriptor: the same bits.
    out_t.zero_()
    engine.decode_device(fab.decode_desc(q_t, out_t, refs_t, hot_count=H, cold_count=C, scale=0.125), stream=stream)
    engine.check_device_errors(stream)
    assert torch.equal(out_t.view(torch.int16), first.view(torch.int16))
    fab.attach_device(0, regions=("cold",), cold_head_blocked=True)
    desc = make_desc(layers=1, batch=1, queries=1, q_heads=4, kv_heads=2, head_dim=64, dict_size=64, dict_heads=2,
                     hot_count=H, cold_count=C, refs_stride=H + C, hot_blocks=8192, cold_blocks=32768, q=q_t,
                     out=out_t, hot_k=fab.device_region("hot")[0], cold=fab.device_region("cold")[0], refs=refs_t,
                     dictionary=fab.device_region("dict")[0], scale=0.125, cold_head_blocked=fab.cold_head_blocked)
    out_t.zero_()
    print("fabric: decode from the head-blocked device cold pool", flush=True)
    engine.decode_device(desc, stream=stream)
    engine.check_device_errors(stream)
    assert torch.equal(out_t.view(torch.int16), first.view(torch.int16))
    out_t.zero_()  # the fabric's descriptor carries the head-blocked flag by itself
    engine.decode_device(fab.decode_desc(q_t, out_t, refs_t, hot_count=H, cold_count=C, scale=0.125), stream=stream)
    engine.check_device_errors(stream)
    assert torch.equal(out_t.view(torch.int16), first.view(torch.int16))
    fab.close()


@pytest.mark.parametrize("hb", [False, True], ids=["file_order", "cold_head_blocked"])
def test_distill_cycle_matches_oracle(tmp_path, engine, hb):
    """One REM cycle on the device copies: every proxy bit-exact, the candidates
    (0 < proxy < 0.15) exactly the low-variance blocks, their codes bit-exact at
    the same cold block index, every other cold block untouched, and the codes
    persisted through a checkpoint and a fresh boot; the file's bytes are the
    same when the device cold pool is kept head-blocked."""
    path, fab = booted(tmp_path)
    rng = np.random.default_rng(13)
    low = sorted(rng.choice(np.arange(8, 8192), 60, replace=False).tolist())
    fill_pools(fab, rng, low=low, zero=(0, 5), const=(7,))
    fab.region_mut("cold")[...] = 0xAB  # untouched blocks keep this pattern
    fab.force_checkpoint()
    fab.attach_device(0, cold_head_blocked=hb)
    print(f"fabric: distill cycle (cold head-blocked {hb})", flush=True)
    n, ent = fab.distill(engine, F.DISTILL_ENTROPY_THRESHOLD)
    hot = fab.hot_pool_blocks()
    want = np.array([oracle.block_entropy(hot[b]) for b in range(8192)], np.float32)
    assert np.array_equal(ent.view(np.uint32), want.view(np.uint32))
    cands = FO.candidates(want, F.DISTILL_ENTROPY_THRESHOLD)
    assert cands == low and n == len(low)  # zero and constant blocks have proxy 0: skipped
    expect = np.full((32768, 16, 2, 8), 0xABAB, np.uint16)
    expect = oracle.encode_blocks(hot, fab.dictionary_atoms(), cands, cold=expect)
    got = fab.cold_pool().view(np.uint16).reshape(32768, 16, 2, 8)
    assert np.array_equal(got, expect)
    fab.force_checkpoint()
    del hot, got
    fab.close()
    with F.Fabric(path, F.model_dims("llama8b", **SMALL)) as again:
        assert np.array_equal(again.cold_pool().view(np.uint16).reshape(32768, 16, 2, 8), expect)


def test_block_entropy_device_lists(engine, stream):
    """aw_block_entropy_device with a block list (bit 31 masked), without one, and
    with an out-of-range block (proxy 0 and the engine's out-of-range flag)."""
    rng = np.random.default_rng(14)
    hot = rng.standard_normal((64, 16, 2, 64)).astype(np.float16)
    hot[9] = 0
    hot_t = torch.from_numpy(hot.view(np.int16)).cuda()
    bits = hot.view(np.uint16)
    want = np.array([oracle.block_entropy(bits[b]) for b in range(64)], np.float32)
    ent = torch.zeros(64, dtype=torch.float32, device="cuda:0")
    engine.block_entropy_device(hot_t, 64, 2, 64, None, 64, ent, stream=stream)
    assert np.array_equal(ent.cpu().numpy().view(np.uint32), want.view(np.uint32))
    lst = np.array([5, 3 | (1 << 31), 63, 9, 0], np.uint32)
    lst_t = torch.from_numpy(lst.view(np.int32)).cuda()
    ent5 = torch.zeros(5, dtype=torch.float32, device="cuda:0")
    engine.block_entropy_device(hot_t, 64, 2, 64, lst_t, 5, ent5, stream=stream)
    assert np.array_equal(ent5.cpu().numpy().view(np.uint32), want[[5, 3, 63, 9, 0]].view(np.uint32))
    engine.check_device_errors(stream)
    bad_t = torch.tensor([64], dtype=torch.int32, device="cuda:0")
    ent1 = torch.full((1,), 7.0, dtype=torch.float32, device="cuda:0")
    engine.block_entropy_device(hot_t, 64, 2, 64, bad_t, 1, ent1, stream=stream)
    assert ent1.item() == 0.0
    with pytest.raises(WeaverError) as e:
        engine.check_device_errors(stream)
    assert e.value.status == AW_E_OOB
