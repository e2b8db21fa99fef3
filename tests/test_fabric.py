"""The `.aether` Fabric on the CPU (include/aether_fabric.h): region map,
genesis, boot and its errors, looms, host views, dirty tracking and
checkpoints.  The product (aether_nexus_amd/csrc/fabric.hip) is checked
against the oracle restatement (oracle/fabric_oracle.py), which the first tests
pin to the reference's own tests and published numbers."""
from __future__ import annotations

import os
import struct
import time

import numpy as np
import pytest

from aether_nexus_amd import fabric as F
from aether_nexus_amd.types import (AW_E_BAD_MAGIC, AW_E_IO, AW_E_TOO_SMALL, AW_E_UNSUPPORTED, AW_E_VERSION,
                                    LoomDescriptor)
from oracle import fabric_oracle as FO

# A small geometry: the fixed regions (observation buffers, trace) still make
# the file ~435 MB, almost all of it holes.
SMALL = dict(layers=1, q_heads=4, kv_heads=2, head_dim=64, hidden_size=256, intermediate_size=512, vocab_size=1000,
             block_size=16, sparsity_k=4, dict_size=64)


def dims(d: dict):
    return F.model_dims("llama8b", **d)


@pytest.fixture
def genesis(tmp_path):
    path = tmp_path / "small.aether"
    F.create_genesis(path, dims(SMALL))
    return path


# ------------------------------------------------------------ oracle pins


def test_oracle_regions_pinned_by_reference():
    """The oracle's layout against what the reference fixes independently."""
    # align_up (fabric.rs:868-874).
    assert [FO.align_up(v, a) for v, a in ((0, 16384), (1, 16384), (16384, 16384), (16385, 16384), (100, 4096))] == \
        [0, 16384, 16384, 32768, 4096]
    r = FO.compute_regions(FO.PRESETS["llama8b"])
    # Boot log of the Llama8B fabric: "Hot pool: 256 MB | Cold pool: 64 MB | Dict: 1024 KB"
    # (docs/walkthrough.md.resolved:70).
    assert (r["hot_pool_size"], r["cold_pool_size"], r["dict_size"]) == (256 << 20, 64 << 20, 1024 << 10)
    # The weight estimate is 2 bytes per parameter x 1.25.  Llama-3.1-8B has
    # 8,030,261,248 parameters, of which the untied lm_head is 128256 x 4096 and is
    # not among the tensors the estimate sums (embedding, per-layer projections, norms).
    params = 8_030_261_248 - 128256 * 4096
    assert FO.estimated_weight_bytes(FO.PRESETS["llama8b"]) == 2 * params + (2 * params) // 4
    for name, d in FO.PRESETS.items():
        r = FO.compute_regions(d)
        # 16 KiB alignment (fabric.rs:756-796) and no overlap (fabric.rs:798-809).
        for k in ("weights_offset", "hot_pool_offset", "cold_pool_offset", "dict_offset", "obs_offset",
                  "trace_offset", "total_size"):
            assert r[k] % 16384 == 0, (name, k)
        order = ("weights", "hot_pool", "cold_pool", "dict", "looms", "radix", "obs", "trace")
        for a, b in zip(order, order[1:]):
            assert r[f"{a}_offset"] + r[f"{a}_size"] <= r[f"{b}_offset"], (name, a, b)
        assert r["trace_offset"] + r["trace_size"] + FO.SIGNATURE_LEN <= r["total_size"]


def test_oracle_parse_looms_known_bytes():
    """parse_looms on hand-made bytes: persona bytes 2, 7 (unknown: Planner), 0, 3
    and little-endian fields."""
    raw = bytearray(128)
    raw[0], raw[32], raw[64], raw[96] = 2, 7, 0, 3
    struct.pack_into("<5I", raw, 4, 1, 2, 3, 4, 5)
    struct.pack_into("<5I", raw, 36, 0x01020304, 0, 0, 0, 0xFFFFFFFF)
    got = FO.parse_looms(bytes(raw))
    assert got == [(2, 1, 2, 3, 4, 5), (0, 0x01020304, 0, 0, 0, 0xFFFFFFFF), (0, 0, 0, 0, 0, 0), (3, 0, 0, 0, 0, 0)]


# ------------------------------------------------------------ product vs oracle


@pytest.mark.parametrize("name", sorted(FO.PRESETS))
def test_regions_match_oracle(name):
    assert F.compute_regions(F.model_dims(name)).as_dict() == FO.compute_regions(FO.PRESETS[name])


def test_regions_random_dims_match_oracle():
    rng = np.random.default_rng(5)
    for _ in range(200):
        d = dict(layers=int(rng.integers(1, 128)), q_heads=int(rng.integers(1, 128)),
                 kv_heads=int(rng.integers(1, 64)), head_dim=int(rng.choice([32, 64, 96, 128, 256])),
                 hidden_size=int(rng.integers(1, 16384)), intermediate_size=int(rng.integers(1, 65536)),
                 vocab_size=int(rng.integers(1, 300000)), block_size=16, sparsity_k=4,
                 dict_size=int(rng.integers(1, 65536)))
        assert F.compute_regions(dims(d)).as_dict() == FO.compute_regions(d), d


def test_regions_overflow_rejected():
    with pytest.raises(F.FabricError):
        F.compute_regions(dims(dict(SMALL, hidden_size=4_000_000_000, intermediate_size=4_000_000_000,
                                    layers=4_000_000_000)))


def test_presets_and_params_from_loom():
    for name, d in FO.PRESETS.items():
        got = F.model_dims(name)
        assert {k: getattr(got, k) for k in d} == d
    with pytest.raises(F.FabricError):
        F.model_dims("gpt2")
    loom = LoomDescriptor(persona=1, hot_count=256, cold_count=2048, token_pos=77)
    p = F.weaver_params_from_loom(F.model_dims("llama8b"), loom)
    want = FO.params_from_loom(FO.PRESETS["llama8b"], loom.as_tuple())
    assert {k: getattr(p, k) for k in want} == want
    assert want["gqa_group"] == 4  # types.rs:601-604: 32 q heads / 8 kv heads


def test_genesis_bytes_and_boot(genesis):
    """create_genesis -> boot (fabric.rs:812-866): the file is zero except the
    header and the persona bytes; the looms read Planner, Coder, Critic, Reviewer;
    the cold pool reads as zero SparseCodes."""
    r = FO.compute_regions(SMALL)
    assert genesis.stat().st_size == r["total_size"]
    data = np.memmap(genesis, np.uint8, "r")
    expect = FO.genesis_bytes(SMALL)
    for off, b in expect.items():
        assert bytes(data[off:off + len(b)]) == b, off
    assert int(np.count_nonzero(data)) == sum(np.count_nonzero(np.frombuffer(b, np.uint8)) for b in expect.values())
    del data
    with F.Fabric(genesis, dims(SMALL)) as fab:
        assert fab.regions.as_dict() == r
        assert [lm.as_tuple() for lm in fab.looms] == [(i, 0, 0, 0, 0, 0) for i in range(4)]
        codes = fab.cold_pool_codes()
        assert codes.size == r["cold_pool_size"] // 16
        assert not codes["indices"].any() and not codes["coeffs"].view(np.uint16).any()
        assert not fab.dirty


def test_llama8b_genesis_roundtrip(tmp_path):
    """The reference's genesis -> boot round trip on its own geometry (fabric.rs:812-841,
    Llama8B: an 18.6 GB file, almost all holes): personas in order, zero codes at both
    ends of the cold pool, the header bytes, and the regions of the layout."""
    d = F.model_dims("llama8b")
    path = tmp_path / "llama8b.aether"
    F.create_genesis(path, d)
    r = FO.compute_regions(FO.PRESETS["llama8b"])
    assert path.stat().st_size == r["total_size"]
    with open(path, "rb") as fh:
        assert fh.read(13) == FO.MAGIC + struct.pack("<I", FO.FORMAT_VERSION)
        for i in range(4):
            fh.seek(r["looms_offset"] + 32 * i)
            assert fh.read(32) == bytes([i]) + bytes(31)
    with F.Fabric(path, d) as fab:
        assert fab.regions.as_dict() == r
        assert [lm.persona for lm in fab.looms] == [0, 1, 2, 3]
        codes = fab.cold_pool_codes()
        assert codes.size == 32768 * 16 * 8
        assert not codes[:64].view(np.uint16).any() and not codes[-64:].view(np.uint16).any()
        assert fab.hot_pool_blocks().shape == (8192, 16, 8, 128)
        assert fab.dictionary_atoms().shape == (8, 512, 128)
    path.unlink()


def test_boot_errors(genesis, tmp_path):
    """FabricError cases of boot_with_mode (fabric.rs:273-344), with the reference's messages."""
    d = dims(SMALL)
    total = FO.compute_regions(SMALL)["total_size"]
    with pytest.raises(F.FabricError) as e:
        F.Fabric(tmp_path / "missing.aether", d)
    assert e.value.status == AW_E_IO and "(os error 2)" in str(e.value)
    os.truncate(genesis, total - 1)
    with pytest.raises(F.FabricError) as e:
        F.Fabric(genesis, d)
    assert e.value.status == AW_E_TOO_SMALL
    assert f"file too small: expected at least {total} bytes, got {total - 1}" in str(e.value)
    os.truncate(genesis, total + 4096)  # larger files boot (only a short file is an error)
    F.Fabric(genesis, d).close()
    with open(genesis, "r+b") as fh:
        fh.write(b"AETHER1.2")
    with pytest.raises(F.FabricError) as e:
        F.Fabric(genesis, d)
    assert e.value.status == AW_E_BAD_MAGIC and "invalid magic bytes" in str(e.value)
    with open(genesis, "r+b") as fh:
        fh.write(b"AETHER1.3" + struct.pack("<I", 0x00010002))
    with pytest.raises(F.FabricError) as e:
        F.Fabric(genesis, d)
    assert e.value.status == AW_E_VERSION
    assert "version mismatch: expected 0x00010003, got 0x00010002" in str(e.value)
    with open(genesis, "r+b") as fh:
        fh.seek(9)
        fh.write(struct.pack("<I", 0x00010003))
    with pytest.raises(F.FabricError) as e:  # BootMode::Verified: Ed25519 is not implemented here
        F.Fabric(genesis, d, public_key=bytes(32))
    assert e.value.status == AW_E_UNSUPPORTED
    F.Fabric(genesis, d).close()


def test_looms_parsed_like_the_reference(genesis):
    r = FO.compute_regions(SMALL)
    rng = np.random.default_rng(3)
    raw = bytearray(rng.integers(0, 256, 128, dtype=np.uint8).tobytes())
    raw[0], raw[32], raw[64], raw[96] = 3, 200, 1, 4
    with open(genesis, "r+b") as fh:
        fh.seek(r["looms_offset"])
        fh.write(raw)
    with F.Fabric(genesis, dims(SMALL)) as fab:
        got = [lm.as_tuple() for lm in fab.looms]
        assert got == FO.parse_looms(bytes(raw))
        for lm, want in zip(fab.looms, got):
            p = F.weaver_params_from_loom(fab.dims, lm)
            assert (p.hot_count, p.cold_count) == want[1:3]


def test_views_dirty_and_checkpoints(genesis):
    """Accessors mark the fabric dirty as the reference's mutable ones do;
    checkpoint flushes only when dirty and >= 300 ms after the last flush;
    force_checkpoint always flushes; the writes reach the file."""
    r = FO.compute_regions(SMALL)
    fab = F.Fabric(genesis, dims(SMALL))
    booted = time.monotonic()
    hot = fab.hot_pool()
    assert hot.size == r["hot_pool_size"] and not hot.flags.writeable
    assert fab.hot_pool_blocks().shape == (8192, 16, 2, 64)
    assert fab.cold_pool_blocks().shape == (32768, 16, 2)
    assert fab.dictionary_atoms().shape == (2, 64, 64)
    trace = fab.trace_log_mut()
    trace[:4] = [1, 2, 3, 4]
    assert not fab.dirty  # trace_log_mut does not mark (fabric.rs:416-421)
    cold = fab.cold_pool_mut()
    assert fab.dirty
    cold[:16] = 7
    fab.checkpoint()  # < 300 ms since boot: nothing flushed
    if time.monotonic() - booted < 0.2:  # a loaded host can take longer to get here
        assert fab.dirty
    time.sleep(0.35)
    fab.checkpoint()
    assert not fab.dirty
    fab.checkpoint()  # clean: a no-op
    obs = fab.observation_bufs_mut()
    assert fab.dirty
    obs[-1] = 9
    fab.force_checkpoint()
    assert not fab.dirty
    del hot, trace, cold, obs
    fab.close()
    with open(genesis, "rb") as fh:
        fh.seek(r["cold_pool_offset"])
        assert fh.read(17) == bytes([7] * 16 + [0])
        fh.seek(r["obs_offset"] + r["obs_size"] - 1)
        assert fh.read(1) == b"\x09"
        fh.seek(r["trace_offset"])
        assert fh.read(4) == bytes([1, 2, 3, 4])
    with F.Fabric(genesis, dims(SMALL)) as fab:
        assert fab.cold_pool_codes()["indices"][0].tolist() == [0x0707] * 4


def test_device_calls_need_attach(genesis):
    with F.Fabric(genesis, dims(SMALL)) as fab:
        with pytest.raises(F.FabricError):
            fab.device_region("hot")
        with pytest.raises(F.FabricError):
            fab.push("hot", 0, 16)
        with pytest.raises(F.FabricError):
            fab.pull("cold", 0, 16)
