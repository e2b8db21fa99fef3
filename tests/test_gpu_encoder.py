"""GPU parity of the SparseCode encoder (Distiller::distill_block,
distiller.rs:171-246) and the block entropy proxy (distiller.rs:126-159)
against the CPU oracle, bit for bit, through the C ABI (aw_encode_device,
aw_encode) on cuda:0."""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from aether_nexus_amd.types import AW_E_OOB, SPARSE_CODE_DTYPE
from aether_nexus_amd.weaver import WeaverError, make_encode_desc
from oracle import oracle

pytestmark = pytest.mark.gpu


def pools(seed, hot_blocks, hkv, hd, a, dh, zero_dict=False, scale=1.0):
    rng = np.random.default_rng(seed)
    hot = (rng.standard_normal((hot_blocks, 16, hkv, hd)) * scale).astype(np.float16).view(np.uint16)
    if zero_dict:
        d = np.zeros((dh, a, hd), np.uint16)
    else:
        dd = rng.standard_normal((dh, a, hd))
        d = (dd / np.linalg.norm(dd, axis=-1, keepdims=True)).astype(np.float16).view(np.uint16)
    return rng, hot, d


def run_device(engine, stream, hot, d, src, dst, cold0, head_blocked, entropy, full_scan=False):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16 else a).cuda()
    hot_t, d_t = dev(hot), dev(d)
    src_t = torch.from_numpy(np.asarray(src, np.uint32).view(np.int32)).cuda()
    dst_t = None if dst is None else torch.from_numpy(np.asarray(dst, np.uint32).view(np.int32)).cuda()
    cold_t = dev(cold0)
    ent_t = torch.zeros(len(src), dtype=torch.float32, device="cuda:0") if entropy else None
    hkv, hd = hot.shape[2], hot.shape[3]
    desc = make_encode_desc(kv_heads=hkv, head_dim=hd, dict_size=d.shape[1], dict_heads=d.shape[0],
                            hot_blocks=hot.shape[0], cold_blocks=cold0.shape[0], hot=hot_t, dictionary=d_t,
                            src_blocks=src_t, dst_blocks=dst_t, cold=cold_t, entropy=ent_t,
                            cold_head_blocked=head_blocked, full_scan=full_scan)
    engine.encode_device(desc, stream=stream)
    engine.check_device_errors(stream)
    cold = cold_t.cpu().numpy().view(np.uint16)
    return cold, (None if ent_t is None else ent_t.cpu().numpy())


@pytest.mark.parametrize("hkv,hd,a,dh,head_blocked", [
    (8, 128, 512, 8, False),    # the reference geometry (Llama8B, per-kv-head dictionary)
    (8, 128, 4096, 1, False),   # the benchmark dictionary (4096 atoms, shared)
    (2, 64, 256, 2, True),
    (4, 64, 528, 1, True),      # dict_size not a power of two
])
def test_encode_device_bit_exact(engine, stream, hkv, hd, a, dh, head_blocked):
    rng, hot, d = pools(11, 24, hkv, hd, a, dh)
    src = rng.permutation(24)[:9]
    dst = rng.permutation(30)[:9]
    shape = (30, hkv, 16, 8) if head_blocked else (30, 16, hkv, 8)
    cold0 = rng.integers(0, 65535, shape, dtype=np.uint16)
    got, ent = run_device(engine, stream, hot, d, src, dst, cold0, head_blocked, True)
    want, went = oracle.encode_blocks(hot, d, src, dst=dst, cold=cold0.copy(), head_blocked=head_blocked, entropy=True)
    assert (got == want).all(), f"{int((got != want).any(axis=-1).sum())} codes differ"
    assert (ent.view(np.uint32) == went.view(np.uint32)).all()


def test_encode_zero_dictionary_picks_first_atoms(engine, stream):
    """distiller.rs:286-310: equal scores keep atoms 0, 1, 2, 3."""
    rng, hot, d = pools(12, 3, 8, 128, 512, 8, zero_dict=True)
    cold0 = np.zeros((3, 16, 8, 8), np.uint16)
    got, _ = run_device(engine, stream, hot, d, [0, 1, 2], None, cold0, False, False)
    assert (got[..., :4] == np.array([0, 1, 2, 3], np.uint16)).all()
    want = oracle.encode_blocks(hot, d, [0, 1, 2])
    assert (got == want).all()


def test_encode_entropy_edge_blocks(engine, stream):
    """All-zero block -> 0 (also with -0.0), constant block -> 0, tiny and large values."""
    rng, hot, d = pools(13, 4, 4, 64, 256, 4)
    hot[0] = 0
    hot[1] = 0x8000
    hot[2] = np.float16(1.0).view(np.uint16)
    hot[3] = (rng.standard_normal(hot[3].shape) * 1e-4).astype(np.float16).view(np.uint16)
    cold0 = np.zeros((4, 16, 4, 8), np.uint16)
    got, ent = run_device(engine, stream, hot, d, [0, 1, 2, 3], None, cold0, False, True)
    _, went = oracle.encode_blocks(hot, d, [0, 1, 2, 3], entropy=True)
    assert ent[0] == 0 and ent[1] == 0 and ent[2] == 0
    assert (ent.view(np.uint32) == went.view(np.uint32)).all()


def test_entropy_sequential_fallback_blocks(engine, stream):
    """Blocks outside the exact-sum case (sum of magnitudes >= 2^29, inf, NaN, -inf)
    in the same waves as ordinary blocks: every proxy bit-exact against the
    oracle's sequential f64 sums, except that a NaN proxy only has to be NaN (the
    sign of a NaN that inf - inf creates is the platform's: negative on the
    oracle's x86, positive on ARM, where the reference runs, and on this GPU; the
    candidate rule 0 < e < 0.15 rejects either)."""
    rng = np.random.default_rng(15)
    nb = 40
    hot = (rng.standard_normal((nb, 16, 8, 128)) * 3).astype(np.float16)
    hot[3] = (np.sign(rng.standard_normal(hot[3].shape)) * 60000).astype(np.float16)  # |sum| >= 2^29
    hot[7, 5, 2, 9] = np.inf
    hot[20, 0, 0, 0] = np.nan
    hot[21, 15, 7, 127] = -np.inf
    big = rng.standard_normal(hot[33].shape) * 30000  # past 65504: infinities of both signs
    hot[33] = np.where(np.abs(big) > 65504, np.copysign(np.inf, big), big).astype(np.float16)
    bits = hot.view(np.uint16)
    want = np.array([oracle.block_entropy(bits[b]) for b in range(nb)], np.float32)
    hot_t = torch.from_numpy(bits.view(np.int16)).cuda()
    ent = torch.zeros(nb, dtype=torch.float32, device="cuda:0")
    print("encoder: entropy fallback blocks", flush=True)
    engine.block_entropy_device(hot_t, nb, 8, 128, None, nb, ent, stream=stream)
    engine.check_device_errors(stream)
    got = ent.cpu().numpy()
    nan = np.isnan(want)
    assert nan[[7, 20, 21, 33]].all() and np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), np.nonzero(got != want)
    assert want[3] > 1e9  # the 2^29 case took the sequential sums


def test_encode_host_slices(engine):
    """aw_encode: copy in, encode, copy back; hot block b -> cold block b."""
    rng, hot, d = pools(14, 6, 8, 128, 512, 8)
    cold = np.zeros(6 * 16 * 8, dtype=SPARSE_CODE_DTYPE)
    ent = engine.encode(hot, d, [4, 1], cold, kv_heads=8, head_dim=128, dict_size=512, dict_heads=8, entropy=True)
    want, went = oracle.encode_blocks(hot, d, [4, 1], cold=np.zeros((6, 16, 8, 8), np.uint16), entropy=True)
    assert (cold.view(np.uint16).reshape(6, 16, 8, 8) == want).all()
    assert (ent.view(np.uint32) == went.view(np.uint32)).all()


def test_encode_bad_block_reported(engine, stream):
    """A source block past the hot pool is skipped and reported (AW_E_OOB);
    the host form rejects it before launch."""
    rng, hot, d = pools(15, 2, 4, 64, 256, 4)
    cold0 = np.zeros((2, 16, 4, 8), np.uint16)
    with pytest.raises(WeaverError) as e:
        run_device(engine, stream, hot, d, [0, 7], None, cold0, False, False)
    assert e.value.status == AW_E_OOB
    cold = np.zeros((2, 16, 4, 8), np.uint16)
    with pytest.raises(WeaverError) as e:
        engine.encode(hot, d, [5], cold, kv_heads=4, head_dim=64, dict_size=256, dict_heads=4)
    assert e.value.status == AW_E_OOB


def _unit(rng, shape):
    dd = rng.standard_normal(shape)
    return (dd / np.linalg.norm(dd, axis=-1, keepdims=True)).astype(np.float16)


@pytest.mark.parametrize("case", ["subnormal_atoms", "subnormal_tokens", "inf_nan", "near_ties", "overflow_ties",
                                  "dict_80", "dict_16"])
def test_encode_prefilter_matches_full_scan(engine, stream, case):
    """The MFMA prefilter with exact rescoring against the plain exact scan
    (AW_F_ENCODE_FULL_SCAN) and the oracle, bit for bit, on inputs built to
    stress it: subnormal components (the bound's flush slack, the token
    fallback), inf / NaN components (always-candidate atoms, fallback tokens),
    atoms one f16 ulp apart (MFMA and exact orders disagree), more tied atoms
    than the candidate list holds (overflow fallback), and dictionary sizes
    that leave a partial 64-atom chunk."""
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    hkv, hd, a, nb = 4, 128, 256, 6
    if case == "dict_80":
        hd, a = 64, 80
    if case == "dict_16":
        a = 16
    hot = rng.standard_normal((nb, 16, hkv, hd)).astype(np.float16)
    d = _unit(rng, (hkv, a, hd))
    if case == "subnormal_atoms":
        mask = rng.random(d.shape) < 0.05
        d[mask] = (rng.choice([-1, 1], mask.sum()) * rng.integers(1, 1024, mask.sum()) * 2.0 ** -24).astype(np.float16)
    elif case == "subnormal_tokens":
        mask = rng.random(hot.shape) < 0.01
        hot[mask] = np.float16(2.0 ** -20)
    elif case == "inf_nan":
        d[0, 7, 3] = np.inf
        d[1, 9, 0] = np.nan
        d[2, 11, 5] = -np.inf
        hot[1, 3, 0, 10] = np.nan
        hot[2, 5, 1, 20] = np.inf
        hot[3, 0, 3, :] = np.float16(-np.inf)
    elif case == "near_ties":
        # Atoms close to the tokens' best directions, and copies of them one ulp apart.
        x = hot[:, :, 0, :].reshape(-1, hd).astype(np.float32)
        best = x[rng.choice(x.shape[0], 8, replace=False)]
        base = (best / np.linalg.norm(best, axis=-1, keepdims=True)).astype(np.float16)
        for h in range(hkv):
            for k in range(8):
                d[h, 8 * k] = base[k]
                for j in range(1, 8):
                    v = base[k].view(np.uint16).copy()
                    v[rng.integers(0, hd)] += np.uint16(1)
                    d[h, 8 * k + j] = v.view(np.float16)
    elif case == "overflow_ties":
        d[:, 40:80] = d[:, 3:4]  # 41 identical atoms
    hb = hot.view(np.uint16)
    db = d.view(np.uint16)
    src = rng.permutation(nb)
    cold0 = np.zeros((nb, 16, hkv, 8), np.uint16)
    got, _ = run_device(engine, stream, hb, db, src, None, cold0.copy(), False, False)
    scan, _ = run_device(engine, stream, hb, db, src, None, cold0.copy(), False, False, full_scan=True)
    want = oracle.encode_blocks(hb, db, src, cold=cold0.copy())
    assert (scan == want).all()
    assert (got == want).all(), f"{int((got != want).any(axis=-1).sum())} codes differ"
