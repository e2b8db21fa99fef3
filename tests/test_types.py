"""Layout contract (CPU only): SparseCode and WeaverParams as the reference
defines them (nexus-core/src/types.rs:150-244, 351-396, tests :516-606), the
ctypes mirrors against the compiled library, and the bit-exact binary16
conversions of the oracle against numpy."""
from __future__ import annotations

import ctypes

import numpy as np

from aether_nexus_amd import types as T
from oracle import oracle


def test_sparse_code_known_answer_bytes():
    """types.rs:547-557: indices [1,42,255,511], coeffs [0.5,-0.25,1.0,0.0]."""
    b = T.code_bytes([1, 42, 255, 511], [0.5, -0.25, 1.0, 0.0])
    assert b == bytes([0x01, 0x00, 0x2A, 0x00, 0xFF, 0x00, 0xFF, 0x01,
                       0x00, 0x38, 0x00, 0xB4, 0x00, 0x3C, 0x00, 0x00])
    idx, coef = T.unpack_codes(np.frombuffer(b, dtype="<u2").reshape(1, 8))
    assert idx.tolist() == [[1, 42, 255, 511]]
    assert coef.astype(np.float32).tolist() == [[0.5, -0.25, 1.0, 0.0]]


def test_sparse_code_size_alignment_and_zero():
    """types.rs:227-228, 537-541: 16 bytes, align 16, default is all-zero bytes."""
    assert T.SPARSE_CODE_DTYPE.itemsize == 16
    assert ctypes.sizeof(T.CSparseCode) == 16
    z = np.zeros(1, T.SPARSE_CODE_DTYPE)
    assert z.tobytes() == bytes(16)
    assert T.SPARSE_CODE_DTYPE.fields["coeffs"][1] == 8


def test_weaver_params_layout():
    """types.rs:351-374: 12 x u32 in reference order; types.rs:563-579 values."""
    p = T.WeaverParams(q_heads=32, kv_heads=8, head_dim=128, block_size=16, gqa_group=4, hot_count=100,
                       cold_count=500, dict_size=512, sparsity_k=4)
    raw = bytes(p)
    assert len(raw) == 48
    assert np.frombuffer(raw, "<u4").tolist() == [32, 8, 128, 16, 4, 100, 500, 512, 4, 0, 0, 0]
    assert T.WeaverParams.hot_count.offset == 20 and T.WeaverParams.sparsity_k.offset == 32


def test_model_dims_and_from_loom():
    assert T.Llama8B.gqa_group() == 4  # types.rs:593-597
    assert T.Llama8B.hidden_size() == 4096
    assert (T.Qwen05B.Q_HEADS, T.Qwen05B.KV_HEADS, T.Qwen05B.HEAD_DIM) == (14, 2, 64)
    p = T.WeaverParams.from_loom(T.Llama8B, T.LoomDescriptor(hot_count=7, cold_count=9))
    assert p.as_dict() == {"q_heads": 32, "kv_heads": 8, "head_dim": 128, "block_size": 16, "gqa_group": 4,
                           "hot_count": 7, "cold_count": 9, "dict_size": 512, "sparsity_k": 4}


def test_pack_unpack_round_trip():
    rng = np.random.default_rng(0)
    idx = rng.integers(0, 65536, size=(100, 4))
    coef = rng.normal(0, 1, size=(100, 4)).astype(np.float16)
    i2, c2 = T.unpack_codes(T.pack_codes(idx, coef))
    np.testing.assert_array_equal(i2, idx)
    np.testing.assert_array_equal(c2.view(np.uint16), coef.view(np.uint16))


def test_f16_to_f32_exhaustive():
    """Every one of the 65536 binary16 patterns, against numpy (NaN payloads
    compared as NaN)."""
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.h2f(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    """Random floats over the whole range plus every tie point and boundary,
    against numpy's IEEE round-to-nearest-even."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200_000) * np.exp2(rng.uniform(-30, 20, 200_000))).astype(np.float32)
    halves = np.arange(0, 0x7C00, dtype=np.uint32)
    lo = halves.astype(np.uint16).view(np.float16).astype(np.float32)
    hi = (halves + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    ties = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    edges = np.array([65504, 65519.99, 65520, 65536, 1e9, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                      2.9802326e-08, 0.0, -0.0, np.inf, -np.inf], dtype=np.float32)
    allx = np.concatenate([x, -x, ties, -ties, edges])
    with np.errstate(over="ignore"):
        expect = allx.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.f2h(allx), expect)
    assert np.all(np.isnan(oracle.f2h(np.array([np.nan], np.float32)).view(np.float16)))
