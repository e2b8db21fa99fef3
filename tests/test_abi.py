"""The C ABI without a GPU (CPU only): the library loads, exports every
function include/*.h declares, its structs match the ctypes
mirrors, and the host-side validation and planning behave as documented.
No compute entry point is called."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from aether_nexus_amd import _lib
from aether_nexus_amd import workloads as W
from aether_nexus_amd.types import (AW_E_ALIGN, AW_PROJECT_AUTO, AW_PROJECT_MFMA, AW_PROJECT_VALU, AW_E_INVALID_ARG, AW_E_OOB, AW_E_UNSUPPORTED, SPARSE_CODE_DTYPE,
                                    STRUCT_SIZES, DecodeDesc, PlanInfo, WeaverParams)
from aether_nexus_amd.weaver import WeaverError, plan, validate_params

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"#define[^\n]*", "", text)
        names |= set(re.findall(r"\b(aw_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert len(HEADERS) >= 2 and len(names) >= 40
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_struct_sizes_match():
    lib = _lib.load()
    sizes = (ctypes.c_size_t * 4)()
    lib.aw_abi_struct_sizes(sizes)
    assert tuple(sizes) == STRUCT_SIZES == (16, 48, ctypes.sizeof(DecodeDesc), ctypes.sizeof(PlanInfo))
    assert lib.aw_abi_version() == 2
    assert lib.aw_status_string(AW_E_OOB).decode().startswith("block ref")


def params(**kw):
    p = dict(q_heads=32, kv_heads=8, head_dim=128, block_size=16, gqa_group=4, hot_count=2, cold_count=1,
             dict_size=512, sparsity_k=4)
    p.update(kw)
    return WeaverParams(**p)


def good_args(p):
    n_hot = max(p.hot_count, 1) * 16 * p.kv_heads * p.head_dim
    cold = np.zeros(max(p.cold_count, 1) * 16 * p.kv_heads, SPARSE_CODE_DTYPE)
    refs = np.arange(p.hot_count + p.cold_count, dtype=np.uint32)
    refs[p.hot_count:] -= p.hot_count  # cold refs count from block 0 of the cold pool
    return dict(n_q_exact=p.q_heads * p.head_dim, n_q_latent=p.q_heads * p.dict_size, n_hot_pool=n_hot,
                cold_pool=cold, loom_refs=refs, n_dictionary=p.kv_heads * p.dict_size * p.head_dim,
                n_out=p.q_heads * p.head_dim)


def test_validate_accepts_reference_shapes():
    p = params()
    validate_params(p, **good_args(p))
    p0 = params(hot_count=0, cold_count=0)
    validate_params(p0, n_q_exact=4096, n_q_latent=0, n_hot_pool=0, cold_pool=None, loom_refs=None, n_dictionary=0,
                    n_out=4096)


@pytest.mark.parametrize("change,code", [
    (dict(gqa_group=3), AW_E_INVALID_ARG),
    (dict(block_size=32), AW_E_UNSUPPORTED),
    (dict(sparsity_k=8), AW_E_UNSUPPORTED),
    (dict(head_dim=96), AW_E_UNSUPPORTED),
    (dict(dict_size=100), AW_E_UNSUPPORTED),
])
def test_validate_rejects_bad_params(change, code):
    p = params(**change)
    args = good_args(params())
    with pytest.raises(WeaverError) as e:
        validate_params(p, **args)
    assert e.value.status == code


def test_validate_rejects_short_buffers_and_bad_refs():
    p = params()
    args = good_args(p)
    for k in ("n_q_exact", "n_q_latent", "n_dictionary", "n_out"):
        bad = dict(args)
        bad[k] = args[k] - 1
        with pytest.raises(WeaverError) as e:
            validate_params(p, **bad)
        assert e.value.status == AW_E_INVALID_ARG, k
    refs = args["loom_refs"].copy()
    refs[0] = 2  # hot pool holds 2 blocks
    with pytest.raises(WeaverError) as e:
        validate_params(p, **{**args, "loom_refs": refs})
    assert e.value.status == AW_E_OOB
    refs = args["loom_refs"].copy()
    refs[0] = 1 | (1 << 31)  # bit 31 is masked: still block 1
    validate_params(p, **{**args, "loom_refs": refs})
    cold = args["cold_pool"].copy()
    cold["indices"][5, 2] = 512  # atom index == dict_size
    with pytest.raises(WeaverError) as e:
        validate_params(p, **{**args, "cold_pool": cold})
    assert e.value.status == AW_E_OOB


def test_validate_rejects_misaligned_codes():
    lib = _lib.load()
    p = params()
    args = good_args(p)
    buf = np.zeros(args["cold_pool"].nbytes + 32, np.uint8)
    off = (-buf.ctypes.data) % 16 + 8  # 8 bytes past a 16-byte boundary
    refs = args["loom_refs"]
    msg = ctypes.create_string_buffer(256)
    rc = lib.aw_validate_params(ctypes.byref(p), args["n_q_exact"], args["n_q_latent"], args["n_hot_pool"],
                                buf.ctypes.data + off, args["cold_pool"].size, refs.ctypes.data, refs.size,
                                args["n_dictionary"], args["n_out"], msg, 256)
    assert rc == AW_E_ALIGN


def test_plan_splits_and_workspace():
    """aw_decode_plan: geometry checks and the split plan for the benchmark shapes."""
    out = np.zeros(1, np.uint16)
    g = W.hot_cold(batch=64)
    d = W.make_desc if hasattr(W, "make_desc") else None
    from aether_nexus_amd.weaver import make_desc
    desc = make_desc(layers=1, batch=64, queries=1, q_heads=32, kv_heads=8, head_dim=128, dict_size=4096,
                     dict_heads=1, hot_count=g.hot_count, cold_count=g.cold_count, refs_stride=g.refs_stride,
                     hot_blocks=g.hot_blocks, cold_blocks=g.cold_blocks, q=1, out=1)
    info = plan(desc)
    assert info.rows_per_kv_head == 4
    assert info.hot_splits >= 1 and info.hot_tokens_per_split % 32 == 0
    assert info.hot_splits * info.hot_tokens_per_split >= g.hot_count * 16
    assert info.cold_splits >= 1 and info.cold_splits * info.cold_tokens_per_split >= g.cold_count * 16
    assert info.cold_row_chunk == 4 and info.computes_q_latent == 1
    assert info.workspace_bytes > 0
    del out, d
    bad = make_desc(layers=1, batch=1, queries=20, q_heads=32, kv_heads=8, head_dim=128, dict_size=4096,
                    dict_heads=1, hot_count=1, cold_count=0, refs_stride=1, hot_blocks=1, cold_blocks=0, q=1, out=1)
    with pytest.raises(WeaverError) as e:  # 4 heads x 20 queries = 80 rows per kv head > 64
        plan(bad)
    assert e.value.status == AW_E_UNSUPPORTED


def test_plan_small_batch_fills_cus():
    """Few sequences: the cold plan halves the row chunk and adds splits until the
    work-groups (items x splits) cover the 256 CUs, within the partial-bins bound
    (A*rc*4 bytes per split <= half the sequence's code bytes); one-row chunks take
    half a round (B = 1: 32 items x 4 splits)."""
    from aether_nexus_amd.weaver import make_desc
    for B, want_rc, want_splits in ((1, 1, 4), (4, 2, 4), (16, 4, 2), (64, 4, 1)):
        g = W.hot_cold(batch=B)
        info = plan(make_desc(layers=1, batch=B, queries=1, q_heads=32, kv_heads=8, head_dim=128, dict_size=4096,
                              dict_heads=1, hot_count=g.hot_count, cold_count=g.cold_count,
                              refs_stride=g.refs_stride, hot_blocks=g.hot_blocks, cold_blocks=g.cold_blocks,
                              q=1, out=1))
        assert (info.cold_row_chunk, info.cold_splits) == (want_rc, want_splits), B
        items = B * 8 * (4 // info.cold_row_chunk)
        assert items * info.cold_splits >= (128 if info.cold_row_chunk == 1 else 256)
        assert 4096 * info.cold_row_chunk * 4 * 2 <= info.cold_tokens_per_split * info.cold_splits * 16


def test_plan_full_hot_region():
    """The reference's whole hot region, MAX_HOT_BLOCKS = 8192 blocks (types.rs:500),
    plans at Llama-8B geometry with and without a cold pool, and so does a
    131072-token contiguous cache; the limit is 64 splits of 4096 blocks."""
    from aether_nexus_amd.weaver import make_desc
    for hot, cold, B in ((4097, 0, 1), (8192, 0, 1), (8192, 2048, 1), (8192, 2048, 4), (8192, 0, 64)):
        info = plan(make_desc(layers=1, batch=B, queries=1, q_heads=32, kv_heads=8, head_dim=128,
                              dict_size=4096 if cold else 0, dict_heads=1, hot_count=hot, cold_count=cold,
                              refs_stride=hot + cold, hot_blocks=hot, cold_blocks=max(cold, 1), q=1, out=1))
        assert 1 <= info.hot_splits <= 64, (hot, cold, B)
        assert info.hot_tokens_per_split % 32 == 0 and info.hot_tokens_per_split <= 4096 * 16
        assert info.hot_splits * info.hot_tokens_per_split >= hot * 16
        assert (info.hot_splits - 1) * info.hot_tokens_per_split < hot * 16  # no empty split
    # Causal verify step over a 131072-token cache (aw_multihead_attention_device's decode).
    info = plan(make_desc(layers=1, batch=1, queries=4, q_heads=32, kv_heads=8, head_dim=128, dict_size=0,
                          dict_heads=1, hot_count=8192, cold_count=0, refs_stride=8192, hot_blocks=8192,
                          cold_blocks=0, q=1, out=1, causal=True, hot_tokens=131072))
    assert info.hot_splits == 64 and info.hot_tokens_per_split == 2048
    top = 64 * 4096
    info = plan(make_desc(layers=1, batch=1, queries=1, q_heads=32, kv_heads=8, head_dim=128, dict_size=0,
                          dict_heads=1, hot_count=top, cold_count=0, refs_stride=top, hot_blocks=top,
                          cold_blocks=0, q=1, out=1))
    assert info.hot_splits == 64 and info.hot_tokens_per_split == 4096 * 16
    with pytest.raises(WeaverError) as e:
        plan(make_desc(layers=1, batch=1, queries=1, q_heads=32, kv_heads=8, head_dim=128, dict_size=0,
                       dict_heads=1, hot_count=top + 1, cold_count=0, refs_stride=top + 1, hot_blocks=top + 1,
                       cold_blocks=0, q=1, out=1))
    assert e.value.status == AW_E_UNSUPPORTED and "4096 blocks" in str(e.value)


def test_plan_cold_output():
    """The cold kernel writes value partials for dictionary heads of at most
    128 KiB of f16 (512 atoms at head_dim 128, 1024 at 64) and bins elsewhere; the
    value path's workspace holds no bins and no D^T, its hot partial arrays hold
    the cold splits too, and a pool past the buffer-load window keeps bins."""
    from aether_nexus_amd.types import AW_COLD_OUT_BINS, AW_COLD_OUT_VALUES
    from aether_nexus_amd.weaver import make_desc

    def info(A, hd=128, dh=8, B=1, cold_blocks=None, hot=128, cold=2048):
        return plan(make_desc(layers=1, batch=B, queries=1, q_heads=32, kv_heads=8, head_dim=hd, dict_size=A,
                              dict_heads=dh, hot_count=hot, cold_count=cold, refs_stride=hot + cold,
                              hot_blocks=hot * B, cold_blocks=cold_blocks or cold * B, q=1, out=1))
    v, b = info(512), info(4096, dh=1)
    assert v.cold_output == AW_COLD_OUT_VALUES and b.cold_output == AW_COLD_OUT_BINS
    assert info(1024, hd=64).cold_output == AW_COLD_OUT_VALUES
    assert info(1024).cold_output == AW_COLD_OUT_BINS and info(528).cold_output == AW_COLD_OUT_BINS
    assert info(512, B=64).cold_output == AW_COLD_OUT_VALUES
    # Hot splits hold >= 64 tokens (2048 hot tokens: 32 splits) beside either cold output.
    # The value path's scratch: q_latent (f16), D^T, and the partials of every hot and
    # cold split (m, l, 128 floats per row).
    assert (v.cold_splits, v.hot_splits) == (4, 32) and b.hot_splits == 32
    rows = 8 * 4
    parts = rows * (v.hot_splits + v.cold_splits)
    assert v.workspace_bytes <= 32 * 512 * 2 + 8 * (512 + 64) * 128 * 2 + parts * (2 * 4 + 128 * 4) + 5 * 4096
    # A dictionary size that is not a multiple of 32 atoms keeps bins (the product's k-steps).
    assert info(496).cold_output == AW_COLD_OUT_BINS and info(480).cold_output == AW_COLD_OUT_VALUES
    # A cold pool over the 4 GiB window of buffer loads (2^21 blocks x 8 kv heads x 16 codes x 16 B).
    assert info(512, cold_blocks=1 << 21).cold_output == AW_COLD_OUT_BINS
    # No cold pool: neither.
    assert info(0, dh=1, cold=0).cold_output == 0


def test_plan_flags():
    """The head-blocked cold layout plans like the reference layout; unknown flag bits are rejected."""
    from aether_nexus_amd.types import AW_E_INVALID_ARG, AW_F_CAUSAL, AW_F_COLD_HEAD_BLOCKED
    from aether_nexus_amd.weaver import make_desc
    g = W.hot_cold(batch=64)
    kw = dict(layers=1, batch=64, queries=1, q_heads=32, kv_heads=8, head_dim=128, dict_size=4096, dict_heads=1,
              hot_count=g.hot_count, cold_count=g.cold_count, refs_stride=g.refs_stride, hot_blocks=g.hot_blocks,
              cold_blocks=g.cold_blocks, q=1, out=1)
    ref = plan(make_desc(**kw))
    hb = plan(make_desc(**kw, cold_head_blocked=True))
    assert (hb.cold_splits, hb.cold_tokens_per_split, hb.workspace_bytes) == \
        (ref.cold_splits, ref.cold_tokens_per_split, ref.workspace_bytes)
    assert AW_F_COLD_HEAD_BLOCKED == 2 and AW_F_CAUSAL == 1
    bad = make_desc(**kw)
    bad.flags = 4
    with pytest.raises(WeaverError) as e:
        plan(bad)
    assert e.value.status == AW_E_INVALID_ARG


def test_descriptors_keep_their_tensors_alive():
    """A descriptor holds raw addresses, so it keeps the tensors behind them
    alive: a temporary (a pool reordered for the call) is not returned to
    torch's cache while the descriptor, or a graph captured from it, may still
    read it."""
    import gc
    import weakref
    import torch
    from aether_nexus_amd.weaver import make_desc, make_encode_desc
    reordered = torch.zeros(64, 16, 8, 8, dtype=torch.int16).permute(0, 2, 1, 3).contiguous()
    ref = weakref.ref(reordered)
    d = make_desc(layers=1, batch=1, queries=1, q_heads=32, kv_heads=8, head_dim=128, dict_size=4096, dict_heads=1,
                  hot_count=0, cold_count=64, refs_stride=64, hot_blocks=0, cold_blocks=64, q=1, out=1,
                  cold=reordered)
    del reordered
    gc.collect()
    assert ref() is not None and d.cold == d._keep[4].data_ptr()
    src = torch.arange(4, dtype=torch.int32)
    sref = weakref.ref(src)
    e = make_encode_desc(kv_heads=8, head_dim=128, dict_size=512, dict_heads=8, hot_blocks=4, cold_blocks=4,
                         hot=1, dictionary=1, src_blocks=src, cold=1)
    del src
    gc.collect()
    assert sref() is not None and e.src_blocks == e._keep[2].data_ptr()
    del d, e
    gc.collect()
    assert sref() is None


def test_engine_create_without_gpu_fails_cleanly():
    """No GPU in this container: creation reports an error instead of crashing."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.aw_engine_create(0, ctypes.byref(h))
    assert rc != 0 and not h.value


def test_headers_compile_as_c_and_match_the_library(tmp_path):
    """A C99 host (the way a Rust or C binding sees the ABI): the headers
    compile with -pedantic -Werror, and a program linked against the library
    finds the struct sizes it reports and the field offsets the Python
    bindings use."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    src = tmp_path / "abi.c"
    src.write_text("""
#include <stddef.h>
#include <stdio.h>
#include "aether_weaver.h"
#include "aether_fabric.h"
#include "aether_ops.h"
int main(void) {
    size_t s[4];
    aw_abi_struct_sizes(s);
    printf("%zu %zu %zu %zu %zu %zu %zu %u %d %d %d\\n", sizeof(aw_sparse_code), sizeof(aw_weaver_params),
           sizeof(aw_decode_desc), sizeof(aw_decode_plan_info), offsetof(aw_decode_desc, hot_tokens),
           offsetof(aw_decode_desc, q), offsetof(aw_decode_desc, out), aw_abi_version(), AW_PROJECT_AUTO,
           AW_PROJECT_MFMA, AW_PROJECT_VALU);
    return !(s[0] == sizeof(aw_sparse_code) && s[1] == sizeof(aw_weaver_params) && s[2] == sizeof(aw_decode_desc) &&
             s[3] == sizeof(aw_decode_plan_info));
}
""")
    lib = Path(_lib.lib_path()).resolve()
    exe = tmp_path / "abi"
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{ROOT / 'include'}", str(src),
                        "-o", str(exe), f"-L{lib.parent}", "-laether_weaver", f"-Wl,-rpath,{lib.parent}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, (r.stdout, r.stderr)
    vals = [int(x) for x in r.stdout.split()]
    assert vals[:4] == list(STRUCT_SIZES)
    assert vals[4:7] == [DecodeDesc.hot_tokens.offset, DecodeDesc.q.offset, DecodeDesc.out.offset]
    assert vals[7] == lib_abi_version()
    assert vals[8:11] == [AW_PROJECT_AUTO, AW_PROJECT_MFMA, AW_PROJECT_VALU]


def lib_abi_version() -> int:
    return _lib.load().aw_abi_version()
