"""Loader for the gfx950 Weaver library (``libaether_weaver.so``).

The reference loads its kernels from a metallib whose path build.rs exports
(``WeaverEngine::new(metallib_path)``, nexus-core/src/weaver.rs:85-95,
build.rs:75).  Here the kernels live in a shared library built in-tree by
``aether_nexus_amd.build``; its path can be overridden with ``AETHER_WEAVER_LIB``.
A missing library is an error: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_NAME = "libaether_weaver.so"
DEFAULT_LIB = PKG_DIR / LIB_NAME

_c_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64

#: Every function declared in include/*.h with its ctypes signature.
SIGNATURES = {
    "aw_abi_version": (_u32, []),
    "aw_abi_struct_sizes": (None, [ctypes.POINTER(_sz)]),
    "aw_status_string": (ctypes.c_char_p, [_c_int]),
    "aw_validate_params": (_c_int, [_vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _sz, _sz, ctypes.c_char_p, _sz]),
    "aw_decode_plan": (_c_int, [_vp, _vp, ctypes.c_char_p, _sz]),
    "aw_engine_create": (_c_int, [_c_int, ctypes.POINTER(_vp)]),
    "aw_engine_destroy": (None, [_vp]),
    "aw_engine_last_error": (ctypes.c_char_p, [_vp]),
    "aw_engine_device_name": (ctypes.c_char_p, [_vp]),
    "aw_engine_max_threads_per_threadgroup": (_u64, [_vp]),
    "aw_decode": (_c_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _sz]),
    "aw_decode_device": (_c_int, [_vp, _vp, _vp]),
    "aw_decode_device_noalloc": (_c_int, [_vp, _vp, _vp]),
    "aw_debug_read_stream": (_c_int, [_vp, _vp, ctypes.c_uint64, ctypes.c_uint32, _vp, _vp]),
    "aw_debug_read_pools": (_c_int, [_vp, _vp, _vp, _vp]),
    "aw_debug_project": (_c_int, [_vp, _vp, _vp, _vp]),
    "aw_multihead_attention_device": (_c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u64, _vp]),
    "aw_engine_check_device_errors": (_c_int, [_vp, _vp]),
    "aw_debug_gather_codes": (_c_int, [_vp, _vp, _sz, _vp, _u32, _u32, _vp, _vp, _vp, _vp]),
    "aw_engine_set_profiling": (_c_int, [_vp, _c_int]),
    "aw_engine_set_projection": (_c_int, [_vp, _c_int]),
    "aw_engine_set_cold_output": (_c_int, [_vp, _c_int]),
    "aw_engine_stage_stats": (_c_int, [_vp, _c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_u64)]),
    "aw_engine_reset_stage_stats": (_c_int, [_vp]),
    "aw_abi_encode_desc_size": (_sz, []),
    "aw_encode_device": (_c_int, [_vp, _vp, _vp]),
    "aw_encode": (_c_int, [_vp, _vp, _sz, _vp, _sz, _u32, _u32, _u32, _u32, _vp, _sz, _vp, _sz, _vp]),
    "aw_block_entropy_device": (_c_int, [_vp, _vp, _u64, _u32, _u32, _vp, _u32, _vp, _vp]),
    # include/aether_fabric.h
    "aw_model_dims_preset": (_c_int, [ctypes.c_char_p, _vp]),
    "aw_fabric_regions_compute": (_c_int, [_vp, _vp]),
    "aw_weaver_params_from_loom": (_c_int, [_vp, _vp, _vp]),
    "aw_fabric_create_genesis": (_c_int, [ctypes.c_char_p, _vp, ctypes.c_char_p, _sz]),
    "aw_fabric_boot": (_c_int, [ctypes.c_char_p, _vp, _vp, ctypes.POINTER(_vp), ctypes.c_char_p, _sz]),
    "aw_fabric_close": (None, [_vp]),
    "aw_fabric_last_error": (ctypes.c_char_p, [_vp]),
    "aw_fabric_regions_of": (_c_int, [_vp, _vp]),
    "aw_fabric_looms": (_c_int, [_vp, _vp]),
    "aw_fabric_region": (_c_int, [_vp, _u32, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_u64)]),
    "aw_fabric_checkpoint": (_c_int, [_vp]),
    "aw_fabric_force_checkpoint": (_c_int, [_vp]),
    "aw_fabric_is_dirty": (_c_int, [_vp]),
    "aw_fabric_attach_device": (_c_int, [_vp, _c_int, _u32]),
    "aw_fabric_device_flags": (_u32, [_vp]),
    "aw_fabric_device_region": (_c_int, [_vp, _u32, ctypes.POINTER(_vp), ctypes.POINTER(_u64)]),
    "aw_fabric_push": (_c_int, [_vp, _u32, _u64, _u64]),
    "aw_fabric_pull": (_c_int, [_vp, _u32, _u64, _u64]),
    "aw_fabric_detach_device": (_c_int, [_vp]),
    "aw_fabric_distill": (_c_int, [_vp, _vp, ctypes.c_float, _vp, ctypes.POINTER(_u32)]),
    # include/aether_ops.h
    "aw_ops_copy_buffer": (_c_int, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "aw_ops_embed_lookup": (_c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "aw_ops_rms_norm": (_c_int, [_vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float, _vp]),
    "aw_ops_rope": (_c_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, ctypes.c_float, _vp]),
    "aw_ops_matmul": (_c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "aw_ops_matmul_scaled": (_c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, ctypes.c_float, _vp]),
    "aw_ops_silu_gate": (_c_int, [_vp, _vp, _vp, _vp, _u32, _vp]),
    "aw_ops_add_residual": (_c_int, [_vp, _vp, _vp, _u32, _vp]),
    "aw_ops_add_bias": (_c_int, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "aw_ops_scale_f16": (_c_int, [_vp, _vp, _u32, ctypes.c_float, _vp]),
    "aw_ops_causal_attention": (_c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u64, _vp]),
    "aw_ops_matmul_add_residual": (_c_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, ctypes.c_float, _vp]),
    "aw_ops_matmul_silu_gate": (_c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "aw_ops_matmul_qkv": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
}

_cache: dict[str, ctypes.CDLL] = {}


def lib_path(path: str | os.PathLike | None = None) -> Path:
    if path is not None:
        return Path(path)
    env = os.environ.get("AETHER_WEAVER_LIB")
    return Path(env) if env else DEFAULT_LIB


def _share_torch_runtime() -> None:
    """Put PyTorch's HIP runtime in the process before this library is opened.

    PyTorch-ROCm ships its own libamdhip64 and loads it into the global symbol
    scope, so a library opened after ``import torch`` binds its HIP calls to that
    runtime and both share one device context (streams and pointers pass freely
    between them).  Opened first, this library would start the system runtime,
    and a second runtime started later in the same process then finds no device.
    Without PyTorch the library uses the system runtime alone."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load the library and declare every exported signature.

    Raises ``FileNotFoundError`` when the library was not built and ``OSError``
    when it cannot be loaded, like ``new_library_with_file`` failing in the
    reference (weaver.rs:89)."""
    p = lib_path(path).resolve()
    key = str(p)
    if key in _cache:
        return _cache[key]
    if not p.is_file():
        raise FileNotFoundError(
            f"{p} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    _share_torch_runtime()
    lib = ctypes.CDLL(key)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _cache[key] = lib
    return lib
