"""The ``.aether`` Fabric: one mapped file holding the Weaver's pools, with
device copies of those pools kept in HBM.

Mirrors the reference's ``Fabric`` (nexus-core/src/fabric.rs): ``boot``,
region accessors, ``checkpoint`` / ``force_checkpoint``, ``create_genesis``,
``FabricRegions::compute`` and the parsed looms, through the C ABI of
include/aether_fabric.h.  The reference runs on unified memory and hands the
mapping to its GPU kernel in place; on a discrete MI355X the hot pool, cold
pool and dictionary are uploaded once (``attach_device``), decoded and
distilled on the device, and written back (``pull``) before a checkpoint.
"""
from __future__ import annotations

import ctypes
import os
from typing import Iterable, Optional

import numpy as np

from . import _lib
from .types import (AW_F_COLD_HEAD_BLOCKED, REGION_IDS, SPARSE_CODE_DTYPE, FabricRegions, LoomDescriptor, ModelDims,
                    WeaverParams)
from .weaver import WeaverError, _status_text, make_desc

#: ModelDims presets (nexus-core/src/types.rs:166-202).
PRESETS = ("llama8b", "granite2b", "qwen05b", "deepseek_r1_1_5b")
#: Default distillation threshold (types.rs:52, types.rs:483).
DISTILL_ENTROPY_THRESHOLD = 0.15
MAX_HOT_BLOCKS = 8192
MAX_COLD_BLOCKS = 32768
#: aw_fabric_attach_device mask flag (include/aether_fabric.h).
AW_FABRIC_COLD_HEAD_BLOCKED = 1 << 31


class FabricError(WeaverError):
    """A failed Fabric call (FabricError, types.rs:430-454); ``status`` is the AW_E_* code."""


def _msg_call(lib, fn, *args) -> None:
    msg = ctypes.create_string_buffer(512)
    rc = fn(*args, msg, 512)
    if rc:
        raise FabricError(f"{_status_text(lib, rc)}: {msg.value.decode()}", rc)


def model_dims(name: str = "llama8b", **overrides) -> ModelDims:
    """A preset's dimensions (``aw_model_dims_preset``), with fields overridden by keyword."""
    lib = _lib.load()
    d = ModelDims()
    rc = lib.aw_model_dims_preset(name.encode(), ctypes.byref(d))
    if rc:
        raise FabricError(f"unknown model preset {name!r} (one of {PRESETS})", rc)
    for k, v in overrides.items():
        if not hasattr(d, k):
            raise TypeError(f"ModelDims has no field {k!r}")
        setattr(d, k, v)
    return d


def compute_regions(dims: ModelDims) -> FabricRegions:
    """``FabricRegions::compute`` (fabric.rs:124-186)."""
    lib = _lib.load()
    r = FabricRegions()
    rc = lib.aw_fabric_regions_compute(ctypes.byref(dims), ctypes.byref(r))
    if rc:
        raise FabricError("layout mismatch: region sizes overflow", rc)
    return r


def weaver_params_from_loom(dims: ModelDims, loom: LoomDescriptor) -> WeaverParams:
    """``WeaverParams::from_loom`` (types.rs:382-395)."""
    lib = _lib.load()
    p = WeaverParams()
    rc = lib.aw_weaver_params_from_loom(ctypes.byref(dims), ctypes.byref(loom), ctypes.byref(p))
    if rc:
        raise FabricError(_status_text(lib, rc), rc)
    return p


def create_genesis(path: str | os.PathLike, dims: ModelDims) -> None:
    """``create_genesis`` (fabric.rs:695-750), unsigned: the signature bytes stay zero."""
    lib = _lib.load()
    _msg_call(lib, lib.aw_fabric_create_genesis, os.fsencode(path), ctypes.byref(dims))


class Fabric:
    """A booted ``.aether`` file (``Fabric<D>``, fabric.rs:234-252)."""

    def __init__(self, path: str | os.PathLike, dims: ModelDims, public_key: Optional[bytes] = None):
        """``Fabric::boot_with_mode`` (fabric.rs:273-344); ``public_key`` None is BootMode::Dev."""
        self._lib = _lib.load()
        self.dims = dims
        key = None
        if public_key is not None:
            if len(public_key) != 32:
                raise ValueError("an Ed25519 public key is 32 bytes")
            key = ctypes.create_string_buffer(bytes(public_key), 32)
        h = ctypes.c_void_p()
        _msg_call(self._lib, self._lib.aw_fabric_boot, os.fsencode(path), ctypes.byref(dims), key, ctypes.byref(h))
        self._h = h
        self.path = os.fspath(path)

    @classmethod
    def boot(cls, path: str | os.PathLike, dims: ModelDims, public_key: Optional[bytes] = None) -> "Fabric":
        """``Fabric::boot`` (fabric.rs:268-271) / ``boot_with_mode``."""
        return cls(path, dims, public_key)

    # -- lifetime
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.aw_fabric_close(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, rc: int, what: str) -> None:
        if rc:
            msg = self._lib.aw_fabric_last_error(self._h).decode()
            raise FabricError(f"{what}: {_status_text(self._lib, rc)}: {msg}", rc)

    # -- layout
    @property
    def regions(self) -> FabricRegions:
        r = FabricRegions()
        self._check(self._lib.aw_fabric_regions_of(self._h, ctypes.byref(r)), "regions")
        return r

    @property
    def looms(self) -> list[LoomDescriptor]:
        arr = (LoomDescriptor * 4)()
        self._check(self._lib.aw_fabric_looms(self._h, arr), "looms")
        return list(arr)

    def total_size(self) -> int:
        return self.regions.total_size

    # -- host views (zero copy over the mapping)
    def _view(self, region: str, writable: bool) -> np.ndarray:
        ptr, n = ctypes.c_void_p(), ctypes.c_uint64()
        self._check(self._lib.aw_fabric_region(self._h, REGION_IDS[region], int(writable), ctypes.byref(ptr),
                                               ctypes.byref(n)), f"region {region}")
        arr = np.ctypeslib.as_array((ctypes.c_uint8 * n.value).from_address(ptr.value))
        if not writable:
            arr.flags.writeable = False
        return arr

    def weights(self) -> np.ndarray:
        return self._view("weights", False)

    def hot_pool(self) -> np.ndarray:
        """The hot pool bytes (fabric.rs:359-363)."""
        return self._view("hot", False)

    def cold_pool(self) -> np.ndarray:
        return self._view("cold", False)

    def cold_pool_codes(self) -> np.ndarray:
        """The cold pool as SparseCodes (fabric.rs:371-375)."""
        return self.cold_pool().view(SPARSE_CODE_DTYPE)

    def dictionary(self) -> np.ndarray:
        return self._view("dict", False)

    def radix_metadata(self) -> np.ndarray:
        return self._view("radix", False)

    def observation_bufs(self) -> np.ndarray:
        return self._view("obs", False)

    def cold_pool_mut(self) -> np.ndarray:
        """Writable cold pool; marks the fabric dirty (fabric.rs:408-414)."""
        return self._view("cold", True)

    def observation_bufs_mut(self) -> np.ndarray:
        return self._view("obs", True)

    def trace_log_mut(self) -> np.ndarray:
        """Writable trace log; does not mark the fabric dirty (fabric.rs:416-421)."""
        return self._view("trace", True)

    def region_mut(self, region: str) -> np.ndarray:
        """Writable view of any region; marks the fabric dirty except for the trace."""
        return self._view(region, True)

    # Shaped views of the pools the Weaver reads.
    def hot_pool_blocks(self, writable: bool = False) -> np.ndarray:
        """[8192][block][kv_heads][head_dim] f16 bit patterns (uint16)."""
        d = self.dims
        v = self._view("hot", writable).view(np.uint16)
        return v.reshape(MAX_HOT_BLOCKS, d.block_size, d.kv_heads, d.head_dim)

    def cold_pool_blocks(self, writable: bool = False) -> np.ndarray:
        """[32768][block][kv_heads] SparseCodes."""
        d = self.dims
        return self._view("cold", writable).view(SPARSE_CODE_DTYPE).reshape(MAX_COLD_BLOCKS, d.block_size,
                                                                           d.kv_heads)

    def dictionary_atoms(self, writable: bool = False) -> np.ndarray:
        """[kv_heads][dict_size][head_dim] f16 bit patterns (uint16)."""
        d = self.dims
        return self._view("dict", writable).view(np.uint16).reshape(d.kv_heads, d.dict_size, d.head_dim)

    # -- persistence
    def checkpoint(self) -> None:
        """``Fabric::checkpoint`` (fabric.rs:463-483)."""
        self._check(self._lib.aw_fabric_checkpoint(self._h), "checkpoint")

    def force_checkpoint(self) -> None:
        """``Fabric::force_checkpoint`` (fabric.rs:485-493)."""
        self._check(self._lib.aw_fabric_force_checkpoint(self._h), "force_checkpoint")

    @property
    def dirty(self) -> bool:
        return bool(self._lib.aw_fabric_is_dirty(self._h))

    # -- residency in HBM
    def attach_device(self, device: int = 0, regions: Iterable[str] = ("hot", "cold", "dict"),
                      cold_head_blocked: bool = False) -> None:
        """Device copies of `regions`; ``cold_head_blocked`` keeps the device cold
        pool in the [blocks][kv_heads][16] order (AW_FABRIC_COLD_HEAD_BLOCKED)."""
        mask = AW_FABRIC_COLD_HEAD_BLOCKED if cold_head_blocked else 0
        for r in regions:
            mask |= 1 << REGION_IDS[r]
        self._check(self._lib.aw_fabric_attach_device(self._h, device, mask), "attach_device")

    @property
    def device_flags(self) -> int:
        """aw_decode_desc / aw_encode_desc flags of the attached pools (AW_F_COLD_HEAD_BLOCKED or 0)."""
        return int(self._lib.aw_fabric_device_flags(self._h))

    @property
    def cold_head_blocked(self) -> bool:
        return bool(self.device_flags & AW_F_COLD_HEAD_BLOCKED)

    def decode_desc(self, q, out, refs, *, hot_count: int, cold_count: int, batch: int = 1, queries: int = 1,
                    refs_stride: Optional[int] = None, scale: float = 1.0, causal: bool = False, q_latent=None,
                    seq_hot=None, seq_cold=None, hot_tokens: int = 0, seq_hot_tokens: bool = False):
        """An ``aw_decode_desc`` over this fabric's device pools, the way the
        reference's kernel reads the mapped pools (one layer; per-kv-head
        dictionary; score scale 1.0 unless given): pool addresses, capacities
        (MAX_HOT_BLOCKS, MAX_COLD_BLOCKS) and the cold order flag come from the
        attachment, so a head-blocked device cold pool is always read as such.
        ``q``, ``out``, ``refs`` and the optional arrays are the caller's device
        tensors or pointers, as for ``make_desc``."""
        dm = self.dims
        return make_desc(layers=1, batch=batch, queries=queries, q_heads=dm.q_heads, kv_heads=dm.kv_heads,
                         head_dim=dm.head_dim, dict_size=dm.dict_size, dict_heads=dm.kv_heads, hot_count=hot_count,
                         cold_count=cold_count,
                         refs_stride=hot_count + cold_count if refs_stride is None else refs_stride,
                         hot_blocks=MAX_HOT_BLOCKS, cold_blocks=MAX_COLD_BLOCKS, q=q, out=out,
                         hot_k=self.device_region("hot")[0] if hot_count else None,
                         cold=self.device_region("cold")[0] if cold_count else None, refs=refs,
                         dictionary=self.device_region("dict")[0] if cold_count else None, q_latent=q_latent,
                         seq_hot=seq_hot, seq_cold=seq_cold, scale=scale, causal=causal,
                         cold_head_blocked=self.cold_head_blocked, hot_tokens=hot_tokens,
                         seq_hot_tokens=seq_hot_tokens)

    def device_region(self, region: str) -> tuple[int, int]:
        """(device address, bytes) of an attached region."""
        ptr, n = ctypes.c_void_p(), ctypes.c_uint64()
        rc = self._lib.aw_fabric_device_region(self._h, REGION_IDS[region], ctypes.byref(ptr), ctypes.byref(n))
        if rc:
            raise FabricError(f"region {region} is not attached", rc)
        return ptr.value, n.value

    def push(self, region: str, offset: int = 0, nbytes: Optional[int] = None) -> None:
        """Host -> device copy of part of an attached region."""
        if nbytes is None:
            nbytes = self.device_region(region)[1] - offset
        self._check(self._lib.aw_fabric_push(self._h, REGION_IDS[region], offset, nbytes), "push")

    def pull(self, region: str, offset: int = 0, nbytes: Optional[int] = None) -> None:
        """Device -> host copy of part of an attached region; marks the fabric dirty."""
        if nbytes is None:
            nbytes = self.device_region(region)[1] - offset
        self._check(self._lib.aw_fabric_pull(self._h, REGION_IDS[region], offset, nbytes), "pull")

    def detach_device(self) -> None:
        self._check(self._lib.aw_fabric_detach_device(self._h), "detach_device")

    def distill(self, engine, threshold: float = DISTILL_ENTROPY_THRESHOLD) -> tuple[int, np.ndarray]:
        """One Distiller REM cycle on the device copies (distiller.rs:60-120):
        returns (blocks distilled, the proxy of every scanned hot block)."""
        n = min(MAX_HOT_BLOCKS, self.regions.hot_pool_size //
                (self.dims.block_size * self.dims.kv_heads * self.dims.head_dim * 2))
        ent = np.zeros(n, np.float32)
        cnt = ctypes.c_uint32()
        self._check(self._lib.aw_fabric_distill(self._h, engine._h, ctypes.c_float(threshold), ent.ctypes.data,
                                                ctypes.byref(cnt)), "distill")
        return cnt.value, ent
