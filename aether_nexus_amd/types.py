"""Layout contract of the Weaver decode path.

Mirrors the reference's types (nexus-core/src/types.rs):
  * ``ModelDims`` / ``Llama8B`` / ``Granite2B`` / ``Qwen05B`` / ``DeepSeekR1_1_5B``
    geometry constants (types.rs:150-204);
  * ``SparseCode`` — 16 bytes, ``u16 indices[4]`` then f16 ``coeffs[4]``,
    little-endian, size and alignment 16 (types.rs:218-244);
  * ``WeaverParams`` — 12 x u32, 48 bytes, reference field order (types.rs:351-396);
  * ``LoomDescriptor`` — per-persona block-table descriptor (types.rs:311-342).
The ctypes structures match include/aether_weaver.h; tests compare their sizes
with what the compiled library reports.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

BLOCK_SIZE = 16
SPARSITY_K = 4
REF_MASK = 0x7FFFFFFF

# --------------------------------------------------------------- ModelDims


class ModelDims:
    """Compile-time geometry of types.rs:150-164 (defaults: Llama-3.1-8B)."""

    LAYERS = 32
    Q_HEADS = 32
    KV_HEADS = 8
    HEAD_DIM = 128
    INTERMEDIATE_SIZE = 14336
    VOCAB_SIZE = 128256
    BLOCK_SIZE = BLOCK_SIZE
    SPARSITY_K = SPARSITY_K
    DICT_SIZE = 512

    @classmethod
    def hidden_size(cls) -> int:
        return cls.Q_HEADS * cls.HEAD_DIM

    @classmethod
    def gqa_group(cls) -> int:
        return cls.Q_HEADS // cls.KV_HEADS


class Llama8B(ModelDims):
    """types.rs:167-168."""


class Granite2B(ModelDims):
    """types.rs:171-180."""

    LAYERS = 40
    HEAD_DIM = 64
    INTERMEDIATE_SIZE = 8192
    VOCAB_SIZE = 49155


class Qwen05B(ModelDims):
    """types.rs:183-192."""

    LAYERS = 24
    Q_HEADS = 14
    KV_HEADS = 2
    HEAD_DIM = 64
    INTERMEDIATE_SIZE = 4864
    VOCAB_SIZE = 151936


class DeepSeekR1_1_5B(ModelDims):
    """types.rs:195-204."""

    LAYERS = 28
    Q_HEADS = 12
    KV_HEADS = 2
    HEAD_DIM = 128
    INTERMEDIATE_SIZE = 8960
    VOCAB_SIZE = 151936


# -------------------------------------------------------------- SparseCode

#: numpy view of a SparseCode; ``np.zeros(n, SPARSE_CODE_DTYPE)`` is n zero codes.
SPARSE_CODE_DTYPE = np.dtype({"names": ["indices", "coeffs"],
                              "formats": [("<u2", (4,)), ("<f2", (4,))],
                              "offsets": [0, 8], "itemsize": 16, "aligned": True})
assert SPARSE_CODE_DTYPE.itemsize == 16


class CSparseCode(ctypes.Structure):
    """``aw_sparse_code``: coefficients carried as raw binary16 bits."""

    _fields_ = [("indices", ctypes.c_uint16 * 4), ("coeffs", ctypes.c_uint16 * 4)]


def pack_codes(indices: np.ndarray, coeffs: np.ndarray) -> np.ndarray:
    """Pack ``indices[..., 4]`` (u16) and ``coeffs[..., 4]`` (f16-representable)
    into SparseCodes, returned as a ``uint16`` array of shape ``[..., 8]``
    (the 16 bytes of each code, indices first)."""
    indices = np.asarray(indices)
    coeffs = np.asarray(coeffs)
    if indices.shape != coeffs.shape or indices.shape[-1] != SPARSITY_K:
        raise ValueError("indices and coeffs must both have shape [..., 4]")
    if indices.size and (indices.min() < 0 or indices.max() > 0xFFFF):
        raise ValueError("atom indices must fit in u16")
    out = np.empty(indices.shape[:-1] + (8,), dtype=np.uint16)
    out[..., :4] = indices.astype(np.uint16)
    out[..., 4:] = coeffs.astype(np.float16).view(np.uint16)
    return out


def unpack_codes(words: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of :func:`pack_codes`: ``(indices u16 [...,4], coeffs f16 [...,4])``."""
    words = np.asarray(words, dtype=np.uint16)
    if words.shape[-1] != 8:
        raise ValueError("codes must have shape [..., 8] (u16 words)")
    return words[..., :4].copy(), words[..., 4:].copy().view(np.float16)


def code_bytes(indices, coeffs) -> bytes:
    """The 16 little-endian bytes of one SparseCode."""
    return pack_codes(np.asarray(indices).reshape(1, 4), np.asarray(coeffs).reshape(1, 4)).astype("<u2").tobytes()


# ------------------------------------------------------------ WeaverParams


class WeaverParams(ctypes.Structure):
    """``aw_weaver_params`` / reference ``WeaverParams`` (types.rs:351-374)."""

    _fields_ = [
        ("q_heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("block_size", ctypes.c_uint32),
        ("gqa_group", ctypes.c_uint32),
        ("hot_count", ctypes.c_uint32),
        ("cold_count", ctypes.c_uint32),
        ("dict_size", ctypes.c_uint32),
        ("sparsity_k", ctypes.c_uint32),
        ("_pad", ctypes.c_uint32 * 3),
    ]

    @classmethod
    def from_loom(cls, dims: type[ModelDims], loom: "LoomDescriptor") -> "WeaverParams":
        """``WeaverParams::from_loom`` (types.rs:381-395)."""
        return cls(q_heads=dims.Q_HEADS, kv_heads=dims.KV_HEADS, head_dim=dims.HEAD_DIM,
                   block_size=dims.BLOCK_SIZE, gqa_group=dims.gqa_group(),
                   hot_count=loom.hot_count, cold_count=loom.cold_count,
                   dict_size=dims.DICT_SIZE, sparsity_k=dims.SPARSITY_K)

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_ if name != "_pad"}


@dataclass
class LoomDescriptor:
    """Per-persona block-table descriptor (types.rs:311-342)."""

    persona: int = 0
    hot_count: int = 0
    cold_count: int = 0
    hot_refs_offset: int = 0
    cold_refs_offset: int = 0
    token_pos: int = 0


# --------------------------------------------------- device request (C ABI)

AW_F_CAUSAL = 1
AW_F_COLD_HEAD_BLOCKED = 2
AW_F_ENCODE_FULL_SCAN = 4
AW_F_SEQ_HOT_TOKENS = 8
AW_F_QLATENT_F32 = 16
AW_NOALLOC_SCRATCH_BYTES = 96 << 20  # scratch of aw_decode_device_noalloc
AW_PROJECT_AUTO, AW_PROJECT_MFMA, AW_PROJECT_VALU = 0, 1, 2  # aw_engine_set_projection
AW_COLD_OUT_AUTO, AW_COLD_OUT_BINS, AW_COLD_OUT_VALUES = 0, 1, 2  # aw_engine_set_cold_output

AW_OK = 0
AW_E_INVALID_ARG = -1
AW_E_ALIGN = -2
AW_E_OOB = -3
AW_E_HIP = -4
AW_E_LOAD = -5
AW_E_UNSUPPORTED = -6
# include/aether_fabric.h: one code per FabricError variant (nexus-core/src/types.rs:430-454)
AW_E_IO = -7
AW_E_BAD_MAGIC = -8
AW_E_VERSION = -9
AW_E_TOO_SMALL = -10
AW_E_SIGNATURE = -11

STAGES = ("project", "hot", "cold", "finish", "merge")


class DecodeDesc(ctypes.Structure):
    """``aw_decode_desc`` (include/aether_weaver.h)."""

    _fields_ = [
        ("layers", ctypes.c_uint32), ("batch", ctypes.c_uint32), ("queries", ctypes.c_uint32),
        ("q_heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
        ("dict_size", ctypes.c_uint32), ("dict_heads", ctypes.c_uint32),
        ("hot_count", ctypes.c_uint32), ("cold_count", ctypes.c_uint32),
        ("refs_stride", ctypes.c_uint32), ("flags", ctypes.c_uint32),
        ("scale", ctypes.c_float), ("hot_tokens", ctypes.c_uint32),
        ("hot_blocks", ctypes.c_uint64), ("cold_blocks", ctypes.c_uint64),
        ("q", ctypes.c_void_p), ("q_latent", ctypes.c_void_p),
        ("hot_k", ctypes.c_void_p), ("hot_v", ctypes.c_void_p),
        ("cold", ctypes.c_void_p), ("refs", ctypes.c_void_p),
        ("seq_hot", ctypes.c_void_p), ("seq_cold", ctypes.c_void_p),
        ("dict", ctypes.c_void_p), ("out", ctypes.c_void_p),
    ]


class EncodeDesc(ctypes.Structure):
    """``aw_encode_desc`` (include/aether_weaver.h): a SparseCode encoder request."""

    _fields_ = [
        ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
        ("dict_size", ctypes.c_uint32), ("dict_heads", ctypes.c_uint32),
        ("n_blocks", ctypes.c_uint32), ("flags", ctypes.c_uint32),
        ("hot_blocks", ctypes.c_uint64), ("cold_blocks", ctypes.c_uint64),
        ("hot", ctypes.c_void_p), ("dict", ctypes.c_void_p),
        ("src_blocks", ctypes.c_void_p), ("dst_blocks", ctypes.c_void_p),
        ("cold", ctypes.c_void_p), ("entropy", ctypes.c_void_p),
    ]


class PlanInfo(ctypes.Structure):
    """``aw_decode_plan_info``."""

    _fields_ = [
        ("rows_per_kv_head", ctypes.c_uint32), ("hot_splits", ctypes.c_uint32),
        ("hot_tokens_per_split", ctypes.c_uint32), ("cold_splits", ctypes.c_uint32),
        ("cold_tokens_per_split", ctypes.c_uint32), ("cold_row_chunk", ctypes.c_uint32),
        ("computes_q_latent", ctypes.c_uint32), ("projection", ctypes.c_uint32),
        ("workspace_bytes", ctypes.c_uint64), ("cold_output", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
    ]


STRUCT_SIZES = (ctypes.sizeof(CSparseCode), ctypes.sizeof(WeaverParams),
                ctypes.sizeof(DecodeDesc), ctypes.sizeof(PlanInfo))


# ---------------------------------------------------------------- the .aether Fabric

REGION_IDS = {"weights": 0, "hot": 1, "cold": 2, "dict": 3, "looms": 4, "radix": 5, "obs": 6, "trace": 7}
PERSONAS = ("Planner", "Coder", "Critic", "Reviewer")  # types.rs:293-300


class ModelDims(ctypes.Structure):
    """``aw_model_dims``: the ModelDims constants (nexus-core/src/types.rs:150-164) as fields."""

    _fields_ = [(n, ctypes.c_uint32) for n in (
        "layers", "q_heads", "kv_heads", "head_dim", "hidden_size", "intermediate_size", "vocab_size",
        "block_size", "sparsity_k", "dict_size")]


class FabricRegions(ctypes.Structure):
    """``aw_fabric_regions``: FabricRegions (nexus-core/src/fabric.rs:74-117)."""

    _fields_ = [(n, ctypes.c_uint64) for n in (
        "weights_offset", "weights_size", "hot_pool_offset", "hot_pool_size", "cold_pool_offset",
        "cold_pool_size", "dict_offset", "dict_size", "looms_offset", "looms_size", "radix_offset",
        "radix_size", "obs_offset", "obs_size", "trace_offset", "trace_size", "total_size")]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class LoomDescriptor(ctypes.Structure):
    """``aw_loom_descriptor``: LoomDescriptor (nexus-core/src/types.rs:311-328), 32 bytes."""

    _fields_ = [
        ("persona", ctypes.c_uint8), ("_pad0", ctypes.c_uint8 * 3),
        ("hot_count", ctypes.c_uint32), ("cold_count", ctypes.c_uint32),
        ("hot_refs_offset", ctypes.c_uint32), ("cold_refs_offset", ctypes.c_uint32),
        ("token_pos", ctypes.c_uint32), ("_pad", ctypes.c_uint32 * 2),
    ]

    def as_tuple(self) -> tuple:
        return (self.persona, self.hot_count, self.cold_count, self.hot_refs_offset, self.cold_refs_offset,
                self.token_pos)


assert ctypes.sizeof(LoomDescriptor) == 32 and ctypes.sizeof(ModelDims) == 40
