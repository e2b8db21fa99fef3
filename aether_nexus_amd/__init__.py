"""MI355X (gfx950) implementation of AetherNexus's Weaver decode hot path.

GQA decode attention over an exact f16 hot pool and a cold pool of 16-byte
SparseCodes attended without decompression, as hand-written HIP kernels
behind the C ABI of include/aether_weaver.h.

  types      layout contract (SparseCode, WeaverParams, ModelDims, aw_decode_desc)
  weaver     WeaverEngine: mirror of the reference engine over the C ABI
  workloads  seeded synthetic decode workloads
  fabric     the .aether file's pools resident in HBM, and the Distiller's REM cycle
  inference  KV cache over aw_multihead_attention_device and the speculative-verify rule
  build      hipcc build of libaether_weaver.so
"""
from .types import (SPARSE_CODE_DTYPE, DecodeDesc, Granite2B, Llama8B, LoomDescriptor, ModelDims, PlanInfo,
                    WeaverParams, pack_codes, unpack_codes)
from .weaver import DecodeOutput, WeaverEngine, WeaverError, make_desc, plan, validate_params

__all__ = ["SPARSE_CODE_DTYPE", "DecodeDesc", "DecodeOutput", "Granite2B", "Llama8B", "LoomDescriptor",
           "ModelDims", "PlanInfo", "WeaverEngine", "WeaverError", "WeaverParams", "make_desc", "pack_codes",
           "plan", "unpack_codes", "validate_params"]
