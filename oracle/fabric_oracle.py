"""CPU restatement of the reference's `.aether` Fabric layout and loom parsing.

TEST INFRASTRUCTURE ONLY: imported by tests/ to check the product's
fabric code (aether_nexus_amd/csrc/fabric.hip through include/aether_fabric.h),
never by the product package.  Plain integer arithmetic on Python ints.

Pins (tests/test_fabric.py):
  * compute_regions: the reference's own tests on the layout (fabric.rs:756-809:
    16 KiB alignment, no overlap; align_up values fabric.rs:868-874), the pool
    sizes its boot log printed for Llama8B (docs/walkthrough.md.resolved:70:
    hot 256 MB, cold 64 MB, dictionary 1024 KB), and, for the weight estimate, the
    published parameter count of Llama-3.1-8B (8,030,261,248 with its untied
    128256 x 4096 lm_head, which the estimate leaves to the 1.25 factor).
  * genesis_bytes / parse_looms: the genesis -> boot round trip of
    fabric.rs:812-841 (personas Planner, Coder, Critic, Reviewer in order) and
    the zero cold pool of fabric.rs:844-866.
  * candidates: the threshold rule of distiller.rs:112-115 on proxies from
    oracle.block_entropy, itself pinned by the reference's entropy tests.
"""
from __future__ import annotations

import struct

MAGIC = b"AETHER1.3"                   # types.rs:461
FORMAT_VERSION = 0x0001_0003           # types.rs:464
SIGNATURE_LEN = 64                     # types.rs:467
HEADER_SIZE = len(MAGIC) + 4 + SIGNATURE_LEN  # types.rs:497
MAX_HOT_BLOCKS = 8192                  # types.rs:500
MAX_COLD_BLOCKS = 32768                # types.rs:503
OBS_BUF_SIZE = 256 * 1024 * 1024       # types.rs:506
TRACE_LOG_SIZE = 128 * 1024 * 1024     # types.rs:509
PERSONA_COUNT = 4                      # types.rs:303-305
LOOM_DESCRIPTOR_SIZE = 32              # repr(C): u8 + pad 3, 5 x u32, [u32; 2] (types.rs:311-328)
SPARSE_CODE_SIZE = 16                  # types.rs:227-228

# ModelDims defaults and presets (types.rs:150-202), as plain dicts.
DEFAULTS = dict(layers=32, q_heads=32, kv_heads=8, head_dim=128, hidden_size=32 * 128, intermediate_size=14336,
                vocab_size=128256, block_size=16, sparsity_k=4, dict_size=512)
PRESETS = {
    "llama8b": dict(DEFAULTS),
    "granite2b": dict(DEFAULTS, layers=40, q_heads=32, kv_heads=8, head_dim=64, hidden_size=2048,
                      intermediate_size=8192, vocab_size=49155),
    "qwen05b": dict(DEFAULTS, layers=24, q_heads=14, kv_heads=2, head_dim=64, hidden_size=896,
                    intermediate_size=4864, vocab_size=151936),
    "deepseek_r1_1_5b": dict(DEFAULTS, layers=28, q_heads=12, kv_heads=2, head_dim=128, hidden_size=1536,
                             intermediate_size=8960, vocab_size=151936),
}


def align_up(value: int, alignment: int) -> int:
    """fabric.rs:683-685 (power-of-two alignment)."""
    return (value + alignment - 1) & ~(alignment - 1)


def estimated_weight_bytes(d: dict) -> int:
    """fabric.rs:190-222: 2 bytes x (per-layer projections and norms x layers +
    embedding and final norm), x 1.25 in f64, truncated."""
    h, inter, vocab = d["hidden_size"], d["intermediate_size"], d["vocab_size"]
    q, kv, hd = d["q_heads"], d["kv_heads"], d["head_dim"]
    per_layer = 2 * (q * hd * h + 2 * kv * hd * h + q * hd * h + 3 * h * inter + 2 * h)
    glob = 2 * (vocab * h + h)
    raw = d["layers"] * per_layer + glob
    return int(float(raw) * 1.25)


def compute_regions(d: dict) -> dict:
    """FabricRegions::compute (fabric.rs:124-186)."""
    r = {}
    r["weights_offset"] = align_up(HEADER_SIZE, 16384)
    r["weights_size"] = align_up(estimated_weight_bytes(d), 16384)
    r["hot_pool_offset"] = align_up(r["weights_offset"] + r["weights_size"], 16384)
    r["hot_pool_size"] = MAX_HOT_BLOCKS * d["block_size"] * d["kv_heads"] * d["head_dim"] * 2
    r["cold_pool_offset"] = align_up(r["hot_pool_offset"] + r["hot_pool_size"], 16384)
    r["cold_pool_size"] = MAX_COLD_BLOCKS * d["block_size"] * d["kv_heads"] * SPARSE_CODE_SIZE
    r["dict_offset"] = align_up(r["cold_pool_offset"] + r["cold_pool_size"], 16384)
    r["dict_size"] = d["kv_heads"] * d["dict_size"] * d["head_dim"] * 2
    r["looms_offset"] = align_up(r["dict_offset"] + r["dict_size"], 4096)
    r["looms_size"] = PERSONA_COUNT * LOOM_DESCRIPTOR_SIZE
    r["radix_offset"] = align_up(r["looms_offset"] + r["looms_size"], 4096)
    r["radix_size"] = (MAX_HOT_BLOCKS + MAX_COLD_BLOCKS) * 3 * 4
    r["obs_offset"] = align_up(r["radix_offset"] + r["radix_size"], 16384)
    r["obs_size"] = OBS_BUF_SIZE
    r["trace_offset"] = align_up(r["obs_offset"] + r["obs_size"], 16384)
    r["trace_size"] = TRACE_LOG_SIZE
    r["total_size"] = align_up(r["trace_offset"] + r["trace_size"] + SIGNATURE_LEN, 16384)
    return r


def genesis_bytes(d: dict) -> dict:
    """create_genesis (fabric.rs:695-750) as {offset: bytes} of every non-zero
    byte run, without the signature (which this oracle does not compute)."""
    r = compute_regions(d)
    out = {0: MAGIC + struct.pack("<I", FORMAT_VERSION)}
    for i in range(PERSONA_COUNT):
        if i:  # persona 0 is a zero byte
            out[r["looms_offset"] + i * LOOM_DESCRIPTOR_SIZE] = bytes([i])
    return out


def parse_looms(loom_bytes: bytes) -> list:
    """parse_looms (fabric.rs:518-549): (persona, hot_count, cold_count,
    hot_refs_offset, cold_refs_offset, token_pos) per persona; a persona byte
    other than 0-3 reads as Planner (0)."""
    out = []
    for i in range(PERSONA_COUNT):
        off = i * LOOM_DESCRIPTOR_SIZE
        persona = loom_bytes[off]
        persona = persona if persona <= 3 else 0
        fields = struct.unpack_from("<5I", loom_bytes, off + 4)
        out.append((persona,) + fields)
    return out


def params_from_loom(d: dict, loom: tuple) -> dict:
    """WeaverParams::from_loom (types.rs:382-395)."""
    return dict(q_heads=d["q_heads"], kv_heads=d["kv_heads"], head_dim=d["head_dim"], block_size=d["block_size"],
                gqa_group=d["q_heads"] // d["kv_heads"], hot_count=loom[1], cold_count=loom[2],
                dict_size=d["dict_size"], sparsity_k=d["sparsity_k"])


def candidates(entropies, threshold: float) -> list:
    """evaluate_entropy's selection (distiller.rs:112-115): blocks whose proxy
    is below the threshold and above zero, in block order.  `entropies` and the
    threshold are compared as f32, as in the reference."""
    import numpy as np
    e = np.asarray(entropies, dtype=np.float32)
    t = np.float32(threshold)
    return [int(b) for b in range(e.size) if e[b] < t and e[b] > 0]
