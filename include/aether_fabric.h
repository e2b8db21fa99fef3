/*
 * aether_fabric.h — C ABI of the `.aether` Fabric: the one file that holds the
 * Weaver's pools, and their residency in GPU memory (HBM).
 *
 * The reference maps the whole file with mmap and hands sub-slices of it to the
 * Weaver (unified memory, zero copy):
 *   nexus-core/src/fabric.rs:124-222   FabricRegions::compute (region map)
 *   nexus-core/src/fabric.rs:273-344   Fabric::boot_with_mode (open, size, magic,
 *                                       version, signature, looms)
 *   nexus-core/src/fabric.rs:347-422   region accessors (&[u8] / &mut [u8])
 *   nexus-core/src/fabric.rs:463-493   checkpoint / force_checkpoint (mmap flush)
 *   nexus-core/src/fabric.rs:518-549   parse_looms
 *   nexus-core/src/fabric.rs:695-750   create_genesis
 *   nexus-core/src/types.rs:150-202    ModelDims and its presets
 *   nexus-core/src/types.rs:311-342    LoomDescriptor
 *   nexus-core/src/types.rs:382-395    WeaverParams::from_loom
 *   nexus-core/src/types.rs:430-509    FabricError, file-format constants, FabricLayout
 *   nexus-core/src/distiller.rs:60-120 Distiller::run / evaluate_entropy (one REM cycle)
 * On a discrete GPU the pools the decode reads must live in HBM: the
 * aw_fabric_attach_device / push / pull calls below keep device copies of the
 * hot pool, cold pool and dictionary, and write device-side changes (codes the
 * GPU encoder produced) back into the mapped file before a checkpoint.
 *
 * Status codes are those of aether_weaver.h plus the file errors below, one per
 * FabricError variant, so a binding can map them back one to one.
 * Threading: a fabric handle is used by one thread at a time (the reference
 * guards the Fabric with a Mutex, distiller.rs:60).
 */
#ifndef AETHER_FABRIC_H
#define AETHER_FABRIC_H

#include "aether_weaver.h"

#ifdef __cplusplus
extern "C" {
#endif

/* FabricError (types.rs:430-454) beyond the codes of aether_weaver.h.
 * MmapFailed -> AW_E_IO, InvalidFile / LayoutMismatch -> AW_E_INVALID_ARG,
 * CheckpointFailed -> AW_E_IO. */
#define AW_E_IO          (-7)  /* open, mmap, read, write or msync failed         */
#define AW_E_BAD_MAGIC   (-8)  /* BadMagic: the file does not start with AETHER1.3 */
#define AW_E_VERSION     (-9)  /* VersionMismatch                                  */
#define AW_E_TOO_SMALL   (-10) /* FileTooSmall                                     */
#define AW_E_SIGNATURE   (-11) /* SignatureInvalid                                 */

/* File-format constants (types.rs:461-509). */
#define AW_FABRIC_MAGIC            "AETHER1.3" /* 9 bytes at offset 0, no terminator */
#define AW_FABRIC_MAGIC_LEN        9u
#define AW_FABRIC_VERSION          0x00010003u /* u32 LE at offset 9 */
#define AW_FABRIC_SIGNATURE_LEN    64u
#define AW_FABRIC_MAX_HOT_BLOCKS   8192u
#define AW_FABRIC_MAX_COLD_BLOCKS  32768u
#define AW_FABRIC_CHECKPOINT_MS    300u
#define AW_FABRIC_PERSONAS         4u

/* Model geometry; replaces the ModelDims trait (types.rs:150-164), whose
 * associated constants become fields.  gqa_group is q_heads / kv_heads. */
typedef struct aw_model_dims {
    uint32_t layers, q_heads, kv_heads, head_dim;
    uint32_t hidden_size, intermediate_size, vocab_size;
    uint32_t block_size;  /* tokens per block, 16 */
    uint32_t sparsity_k;  /* codes per token, 4 */
    uint32_t dict_size;   /* dictionary atoms per kv head */
} aw_model_dims;

/* The presets of types.rs:166-202 by name: "llama8b", "granite2b", "qwen05b",
 * "deepseek_r1_1_5b".  AW_E_INVALID_ARG for another name. */
int aw_model_dims_preset(const char* name, aw_model_dims* out);

/* Byte offset and size of every region; replaces FabricRegions
 * (fabric.rs:74-117).  Layout order: header | weights | hot pool | cold pool |
 * dictionary | looms | radix | observation buffers | trace | signature. */
typedef struct aw_fabric_regions {
    uint64_t weights_offset, weights_size;
    uint64_t hot_pool_offset, hot_pool_size;
    uint64_t cold_pool_offset, cold_pool_size;
    uint64_t dict_offset, dict_size;
    uint64_t looms_offset, looms_size;
    uint64_t radix_offset, radix_size;
    uint64_t obs_offset, obs_size;
    uint64_t trace_offset, trace_size;
    uint64_t total_size;
} aw_fabric_regions;

/* Region ids for the accessors. */
#define AW_REGION_WEIGHTS 0u
#define AW_REGION_HOT     1u /* [8192][block_size][kv_heads][head_dim] f16      */
#define AW_REGION_COLD    2u /* [32768][block_size][kv_heads] aw_sparse_code    */
#define AW_REGION_DICT    3u /* [kv_heads][dict_size][head_dim] f16             */
#define AW_REGION_LOOMS   4u
#define AW_REGION_RADIX   5u
#define AW_REGION_OBS     6u
#define AW_REGION_TRACE   7u
#define AW_REGION_COUNT   8u
#define AW_REGION_BIT(r)  (1u << (r))

/* Replaces FabricRegions::compute (fabric.rs:124-186) with
 * estimated_weight_bytes (fabric.rs:190-222): the same offsets, alignments
 * (16 KiB; 4 KiB for looms and radix) and sizes, in 64-bit arithmetic.
 * AW_E_INVALID_ARG when a size overflows 2^62. */
int aw_fabric_regions_compute(const aw_model_dims* dims, aw_fabric_regions* out);

/* One persona's attention pathway, 32 bytes in the reference's repr(C) layout
 * (types.rs:311-328): persona byte, 3 padding bytes, 5 u32, 2 u32 padding. */
typedef struct aw_loom_descriptor {
    uint8_t  persona;  /* 0 Planner, 1 Coder, 2 Critic, 3 Reviewer */
    uint8_t  _pad0[3];
    uint32_t hot_count;
    uint32_t cold_count;
    uint32_t hot_refs_offset;
    uint32_t cold_refs_offset;
    uint32_t token_pos;
    uint32_t _pad[2];
} aw_loom_descriptor;

/* Replaces WeaverParams::from_loom (types.rs:382-395). */
int aw_weaver_params_from_loom(const aw_model_dims* dims, const aw_loom_descriptor* loom,
                               aw_weaver_params* out);

typedef struct aw_fabric aw_fabric;

/* Replaces create_genesis (fabric.rs:695-750): creates (truncating) a file of
 * total_size bytes, all zero (a sparse file) except the magic, the version and
 * the four persona bytes of the loom region.  The reference signs the file with
 * an Ed25519 key; this library has no signer and leaves the 64 signature bytes
 * zero.  `msg` (may be NULL) receives a description of a failure. */
int aw_fabric_create_genesis(const char* path, const aw_model_dims* dims, char* msg, size_t msg_len);

/* Replaces Fabric::boot / boot_with_mode (fabric.rs:268-344): opens `path`
 * read-write, checks that it holds at least total_size bytes
 * (AW_E_TOO_SMALL), maps it shared, checks the magic (AW_E_BAD_MAGIC) and the
 * version (AW_E_VERSION), and parses the looms.  public_key NULL is
 * BootMode::Dev; a key (BootMode::Verified) returns AW_E_UNSUPPORTED: this
 * library does not implement Ed25519.  Messages follow FabricError's texts. */
int aw_fabric_boot(const char* path, const aw_model_dims* dims, const uint8_t* public_key,
                   aw_fabric** out, char* msg, size_t msg_len);

/* Unmaps the file and frees the device copies.  No implicit flush: call
 * aw_fabric_force_checkpoint first to persist (the reference's Drop of the
 * mmap does not flush either). */
void aw_fabric_close(aw_fabric* fabric);

/* Text of the last failure on this handle. */
const char* aw_fabric_last_error(const aw_fabric* fabric);

int aw_fabric_regions_of(const aw_fabric* fabric, aw_fabric_regions* out);

/* The 4 looms parsed at boot (fabric.rs:518-549: a persona byte above 3 reads
 * as Planner; the 5 u32 fields are read little-endian at +4). */
int aw_fabric_looms(const aw_fabric* fabric, aw_loom_descriptor out[4]);

/* Host view of one region of the mapping (fabric.rs:347-422).  writable != 0
 * marks the fabric dirty, as cold_pool_mut and observation_bufs_mut do
 * (fabric.rs:395-414), except for the trace region, whose mutable accessor
 * does not (fabric.rs:416-421). */
int aw_fabric_region(aw_fabric* fabric, uint32_t region, int writable, void** ptr, uint64_t* bytes);

/* Replaces Fabric::checkpoint (fabric.rs:463-483): when dirty and at least
 * 300 ms after the last flush, starts an asynchronous flush of the mapping
 * (msync MS_ASYNC) and clears the dirty flag; otherwise does nothing. */
int aw_fabric_checkpoint(aw_fabric* fabric);

/* Replaces Fabric::force_checkpoint (fabric.rs:485-493): a synchronous flush
 * (msync MS_SYNC), clears the dirty flag. */
int aw_fabric_force_checkpoint(aw_fabric* fabric);

/* 1 when a write is pending a checkpoint, else 0. */
int aw_fabric_is_dirty(const aw_fabric* fabric);

/* ---- residency in GPU memory (no reference counterpart: the reference runs on
 * unified memory and reads the mapping in place) ---------------------------- */

/* Flag in aw_fabric_attach_device's region_mask: keep the device copy of the
 * cold pool in the head-blocked order [blocks][kv_heads][block_size] instead of
 * the file's [blocks][block_size][kv_heads].  The decode and the encoder read
 * and write that order with AW_F_COLD_HEAD_BLOCKED (aw_fabric_device_flags);
 * it gives the same output bits and shorter decode steps (one kv head's codes
 * of a block fill whole 64-byte L2 sectors).  The file keeps its format: copies
 * reorder whole blocks on the device, and push / pull still take byte ranges of
 * the file's cold region.  A cold-pool push then writes whole blocks: the bytes
 * of its first and last block outside the range come from the mapping too; a
 * pull writes only the requested bytes into the mapping. */
#define AW_FABRIC_COLD_HEAD_BLOCKED (1u << 31)

/* Allocates device copies of the regions in region_mask (AW_REGION_BIT of
 * HOT, COLD, DICT, ..., optionally | AW_FABRIC_COLD_HEAD_BLOCKED) on HIP device
 * `device` and uploads them.  Uploads go through two pinned staging buffers:
 * host threads copy the mapping into one while the DMA engine copies the
 * other.  A region already attached is uploaded again (in the order the flag
 * now names).  All regions of one fabric live on one device. */
int aw_fabric_attach_device(aw_fabric* fabric, int device, uint32_t region_mask);

/* The aw_decode_desc / aw_encode_desc flags that describe the attached device
 * pools: AW_F_COLD_HEAD_BLOCKED when the cold pool is attached head-blocked,
 * else 0. */
uint32_t aw_fabric_device_flags(const aw_fabric* fabric);

/* Device address and size of an attached region (AW_E_INVALID_ARG if it is
 * not attached).  The device copies are ordinary device memory, 256-byte
 * aligned: pass them to aw_decode_desc / aw_encode_desc. */
int aw_fabric_device_region(const aw_fabric* fabric, uint32_t region, void** dptr, uint64_t* bytes);

/* Host -> device copy of bytes [offset, offset + bytes) of an attached region,
 * after host writes to the mapping.  Blocking. */
int aw_fabric_push(aw_fabric* fabric, uint32_t region, uint64_t offset, uint64_t bytes);

/* Device -> host copy of bytes [offset, offset + bytes) of an attached region
 * into the mapping, after device writes; marks the fabric dirty (except for
 * the trace region).  Blocking. */
int aw_fabric_pull(aw_fabric* fabric, uint32_t region, uint64_t offset, uint64_t bytes);

/* Frees the device copies (the mapping is unchanged). */
int aw_fabric_detach_device(aw_fabric* fabric);

/* One Distiller REM cycle (distiller.rs:60-88) on the device copies:
 *   1. the variance proxy of every hot block b < min(8192, hot blocks)
 *      (evaluate_entropy, distiller.rs:97-120; compute_block_entropy :126-159);
 *   2. each block with 0 < proxy < threshold, in ascending order, encoded into
 *      cold block b (distill_block, distiller.rs:171-246, as aw_encode_device
 *      with the per-head dictionary of the dictionary region);
 *   3. the changed cold blocks written back into the mapping, then
 *      aw_fabric_checkpoint (distiller.rs:81-86).
 * Needs HOT, COLD and DICT attached.  `entropy` (may be NULL) receives the
 * min(8192, hot blocks) proxies; n_distilled (may be NULL) the candidate count.
 * The reference's default threshold is 0.15 (types.rs:52, types.rs:483). */
int aw_fabric_distill(aw_fabric* fabric, aw_engine* engine, float threshold, float* entropy,
                      uint32_t* n_distilled);

#ifdef __cplusplus
}
#endif

#endif /* AETHER_FABRIC_H */
