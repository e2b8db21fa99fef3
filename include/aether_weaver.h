/*
 * aether_weaver.h — C ABI of the MI355X (gfx950) Weaver decode library.
 *
 * Weaver decode is GQA decode attention over two KV pools:
 *   - a hot pool of exact f16 rows, blocks of 16 tokens  [blocks][16][kv_heads][head_dim];
 *   - a cold pool of 16-byte SparseCodes (4 dictionary atom indices + 4 f16
 *     coefficients per token and kv head)              [blocks][16][kv_heads],
 *     attended directly on the codes, without decompression.
 * Blocks are addressed through a block table ("loom refs"): hot refs first,
 * then cold refs; the physical block is ref & 0x7FFFFFFF.
 *
 * The reference dispatches one Metal kernel through a Rust engine:
 *   nexus-core/src/weaver.rs:85        WeaverEngine::new(metallib_path)
 *   nexus-core/src/weaver.rs:139-237   WeaverEngine::decode(q_exact, q_latent, hot_pool,
 *                                        cold_pool, loom_refs, dictionary, params)
 *   nexus-core/src/weaver.rs:314-321   device_name(), max_threads_per_threadgroup()
 *   nexus-core/src/weaver_kernel.metal:118-240  weaver_decode (8 buffer bindings)
 * Each entry point below names the reference interface it replaces.  All
 * pointers are plain host or device pointers; no framework types cross this
 * boundary.  Every function returns AW_OK (0) or a negative AW_E_* code; the
 * engine keeps a text description of the last failure (aw_engine_last_error).
 *
 * Threading: calls on one engine must be serialised by the caller (the
 * reference's decode takes &mut self, weaver.rs:139).  Use one engine per
 * host thread, or lock around it.
 */
#ifndef AETHER_WEAVER_H
#define AETHER_WEAVER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AW_ABI_VERSION 2u

/* ---- status codes -------------------------------------------------------- */
#define AW_OK             0
#define AW_E_INVALID_ARG (-1) /* bad geometry, null pointer, short buffer          */
#define AW_E_ALIGN       (-2) /* SparseCode pointer not 16-byte aligned            */
#define AW_E_OOB         (-3) /* block ref or atom index beyond its buffer         */
#define AW_E_HIP         (-4) /* HIP runtime failure (no device, launch, copy ...) */
#define AW_E_LOAD        (-5) /* kernels for this device are not in the library    */
#define AW_E_UNSUPPORTED (-6) /* valid request the library does not implement      */

/* ---- reference layouts ---------------------------------------------------- */

/* One token's compressed K(=V) row for one kv head: V = sum_k coeffs[k] * D[indices[k]].
 * 16 bytes, little-endian: u16 indices[4] at bytes 0-7, IEEE binary16 coeffs[4]
 * at bytes 8-15.  Replaces SparseCode (nexus-core/src/types.rs:218-228,
 * weaver_kernel.metal:34-37).  Coefficients are carried as raw binary16 bits. */
typedef struct aw_sparse_code {
    uint16_t indices[4];
    uint16_t coeffs[4];
} aw_sparse_code;

/* Dispatch parameters, 12 x u32 = 48 bytes in the reference field order.
 * Replaces WeaverParams (nexus-core/src/types.rs:351-374, weaver_kernel.metal:40-51).
 * hot_count / cold_count are numbers of 16-token blocks. */
typedef struct aw_weaver_params {
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t block_size;  /* must be 16 */
    uint32_t gqa_group;   /* q_heads / kv_heads */
    uint32_t hot_count;
    uint32_t cold_count;
    uint32_t dict_size;
    uint32_t sparsity_k;  /* must be 4 */
    uint32_t _pad[3];
} aw_weaver_params;

/* ---- device-resident, batched / multi-query request ------------------------ */

/* Flags for aw_decode_desc.flags. */
#define AW_F_CAUSAL 1u /* query j of Q sees hot tokens p < n_hot_tokens - Q + 1 + j
                          (the rule of nexus-core/src/ops.metal:549); cold tokens are
                          all older than the drafts and always visible */
#define AW_F_COLD_HEAD_BLOCKED 2u /* cold pool laid out [L][cold_blocks][kv_heads][16]:
                          each kv head's 16 codes of a block contiguous (256 bytes).
                          No reference counterpart: the reference pool is
                          [blocks][16][kv_heads] (fabric.rs:124-186), where one kv
                          head's code is 16 bytes of every 128-byte token line, so a
                          cold work-group reads a 64-byte sector per code.  For
                          producers that can write it (an encoder on the device),
                          the head-blocked order reads whole sectors; the results
                          are identical bit for bit. */
/* aw_encode_desc only: score every atom exactly (the plain sequential scan)
 * instead of an MFMA prefilter with exact rescoring of the atoms that can reach
 * the top 4.  Both give the same codes; the scan is the slower reference form. */
#define AW_F_ENCODE_FULL_SCAN 4u
/* aw_decode_desc: seq_hot entries count hot TOKENS (<= hot_count * 16) instead
 * of blocks, so a sequence may end inside its last block (the reference's
 * contiguous KV cache, inference.rs:470-483).  Needs seq_hot. */
#define AW_F_SEQ_HOT_TOKENS 8u
/* aw_decode_desc: when q_latent is NULL (computed on the device), keep it in
 * fp32 (workspace and the cold kernel's LDS table) instead of rounding it to
 * f16 like the reference's q_latent buffer (weaver_kernel.metal:111).  A
 * score moves by up to 2^-11 of sum_k |c_k q_latent[idx_k]| under f16
 * rounding; peaked softmaxes (large coefficients, large q) amplify that past
 * the 2e-3 tolerance.  Costs about a tenth of the cold kernel's time (16-byte
 * table reads per term instead of 8).  Ignored when q_latent is given. */
#define AW_F_QLATENT_F32 16u

/* One decode call over L layers x B sequences x Q query tokens.  All pointers
 * are DEVICE pointers.  Element layouts (f16 = raw binary16 bits):
 *   q        [L][B][Q][q_heads][head_dim]
 *   q_latent [L][B][Q][q_heads][dict_size] or NULL (then q . D^T is computed
 *            on the device, fp32 accumulation, stored as f16 like the
 *            reference's q_latent buffer, weaver_kernel.metal:111, or kept in
 *            fp32 with AW_F_QLATENT_F32)
 *   hot_k    [L][hot_blocks][16][kv_heads][head_dim]
 *   hot_v    same as hot_k, or NULL: V is the K row (reference, metal:162-166)
 *   cold     [L][cold_blocks][16][kv_heads]   (16-byte aligned; with
 *            AW_F_COLD_HEAD_BLOCKED [L][cold_blocks][kv_heads][16])
 *   refs     [L][B][refs_stride]: hot refs [0, hot_count), cold refs
 *            [hot_count, hot_count + cold_count) of each sequence
 *   seq_hot, seq_cold  optional [L][B] per-sequence block counts
 *            (<= hot_count / cold_count); NULL = every sequence uses the maximum;
 *            with AW_F_SEQ_HOT_TOKENS seq_hot counts tokens
 *   dict     [L][dict_heads][dict_size][head_dim]; dict_heads is 1 (one shared
 *            dictionary) or kv_heads (the reference's per-kv-head dictionary,
 *            weaver_kernel.metal:212-215)
 *   out      [L][B][Q][q_heads][head_dim]
 * scale multiplies every score; 1.0 reproduces the reference, which applies
 * none (weaver_kernel.metal:153-160,186-190).
 * Hot pools: a sequence's hot tokens run in at most 64 splits of at most 4096
 * blocks, so hot_count (or hot_tokens / 16) may reach 262144 blocks = 4 Mi
 * tokens per sequence; the reference Fabric holds MAX_HOT_BLOCKS = 8192
 * (types.rs:500).  Larger requests return AW_E_UNSUPPORTED.
 * hot_tokens: 0, or the hot tokens of every sequence (1 .. hot_count * 16);
 * hot tokens past it are neither scored nor read as values (nor past a
 * seq_hot entry).  Loads still cover whole blocks, so the pool must hold every
 * referenced block in full. */
typedef struct aw_decode_desc {
    uint32_t layers, batch, queries;
    uint32_t q_heads, kv_heads, head_dim;
    uint32_t dict_size, dict_heads;
    uint32_t hot_count, cold_count;   /* max blocks per sequence */
    uint32_t refs_stride;             /* >= hot_count + cold_count */
    uint32_t flags;
    float    scale;
    uint32_t hot_tokens;              /* 0 = hot_count * 16 */
    uint64_t hot_blocks, cold_blocks; /* pool capacity per layer, in blocks */
    const uint16_t*       q;
    const uint16_t*       q_latent;
    const uint16_t*       hot_k;
    const uint16_t*       hot_v;
    const aw_sparse_code* cold;
    const uint32_t*       refs;
    const uint32_t*       seq_hot;
    const uint32_t*       seq_cold;
    const uint16_t*       dict;
    uint16_t*             out;
} aw_decode_desc;

/* How a request is split across the GPU; filled by aw_decode_plan. */
typedef struct aw_decode_plan_info {
    uint32_t rows_per_kv_head;   /* R = gqa_group * queries */
    uint32_t hot_splits;         /* work items per (layer, seq, kv head) on the hot pool */
    uint32_t hot_tokens_per_split;
    uint32_t cold_splits;
    uint32_t cold_tokens_per_split;
    uint32_t cold_row_chunk;     /* query rows binned together in one cold work-group */
    uint32_t computes_q_latent;  /* 1 when q . D^T runs on the device */
    uint32_t projection;         /* its kernel by the planner's choice: AW_PROJECT_MFMA or _VALU (0: none) */
    uint64_t workspace_bytes;    /* device scratch this request needs */
    uint32_t cold_output;        /* what the cold kernel writes: AW_COLD_OUT_BINS or _VALUES (0: no cold pool) */
    uint32_t reserved;
} aw_decode_plan_info;

/* Kernel stages, for aw_engine_stage_stats. */
#define AW_STAGE_PROJECT 0 /* q_latent = q . D^T (MFMA) */
#define AW_STAGE_HOT     1 /* split-K exact attention over the hot pool (MFMA) */
#define AW_STAGE_COLD    2 /* scores on the codes + per-atom softmax-weight bins */
#define AW_STAGE_FINISH  3 /* bins . D (MFMA); fused log-sum-exp merge when it fits */
#define AW_STAGE_MERGE   4 /* log-sum-exp merge of hot and cold partials, f16 out */
#define AW_STAGE_COUNT   5

typedef struct aw_engine aw_engine;

/* ---- pure host functions (no GPU needed) ---------------------------------- */

/* ABI version and sizeof() of the public structs, for bindings to check their
 * layouts: sizes[0..3] = aw_sparse_code, aw_weaver_params, aw_decode_desc,
 * aw_decode_plan_info.  No reference counterpart. */
uint32_t aw_abi_version(void);
void     aw_abi_struct_sizes(size_t sizes[4]);

/* Text for a status code.  No reference counterpart (the reference returns String). */
const char* aw_status_string(int status);

/* Validate reference parameters against the slice lengths that
 * WeaverEngine::decode receives (weaver.rs:139-148), including every block ref
 * and every referenced atom index.  The reference validates nothing and reads
 * past short buffers; this library rejects such calls before launch.
 * msg (may be NULL) receives a description of the first failure. */
int aw_validate_params(const aw_weaver_params* params,
                       size_t n_q_exact, size_t n_q_latent, size_t n_hot_pool,
                       const aw_sparse_code* cold_pool, size_t n_cold_pool,
                       const uint32_t* loom_refs, size_t n_loom_refs,
                       size_t n_dictionary, size_t n_out,
                       char* msg, size_t msg_len);

/* Validate a device request's geometry and report how it will be split and how
 * much scratch it needs.  Reads only the numeric fields of desc. */
int aw_decode_plan(const aw_decode_desc* desc, aw_decode_plan_info* info,
                   char* msg, size_t msg_len);

/* ---- engine ------------------------------------------------------------------ */

/* Replaces WeaverEngine::new (weaver.rs:85-132): selects HIP device `device`,
 * checks that the library holds gfx950 kernels for it, creates the engine's
 * stream and persistent buffers.  The reference's metallib path becomes the
 * path of this shared library, which the host loads (dlopen) before calling. */
int  aw_engine_create(int device, aw_engine** out);
void aw_engine_destroy(aw_engine* engine);

/* Last failure on this engine (engine-owned, valid until the next call). */
const char* aw_engine_last_error(const aw_engine* engine);

/* Replaces WeaverEngine::device_name (weaver.rs:314-316). */
const char* aw_engine_device_name(const aw_engine* engine);

/* Replaces WeaverEngine::max_threads_per_threadgroup (weaver.rs:319-321). */
uint64_t aw_engine_max_threads_per_threadgroup(const aw_engine* engine);

/* Replaces WeaverEngine::decode (weaver.rs:139-237) with the same semantics:
 * host slices are copied into engine-owned device buffers that grow only on
 * overflow (weaver.rs:241-311), one decode of one token runs with
 * reference-literal math (no score scale, per-kv-head dictionary
 * [kv_heads][dict_size][head_dim], bit 31 of refs masked), the call waits for
 * the GPU and copies q_heads*head_dim f16 values to `out`.
 * q_latent may be NULL (n_q_latent 0): it is then computed as q . D^T on the
 * device.  Zero-length slices are allowed where the params need no data. */
int aw_decode(aw_engine* engine,
              const uint16_t* q_exact, size_t n_q_exact,
              const uint16_t* q_latent, size_t n_q_latent,
              const uint16_t* hot_pool, size_t n_hot_pool,
              const aw_sparse_code* cold_pool, size_t n_cold_pool,
              const uint32_t* loom_refs, size_t n_loom_refs,
              const uint16_t* dictionary, size_t n_dictionary,
              const aw_weaver_params* params,
              uint16_t* out, size_t n_out);

/* Device-resident batched / multi-query / multi-layer decode, asynchronous on
 * `hip_stream` (a hipStream_t; NULL is HIP's null stream).  Extends the
 * reference kernel (weaver_kernel.metal:118-240) with batch, queries, layers,
 * causal drafts, score scale, shared dictionary and separate V.  Scratch comes
 * from an engine-owned workspace that grows on demand (the growth allocates).
 * Block refs and atom indices are checked on the device: a bad one is skipped
 * and recorded; aw_engine_check_device_errors reports it.
 * The call may be captured into a HIP graph (stream capture): the graph keeps
 * the workspace that call used, and the engine frees no workspace before
 * aw_engine_destroy, so later, larger calls leave captured graphs valid.  A
 * call being captured cannot grow the workspace (that allocates): it returns
 * AW_E_UNSUPPORTED, enqueueing nothing; make one eager call of the same (or a
 * larger) request first.
 * Replays and other calls on one engine share that workspace: run them one at
 * a time (stream-ordered, or synchronised between). */
int aw_decode_device(aw_engine* engine, const aw_decode_desc* desc, void* hip_stream);

/* No reference counterpart.  For callers that cannot allocate device memory:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  The same decode as aw_decode_device (same kernels, same output
 * bits), but it allocates nothing: its scratch is a fixed device array of
 * AW_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the
 * process ends (its address is looked up once per device, at
 * aw_engine_create).  A request whose scratch (aw_decode_plan_info.
 * workspace_bytes) exceeds it returns AW_E_UNSUPPORTED: 96 MiB covers a
 * one-layer decode of 64 sequences at hot 2048 + cold 32768 tokens (55.1 MiB),
 * not two such layers in one call (106.2 MiB) nor a 32-layer call.  Stage timing (aw_engine_set_profiling) is
 * not recorded for these calls.  Every call on one GPU, from any engine,
 * shares that GPU's array and leaves its contents behind: calls (and graph
 * replays) that overlap on one GPU race; order them on one stream or
 * synchronise between them. */
#define AW_NOALLOC_SCRATCH_BYTES ((uint64_t)96 << 20)
int aw_decode_device_noalloc(aw_engine* engine, const aw_decode_desc* desc, void* hip_stream);

/* Replaces Ops::multihead_attention (nexus-core/src/ops.rs:433-462, kernel
 * ops.metal:528-616), the attention of InferenceEngine::forward_batch
 * (inference.rs:546-556): causal GQA attention of num_queries new tokens over
 * a contiguous KV cache, asynchronous on `hip_stream`.  Device pointers, f16:
 *   q                [num_queries][q_heads][head_dim]
 *   k_cache, v_cache [cache_tokens][kv_heads][head_dim] (positions 0 .. kv_len-1 hold
 *                    the sequence, the new tokens last, as forward_batch writes them)
 *   out              [num_queries][q_heads][head_dim]
 * Query i sees cache positions p < kv_len - num_queries + 1 + i (ops.metal:549),
 * scores scaled by 1/sqrt(head_dim) (ops.metal:557).  The cache is read as the
 * hot pool (16-token blocks, identity block table), so cache_tokens must cover
 * kv_len rounded up to 16 (the reference allocates MAX_SEQ_LEN = 4096 tokens,
 * inference.rs:219,256-266).  Unlike the reference (threadgroup scores[4096],
 * ops.metal:564) kv_len is not limited to 4096: it may reach 4 Mi positions
 * (the hot-pool limit of aw_decode_device), and kv_len + 1 < num_queries is
 * rejected instead of wrapping.  Queries beyond 64 / (q_heads / kv_heads) per
 * call are processed in consecutive groups.  Like aw_decode_device, a call
 * being captured into a HIP graph cannot grow the engine's workspace or its
 * block table: make one eager call with that kv_len (or longer) first. */
int aw_multihead_attention_device(aw_engine* engine, const uint16_t* q, const uint16_t* k_cache,
                                  const uint16_t* v_cache, uint16_t* out, uint32_t kv_len,
                                  uint32_t head_dim, uint32_t q_heads, uint32_t kv_heads,
                                  uint32_t num_queries, uint64_t cache_tokens, void* hip_stream);

/* Wait for `hip_stream` and report AW_E_OOB if any kernel since the last check
 * met an out-of-range block ref or atom index (then clears the record). */
int aw_engine_check_device_errors(aw_engine* engine, void* hip_stream);

/* Bit-exact SparseCode decode and atom gather, for testing the codec on the
 * device: for code i and slot k, idx[4i+k] = indices[k], coef[4i+k] =
 * (float)coeffs[k], atoms[(4i+k)*head_dim + j] = dict[indices[k]*head_dim + j]
 * (raw bits).  Device pointers; the dictionary is one [dict_size][head_dim]
 * table.  Indices >= dict_size yield atoms of 0xFFFF and are recorded like
 * aw_decode_device.  Mirrors the gathers of weaver_kernel.metal:182-216. */
int aw_debug_gather_codes(aw_engine* engine, const aw_sparse_code* codes, size_t n_codes,
                          const uint16_t* dict, uint32_t dict_size, uint32_t head_dim,
                          uint32_t* idx, float* coef, uint16_t* atoms, void* hip_stream);

/* ---- SparseCode encoder (distillation of hot blocks) ------------------------ */

/* One encoder request over n_blocks hot blocks.  All pointers are DEVICE
 * pointers.  Element layouts (f16 = raw binary16 bits):
 *   hot        [hot_blocks][16][kv_heads][head_dim] f16 (the hot pool, fabric.rs:131-134)
 *   dict       [dict_heads][dict_size][head_dim] f16; dict_heads is kv_heads (the
 *              reference's per-kv-head dictionary, distiller.rs:201-202) or 1 (shared)
 *   src_blocks [n_blocks] hot block indices to encode (bit 31 masked, as in a ref)
 *   dst_blocks [n_blocks] cold block indices that receive the codes, or NULL: the
 *              source index (distiller.rs:177 writes hot block b's codes at cold block b)
 *   cold       [cold_blocks][16][kv_heads] SparseCodes; with AW_F_COLD_HEAD_BLOCKED
 *              [cold_blocks][kv_heads][16]
 *   entropy    optional [n_blocks] f32: the block's variance proxy (distiller.rs:126-159)
 * flags: 0, AW_F_COLD_HEAD_BLOCKED, AW_F_ENCODE_FULL_SCAN (either or both). */
typedef struct aw_encode_desc {
    uint32_t kv_heads, head_dim, dict_size, dict_heads;
    uint32_t n_blocks, flags;
    uint64_t hot_blocks, cold_blocks;
    const uint16_t*  hot;
    const uint16_t*  dict;
    const uint32_t*  src_blocks;
    const uint32_t*  dst_blocks;
    aw_sparse_code*  cold;
    float*           entropy;
} aw_encode_desc;

/* sizeof(aw_encode_desc), for bindings to check their layout.  No reference counterpart. */
size_t aw_abi_encode_desc_size(void);

/* Replaces Distiller::distill_block (distiller.rs:171-246) for a batch of
 * blocks, asynchronous on `hip_stream`.  For every token t and kv head g of
 * each source block, with x = hot[b][t][g][:] and D = the dictionary of head g:
 *   s_a = sum_j f32(x_j) * f32(D[a][j]), summed in j order from -0.0 in f32
 *         (distiller.rs:212-216; Rust >= 1.82 folds f32 sums from -0.0,
 *         rust-version 1.85 in Cargo.toml), exactly: each step is one FMA of an
 *         exact f16 x f16 product;
 *   the 4 atoms with the largest s_a, ordered by s_a descending and, among
 *   equal scores, by atom index ascending (a stable order; the reference's
 *   sort_unstable_by at distiller.rs:221-223 leaves ties unordered, and its
 *   test at :299-307 expects indices [0,1,2,3] for equal scores); NaN and
 *   -inf scores are never chosen (a slot left unfilled holds the zero code's
 *   index 0 and coefficient 0);
 *   code = {indices: those atoms, coeffs: f16(s_a) rounded to nearest even}
 *   (distiller.rs:225-233), written to the destination block, token t, head g.
 * When `entropy` is set it also writes each block's variance proxy: the mean
 * and variance of its f16 values summed in f64 in memory order, returned as f32,
 * 0 for an all-zero block (distiller.rs:126-159). */
int aw_encode_device(aw_engine* engine, const aw_encode_desc* desc, void* hip_stream);

/* Host-slice form of aw_encode_device with copy-in / copy-out and a blocking
 * wait, for a host that owns the pools in memory (the mmap'd Fabric,
 * fabric.rs:359-379).  Sizes count elements: n_hot and n_dict f16 values,
 * n_cold SparseCodes.  `hot` holds whole blocks, `dict` dict_heads
 * dictionaries, `cold` whole blocks (read and written back in full),
 * `blocks` the hot block indices to encode (each written to the same cold
 * block index, distiller.rs:177), `entropy` may be NULL. */
int aw_encode(aw_engine* engine,
              const uint16_t* hot, size_t n_hot, const uint16_t* dict, size_t n_dict,
              uint32_t kv_heads, uint32_t head_dim, uint32_t dict_size, uint32_t dict_heads,
              const uint32_t* blocks, size_t n_blocks,
              aw_sparse_code* cold, size_t n_cold, float* entropy);

/* The variance proxy of hot blocks alone, asynchronous on `hip_stream`:
 * entropy[i] = the proxy of hot block blocks[i] & 0x7FFFFFFF (blocks NULL:
 * block i), as aw_encode_device computes it; a block index >= hot_blocks gives
 * 0 and sets the engine's out-of-range flag (aw_engine_check_device_errors).
 * `hot` holds [hot_blocks][16][kv_heads][head_dim] f16, 16-byte aligned.
 * Replaces the per-block loop of Distiller::evaluate_entropy
 * (distiller.rs:97-120). */
int aw_block_entropy_device(aw_engine* engine, const uint16_t* hot, uint64_t hot_blocks, uint32_t kv_heads,
                            uint32_t head_dim, const uint32_t* blocks, uint32_t n_blocks, float* entropy,
                            void* hip_stream);

/* No reference counterpart: a read-only HBM stream, for measuring the
 * attainable read bandwidth beside the 8 TB/s nominal peak (the decode's
 * pools are only read).  Reads `bytes` (a multiple of 16) from the 16-byte
 * aligned device buffer `buf` with 16-byte loads, 8 in flight per lane,
 * `waves_per_cu` waves per CU (a multiple of 4, 4 .. 64), XOR-folding each
 * wave's data into one word; a wave writes its word into `sink` (64 u32,
 * device) only when it equals 0xA5A5A5A5, so the loads cannot be elided and
 * the stream writes (almost) nothing.  Asynchronous on `hip_stream`. */
int aw_debug_read_stream(aw_engine* engine, const void* buf, uint64_t bytes, uint32_t waves_per_cu,
                         uint32_t* sink, void* hip_stream);

/* No reference counterpart: the q_latent = q . D^T projection of a request on
 * its own, for checking it directly.  `desc` is a request that computes
 * q_latent (a cold pool and q_latent NULL); the projection runs as in
 * aw_decode_device and its result, [L][B][Q][Hq][A] f16 (fp32 with
 * AW_F_QLATENT_F32), is copied into `q_latent` (device).  Asynchronous on
 * `hip_stream`; may grow the engine workspace. */
int aw_debug_project(aw_engine* engine, const aw_decode_desc* desc, void* q_latent, void* hip_stream);

/* No reference counterpart: the attainable HBM rate of a decode's own pool
 * reads.  Reads every hot K (and V) row and every cold code of the request
 * `desc` describes (its pools, block refs, counts and cold order; q, dict and
 * out are not used), through the block table, in the pools' layouts, one wave
 * per stretch of 32 hot or 256 cold blocks of a (layer, sequence, kv head),
 * nothing computed; a wave writes its XOR fold into `sink` (64 u32, device)
 * only when it equals 0xA5A5A5A5.  Per-sequence counts (seq_hot, seq_cold) are
 * ignored: every sequence's hot_count and cold_count blocks are read.
 * Asynchronous on `hip_stream`. */
int aw_debug_read_pools(aw_engine* engine, const aw_decode_desc* desc, uint32_t* sink, void* hip_stream);

/* Per-stage kernel timing with HIP events recorded on the stream each kernel
 * runs on: every launch is bracketed by a pair of events.  AW_PROFILE_ON keeps
 * the pipeline as it runs unprofiled (the hot kernel on the engine's side
 * stream, concurrent with q.D^T and the cold kernel); AW_PROFILE_SERIAL runs
 * every stage on the caller's stream, one after another.  No reference
 * counterpart (the reference times whole calls, bench.rs:149-168). */
#define AW_PROFILE_OFF 0
#define AW_PROFILE_ON 1
#define AW_PROFILE_SERIAL 2
int aw_engine_set_profiling(aw_engine* engine, int mode);

/* Which kernel computes q_latent = q . D^T (spec YELLOWPAPER.md:86-92; the
 * reference's caller supplies it, weaver_kernel.metal:111).  AW_PROJECT_AUTO
 * is the planner's choice by rows per dictionary group: MFMA tiles at every
 * row count, the VALU kernel having measured slower at each one (4 rows per
 * group with 512 atoms: 10.9 against 6.6 us; 32 rows with 4096 atoms: 9.0
 * against 6.5; 2048 rows: 56 against 12.3).  AW_PROJECT_MFMA and
 * AW_PROJECT_VALU force one path, for measuring the other.  No reference
 * counterpart. */
#define AW_PROJECT_AUTO 0
#define AW_PROJECT_MFMA 1
#define AW_PROJECT_VALU 2
int aw_engine_set_projection(aw_engine* engine, int mode);

/* What the cold kernel hands on (weaver_kernel.metal:206-222 forms the cold
 * output per token; here it is formed per atom).  AW_COLD_OUT_BINS: per-atom
 * softmax-weight bins, which a finish kernel multiplies by the dictionary on
 * MFMA before the merge.  AW_COLD_OUT_VALUES: each work item multiplies its own
 * bins by the dictionary on MFMA (D^T read from L2) and hands value partials
 * straight to the merge, so no bins reach HBM and no finish runs; only for
 * dictionaries of at most 128 KiB per head with a multiple of 32 atoms (512
 * atoms at head_dim 128), elsewhere bins.  AW_COLD_OUT_AUTO is the planner's
 * choice (values wherever allowed).  Both forms are exact rewrites of the same
 * sums, with the same f16 hi + lo split of the bins.  No reference
 * counterpart. */
#define AW_COLD_OUT_AUTO 0
#define AW_COLD_OUT_BINS 1
#define AW_COLD_OUT_VALUES 2
int aw_engine_set_cold_output(aw_engine* engine, int mode);
int aw_engine_stage_stats(aw_engine* engine, int stage, double* total_ms, uint64_t* launches);
int aw_engine_reset_stage_stats(aw_engine* engine);

#ifdef __cplusplus
}
#endif

#endif /* AETHER_WEAVER_H */
