// weaver_engine.hip — C ABI of the gfx950 Weaver decode library.
//
// Replaces WeaverEngine (nexus-core/src/weaver.rs:31-322): engine creation,
// the reference-compatible host-slice decode, plus a device-resident batched
// entry point.  Kernels live in weaver_kernels.hpp.  There is no CPU fallback:
// without a gfx950 device every compute entry point returns an error.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/aether_fabric.h"
#include "engine_internal.hpp"
#include "weaver_kernels.hpp"

static_assert(sizeof(aw_sparse_code) == 16, "SparseCode is 16 bytes (types.rs:227)");
static_assert(sizeof(aw_weaver_params) == 48, "WeaverParams is 12 x u32 (types.rs:351-374)");
static_assert(offsetof(aw_weaver_params, hot_count) == 20, "WeaverParams field order");
static_assert(offsetof(aw_weaver_params, sparsity_k) == 32, "WeaverParams field order");

namespace {

constexpr uint32_t kBlock = aw::kBlockTokens;
constexpr size_t kAlign = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

void put_msg(char* msg, size_t len, const char* fmt, ...) {
    if (!msg || !len) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, len, fmt, ap);
    va_end(ap);
}

struct DevBuf {
    void* ptr = nullptr;
    size_t cap = 0;
};

// Grow-only device buffer (weaver.rs:252-255 reallocates only on overflow).
int ensure(DevBuf& b, size_t bytes, std::string& err) {
    if (bytes <= b.cap && b.ptr) return AW_OK;
    if (b.ptr) (void)hipFree(b.ptr);
    b.ptr = nullptr;
    b.cap = 0;
    size_t want = std::max<size_t>(align_up(bytes, kAlign), kAlign);
    hipError_t e = hipMalloc(&b.ptr, want);
    if (e != hipSuccess) {
        err = std::string("hipMalloc(") + std::to_string(want) + ") failed: " + hipGetErrorString(e);
        b.ptr = nullptr;
        return AW_E_HIP;
    }
    b.cap = want;
    return AW_OK;
}

// True when `st` is being captured into a HIP graph (then nothing may be
// allocated or copied synchronously on its behalf).
bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// The decode workspace grows like ensure(), but an outgrown buffer is kept
// until the engine is destroyed instead of freed: a decode captured into a HIP
// graph holds the address it was captured with, and a later, larger request
// must not free it under the graph.  Growth is geometric (1.5x), so the kept
// buffers add up to at most twice the largest one.  A call being captured
// cannot grow it: it returns AW_E_UNSUPPORTED, asking for an eager call of
// that size first.
int ensure_keep(DevBuf& b, size_t bytes, std::vector<void*>& retired, std::string& err, hipStream_t st) {
    if (bytes <= b.cap && b.ptr) return AW_OK;
    if (capturing(st)) {
        err = "the workspace must grow to " + std::to_string(bytes) +
              " bytes during stream capture: make one eager call of this size (or larger) before capturing";
        return AW_E_UNSUPPORTED;
    }
    const size_t want = std::max({align_up(bytes, kAlign), kAlign, align_up(b.cap + b.cap / 2, kAlign)});
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        err = std::string("hipMalloc(") + std::to_string(want) + ") failed: " + hipGetErrorString(e);
        return AW_E_HIP;
    }
    if (b.ptr) retired.push_back(b.ptr);
    b.ptr = p;
    b.cap = want;
    return AW_OK;
}

// Workspace sub-allocation offsets for one request.
struct Layout {
    aw_decode_plan_info info{};
    uint32_t rc = 4;       // cold rows per work-group
    uint32_t n_chunks = 1; // ceil(R / rc)
    uint32_t n_ar = 1;     // atom ranges of the finish
    bool sep_merge = false; // a merge kernel after the finish even with one atom range
    bool fin_rows = false; // finish_rows_kernel (16-row tiles, waves over atoms) instead of finish_kernel
    uint32_t atoms_per_range = 0;
    uint32_t tiles_per_group = 0, rows_per_group = 0, n_groups = 0;
    bool qf32 = false;     // q_latent computed on the device, kept in fp32
    bool cold_out = false; // the cold kernel writes value partials for the merge (no bins, no finish)
    size_t cold_smem = 0, w_lds_off = 0; // the cold kernel's LDS bytes; with cold_out, where its W staging starts
    uint32_t part_splits = 0; // partials per row in the hot arrays: hot splits (+ cold splits when cold_out)
    size_t off_ql = 0, off_dt = 0, off_hm = 0, off_hl = 0, off_ho = 0;
    size_t off_cm = 0, off_cl = 0, off_ca = 0, off_cw = 0, off_ocp = 0;
};

bool supported_head_dim(uint32_t d) { return d == 64 || d == 128; }

// Query rows per kv head from which the merge runs as its own kernel after the
// finish, whatever the finish's atom ranges.
constexpr uint32_t kSepMergeRows = 16;
// Cold splits per row before the row chunk is halved instead.
constexpr uint64_t kColdSplitsBeforeRc = 8;
// Largest dictionary head (bytes of f16) for which the cold kernel writes value
// partials (AW_COLD_OUT_VALUES): every work item reads its head's D^T (the
// projection's tiled copy) from L2 once, in place of the bins' round trip through
// HBM and the finish kernel.
constexpr uint64_t kColdOutMaxDictBytes = 128u << 10;

// q . D^T on the vector ALUs (project_valu_kernel: kProjValuTa atoms x
// kProjValuRb rows per work-group) for groups of at most kProjValuRows rows
// sharing a dictionary, on MFMA (project_kernel) above.  0: MFMA at every row
// count.  Measured (serialized, MI355X): 4 rows per group over 512 atoms 10.9
// against 6.6 us; 16 rows 10.5 against 6.6; 32 rows over 4096 atoms 9.0 against
// 6.5; 256 rows 11.1 against 6.7; 2048 rows 56 against 12.3.  At small row
// counts both are a chain of one dictionary load, the products and the stores;
// the MFMA kernel's 512-thread tiles issue more of the loads at once.
constexpr int kProjValuRb = 8;
constexpr int kProjValuTa = 64;
constexpr uint32_t kProjValuRows = 0;

// Row pitches of D^T (halves) and of the cold bins W (floats): one 128-byte line
// of padding, so rows whose natural stride is a power of two (8 or 16 KiB at
// 4096 atoms) spread over the L2 channels instead of landing on one.
uint32_t dt_pitch(uint32_t A) { return A + 64; }
uint32_t w_pitch(uint32_t A) { return A + 32; }

// Buffer loads cover the codes when a layer's pool fits the resource window and
// the largest in-block token offset added to the "no code" offset stays below 2^32.
bool cold_uses_buffer(const aw_decode_desc* d) {
    const uint64_t blk_bytes = (uint64_t)kBlock * d->kv_heads * 16u;
    return d->kv_heads <= 256 && d->cold_blocks * blk_bytes <= aw::kColdWindow;
}

// Largest cold row chunk (1, 2 or 4) whose LDS tables fit (with at least one
// 1024-token split's block refs), for a q_latent table of qbytes per entry.
uint32_t pick_rc(uint32_t R, uint32_t A, size_t max_lds, uint32_t qbytes) {
    uint32_t rc = R >= 4 ? 4 : (R >= 2 ? 2 : 1);
    while (rc > 1 && aw::cold_smem_bytes(A, (int)rc, 1024, qbytes) > max_lds) rc /= 2;
    return rc;
}

// hot_waves_per_cu[rt]: resident hot waves per CU for RT = 1, 2, 4 row tiles (0, 1, 2).
// cold_out_mode: AW_COLD_OUT_* (the engine's setting; AUTO for aw_decode_plan).
int plan(const aw_decode_desc* d, size_t max_lds, uint32_t n_cu, const uint32_t hot_waves_per_cu[3], int cold_out_mode,
         Layout* L, char* msg, size_t mlen) {
    if (!d) {
        put_msg(msg, mlen, "null descriptor");
        return AW_E_INVALID_ARG;
    }
    if (d->layers == 0 || d->batch == 0 || d->queries == 0) {
        put_msg(msg, mlen, "layers, batch and queries must be >= 1");
        return AW_E_INVALID_ARG;
    }
    if (d->kv_heads == 0 || d->q_heads == 0 || d->q_heads % d->kv_heads) {
        put_msg(msg, mlen, "q_heads (%u) must be a positive multiple of kv_heads (%u)", d->q_heads, d->kv_heads);
        return AW_E_INVALID_ARG;
    }
    if (!supported_head_dim(d->head_dim)) {
        put_msg(msg, mlen, "head_dim %u unsupported (64 or 128)", d->head_dim);
        return AW_E_UNSUPPORTED;
    }
    const uint32_t G = d->q_heads / d->kv_heads;
    const uint64_t R64 = (uint64_t)G * d->queries;
    if (R64 > 64) {
        put_msg(msg, mlen, "gqa_group*queries = %llu exceeds 64 query rows per kv head",
                (unsigned long long)R64);
        return AW_E_UNSUPPORTED;
    }
    const uint32_t R = (uint32_t)R64;
    if (d->refs_stride < (uint64_t)d->hot_count + d->cold_count) {
        put_msg(msg, mlen, "refs_stride %u < hot_count + cold_count", d->refs_stride);
        return AW_E_INVALID_ARG;
    }
    constexpr uint32_t kKnown = AW_F_CAUSAL | AW_F_COLD_HEAD_BLOCKED | AW_F_SEQ_HOT_TOKENS | AW_F_QLATENT_F32;
    if (d->flags & ~kKnown) {
        put_msg(msg, mlen, "unknown flags 0x%x", d->flags & ~kKnown);
        return AW_E_INVALID_ARG;
    }
    if ((uint64_t)d->hot_tokens > (uint64_t)d->hot_count * kBlock) {
        put_msg(msg, mlen, "hot_tokens %u exceeds hot_count * 16 (%llu)", d->hot_tokens,
                (unsigned long long)d->hot_count * kBlock);
        return AW_E_INVALID_ARG;
    }
    if (!(d->scale == d->scale) || std::isinf(d->scale)) {
        put_msg(msg, mlen, "scale must be finite");
        return AW_E_INVALID_ARG;
    }
    if (d->cold_count > 0) {
        if (d->dict_size == 0 || d->dict_size > 65536 || d->dict_size % 16) {
            put_msg(msg, mlen, "dict_size %u must be a multiple of 16 in [16, 65536]", d->dict_size);
            return AW_E_UNSUPPORTED;
        }
        if (d->dict_heads != 1 && d->dict_heads != d->kv_heads) {
            put_msg(msg, mlen, "dict_heads must be 1 (shared) or kv_heads");
            return AW_E_INVALID_ARG;
        }
    }
    const uint64_t n_lbg = (uint64_t)d->layers * d->batch * d->kv_heads;
    const uint32_t HD = d->head_dim, A = d->dict_size;
    Layout& o = *L;
    o = Layout{};
    o.info.rows_per_kv_head = R;
    o.info.computes_q_latent = (d->cold_count > 0 && d->q_latent == nullptr) ? 1u : 0u;
    // Computed on the device, q_latent is rounded to f16 like the reference's
    // buffer, or kept in fp32 on request (workspace and the cold kernel's LDS
    // table): f16 rounding moves a score by up to 2^-11 of sum_k |c_k q_latent[idx_k]|.
    o.qf32 = o.info.computes_q_latent != 0 && (d->flags & AW_F_QLATENT_F32) != 0;
    if (o.info.computes_q_latent) {
        const uint32_t per_group = d->batch * d->queries * (d->dict_heads == 1 ? d->q_heads : d->q_heads / d->kv_heads);
        o.info.projection = per_group <= kProjValuRows ? AW_PROJECT_VALU : AW_PROJECT_MFMA;
    }
    const uint32_t qbytes = o.qf32 ? 4u : 2u;

    // Hot: one round of waves filling the resident capacity, splits <= kMaxSplits.
    if (d->hot_count > 0) {
        const uint64_t n_tok = d->hot_tokens ? d->hot_tokens : (uint64_t)d->hot_count * kBlock;
        // Beside the cold kernel (one 8-wave work-group per CU) one hot wave per SIMD fits.
        uint32_t wpc = hot_waves_per_cu[R <= 16 ? 0 : (R <= 32 ? 1 : 2)];
        if (d->cold_count > 0) wpc = std::min(wpc, 4u);
        uint64_t want = cdiv((uint64_t)n_cu * std::max(1u, wpc), n_lbg);
        // Beside the cold kernel, splits of at most ~512 tokens (B = 64 sweep: 4 splits of
        // 512 tokens 0.159 ms, 2 of 1024 0.164 ms; B = 32: 4 of 512 0.089 ms, 8 of 256 0.092 ms).
        if (d->cold_count > 0) want = std::max<uint64_t>(want, cdiv(n_tok, 512));
        // >= 64 tokens per wave: alone, one-sequence attention 11.9 -> 11.1 us per layer
        // against 128; beside the cold kernel's value partials the cache's decode 31.05 ->
        // 30.6 us per layer and verify 43.5 -> 41.9, beside its bins B = 2 40.6 -> 39.9 us
        // and B = 4 44.9 -> 44.4 (other batches unchanged).
        const uint64_t cap = std::max<uint64_t>(1, cdiv(n_tok, 64));
        const uint64_t S = std::max<uint64_t>(1, std::min<uint64_t>({want, cap, (uint64_t)aw::kMaxSplits}));
        // A split's block refs are staged in the hot kernel's LDS (4 bytes each,
        // sized per launch): at most kMaxHotSplitBlocks, so 64 splits cover
        // 64 * 4096 blocks = 4 Mi tokens per sequence.
        const uint64_t tps = align_up(cdiv(n_tok, S), 32);
        if (tps > (uint64_t)aw::kMaxHotSplitBlocks * kBlock) {
            put_msg(msg, mlen, "hot pool of %llu tokens exceeds %d splits of %u blocks (%llu tokens per sequence)",
                    (unsigned long long)n_tok, aw::kMaxSplits, aw::kMaxHotSplitBlocks,
                    (unsigned long long)aw::kMaxSplits * aw::kMaxHotSplitBlocks * kBlock);
            return AW_E_UNSUPPORTED;
        }
        o.info.hot_tokens_per_split = (uint32_t)tps;
        o.info.hot_splits = cdiv(n_tok, tps);
    }
    // Cold: one work-group per CU at a time (LDS bound), one round of work-groups;
    // >= 1024 tokens per split.
    if (d->cold_count > 0) {
        o.rc = pick_rc(R, A, max_lds, qbytes);
        if (aw::cold_smem_bytes(A, (int)o.rc, 1024, qbytes) > max_lds) {
            put_msg(msg, mlen, "dict_size %u needs %zu bytes of LDS, device allows %zu", A,
                    aw::cold_smem_bytes(A, (int)o.rc, 1024, qbytes), max_lds);
            return AW_E_UNSUPPORTED;
        }
        const uint64_t n_tok = (uint64_t)d->cold_count * kBlock;
        // Splits per (layer, sequence, kv head, row chunk) item for a chunk of rc rows:
        // >= 1024 tokens per split, and bin partials (A*rc*4 bytes per split, written here
        // and read again by the finish) at most half the code bytes of the sequence.
        // A row with many cold splits costs the finish ~0.6 us per split (it combines
        // their factors and bins), so while the row chunk can still shrink, at most
        // kColdSplitsBeforeRc splits: a one-sequence decode over 512-atom per-kv-head
        // dictionaries measured 51.6 us with rc 4 x 32 splits, 44.9 with 4 x 16,
        // 38.1 with 2 x 8 and 35.3 with 1 x 8.  One-row chunks take half a round of
        // work-groups, each with twice the tokens: the cache's one-sequence decode over
        // those dictionaries 30.6 -> 28.5 us per layer, the B = 1 step over a shared
        // 4096-atom dictionary 36.8 -> 35.5 us (a quarter of a round: 32.1 and 39.8;
        // the sweep's batches of 2-64 sequences keep chunks of 2 or 4 rows).
        auto splits_for = [&](uint32_t rc) {
            const uint64_t items = n_lbg * cdiv(R, rc);
            const uint64_t want = std::max<uint64_t>(1, cdiv((uint64_t)n_cu, items) / (rc == 1 ? 2u : 1u));
            const uint64_t cap = std::max<uint64_t>(
                1, std::min<uint64_t>(cdiv(n_tok, 1024), (n_tok * 16) / ((uint64_t)A * rc * 4 * 2)));
            const uint64_t lim = rc > 1 ? kColdSplitsBeforeRc : (uint64_t)aw::kMaxSplits;
            return std::max<uint64_t>(1, std::min<uint64_t>({want, cap, lim, (uint64_t)aw::kMaxSplits}));
        };
        // Too few work-groups to fill the CUs: smaller row chunks (each item then reads
        // the codes again, but does less work per token and allows more splits).
        while (o.rc > 1 && n_lbg * cdiv(R, o.rc) * splits_for(o.rc) < (uint64_t)n_cu) o.rc /= 2;
        o.n_chunks = cdiv(R, o.rc);
        // Splits of at least 8192 tokens once the chunk is chosen: each split's set-up,
        // plan, reductions and write-out are paid per item (B = 2, 2-row chunks: 8 -> 4
        // splits, 42.4 -> 40.5 us; the cache's verify step, 4-row chunks: 8 -> 4 splits,
        // 41.7 -> 39.0 us per layer; batches whose splits already hold 8192 tokens or more
        // unchanged, and halving those was slower: B = 8 53.5 -> 57.7 us, B = 16 66.5 -> 76.6).
        uint64_t S = std::min<uint64_t>(splits_for(o.rc), std::max<uint64_t>(1, n_tok / 8192));
        uint64_t tps = align_up(cdiv(n_tok, S), 16);
        // The split's block refs live in LDS too: shorten splits until they fit.
        while (tps > 1024 && aw::cold_smem_bytes(A, (int)o.rc, (uint32_t)tps, qbytes) > max_lds) {
            ++S;
            tps = align_up(cdiv(n_tok, S), 16);
        }
        if (cdiv(n_tok, tps) > (uint64_t)aw::kMaxSplits) {
            put_msg(msg, mlen, "cold pool of %llu tokens needs more than %d splits", (unsigned long long)n_tok,
                    aw::kMaxSplits);
            return AW_E_UNSUPPORTED;
        }
        o.info.cold_tokens_per_split = (uint32_t)tps;
        o.info.cold_splits = cdiv(n_tok, tps);
        o.info.cold_row_chunk = o.rc;
        // Finish tiles: groups of rows that share one dictionary.
        const uint32_t dh = d->dict_heads;
        const uint32_t hg = dh == 1 ? d->kv_heads : 1;
        o.rows_per_group = d->batch * hg * R;
        o.tiles_per_group = cdiv(o.rows_per_group, (uint32_t)aw::kFinishRows);
        o.n_groups = d->layers * dh;
        // About one 8-wave work-group per CU, >= 64 atoms (one super-chunk) per range:
        // a finish work-group is latency-bound per super-chunk, so small batches
        // take many short ranges.
        const uint64_t tiles = (uint64_t)o.tiles_per_group * o.n_groups;
        uint32_t n_ar = 1;
        if (tiles < (uint64_t)n_cu) n_ar = (uint32_t)std::min<uint64_t>(cdiv((uint64_t)n_cu, tiles), std::max(1u, A / 64));
        // One cold split per row and at least a quarter of a work-group per CU of
        // 16-row tiles: finish_rows_kernel, 16 rows per work-group over an atom
        // range, as many ranges as fill the CUs once.
        const uint64_t tiles16 = (uint64_t)cdiv(o.rows_per_group, 16u) * o.n_groups;
        if (o.info.cold_splits == 1 && A % 32 == 0 && tiles16 * 4 >= (uint64_t)n_cu) {
            o.fin_rows = true;
            n_ar = (uint32_t)std::min<uint64_t>(cdiv((uint64_t)n_cu, tiles16), std::max(1u, A / 256));
        }
        o.atoms_per_range = (uint32_t)align_up(cdiv(A, n_ar), 32);
        o.n_ar = cdiv(A, o.atoms_per_range);
        // Many rows per kv head: the hot kernel, starved of LDS beside the cold
        // kernel, ends after it (32-layer verify, R = 32: 4.97 against 4.70 ms), so
        // the finish does not merge and wait for it; a merge kernel follows.
        o.sep_merge = o.n_ar > 1 || (R >= kSepMergeRows && o.info.hot_splits > 0);
        // Value partials from the cold kernel: small dictionary heads, and room for
        // the cold splits beside the hot ones in the merge's partials.
        o.cold_out = cold_out_mode != AW_COLD_OUT_BINS && (uint64_t)A * HD * 2 <= kColdOutMaxDictBytes && A % 32 == 0 &&
                     (uint64_t)o.info.hot_splits + o.info.cold_splits <= (uint64_t)aw::kMaxSplits &&
                     cold_uses_buffer(d);
        o.info.cold_output = o.cold_out ? AW_COLD_OUT_VALUES : AW_COLD_OUT_BINS;
        o.cold_smem = aw::cold_smem_bytes(A, (int)o.rc, o.info.cold_tokens_per_split, qbytes);
        if (o.cold_out) { // the bins' f16 hi + lo terms staged after the tables (A * rc * 4 bytes)
            o.w_lds_off = align_up(o.cold_smem, 16);
            o.cold_smem = o.w_lds_off + (size_t)A * o.rc * 4;
            if (o.cold_smem > max_lds) o.cold_out = false;
            o.info.cold_output = o.cold_out ? AW_COLD_OUT_VALUES : AW_COLD_OUT_BINS;
            if (!o.cold_out) o.cold_smem = aw::cold_smem_bytes(A, (int)o.rc, o.info.cold_tokens_per_split, qbytes);
        }
    }
    o.part_splits = o.info.hot_splits + (o.cold_out ? o.info.cold_splits : 0u);

    // Workspace layout.
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t at = off;
        off = align_up(off + bytes, kAlign);
        return at;
    };
    if (o.info.computes_q_latent) o.off_ql = take((uint64_t)d->layers * d->batch * d->queries * d->q_heads * A * qbytes);
    if (d->cold_count > 0) o.off_dt = take((uint64_t)d->layers * d->dict_heads * dt_pitch(A) * HD * 2);
    if (o.part_splits) {
        const uint64_t n = n_lbg * o.part_splits * R;
        o.off_hm = take(n * 4);
        o.off_hl = take(n * 4);
        o.off_ho = take(n * HD * 4);
    }
    if (o.info.cold_splits && !o.cold_out) {
        const uint64_t n = n_lbg * o.info.cold_splits * R;
        o.off_cm = take(n * 4);
        o.off_cl = take(n * 4);
        o.off_ca = take(n * 4);
        // Tiled for finish_rows_kernel: whole 16-row tiles of each dictionary group.
        const uint64_t tiled = (uint64_t)o.n_groups * cdiv(o.rows_per_group, 16u) * 16 * A;
        o.off_cw = take((o.fin_rows ? tiled : n * w_pitch(A)) * 4);
        if (o.sep_merge) o.off_ocp = take(n_lbg * R * o.n_ar * HD * 4);
    }
    o.info.workspace_bytes = off;
    return AW_OK;
}

} // namespace

// ------------------------------------------------- fixed scratch (no allocation)
//
// Scratch of aw_decode_device_noalloc: one file-scope device array, which every
// GPU the library runs on holds (its own copy, at its own address) until the
// process ends.  Host code never uses the array's name as an address: the name
// is a host-side stand-in.  The device address comes from hipGetSymbolAddress,
// once per device with that device current (at engine creation), and is kept
// per device in g_scratch_ptr.
static_assert(AW_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) unsigned char scratch[AW_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device`, which must be current.
hipError_t scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return err;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

} // namespace

// ------------------------------------------------------------------ engine

struct aw_engine {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t side = nullptr;               // hot kernel, concurrent with q.D^T + cold
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    std::string name, last_error;
    uint64_t max_threads = 0;
    size_t max_lds = 0;
    uint32_t n_cu = 0;
    uint32_t hot_wpc[3] = {12, 4, 4}; // resident hot waves per CU (RT = 1, 2, 4)
    DevBuf q, ql, hot, cold, refs, dict, out; // aw_decode copies (weaver.rs:40-46)
    DevBuf ws;                                // per-request scratch
    std::vector<void*> retired_ws;            // outgrown scratch, kept for captured graphs
    void* scratch = nullptr;                  // this device's `scratch` array (aw_decode_device_noalloc)
    DevBuf enc_ws;                            // encoder scratch: per-atom norms and flags
    DevBuf iota;                              // identity block table for contiguous caches
    uint32_t iota_n = 0;                      // entries of `iota` filled
    uint32_t* err = nullptr;                  // device error word
    int profiling = 0; // AW_PROFILE_*
    int projection = AW_PROJECT_AUTO;
    int cold_output = AW_COLD_OUT_AUTO;
    struct Pending {
        int stage;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> free_events;
    double stage_ms[AW_STAGE_COUNT] = {};
    uint64_t stage_n[AW_STAGE_COUNT] = {};
};

namespace {

int fail(aw_engine* e, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (e) e->last_error = buf;
    return code;
}

int hip_fail(aw_engine* e, hipError_t err, const char* what) {
    return fail(e, AW_E_HIP, "%s: %s", what, hipGetErrorString(err));
}

#define AW_HIP(e, call)                                              \
    do {                                                             \
        hipError_t _err = (call);                                    \
        if (_err != hipSuccess) return hip_fail((e), _err, #call);   \
    } while (0)

hipEvent_t take_event(aw_engine* e) {
    if (!e->free_events.empty()) {
        hipEvent_t ev = e->free_events.back();
        e->free_events.pop_back();
        return ev;
    }
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventReleaseToDevice) != hipSuccess) return nullptr;
    return ev;
}

// Resolve finished event pairs into the per-stage totals.
void drain_events(aw_engine* e) {
    for (auto& p : e->pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            e->stage_ms[p.stage] += ms;
            e->stage_n[p.stage] += 1;
        }
        e->free_events.push_back(p.a);
        e->free_events.push_back(p.b);
    }
    e->pending.clear();
}

struct StageTimer {
    aw_engine* e;
    int stage;
    hipStream_t s;
    hipEvent_t a = nullptr, b = nullptr;
    StageTimer(aw_engine* e_, int st, hipStream_t s_) : e(e_), stage(st), s(s_) {
        if (!e->profiling) return;
        if (e->pending.size() > 8192) drain_events(e);
        a = take_event(e);
        b = take_event(e);
        if (a && b) (void)hipEventRecord(a, s);
    }
    ~StageTimer() {
        if (!a || !b) return;
        (void)hipEventRecord(b, s);
        e->pending.push_back({stage, a, b});
    }
};

template <int HD>
int launch_project(aw_engine* e, const aw_decode_desc* d, const Layout& o, char* ws, hipStream_t st) {
    aw::ProjArgs a{};
    a.q = d->q;
    a.dict = d->dict;
    a.ql = o.info.computes_q_latent && !o.qf32 ? (uint16_t*)(ws + o.off_ql) : nullptr;
    a.qlf = o.qf32 ? (float*)(ws + o.off_ql) : nullptr;
    a.dt = (uint16_t*)(ws + o.off_dt);
    a.dt_pitch = dt_pitch(d->dict_size);
    a.dt_tiled = o.fin_rows || o.cold_out ? 1u : 0u; // the row-tile finish's and the value partials' A operand
    a.batch = d->batch;
    a.queries = d->queries;
    a.q_heads = d->q_heads;
    a.kv_heads = d->kv_heads;
    a.gqa = d->q_heads / d->kv_heads;
    a.rows_r = o.info.rows_per_kv_head;
    a.dict_size = d->dict_size;
    a.dict_heads = d->dict_heads;
    a.rows_per_group = d->batch * d->queries * (d->dict_heads == 1 ? d->q_heads : a.gqa);
    a.dict_layer = (uint64_t)d->dict_heads * d->dict_size * HD;
    // Without q_latent to compute, one row block per atom block only writes D^T.
    const uint32_t rows = (a.ql || a.qlf) ? a.rows_per_group : 1;
    const uint32_t gz = d->layers * d->dict_heads;
    const uint32_t A = d->dict_size;
    StageTimer t(e, AW_STAGE_PROJECT, st);
    const bool valu = e->projection == AW_PROJECT_VALU ||
                      (e->projection == AW_PROJECT_AUTO && o.info.projection == AW_PROJECT_VALU);
    if (valu) {
        hipLaunchKernelGGL((aw::project_valu_kernel<HD, kProjValuTa, kProjValuRb>), dim3(cdiv(A, (uint32_t)kProjValuTa),
                           cdiv(rows, (uint32_t)kProjValuRb), gz), dim3(kProjValuTa),
                           aw::project_valu_smem_bytes(HD, kProjValuTa, kProjValuRb), st, a);
        AW_HIP(e, hipGetLastError());
        return AW_OK;
    }
    const dim3 block(aw::kProjThreads);
    // Tiles as large as keep >= one work-group per CU: fewer re-reads of D and q.
    auto wgs = [&](uint32_t tr, uint32_t ta) { return (uint64_t)cdiv(A, ta) * cdiv(rows, tr) * gz; };
#define AW_LAUNCH_PROJ(TR, TA, WR)                                                                              \
    hipLaunchKernelGGL((aw::project_kernel<HD, TR, TA, WR>), dim3(cdiv(A, TA), cdiv(rows, TR), gz), block,      \
                       aw::project_smem_bytes(HD, TR, TA), st, a)
    if (rows <= 32)
        AW_LAUNCH_PROJ(32, 64, 2);
    else if (wgs(128, 256) >= e->n_cu)
        AW_LAUNCH_PROJ(128, 256, 2);
    else if (wgs(128, 128) >= e->n_cu)
        AW_LAUNCH_PROJ(128, 128, 4);
    else
        AW_LAUNCH_PROJ(128, 64, 8);
#undef AW_LAUNCH_PROJ
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

template <int HD>
int launch_hot(aw_engine* e, const aw_decode_desc* d, const Layout& o, char* ws, hipStream_t st) {
    aw::HotArgs a{};
    a.q = d->q;
    a.hot_k = d->hot_k;
    a.hot_v = d->hot_v;
    a.refs = d->refs;
    a.seq_hot = d->seq_hot;
    a.part_m = (float*)(ws + o.off_hm);
    a.part_l = (float*)(ws + o.off_hl);
    a.part_o = (float*)(ws + o.off_ho);
    a.err = e->err;
    a.batch = d->batch;
    a.queries = d->queries;
    a.q_heads = d->q_heads;
    a.kv_heads = d->kv_heads;
    a.gqa = d->q_heads / d->kv_heads;
    a.rows_r = o.info.rows_per_kv_head;
    a.hot_count = d->hot_count;
    a.refs_stride = d->refs_stride;
    a.splits = o.info.hot_splits;
    a.part_splits = o.part_splits;
    a.tokens_per_split = o.info.hot_tokens_per_split;
    a.refs_cap = (uint32_t)align_up(cdiv(a.tokens_per_split, kBlock), 4);
    // The engine's identity table (contiguous caches, one sequence): the kernel
    // computes the block instead of reading it.
    a.refs_identity = (d->refs == (const uint32_t*)e->iota.ptr && d->batch == 1 && d->layers == 1) ? 1u : 0u;
    a.causal = (d->flags & AW_F_CAUSAL) ? 1u : 0u;
    a.n_tok_max = d->hot_tokens ? d->hot_tokens : d->hot_count * kBlock;
    a.seq_tokens = (d->flags & AW_F_SEQ_HOT_TOKENS) ? 1u : 0u;
    a.scale_log2 = d->scale * aw::kLog2e;
    a.hot_blocks = d->hot_blocks;
    a.hot_layer = d->hot_blocks * kBlock * d->kv_heads * HD;
    a.refs_layer = (uint64_t)d->batch * d->refs_stride;
    const uint64_t grid = (uint64_t)d->layers * d->batch * d->kv_heads * a.splits;
    if (grid > 0x7FFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "hot grid too large");
    StageTimer t(e, AW_STAGE_HOT, st);
    const uint32_t R = a.rows_r;
    const size_t smem = a.refs_identity ? 0 : (size_t)a.refs_cap * 4; // the split's block refs
#define AW_LAUNCH_HOT(RTV, SV) hipLaunchKernelGGL((aw::hot_kernel<HD, RTV, SV>), dim3((uint32_t)grid), dim3(64), smem, st, a)
    const bool sepv = a.hot_v != nullptr;
    if (R <= 16) {
        if (sepv) AW_LAUNCH_HOT(1, true); else AW_LAUNCH_HOT(1, false);
    } else if (R <= 32) {
        if (sepv) AW_LAUNCH_HOT(2, true); else AW_LAUNCH_HOT(2, false);
    } else {
        if (sepv) AW_LAUNCH_HOT(4, true); else AW_LAUNCH_HOT(4, false);
    }
#undef AW_LAUNCH_HOT
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

// Codes per lane per wave tile, and wave tiles of code loads in flight.  2 x 4
// measured faster than 4 x 2, 4 x 3, 4 x 4 and 8 x 2 at B = 64; deeper rings hold
// more VGPRs, which crowd out the hot waves running beside the cold kernel.
constexpr int kColdCPT = 2;
constexpr int kColdPD = 4;

// cold_kernel instance for a row chunk of 1, 2 or 4, a power-of-two dictionary
// or not, an f16 or fp32 q_latent table, buffer loads (a layer's pool within
// aw::kColdWindow bytes) or 64-bit addresses, and bins or value partials out
// (value partials with buffer loads only).
const void* cold_kernel_fn(uint32_t rc, bool pow2, bool qf32, bool buf, bool out) {
#define AW_COLD_B(RCV, P2, OUT)                                                                  \
    { {(const void*)aw::cold_kernel<RCV, kColdCPT, kColdPD, P2, false, false, false>,          \
       (const void*)aw::cold_kernel<RCV, kColdCPT, kColdPD, P2, false, true, OUT>},            \
      {(const void*)aw::cold_kernel<RCV, kColdCPT, kColdPD, P2, true, false, false>,           \
       (const void*)aw::cold_kernel<RCV, kColdCPT, kColdPD, P2, true, true, OUT>} }
#define AW_COLD(RCV) {{AW_COLD_B(RCV, false, false), AW_COLD_B(RCV, true, false)}, \
                      {AW_COLD_B(RCV, false, true), AW_COLD_B(RCV, true, true)}}
    static const void* const table[3][2][2][2][2] = {AW_COLD(1), AW_COLD(2), AW_COLD(4)};
#undef AW_COLD
#undef AW_COLD_B
    return table[rc == 4 ? 2 : (rc == 2 ? 1 : 0)][out ? 1 : 0][pow2 ? 1 : 0][qf32 ? 1 : 0][buf ? 1 : 0];
}

int launch_cold(aw_engine* e, const aw_decode_desc* d, const Layout& o, char* ws, hipStream_t st) {
    aw::ColdArgs a{};
    const uint32_t HD = d->head_dim, A = d->dict_size, G = d->q_heads / d->kv_heads;
    const uint32_t R = o.info.rows_per_kv_head;
    a.cold = (const aw::uint4_t*)d->cold;
    a.refs = d->refs;
    a.seq_cold = d->seq_cold;
    a.part_m = (float*)(ws + o.off_cm);
    a.part_l = (float*)(ws + o.off_cl);
    a.part_amax = (float*)(ws + o.off_ca);
    a.part_w = (float*)(ws + o.off_cw);
    a.w_pitch = w_pitch(d->dict_size);
    a.err = e->err;
    a.batch = d->batch;
    a.kv_heads = d->kv_heads;
    a.gqa = G;
    a.rows_r = R;
    a.hot_count = d->hot_count;
    a.cold_count = d->cold_count;
    a.refs_stride = d->refs_stride;
    a.dict_size = A;
    a.splits = o.info.cold_splits;
    a.tokens_per_split = o.info.cold_tokens_per_split;
    a.n_chunks = o.n_chunks;
    const bool head_blocked = (d->flags & AW_F_COLD_HEAD_BLOCKED) != 0;
    // Sharers on one XCD: the row chunks of a kv head in the head-blocked order
    // (they read the same 256-byte runs), else the kv heads of a chunk (their codes
    // share lines in the reference order).
    a.chunk_xcd = (head_blocked && o.n_chunks > 1) ? 1u : 0u;
    const uint64_t n_units = a.chunk_xcd ? (uint64_t)d->layers * d->batch * a.splits * d->kv_heads
                                         : (uint64_t)d->layers * d->batch * o.n_chunks * a.splits;
    if (n_units > 0xFFFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "cold grid too large");
    a.n_units = (uint32_t)n_units;
    a.scale_log2 = d->scale * aw::kLog2e;
    a.w_tiled = o.fin_rows ? 1u : 0u;
    a.w_rows_per_group = o.rows_per_group;
    a.w_dict_heads = d->dict_heads;
    a.cold_blocks = d->cold_blocks;
    a.cold_layer = d->cold_blocks * kBlock * d->kv_heads;
    a.s_tok = head_blocked ? 1u : d->kv_heads;
    a.s_head = head_blocked ? kBlock : 1u;
    a.refs_layer = (uint64_t)d->batch * d->refs_stride;
    // q_latent [L][B][Q][Hq][A], computed on the device or the caller's.
    a.ql = o.info.computes_q_latent ? nullptr : d->q_latent;
    a.qlf = o.qf32 ? (const float*)(ws + o.off_ql) : nullptr;
    if (o.info.computes_q_latent && !o.qf32) a.ql = (const uint16_t*)(ws + o.off_ql);
    a.s_lb = (uint64_t)d->queries * d->q_heads * A;
    a.s_g = (uint64_t)G * A;
    a.s_q = (uint64_t)d->q_heads * A;
    a.s_j = A;
    a.s_a = 1;
    if (o.cold_out) {
        a.dt = (const uint16_t*)(ws + o.off_dt);
        a.dict_heads = d->dict_heads;
        a.head_dim = HD;
        a.out_splits = o.part_splits;
        a.out_split0 = o.info.hot_splits;
        a.w_lds_off = (uint32_t)o.w_lds_off;
        a.out_m = (float*)(ws + o.off_hm);
        a.out_l = (float*)(ws + o.off_hl);
        a.out_o = (float*)(ws + o.off_ho);
    }
    const uint64_t n_wg = (uint64_t)cdiv(a.n_units, 8) * 8 * (a.chunk_xcd ? o.n_chunks : d->kv_heads);
    if (n_wg > 0x7FFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "cold grid too large");
    a.n_wg = (uint32_t)n_wg;
    const size_t smem = o.cold_smem;
    const bool pow2 = (A & (A - 1u)) == 0u;
    const void* fn = cold_kernel_fn(o.rc, pow2, o.qf32, cold_uses_buffer(d), o.cold_out);
    // One resident round of work-groups (a multiple of 8: each keeps its XCD).
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, aw::kColdThreads, smem) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const uint64_t resident = std::max<uint64_t>(8, ((uint64_t)e->n_cu * per_cu) / 8 * 8);
    const uint64_t grid = std::min<uint64_t>(n_wg, resident);
    StageTimer t(e, AW_STAGE_COLD, st);
    void* args[] = {&a};
    AW_HIP(e, hipLaunchKernel(fn, dim3((uint32_t)grid), dim3(aw::kColdThreads), args, smem, st));
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

template <int HD>
int launch_finish(aw_engine* e, const aw_decode_desc* d, const Layout& o, char* ws, hipStream_t st) {
    aw::FinishArgs a{};
    a.dt = (const uint16_t*)(ws + o.off_dt);
    a.dt_pitch = dt_pitch(d->dict_size);
    a.w_pitch = w_pitch(d->dict_size);
    a.cold_m = (const float*)(ws + o.off_cm);
    a.cold_l = (const float*)(ws + o.off_cl);
    a.cold_w = (const float*)(ws + o.off_cw);
    a.cold_amax = (const float*)(ws + o.off_ca);
    if (o.info.hot_splits) {
        a.hot_m = (const float*)(ws + o.off_hm);
        a.hot_l = (const float*)(ws + o.off_hl);
        a.hot_o = (const float*)(ws + o.off_ho);
    }
    a.ocp = o.sep_merge ? (float*)(ws + o.off_ocp) : nullptr;
    a.sep_merge = o.sep_merge ? 1u : 0u;
    a.out = d->out;
    a.batch = d->batch;
    a.queries = d->queries;
    a.q_heads = d->q_heads;
    a.kv_heads = d->kv_heads;
    a.gqa = d->q_heads / d->kv_heads;
    a.rows_r = o.info.rows_per_kv_head;
    a.dict_size = d->dict_size;
    a.dict_heads = d->dict_heads;
    a.rows_per_group = o.rows_per_group;
    a.tiles_per_group = o.tiles_per_group;
    a.cold_splits = o.info.cold_splits;
    a.hot_splits = o.info.hot_splits;
    a.n_ar = o.n_ar;
    a.atoms_per_range = o.atoms_per_range;
    a.dict_layer = (uint64_t)d->dict_heads * d->dict_size * HD;
    const uint64_t gx = (uint64_t)o.tiles_per_group * o.n_groups;
    if (gx > 0x7FFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "finish grid too large");
    StageTimer t(e, AW_STAGE_FINISH, st);
    if (o.fin_rows) {
        const uint64_t gr = (uint64_t)cdiv(o.rows_per_group, 16u) * o.n_groups;
        if (gr > 0x7FFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "finish grid too large");
        hipLaunchKernelGGL((aw::finish_rows_kernel<HD>), dim3((uint32_t)gr, o.n_ar), dim3(aw::kFinRowsWaves * 64),
                           aw::finish_rows_smem_bytes(HD), st, a);
        AW_HIP(e, hipGetLastError());
        return AW_OK;
    }
    const bool fused = !o.sep_merge && a.hot_splits > 0;
    const uint32_t sneed = std::max(a.cold_splits, fused ? a.hot_splits : 1u);
    uint32_t sf = 1;
    while (sf < sneed) sf *= 2;
    const size_t smem = aw::finish_smem_bytes(HD, sf);
    const dim3 block(aw::kFinishWaves * 64);
    if (a.cold_splits == 1)
        hipLaunchKernelGGL((aw::finish_kernel<HD, true>), dim3((uint32_t)gx, o.n_ar), block, smem, st, a);
    else
        hipLaunchKernelGGL((aw::finish_kernel<HD, false>), dim3((uint32_t)gx, o.n_ar), block, smem, st, a);
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

template <int HD>
int launch_merge(aw_engine* e, const aw_decode_desc* d, const Layout& o, char* ws, hipStream_t st) {
    aw::MergeArgs a{};
    const bool cold = o.info.cold_splits > 0 && !o.cold_out; // value partials come in as splits of the hot arrays
    a.cold_m = cold ? (const float*)(ws + o.off_cm) : nullptr;
    a.cold_l = cold ? (const float*)(ws + o.off_cl) : nullptr;
    a.cold_amax = cold ? (const float*)(ws + o.off_ca) : nullptr;
    a.ocp = cold ? (const float*)(ws + o.off_ocp) : nullptr;
    if (o.part_splits) {
        a.hot_m = (const float*)(ws + o.off_hm);
        a.hot_l = (const float*)(ws + o.off_hl);
        a.hot_o = (const float*)(ws + o.off_ho);
    }
    a.out = d->out;
    a.batch = d->batch;
    a.queries = d->queries;
    a.q_heads = d->q_heads;
    a.kv_heads = d->kv_heads;
    a.gqa = d->q_heads / d->kv_heads;
    a.rows_r = o.info.rows_per_kv_head;
    a.cold_splits = cold ? o.info.cold_splits : 0u;
    a.hot_splits = o.part_splits;
    a.n_ar = cold ? o.n_ar : 0u;
    a.total_rows = (uint64_t)d->layers * d->batch * d->kv_heads * a.rows_r;
    const uint64_t gx = cdiv(a.total_rows, 4);
    if (gx > 0x7FFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "merge grid too large");
    StageTimer t(e, AW_STAGE_MERGE, st);
    // Deep load batches when the rows have many partials (measured at B = 1: 45.2 us
    // a step with 16 float4 loads per batch, 45.9 with 8), shallow ones otherwise
    // (B = 64: 16 ranges, 2 hot splits).
    if (a.total_rows <= 4ull * e->n_cu && (a.n_ar > 8 || a.hot_splits > 8))
        // Few rows with many partials: a work-group per row, its waves splitting them
        // (measured to B = 32; B = 8 step 58.2 -> 55.8 us).
        hipLaunchKernelGGL((aw::merge_row_kernel<HD, 8>), dim3((uint32_t)a.total_rows), dim3(256), 0, st, a);
    else if (a.n_ar > 16 || a.hot_splits > 8)
        hipLaunchKernelGGL((aw::merge_kernel<HD, 16>), dim3((uint32_t)gx), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((aw::merge_kernel<HD, 4>), dim3((uint32_t)gx), dim3(256), 0, st, a);
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

// Stage order on `st`: [q.D^T] -> cold -> finish [-> merge], or [q.D^T] ->
// cold -> merge when the cold kernel writes value partials.  The hot kernel
// (HBM-bound) runs on the engine's side stream, forked after q.D^T, so it starts
// together with the cold kernel (bound by L2 requests: one per 16-byte code, one
// resident work-group per CU) and fills the resources the cold work-groups leave
// free.  It is joined only where its partials are read: before the merge, or
// before the finish when the finish merges.  AW_PROFILE_SERIAL puts everything
// on `st`, one kernel at a time.
template <int HD>
int run_pipeline(aw_engine* e, const aw_decode_desc* d, const Layout& o, char* ws, hipStream_t st) {
    int rc = AW_OK;
    const bool cold = o.info.cold_splits > 0;
    const bool hot = o.info.hot_splits > 0;
    const bool fork = hot && cold && e->profiling != AW_PROFILE_SERIAL;
    if (!cold) {
        if (hot && (rc = launch_hot<HD>(e, d, o, ws, st))) return rc;
        return launch_merge<HD>(e, d, o, ws, st);
    }
    if (hot && !fork)
        if ((rc = launch_hot<HD>(e, d, o, ws, st))) return rc;
    if ((rc = launch_project<HD>(e, d, o, ws, st))) return rc;
    // The cold launch goes in before the hot branch: a captured graph then
    // dispatches the critical-path kernel first (about 8 us earlier at B = 64).
    if (fork) AW_HIP(e, hipEventRecord(e->ev_fork, st));
    if ((rc = launch_cold(e, d, o, ws, st))) return rc;
    if (fork) {
        AW_HIP(e, hipStreamWaitEvent(e->side, e->ev_fork, 0));
        if ((rc = launch_hot<HD>(e, d, o, ws, e->side))) return rc;
        AW_HIP(e, hipEventRecord(e->ev_join, e->side));
    }
    if (o.cold_out) { // value partials: the merge reads the hot and cold splits alike
        if (fork) AW_HIP(e, hipStreamWaitEvent(st, e->ev_join, 0));
        return launch_merge<HD>(e, d, o, ws, st);
    }
    const bool merge = o.sep_merge; // otherwise the finish merges
    if (fork && !merge) AW_HIP(e, hipStreamWaitEvent(st, e->ev_join, 0));
    if ((rc = launch_finish<HD>(e, d, o, ws, st))) return rc;
    if (merge) {
        if (fork) AW_HIP(e, hipStreamWaitEvent(st, e->ev_join, 0));
        if ((rc = launch_merge<HD>(e, d, o, ws, st))) return rc;
    }
    return AW_OK;
}

// no_alloc: scratch from the device's fixed `scratch` array instead of the
// engine workspace; nothing is allocated (no workspace growth, no timing events).
int decode_device(aw_engine* e, const aw_decode_desc* d, hipStream_t st, bool no_alloc = false) {
    Layout o;
    char msg[256] = {0};
    int rc = plan(d, e->max_lds, e->n_cu, e->hot_wpc, e->cold_output, &o, msg, sizeof msg);
    if (rc) return fail(e, rc, "%s", msg);
    if (!d->out || !d->q) return fail(e, AW_E_INVALID_ARG, "q and out are required");
    if (d->hot_count && (!d->hot_k || !d->refs)) return fail(e, AW_E_INVALID_ARG, "hot_k and refs are required");
    if ((d->flags & AW_F_SEQ_HOT_TOKENS) && !d->seq_hot)
        return fail(e, AW_E_INVALID_ARG, "AW_F_SEQ_HOT_TOKENS needs seq_hot");
    if (d->cold_count && (!d->cold || !d->refs || !d->dict))
        return fail(e, AW_E_INVALID_ARG, "cold, refs and dict are required");
    if (d->cold_count && d->cold_blocks == 0)
        return fail(e, AW_E_INVALID_ARG, "cold_count > 0 needs cold_blocks > 0");
    if (d->hot_count && d->hot_blocks == 0)
        return fail(e, AW_E_INVALID_ARG, "hot_count > 0 needs hot_blocks > 0");
    if (d->cold_count && ((uintptr_t)d->cold & 15u))
        return fail(e, AW_E_ALIGN, "cold pool pointer is not 16-byte aligned");
    if (no_alloc) {
        if (o.info.workspace_bytes > (uint64_t)AW_NOALLOC_SCRATCH_BYTES)
            return fail(e, AW_E_UNSUPPORTED,
                        "request needs %llu bytes of scratch; the no-allocation entry point has %llu "
                        "(use aw_decode_device, or split the request over layers or sequences)",
                        (unsigned long long)o.info.workspace_bytes, (unsigned long long)AW_NOALLOC_SCRATCH_BYTES);
        if (!e->scratch) return fail(e, AW_E_HIP, "the device's scratch array has no address");
        // Stage timers create events: keep them off for this call.
        const int prof = e->profiling;
        e->profiling = AW_PROFILE_OFF;
        char* ws = (char*)e->scratch;
        rc = d->head_dim == 64 ? run_pipeline<64>(e, d, o, ws, st) : run_pipeline<128>(e, d, o, ws, st);
        e->profiling = prof;
        return rc;
    }
    if ((rc = ensure_keep(e->ws, o.info.workspace_bytes, e->retired_ws, e->last_error, st))) return rc;
    char* ws = (char*)e->ws.ptr;
    return d->head_dim == 64 ? run_pipeline<64>(e, d, o, ws, st) : run_pipeline<128>(e, d, o, ws, st);
}

template <typename F>
int check_kernel(aw_engine* e, F* fn, const char* name) {
    hipFuncAttributes attr;
    hipError_t err = hipFuncGetAttributes(&attr, (const void*)fn);
    if (err != hipSuccess)
        return fail(e, AW_E_LOAD, "kernel %s has no code object for this device: %s", name, hipGetErrorString(err));
    return AW_OK;
}

} // namespace

// ------------------------------------------------------------- C ABI

extern "C" {

uint32_t aw_abi_version(void) { return AW_ABI_VERSION; }

void aw_abi_struct_sizes(size_t sizes[4]) {
    sizes[0] = sizeof(aw_sparse_code);
    sizes[1] = sizeof(aw_weaver_params);
    sizes[2] = sizeof(aw_decode_desc);
    sizes[3] = sizeof(aw_decode_plan_info);
}

size_t aw_abi_encode_desc_size(void) { return sizeof(aw_encode_desc); }

const char* aw_status_string(int status) {
    switch (status) {
    case AW_OK: return "ok";
    case AW_E_INVALID_ARG: return "invalid argument";
    case AW_E_ALIGN: return "misaligned SparseCode pointer";
    case AW_E_OOB: return "block ref or atom index out of range";
    case AW_E_HIP: return "HIP runtime error";
    case AW_E_LOAD: return "kernels not available for this device";
    case AW_E_UNSUPPORTED: return "unsupported request";
    case AW_E_IO: return "file I/O failed";
    case AW_E_BAD_MAGIC: return "invalid magic bytes";
    case AW_E_VERSION: return "version mismatch";
    case AW_E_TOO_SMALL: return "file too small";
    case AW_E_SIGNATURE: return "signature verification failed";
    default: return "unknown status";
    }
}

int aw_validate_params(const aw_weaver_params* p, size_t n_q_exact, size_t n_q_latent, size_t n_hot_pool,
                       const aw_sparse_code* cold_pool, size_t n_cold_pool, const uint32_t* loom_refs,
                       size_t n_loom_refs, size_t n_dictionary, size_t n_out, char* msg, size_t mlen) {
    if (!p) {
        put_msg(msg, mlen, "null params");
        return AW_E_INVALID_ARG;
    }
    if (p->block_size != kBlock) {
        put_msg(msg, mlen, "block_size %u, only 16 is supported (ModelDims::BLOCK_SIZE)", p->block_size);
        return AW_E_UNSUPPORTED;
    }
    if (p->sparsity_k != 4) {
        put_msg(msg, mlen, "sparsity_k %u, a SparseCode holds exactly 4 terms", p->sparsity_k);
        return AW_E_UNSUPPORTED;
    }
    if (p->kv_heads == 0 || p->gqa_group == 0 || (uint64_t)p->gqa_group * p->kv_heads != p->q_heads) {
        put_msg(msg, mlen, "gqa_group (%u) * kv_heads (%u) != q_heads (%u)", p->gqa_group, p->kv_heads, p->q_heads);
        return AW_E_INVALID_ARG;
    }
    if (!supported_head_dim(p->head_dim)) {
        put_msg(msg, mlen, "head_dim %u unsupported (64 or 128)", p->head_dim);
        return AW_E_UNSUPPORTED;
    }
    if (p->gqa_group > 64) {
        put_msg(msg, mlen, "gqa_group %u exceeds 64", p->gqa_group);
        return AW_E_UNSUPPORTED;
    }
    const uint64_t HD = p->head_dim, Hkv = p->kv_heads;
    if (n_q_exact < (uint64_t)p->q_heads * HD) {
        put_msg(msg, mlen, "q_exact holds %zu values, needs %llu", n_q_exact,
                (unsigned long long)p->q_heads * HD);
        return AW_E_INVALID_ARG;
    }
    if (n_out < (uint64_t)p->q_heads * HD) {
        put_msg(msg, mlen, "output holds %zu values, needs %llu", n_out, (unsigned long long)p->q_heads * HD);
        return AW_E_INVALID_ARG;
    }
    const uint64_t nrefs = (uint64_t)p->hot_count + p->cold_count;
    if (n_loom_refs < nrefs || (nrefs && !loom_refs)) {
        put_msg(msg, mlen, "loom_refs holds %zu refs, needs hot_count + cold_count = %llu", n_loom_refs,
                (unsigned long long)nrefs);
        return AW_E_INVALID_ARG;
    }
    const uint64_t hot_blocks = n_hot_pool / (kBlock * Hkv * HD);
    for (uint32_t b = 0; b < p->hot_count; ++b) {
        const uint32_t phys = loom_refs[b] & aw::kRefMask;
        if (phys >= hot_blocks) {
            put_msg(msg, mlen, "hot ref %u -> block %u, hot pool holds %llu blocks", b, phys,
                    (unsigned long long)hot_blocks);
            return AW_E_OOB;
        }
    }
    if (p->cold_count) {
        if (p->dict_size == 0 || p->dict_size > 65536 || p->dict_size % 16) {
            put_msg(msg, mlen, "dict_size %u must be a multiple of 16 in [16, 65536]", p->dict_size);
            return AW_E_UNSUPPORTED;
        }
        if (n_q_latent != 0 && n_q_latent < (uint64_t)p->q_heads * p->dict_size) {
            put_msg(msg, mlen, "q_latent holds %zu values, needs %llu (or 0 to compute it)", n_q_latent,
                    (unsigned long long)p->q_heads * p->dict_size);
            return AW_E_INVALID_ARG;
        }
        if (n_dictionary < Hkv * p->dict_size * HD) {
            put_msg(msg, mlen, "dictionary holds %zu values, needs kv_heads*dict_size*head_dim = %llu", n_dictionary,
                    (unsigned long long)(Hkv * p->dict_size * HD));
            return AW_E_INVALID_ARG;
        }
        if (!cold_pool) {
            put_msg(msg, mlen, "cold pool is empty but cold_count = %u", p->cold_count);
            return AW_E_INVALID_ARG;
        }
        if ((uintptr_t)cold_pool & 15u) {
            put_msg(msg, mlen, "cold pool pointer is not 16-byte aligned");
            return AW_E_ALIGN;
        }
        const uint64_t cold_blocks = n_cold_pool / (kBlock * Hkv);
        for (uint32_t b = 0; b < p->cold_count; ++b) {
            const uint32_t phys = loom_refs[p->hot_count + b] & aw::kRefMask;
            if (phys >= cold_blocks) {
                put_msg(msg, mlen, "cold ref %u -> block %u, cold pool holds %llu blocks", b, phys,
                        (unsigned long long)cold_blocks);
                return AW_E_OOB;
            }
            const aw_sparse_code* c = cold_pool + (uint64_t)phys * kBlock * Hkv;
            for (uint64_t i = 0; i < kBlock * Hkv; ++i)
                for (int k = 0; k < 4; ++k)
                    if (c[i].indices[k] >= p->dict_size) {
                        put_msg(msg, mlen, "cold block %u code %llu: atom index %u >= dict_size %u", phys,
                                (unsigned long long)i, c[i].indices[k], p->dict_size);
                        return AW_E_OOB;
                    }
        }
    }
    return AW_OK;
}

int aw_decode_plan(const aw_decode_desc* desc, aw_decode_plan_info* info, char* msg, size_t mlen) {
    Layout o;
    // Host-side planning assumes the MI355X limits: 160 KiB LDS per work-group, 256 CUs.
    const uint32_t wpc[3] = {12, 4, 4}; // gfx950 residency of the hot kernel variants
    int rc = plan(desc, 160 * 1024, 256, wpc, AW_COLD_OUT_AUTO, &o, msg, mlen);
    if (rc == AW_OK && info) *info = o.info;
    return rc;
}

int aw_engine_create(int device, aw_engine** out) {
    if (!out) return AW_E_INVALID_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return AW_E_HIP;
    if (device < 0 || device >= count) return AW_E_INVALID_ARG;
    aw_engine* e = new aw_engine();
    e->device = device;
    hipDeviceProp_t prop;
    if (hipSetDevice(device) != hipSuccess || hipGetDeviceProperties(&prop, device) != hipSuccess) {
        delete e;
        return AW_E_HIP;
    }
    e->name = prop.name;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        delete e;
        return AW_E_LOAD;
    }
    e->max_threads = (uint64_t)prop.maxThreadsPerBlock;
    e->max_lds = prop.sharedMemPerBlock;
    e->n_cu = (uint32_t)prop.multiProcessorCount;
    int rc = AW_OK;
    if (!rc) rc = check_kernel(e, aw::hot_kernel<128, 1, false>, "hot_kernel");
    if (!rc) rc = check_kernel(e, aw::cold_kernel<4, kColdCPT, kColdPD, true, false, true, false>, "cold_kernel");
    if (!rc) rc = check_kernel(e, aw::finish_kernel<128, true>, "finish_kernel");
    if (rc) {
        delete e;
        return rc;
    }
    // Resident hot waves per CU, from the compiled kernels' resource use (K == V variants).
    {
        const void* hk[3] = {(const void*)aw::hot_kernel<128, 1, false>, (const void*)aw::hot_kernel<128, 2, false>,
                             (const void*)aw::hot_kernel<128, 4, false>};
        for (int i = 0; i < 3; ++i) {
            int nb = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, hk[i], 64, 0) == hipSuccess && nb > 0)
                e->hot_wpc[i] = (uint32_t)nb;
        }
    }
    // Let the cold, finish and projection kernels use the device's full LDS.  A
    // refusal (a kernel whose static LDS leaves less than that) fails the
    // engine here, and its error is cleared so that it does not surface at the
    // caller's next HIP call.
    bool attr_ok = true;
    auto set_lds = [&](const void* f) {
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)e->max_lds) != hipSuccess) {
            attr_ok = false;
            (void)hipGetLastError();
        }
    };
    {
        for (uint32_t rcv : {1u, 2u, 4u})
            for (bool p2 : {false, true})
                for (bool qf : {false, true})
                    for (bool bf : {false, true})
                        for (bool out : {false, true}) set_lds(cold_kernel_fn(rcv, p2, qf, bf, out));
        const void* fin[] = {(const void*)aw::finish_kernel<128, true>, (const void*)aw::finish_kernel<128, false>,
                             (const void*)aw::finish_kernel<64, true>, (const void*)aw::finish_kernel<64, false>};
        for (const void* f : fin) set_lds(f);
        const void* finr[] = {(const void*)aw::finish_rows_kernel<128>, (const void*)aw::finish_rows_kernel<64>};
        for (const void* f : finr) set_lds(f);
        const void* proj[] = {(const void*)aw::project_kernel<128, 32, 64, 2>, (const void*)aw::project_kernel<128, 128, 256, 2>,
                              (const void*)aw::project_kernel<128, 128, 128, 4>, (const void*)aw::project_kernel<128, 128, 64, 8>,
                              (const void*)aw::project_kernel<64, 32, 64, 2>, (const void*)aw::project_kernel<64, 128, 256, 2>,
                              (const void*)aw::project_kernel<64, 128, 128, 4>, (const void*)aw::project_kernel<64, 128, 64, 8>,
                              (const void*)aw::project_valu_kernel<128, kProjValuTa, kProjValuRb>,
                              (const void*)aw::project_valu_kernel<64, kProjValuTa, kProjValuRb>};
        for (const void* f : proj) set_lds(f);
        if (!aw_engine_internal::ops_set_lds_limits(e->max_lds)) attr_ok = false;
    }
    if (!attr_ok) {
        aw_engine_destroy(e);
        return AW_E_HIP;
    }
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&e->side, hipStreamNonBlocking) != hipSuccess ||
        // Fork/join order two streams of this device: a device-scope release is enough,
        // no system-scope cache writeback.
        hipEventCreateWithFlags(&e->ev_fork, hipEventDisableTiming | hipEventDisableSystemFence) != hipSuccess ||
        hipEventCreateWithFlags(&e->ev_join, hipEventDisableTiming | hipEventDisableSystemFence) != hipSuccess ||
        hipMalloc((void**)&e->err, 256) != hipSuccess || hipMemset(e->err, 0, 256) != hipSuccess ||
        // The fixed scratch array's address on this device (current since hipSetDevice above).
        scratch_address(device, &e->scratch) != hipSuccess) {
        aw_engine_destroy(e);
        return AW_E_HIP;
    }
    *out = e;
    return AW_OK;
}

void aw_engine_destroy(aw_engine* e) {
    if (!e) return;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    drain_events(e);
    for (hipEvent_t ev : e->free_events) (void)hipEventDestroy(ev);
    for (DevBuf* b : {&e->q, &e->ql, &e->hot, &e->cold, &e->refs, &e->dict, &e->out, &e->ws, &e->enc_ws, &e->iota})
        if (b->ptr) (void)hipFree(b->ptr);
    for (void* p : e->retired_ws) (void)hipFree(p);
    if (e->err) (void)hipFree(e->err);
    if (e->side) (void)hipStreamSynchronize(e->side);
    if (e->ev_fork) (void)hipEventDestroy(e->ev_fork);
    if (e->ev_join) (void)hipEventDestroy(e->ev_join);
    if (e->side) (void)hipStreamDestroy(e->side);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

const char* aw_engine_last_error(const aw_engine* e) { return e ? e->last_error.c_str() : "null engine"; }
const char* aw_engine_device_name(const aw_engine* e) { return e ? e->name.c_str() : ""; }
uint64_t aw_engine_max_threads_per_threadgroup(const aw_engine* e) { return e ? e->max_threads : 0; }

int aw_decode(aw_engine* e, const uint16_t* q_exact, size_t n_q_exact, const uint16_t* q_latent, size_t n_q_latent,
              const uint16_t* hot_pool, size_t n_hot_pool, const aw_sparse_code* cold_pool, size_t n_cold_pool,
              const uint32_t* loom_refs, size_t n_loom_refs, const uint16_t* dictionary, size_t n_dictionary,
              const aw_weaver_params* p, uint16_t* out, size_t n_out) {
    if (!e) return AW_E_INVALID_ARG;
    char msg[256] = {0};
    int rc = aw_validate_params(p, n_q_exact, n_q_latent, n_hot_pool, cold_pool, n_cold_pool, loom_refs,
                                n_loom_refs, n_dictionary, n_out, msg, sizeof msg);
    if (rc) return fail(e, rc, "%s", msg);
    if (!q_exact || !out) return fail(e, AW_E_INVALID_ARG, "q_exact and out are required");
    AW_HIP(e, hipSetDevice(e->device));
    const uint64_t HD = p->head_dim;
    // Copy the slices into the persistent buffers (weaver.rs:155-196); empty slices are skipped.
    auto fill = [&](DevBuf& b, const void* src, size_t bytes) -> int {
        if (!bytes) return AW_OK;
        int r = ensure(b, bytes, e->last_error);
        if (r) return r;
        AW_HIP(e, hipMemcpyAsync(b.ptr, src, bytes, hipMemcpyHostToDevice, e->stream));
        return AW_OK;
    };
    const bool cold = p->cold_count > 0;
    const bool hot = p->hot_count > 0;
    if ((rc = fill(e->q, q_exact, (size_t)p->q_heads * HD * 2))) return rc;
    if (cold && n_q_latent)
        if ((rc = fill(e->ql, q_latent, (size_t)p->q_heads * p->dict_size * 2))) return rc;
    if (hot && (rc = fill(e->hot, hot_pool, n_hot_pool * 2))) return rc;
    if (cold && (rc = fill(e->cold, cold_pool, n_cold_pool * sizeof(aw_sparse_code)))) return rc;
    if ((rc = fill(e->refs, loom_refs, ((size_t)p->hot_count + p->cold_count) * 4))) return rc;
    if (cold && (rc = fill(e->dict, dictionary, (size_t)p->kv_heads * p->dict_size * HD * 2))) return rc;
    if ((rc = ensure(e->out, (size_t)p->q_heads * HD * 2, e->last_error))) return rc;

    aw_decode_desc d{};
    d.layers = d.batch = d.queries = 1;
    d.q_heads = p->q_heads;
    d.kv_heads = p->kv_heads;
    d.head_dim = p->head_dim;
    d.dict_size = cold ? p->dict_size : 0;
    d.dict_heads = p->kv_heads; // reference layout [kv_heads][dict_size][head_dim]
    d.hot_count = p->hot_count;
    d.cold_count = p->cold_count;
    d.refs_stride = p->hot_count + p->cold_count;
    d.flags = 0;
    d.scale = 1.0f; // the reference applies no score scale
    d.hot_blocks = hot ? n_hot_pool / (kBlock * p->kv_heads * HD) : 0;
    d.cold_blocks = cold ? n_cold_pool / (kBlock * p->kv_heads) : 0;
    d.q = (const uint16_t*)e->q.ptr;
    d.q_latent = (cold && n_q_latent) ? (const uint16_t*)e->ql.ptr : nullptr;
    d.hot_k = hot ? (const uint16_t*)e->hot.ptr : nullptr;
    d.hot_v = nullptr;
    d.cold = cold ? (const aw_sparse_code*)e->cold.ptr : nullptr;
    d.refs = (const uint32_t*)e->refs.ptr;
    d.dict = cold ? (const uint16_t*)e->dict.ptr : nullptr;
    d.out = (uint16_t*)e->out.ptr;
    if ((rc = decode_device(e, &d, e->stream))) return rc;
    AW_HIP(e, hipMemcpyAsync(out, e->out.ptr, (size_t)p->q_heads * HD * 2, hipMemcpyDeviceToHost, e->stream));
    AW_HIP(e, hipStreamSynchronize(e->stream)); // commit + wait_until_completed (weaver.rs:227-228)
    return aw_engine_check_device_errors(e, e->stream);
}

int aw_decode_device(aw_engine* e, const aw_decode_desc* desc, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    AW_HIP(e, hipSetDevice(e->device));
    hipStream_t st = (hipStream_t)stream; // NULL is HIP's null stream
    return decode_device(e, desc, st);
}

int aw_decode_device_noalloc(aw_engine* e, const aw_decode_desc* desc, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    AW_HIP(e, hipSetDevice(e->device));
    hipStream_t st = (hipStream_t)stream; // NULL is HIP's null stream
    return decode_device(e, desc, st, /*no_alloc=*/true);
}

// The contiguous cache [cache_tokens][kv_heads][head_dim] is the hot pool
// [blocks][16][kv_heads][head_dim] with block b at ref b; each group of at most
// 64 / G queries is one causal decode whose hot_tokens place its queries at the
// cache's end (ops.metal:549).
int aw_multihead_attention_device(aw_engine* e, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                  uint16_t* out, uint32_t kv_len, uint32_t head_dim, uint32_t q_heads,
                                  uint32_t kv_heads, uint32_t num_queries, uint64_t cache_tokens, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    if (!q || !k_cache || !v_cache || !out) return fail(e, AW_E_INVALID_ARG, "q, k_cache, v_cache and out are required");
    if (num_queries == 0) return fail(e, AW_E_INVALID_ARG, "num_queries must be >= 1");
    if ((uint64_t)kv_len + 1 < num_queries)
        return fail(e, AW_E_INVALID_ARG, "kv_len %u is shorter than num_queries - 1 (%u): the new tokens are not in the cache",
                    kv_len, num_queries - 1);
    if (kv_heads == 0 || q_heads == 0 || q_heads % kv_heads)
        return fail(e, AW_E_INVALID_ARG, "q_heads (%u) must be a positive multiple of kv_heads (%u)", q_heads, kv_heads);
    const uint32_t G = q_heads / kv_heads;
    if (G > 64) return fail(e, AW_E_UNSUPPORTED, "gqa group %u exceeds 64 query rows per kv head", G);
    const uint64_t blocks = cdiv((uint64_t)kv_len, kBlock);
    if (blocks * kBlock > cache_tokens)
        return fail(e, AW_E_INVALID_ARG, "kv_len %u reads %llu cache tokens (whole 16-token blocks); the cache holds %llu",
                    kv_len, (unsigned long long)(blocks * kBlock), (unsigned long long)cache_tokens);
    if (blocks > 0xFFFFFFFFull / kBlock) return fail(e, AW_E_UNSUPPORTED, "kv_len too large");
    AW_HIP(e, hipSetDevice(e->device));
    hipStream_t st = (hipStream_t)stream; // NULL is HIP's null stream
    if (blocks > e->iota_n) {
        // Grown (and kept, like the workspace) on the host's side: filled with a
        // synchronous copy, so calls on any stream see it complete.
        int rc = ensure_keep(e->iota, blocks * 4, e->retired_ws, e->last_error, st);
        if (rc) return rc;
        const uint32_t n = (uint32_t)std::min<size_t>(e->iota.cap / 4, 0xFFFFFFFFull);
        std::vector<uint32_t> ids(n);
        for (uint32_t i = 0; i < n; ++i) ids[i] = i;
        AW_HIP(e, hipMemcpy(e->iota.ptr, ids.data(), (size_t)n * 4, hipMemcpyHostToDevice));
        e->iota_n = n;
    }
    const uint32_t per = 64 / G; // queries of one call: G * queries <= 64 rows per kv head
    const size_t qrow = (size_t)q_heads * head_dim;
    for (uint32_t j0 = 0; j0 < num_queries; j0 += per) {
        const uint32_t c = std::min(per, num_queries - j0);
        // The group's last query is token kv_len - num_queries + j0 + c - 1 of the cache.
        const uint32_t n_tok = (uint32_t)((uint64_t)kv_len + j0 + c - num_queries);
        aw_decode_desc d{};
        d.layers = 1;
        d.batch = 1;
        d.queries = c;
        d.q_heads = q_heads;
        d.kv_heads = kv_heads;
        d.head_dim = head_dim;
        d.hot_count = (uint32_t)cdiv((uint64_t)n_tok, kBlock);
        d.hot_tokens = n_tok;
        d.refs_stride = d.hot_count;
        d.flags = AW_F_CAUSAL;
        d.scale = 1.0f / std::sqrt((float)head_dim);
        d.hot_blocks = cache_tokens / kBlock;
        d.q = q + j0 * qrow;
        d.hot_k = k_cache;
        d.hot_v = v_cache;
        d.refs = (const uint32_t*)e->iota.ptr;
        d.out = out + j0 * qrow;
        const int rc = decode_device(e, &d, st);
        if (rc) return rc;
    }
    return AW_OK;
}

int aw_engine_check_device_errors(aw_engine* e, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    AW_HIP(e, hipSetDevice(e->device));
    hipStream_t st = (hipStream_t)stream; // NULL is HIP's null stream
    uint32_t word = 0;
    AW_HIP(e, hipMemcpyAsync(&word, e->err, 4, hipMemcpyDeviceToHost, st));
    AW_HIP(e, hipStreamSynchronize(st));
    if (!word) return AW_OK;
    AW_HIP(e, hipMemsetAsync(e->err, 0, 4, st));
    AW_HIP(e, hipStreamSynchronize(st));
    return fail(e, AW_E_OOB, "device saw out-of-range input:%s%s%s%s (the affected tokens or terms were skipped)",
                (word & aw::kErrHotRef) ? " hot block ref" : "", (word & aw::kErrColdRef) ? " cold block ref" : "",
                (word & aw::kErrAtom) ? " atom index" : "",
                (word & aw_engine_internal::kErrTokenBit) ? " token id" : "");
}


int aw_debug_gather_codes(aw_engine* e, const aw_sparse_code* codes, size_t n, const uint16_t* dict,
                          uint32_t dict_size, uint32_t head_dim, uint32_t* idx, float* coef, uint16_t* atoms,
                          void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    if (!n) return AW_OK;
    if (!codes || !dict || !idx || !coef || !atoms || !head_dim || !dict_size)
        return fail(e, AW_E_INVALID_ARG, "null pointer or zero size");
    if ((uintptr_t)codes & 15u) return fail(e, AW_E_ALIGN, "codes pointer is not 16-byte aligned");
    AW_HIP(e, hipSetDevice(e->device));
    hipStream_t st = (hipStream_t)stream; // NULL is HIP's null stream
    const uint64_t threads = (uint64_t)n * 4;
    hipLaunchKernelGGL(aw::gather_codes_kernel, dim3(cdiv(threads, 256)), dim3(256), 0, st,
                       (const aw::uint4_t*)codes, (uint64_t)n, dict, dict_size, head_dim, idx, coef, atoms, e->err);
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

namespace {

// Geometry checks of an encoder request (numeric fields only).
int encode_check(const aw_encode_desc* d, char* msg, size_t mlen) {
    if (d->kv_heads == 0 || !supported_head_dim(d->head_dim)) {
        put_msg(msg, mlen, "kv_heads %u must be >= 1 and head_dim %u 64 or 128", d->kv_heads, d->head_dim);
        return AW_E_UNSUPPORTED;
    }
    if (d->dict_size == 0 || d->dict_size > 65536 || d->dict_size % 16) {
        put_msg(msg, mlen, "dict_size %u must be a multiple of 16 in [16, 65536]", d->dict_size);
        return AW_E_UNSUPPORTED;
    }
    if (d->dict_heads != 1 && d->dict_heads != d->kv_heads) {
        put_msg(msg, mlen, "dict_heads must be 1 (shared) or kv_heads");
        return AW_E_INVALID_ARG;
    }
    if (d->flags & ~(AW_F_COLD_HEAD_BLOCKED | AW_F_ENCODE_FULL_SCAN)) {
        put_msg(msg, mlen, "unknown encoder flags 0x%x", d->flags & ~(AW_F_COLD_HEAD_BLOCKED | AW_F_ENCODE_FULL_SCAN));
        return AW_E_INVALID_ARG;
    }
    if (d->n_blocks >= (1u << 27)) {
        put_msg(msg, mlen, "n_blocks %u too large", d->n_blocks);
        return AW_E_UNSUPPORTED;
    }
    return AW_OK;
}

int encode_device(aw_engine* e, const aw_encode_desc* d, hipStream_t st) {
    char msg[256] = {0};
    int rc = encode_check(d, msg, sizeof msg);
    if (rc) return fail(e, rc, "%s", msg);
    if (!d->n_blocks) return AW_OK;
    if (!d->hot || !d->dict || !d->src_blocks || !d->cold || !d->hot_blocks || !d->cold_blocks)
        return fail(e, AW_E_INVALID_ARG, "hot, dict, src_blocks and cold are required, with hot_blocks and cold_blocks > 0");
    if ((uintptr_t)d->cold & 15u) return fail(e, AW_E_ALIGN, "cold pool pointer is not 16-byte aligned");
    if (((uintptr_t)d->hot | (uintptr_t)d->dict) & 15u)
        return fail(e, AW_E_ALIGN, "hot pool and dictionary pointers must be 16-byte aligned");
    AW_HIP(e, hipSetDevice(e->device));
    aw::EncodeArgs a{};
    a.hot = d->hot;
    a.dict = d->dict;
    a.src = d->src_blocks;
    a.dst = d->dst_blocks;
    a.cold = (aw::uint4_t*)d->cold;
    a.entropy = d->entropy;
    a.err = e->err;
    a.kv_heads = d->kv_heads;
    a.dict_size = d->dict_size;
    a.dict_heads = d->dict_heads;
    a.n_blocks = d->n_blocks;
    const bool head_blocked = (d->flags & AW_F_COLD_HEAD_BLOCKED) != 0;
    a.s_tok = head_blocked ? 1u : d->kv_heads;
    a.s_head = head_blocked ? kBlock : 1u;
    a.hot_blocks = d->hot_blocks;
    a.cold_blocks = d->cold_blocks;
    // Scratch of the MFMA path (the atoms' norms), allocated before any work is queued.
    const bool full_scan = (d->flags & AW_F_ENCODE_FULL_SCAN) != 0;
    const uint64_t n_atoms = (uint64_t)d->dict_heads * d->dict_size;
    if (!full_scan && (rc = ensure_keep(e->enc_ws, n_atoms * sizeof(aw::AtomNorm), e->retired_ws, e->last_error, st)))
        return rc;
    // The entropy proxy (few long lanes) runs on the side stream beside the encoder.
    if (d->entropy) {
        AW_HIP(e, hipEventRecord(e->ev_fork, st));
        AW_HIP(e, hipStreamWaitEvent(e->side, e->ev_fork, 0));
        hipLaunchKernelGGL(aw::entropy_kernel, dim3(cdiv(d->n_blocks, aw::kEntBlocks)), dim3(64), 0, e->side, a, d->head_dim);
        AW_HIP(e, hipGetLastError());
        AW_HIP(e, hipEventRecord(e->ev_join, e->side));
    }
    if (full_scan) {
        const dim3 grid(cdiv((uint64_t)d->n_blocks * kBlock, aw::kEncThreads), d->kv_heads);
        if (d->head_dim == 64)
            hipLaunchKernelGGL(aw::encode_kernel<64>, grid, dim3(aw::kEncThreads), 0, st, a);
        else
            hipLaunchKernelGGL(aw::encode_kernel<128>, grid, dim3(aw::kEncThreads), 0, st, a);
    } else {
        // MFMA prefilter + exact rescoring: the atoms' norms first.
        aw::AtomNorm* dn = (aw::AtomNorm*)e->enc_ws.ptr;
        const dim3 ngrid((uint32_t)cdiv(n_atoms, 256));
        const dim3 grid(cdiv((uint64_t)d->n_blocks * kBlock, aw::kEncMTokens), d->kv_heads);
        if (d->head_dim == 64) {
            hipLaunchKernelGGL(aw::dict_norm_kernel<64>, ngrid, dim3(256), 0, st, d->dict, n_atoms, dn);
            hipLaunchKernelGGL(aw::encode_mfma_kernel<64>, grid, dim3(aw::kEncMThreads), 0, st, a, dn);
        } else {
            hipLaunchKernelGGL(aw::dict_norm_kernel<128>, ngrid, dim3(256), 0, st, d->dict, n_atoms, dn);
            hipLaunchKernelGGL(aw::encode_mfma_kernel<128>, grid, dim3(aw::kEncMThreads), 0, st, a, dn);
        }
    }
    AW_HIP(e, hipGetLastError());
    if (d->entropy) AW_HIP(e, hipStreamWaitEvent(st, e->ev_join, 0));
    return AW_OK;
}

} // namespace

int aw_encode_device(aw_engine* e, const aw_encode_desc* desc, void* stream) {
    if (!e || !desc) return AW_E_INVALID_ARG;
    return encode_device(e, desc, (hipStream_t)stream); // NULL is HIP's null stream
}

int aw_block_entropy_device(aw_engine* e, const uint16_t* hot, uint64_t hot_blocks, uint32_t kv_heads,
                            uint32_t head_dim, const uint32_t* blocks, uint32_t n_blocks, float* entropy,
                            void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    if (!n_blocks) return AW_OK;
    if (!hot || !entropy || !hot_blocks || !kv_heads || !head_dim)
        return fail(e, AW_E_INVALID_ARG, "hot, entropy, hot_blocks, kv_heads and head_dim are required");
    if ((uintptr_t)hot & 15u) return fail(e, AW_E_ALIGN, "hot pool pointer is not 16-byte aligned");
    if (n_blocks >= (1u << 27)) return fail(e, AW_E_UNSUPPORTED, "n_blocks %u too large", n_blocks);
    AW_HIP(e, hipSetDevice(e->device));
    aw::EncodeArgs a{};
    a.hot = hot;
    a.src = blocks;
    a.entropy = entropy;
    a.err = e->err;
    a.kv_heads = kv_heads;
    a.n_blocks = n_blocks;
    a.hot_blocks = hot_blocks;
    hipLaunchKernelGGL(aw::entropy_kernel, dim3(cdiv(n_blocks, aw::kEntBlocks)), dim3(64), 0, (hipStream_t)stream, a,
                       head_dim);
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

int aw_encode(aw_engine* e, const uint16_t* hot, size_t n_hot, const uint16_t* dict, size_t n_dict,
              uint32_t kv_heads, uint32_t head_dim, uint32_t dict_size, uint32_t dict_heads, const uint32_t* blocks,
              size_t n_blocks, aw_sparse_code* cold, size_t n_cold, float* entropy) {
    if (!e) return AW_E_INVALID_ARG;
    aw_encode_desc d{};
    d.kv_heads = kv_heads;
    d.head_dim = head_dim;
    d.dict_size = dict_size;
    d.dict_heads = dict_heads;
    d.n_blocks = (uint32_t)std::min<size_t>(n_blocks, 0xFFFFFFFFu);
    char msg[256] = {0};
    int rc = encode_check(&d, msg, sizeof msg);
    if (rc) return fail(e, rc, "%s", msg);
    if (n_blocks != d.n_blocks) return fail(e, AW_E_UNSUPPORTED, "too many blocks");
    if (!n_blocks) return AW_OK;
    const size_t per_block = (size_t)kBlock * kv_heads * head_dim, codes_per_block = (size_t)kBlock * kv_heads;
    if (!hot || !dict || !blocks || !cold) return fail(e, AW_E_INVALID_ARG, "hot, dict, blocks and cold are required");
    if (n_hot < per_block || n_hot % per_block)
        return fail(e, AW_E_INVALID_ARG, "hot slice of %zu values is not a whole number of %zu-value blocks", n_hot, per_block);
    if (n_dict != (size_t)dict_heads * dict_size * head_dim)
        return fail(e, AW_E_INVALID_ARG, "dictionary slice of %zu values, expected %zu", n_dict,
                    (size_t)dict_heads * dict_size * head_dim);
    if (n_cold < codes_per_block || n_cold % codes_per_block)
        return fail(e, AW_E_INVALID_ARG, "cold slice of %zu codes is not a whole number of %zu-code blocks", n_cold,
                    codes_per_block);
    const uint64_t hot_blocks = n_hot / per_block, cold_blocks = n_cold / codes_per_block;
    for (size_t i = 0; i < n_blocks; ++i) {
        const uint32_t b = blocks[i] & 0x7FFFFFFFu;
        if (b >= hot_blocks || b >= cold_blocks)
            return fail(e, AW_E_OOB, "block %u (entry %zu) outside the hot pool (%llu blocks) or cold pool (%llu blocks)",
                        b, i, (unsigned long long)hot_blocks, (unsigned long long)cold_blocks);
    }
    AW_HIP(e, hipSetDevice(e->device));
    auto fill = [&](DevBuf& b, const void* src, size_t bytes) -> int {
        int r = ensure(b, bytes, e->last_error);
        if (r) return r;
        AW_HIP(e, hipMemcpyAsync(b.ptr, src, bytes, hipMemcpyHostToDevice, e->stream));
        return AW_OK;
    };
    if ((rc = fill(e->hot, hot, n_hot * 2))) return rc;
    if ((rc = fill(e->dict, dict, n_dict * 2))) return rc;
    if ((rc = fill(e->refs, blocks, n_blocks * 4))) return rc;
    if ((rc = fill(e->cold, cold, n_cold * sizeof(aw_sparse_code)))) return rc;
    if (entropy && (rc = ensure(e->out, n_blocks * 4, e->last_error))) return rc;
    d.hot = (const uint16_t*)e->hot.ptr;
    d.dict = (const uint16_t*)e->dict.ptr;
    d.src_blocks = (const uint32_t*)e->refs.ptr;
    d.cold = (aw_sparse_code*)e->cold.ptr;
    d.entropy = entropy ? (float*)e->out.ptr : nullptr;
    d.hot_blocks = hot_blocks;
    d.cold_blocks = cold_blocks;
    if ((rc = encode_device(e, &d, e->stream))) return rc;
    AW_HIP(e, hipMemcpyAsync(cold, e->cold.ptr, n_cold * sizeof(aw_sparse_code), hipMemcpyDeviceToHost, e->stream));
    if (entropy) AW_HIP(e, hipMemcpyAsync(entropy, e->out.ptr, n_blocks * 4, hipMemcpyDeviceToHost, e->stream));
    AW_HIP(e, hipStreamSynchronize(e->stream));
    return aw_engine_check_device_errors(e, e->stream);
}

int aw_debug_read_stream(aw_engine* e, const void* buf, uint64_t bytes, uint32_t waves_per_cu, uint32_t* sink,
                         void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    if (!buf || !sink || !bytes || (bytes & 15u) || ((uintptr_t)buf & 15u))
        return fail(e, AW_E_INVALID_ARG, "buf (16-byte aligned), sink and bytes (a multiple of 16) are required");
    if (waves_per_cu < 4 || waves_per_cu > 64 || (waves_per_cu & 3u))
        return fail(e, AW_E_INVALID_ARG, "waves_per_cu %u must be a multiple of 4 in [4, 64]", waves_per_cu);
    AW_HIP(e, hipSetDevice(e->device));
    const uint32_t grid = e->n_cu * (waves_per_cu / 4); // 4 waves per 256-thread work-group
    hipLaunchKernelGGL(aw::read_stream_kernel<8>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const aw::uint4_t*)buf, bytes / 16, sink);
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

int aw_debug_project(aw_engine* e, const aw_decode_desc* d, void* q_latent, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    if (!d || !q_latent) return fail(e, AW_E_INVALID_ARG, "desc and q_latent are required");
    Layout o;
    char msg[256] = {0};
    int rc = plan(d, e->max_lds, e->n_cu, e->hot_wpc, e->cold_output, &o, msg, sizeof msg);
    if (rc) return fail(e, rc, "%s", msg);
    if (!o.info.computes_q_latent)
        return fail(e, AW_E_INVALID_ARG, "the request does not compute q_latent (it needs a cold pool and q_latent NULL)");
    if (!d->q || !d->dict) return fail(e, AW_E_INVALID_ARG, "q and dict are required");
    AW_HIP(e, hipSetDevice(e->device));
    hipStream_t st = (hipStream_t)stream; // NULL is HIP's null stream
    if ((rc = ensure_keep(e->ws, o.info.workspace_bytes, e->retired_ws, e->last_error, st))) return rc;
    char* ws = (char*)e->ws.ptr;
    rc = d->head_dim == 64 ? launch_project<64>(e, d, o, ws, st) : launch_project<128>(e, d, o, ws, st);
    if (rc) return rc;
    const size_t bytes = (size_t)d->layers * d->batch * d->queries * d->q_heads * d->dict_size * (o.qf32 ? 4 : 2);
    AW_HIP(e, hipMemcpyAsync(q_latent, ws + o.off_ql, bytes, hipMemcpyDeviceToDevice, st));
    return AW_OK;
}

int aw_debug_read_pools(aw_engine* e, const aw_decode_desc* d, uint32_t* sink, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    if (!d || !sink) return fail(e, AW_E_INVALID_ARG, "desc and sink are required");
    if (d->layers == 0 || d->batch == 0 || d->kv_heads == 0 || (d->head_dim != 64 && d->head_dim != 128))
        return fail(e, AW_E_INVALID_ARG, "layers, batch, kv_heads >= 1 and head_dim 64 or 128 are required");
    if (d->refs_stride < d->hot_count + d->cold_count) return fail(e, AW_E_INVALID_ARG, "refs_stride too small");
    if ((d->hot_count && (!d->hot_k || !d->hot_blocks)) || (d->cold_count && (!d->cold || !d->cold_blocks)) ||
        ((d->hot_count || d->cold_count) && !d->refs))
        return fail(e, AW_E_INVALID_ARG, "pools, capacities and refs are required for the blocks asked for");
    if (((uintptr_t)d->hot_k | (uintptr_t)d->hot_v | (uintptr_t)d->cold) & 15u)
        return fail(e, AW_E_ALIGN, "pools must be 16-byte aligned");
    AW_HIP(e, hipSetDevice(e->device));
    aw::GatherArgs a{};
    a.hot_k = (const aw::uint4_t*)d->hot_k;
    a.hot_v = (const aw::uint4_t*)d->hot_v;
    a.cold = (const aw::uint4_t*)d->cold;
    a.refs = d->refs;
    a.sink = sink;
    a.batch = d->batch;
    a.kv_heads = d->kv_heads;
    a.hd16 = d->head_dim / 8;
    a.hot_count = d->hot_count;
    a.cold_count = d->cold_count;
    a.refs_stride = d->refs_stride;
    a.cold_head_blocked = (d->flags & AW_F_COLD_HEAD_BLOCKED) ? 1u : 0u;
    a.hot_units = (uint32_t)cdiv(d->hot_count, aw::kGatherHotBlocks);
    a.cold_units = (uint32_t)cdiv(d->cold_count, aw::kGatherColdBlocks);
    a.hot_blocks = d->hot_blocks;
    a.cold_blocks = d->cold_blocks;
    a.hot_layer16 = d->hot_blocks * kBlock * d->kv_heads * a.hd16;
    a.cold_layer16 = d->cold_blocks * kBlock * d->kv_heads;
    a.refs_layer = (uint64_t)d->batch * d->refs_stride;
    const uint64_t grid = (uint64_t)d->layers * d->batch * d->kv_heads * (a.hot_units + a.cold_units);
    if (grid == 0) return AW_OK;
    if (grid > 0x7FFFFFFFull) return fail(e, AW_E_UNSUPPORTED, "gather grid too large");
    hipLaunchKernelGGL(aw::gather_read_kernel<8>, dim3((uint32_t)grid), dim3(64), 0, (hipStream_t)stream, a);
    AW_HIP(e, hipGetLastError());
    return AW_OK;
}

int aw_engine_set_projection(aw_engine* e, int mode) {
    if (!e) return AW_E_INVALID_ARG;
    if (mode < AW_PROJECT_AUTO || mode > AW_PROJECT_VALU) return fail(e, AW_E_INVALID_ARG, "projection mode %d", mode);
    e->projection = mode;
    return AW_OK;
}

int aw_engine_set_cold_output(aw_engine* e, int mode) {
    if (!e) return AW_E_INVALID_ARG;
    if (mode < AW_COLD_OUT_AUTO || mode > AW_COLD_OUT_VALUES) return fail(e, AW_E_INVALID_ARG, "cold output mode %d", mode);
    e->cold_output = mode;
    return AW_OK;
}

int aw_engine_set_profiling(aw_engine* e, int enable) {
    if (!e) return AW_E_INVALID_ARG;
    if (enable < AW_PROFILE_OFF || enable > AW_PROFILE_SERIAL) return fail(e, AW_E_INVALID_ARG, "profiling mode %d", enable);
    e->profiling = enable;
    return AW_OK;
}

int aw_engine_stage_stats(aw_engine* e, int stage, double* total_ms, uint64_t* launches) {
    if (!e || stage < 0 || stage >= AW_STAGE_COUNT) return AW_E_INVALID_ARG;
    drain_events(e);
    if (total_ms) *total_ms = e->stage_ms[stage];
    if (launches) *launches = e->stage_n[stage];
    return AW_OK;
}

int aw_engine_reset_stage_stats(aw_engine* e) {
    if (!e) return AW_E_INVALID_ARG;
    drain_events(e);
    for (int i = 0; i < AW_STAGE_COUNT; ++i) {
        e->stage_ms[i] = 0;
        e->stage_n[i] = 0;
    }
    return AW_OK;
}

} // extern "C"

// ------------------------------------------------- for the library's other sources

namespace aw_engine_internal {

int device(const aw_engine* e) { return e->device; }
uint32_t compute_units(const aw_engine* e) { return e->n_cu; }
uint32_t* error_word(const aw_engine* e) { return e->err; }
int fail(aw_engine* e, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (e) e->last_error = buf;
    return code;
}

} // namespace aw_engine_internal

