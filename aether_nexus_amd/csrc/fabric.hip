// The `.aether` Fabric: region map, genesis, boot, looms, checkpoint, and the
// residency of its pools in HBM.  Host code; the device work is copies and the
// Weaver library's own entry points (entropy, encoder).
//
// Reference: nexus-core/src/fabric.rs (FabricRegions, Fabric, create_genesis),
// nexus-core/src/types.rs (ModelDims, LoomDescriptor, WeaverParams::from_loom,
// constants), nexus-core/src/distiller.rs:60-120 (one REM cycle).

#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "aether_fabric.h"

namespace {

constexpr uint64_t kHeaderSize = AW_FABRIC_MAGIC_LEN + 4 + AW_FABRIC_SIGNATURE_LEN; // types.rs:497
constexpr uint64_t kObsBufSize = 256ull << 20;                                     // types.rs:506
constexpr uint64_t kTraceLogSize = 128ull << 20;                                   // types.rs:509
constexpr uint64_t kLoomBytes = sizeof(aw_loom_descriptor);                       // 32
constexpr uint64_t kCodeBytes = sizeof(aw_sparse_code);                           // 16
constexpr uint64_t kPage = 16384, kSmallPage = 4096;
constexpr uint64_t kLimit = 1ull << 62;
static_assert(sizeof(aw_loom_descriptor) == 32, "LoomDescriptor is 32 bytes (repr(C))");

// Staging for host <-> device copies: two pinned buffers, filled / drained by
// up to kIoThreads threads copying through the mapping while the DMA engine
// moves the other buffer.
constexpr uint64_t kStageBytes = 32ull << 20;
constexpr unsigned kIoThreads = 8;
constexpr uint64_t kIoMinPerThread = 2ull << 20;

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) & ~(a - 1); }

void put(char* msg, size_t mlen, const char* fmt, ...) {
    if (!msg || !mlen) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, mlen, fmt, ap);
    va_end(ap);
}

// Rust's io::Error text: "<strerror> (os error N)".
std::string os_error(int err) { return std::string(strerror(err)) + " (os error " + std::to_string(err) + ")"; }

// Checked product and sum of sizes (usize arithmetic in the reference).
struct Sz {
    unsigned __int128 v;
    bool ok() const { return v < kLimit; }
};
Sz operator*(Sz a, Sz b) { return Sz{(a.ok() && b.ok()) ? a.v * b.v : (unsigned __int128)kLimit}; }
Sz operator+(Sz a, Sz b) { return Sz{(a.ok() && b.ok()) ? a.v + b.v : (unsigned __int128)kLimit}; }
Sz S(uint64_t x) { return Sz{x}; }

// estimated_weight_bytes (fabric.rs:190-222): 2 bytes per parameter of the
// projections, norms and embedding, times 1.25 (f64, truncated).
bool weight_estimate(const aw_model_dims& d, uint64_t* out) {
    const Sz h = S(d.hidden_size), inter = S(d.intermediate_size), vocab = S(d.vocab_size);
    const Sz q = S(d.q_heads), kv = S(d.kv_heads), hd = S(d.head_dim);
    const Sz per_layer = S(2) * (q * hd * h + kv * hd * h + kv * hd * h + q * hd * h + h * inter + h * inter +
                                 inter * h + h + h);
    const Sz global = S(2) * (vocab * h + h);
    const Sz raw = S(d.layers) * per_layer + global;
    if (!raw.ok()) return false;
    const double scaled = (double)(uint64_t)raw.v * 1.25;
    if (!(scaled < (double)kLimit)) return false;
    *out = (uint64_t)scaled;
    return true;
}

// FabricRegions::compute (fabric.rs:124-186).
bool compute_regions(const aw_model_dims& d, aw_fabric_regions* r) {
    uint64_t w = 0;
    if (!weight_estimate(d, &w)) return false;
    const Sz hot = S(AW_FABRIC_MAX_HOT_BLOCKS) * S(d.block_size) * S(d.kv_heads) * S(d.head_dim) * S(2);
    const Sz cold = S(AW_FABRIC_MAX_COLD_BLOCKS) * S(d.block_size) * S(d.kv_heads) * S(kCodeBytes);
    const Sz dict = S(d.kv_heads) * S(d.dict_size) * S(d.head_dim) * S(2);
    if (!hot.ok() || !cold.ok() || !dict.ok()) return false;
    aw_fabric_regions o{};
    o.weights_offset = align_up(kHeaderSize, kPage);
    o.weights_size = align_up(w, kPage);
    o.hot_pool_offset = align_up(o.weights_offset + o.weights_size, kPage);
    o.hot_pool_size = (uint64_t)hot.v;
    o.cold_pool_offset = align_up(o.hot_pool_offset + o.hot_pool_size, kPage);
    o.cold_pool_size = (uint64_t)cold.v;
    o.dict_offset = align_up(o.cold_pool_offset + o.cold_pool_size, kPage);
    o.dict_size = (uint64_t)dict.v;
    o.looms_offset = align_up(o.dict_offset + o.dict_size, kSmallPage);
    o.looms_size = AW_FABRIC_PERSONAS * kLoomBytes;
    o.radix_offset = align_up(o.looms_offset + o.looms_size, kSmallPage);
    o.radix_size = (uint64_t)(AW_FABRIC_MAX_HOT_BLOCKS + AW_FABRIC_MAX_COLD_BLOCKS) * 3 * 4;
    o.obs_offset = align_up(o.radix_offset + o.radix_size, kPage);
    o.obs_size = kObsBufSize;
    o.trace_offset = align_up(o.obs_offset + o.obs_size, kPage);
    o.trace_size = kTraceLogSize;
    o.total_size = align_up(o.trace_offset + o.trace_size + AW_FABRIC_SIGNATURE_LEN, kPage);
    if (o.total_size >= kLimit) return false;
    *r = o;
    return true;
}

uint32_t rd_u32(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

// parse_looms (fabric.rs:518-549).
void parse_looms(const uint8_t* loom_bytes, aw_loom_descriptor out[4]) {
    for (uint32_t i = 0; i < AW_FABRIC_PERSONAS; ++i) {
        const uint8_t* p = loom_bytes + i * kLoomBytes;
        aw_loom_descriptor l{};
        l.persona = p[0] <= 3 ? p[0] : 0; // unknown persona bytes read as Planner
        l.hot_count = rd_u32(p + 4);
        l.cold_count = rd_u32(p + 8);
        l.hot_refs_offset = rd_u32(p + 12);
        l.cold_refs_offset = rd_u32(p + 16);
        l.token_pos = rd_u32(p + 20);
        out[i] = l;
    }
}

bool region_span(const aw_fabric_regions& r, uint32_t region, uint64_t* off, uint64_t* size) {
    switch (region) {
    case AW_REGION_WEIGHTS: *off = r.weights_offset; *size = r.weights_size; return true;
    case AW_REGION_HOT: *off = r.hot_pool_offset; *size = r.hot_pool_size; return true;
    case AW_REGION_COLD: *off = r.cold_pool_offset; *size = r.cold_pool_size; return true;
    case AW_REGION_DICT: *off = r.dict_offset; *size = r.dict_size; return true;
    case AW_REGION_LOOMS: *off = r.looms_offset; *size = r.looms_size; return true;
    case AW_REGION_RADIX: *off = r.radix_offset; *size = r.radix_size; return true;
    case AW_REGION_OBS: *off = r.obs_offset; *size = r.obs_size; return true;
    case AW_REGION_TRACE: *off = r.trace_offset; *size = r.trace_size; return true;
    default: return false;
    }
}

// Whole-range pwrite with EINTR and short-transfer handling.
bool pwrite_all(int fd, const void* src, uint64_t n, uint64_t off) {
    const uint8_t* p = (const uint8_t*)src;
    while (n) {
        const ssize_t k = pwrite(fd, p, (size_t)std::min<uint64_t>(n, 1ull << 30), (off_t)off);
        if (k < 0 && errno == EINTR) continue;
        if (k <= 0) return false;
        p += k, off += (uint64_t)k, n -= (uint64_t)k;
    }
    return true;
}

// Copies [off, off + n) of the shared mapping into buf (to_map false) or buf
// into the mapping (true) on up to kIoThreads threads.  Through the mapping
// rather than with pread / pwrite: concurrent pwrites to one file serialise on
// its inode lock (write-back of the 64 MiB Llama8B cold pool: ~12 GB/s with
// pwrite against ~37 GB/s with memcpy).
void map_copy(uint8_t* map, uint8_t* buf, uint64_t n, uint64_t off, bool to_map) {
    const unsigned t = (unsigned)std::max<uint64_t>(1, std::min<uint64_t>(kIoThreads, n / kIoMinPerThread));
    if (t == 1) {
        if (to_map) memcpy(map + off, buf, n);
        else memcpy(buf, map + off, n);
        return;
    }
    const uint64_t per = align_up((n + t - 1) / t, 4096);
    std::vector<std::thread> th;
    th.reserve(t);
    for (unsigned i = 0; i < t; ++i) {
        const uint64_t a = (uint64_t)i * per;
        if (a >= n) break;
        const uint64_t len = std::min(per, n - a);
        th.emplace_back([=] {
            if (to_map) memcpy(map + off + a, buf + a, len);
            else memcpy(buf + a, map + off + a, len);
        });
    }
    for (auto& x : th) x.join();
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Reorders whole cold-pool blocks of 16-byte codes between the file's order
// [block][token][kv_head] and the head-blocked order [block][kv_head][token]
// (to_head_blocked 1) or back (0).  One thread per code; reads are coalesced.
__global__ __launch_bounds__(256) void cold_reorder_kernel(const u32x4* src, u32x4* dst, uint64_t n_codes,
                                                           uint32_t block_size, uint32_t kv_heads,
                                                           int to_head_blocked) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_codes) return;
    const uint64_t per = (uint64_t)block_size * kv_heads;
    const uint64_t blk = i / per, r = i % per;
    uint64_t j;
    if (to_head_blocked) {
        const uint64_t t = r / kv_heads, g = r % kv_heads;
        j = g * block_size + t;
    } else {
        const uint64_t g = r / block_size, t = r % block_size;
        j = t * kv_heads + g;
    }
    dst[blk * per + j] = src[i];
}

} // namespace

struct aw_fabric {
    int fd = -1;
    uint8_t* base = nullptr;
    uint64_t map_len = 0;
    aw_model_dims dims{};
    aw_fabric_regions regions{};
    aw_loom_descriptor looms[4]{};
    std::atomic<bool> dirty{false};
    std::mutex ckpt_mu;
    std::chrono::steady_clock::time_point last_ckpt{};
    std::string last_error;
    // Device residency.
    int device = -1;
    hipStream_t stream = nullptr;
    void* dev[AW_REGION_COUNT] = {};
    uint8_t* stage[2] = {nullptr, nullptr};
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
    bool cold_hb = false;       // device cold pool in the head-blocked order
    uint8_t* dstage = nullptr;  // device staging for reordered cold-pool chunks
};

namespace {

int ffail(aw_fabric* f, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (f) f->last_error = buf;
    return code;
}

#define FAB_HIP(f, call)                                                                            \
    do {                                                                                            \
        hipError_t e_ = (call);                                                                     \
        if (e_ != hipSuccess) return ffail(f, AW_E_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

int ensure_staging(aw_fabric* f) {
    for (int i = 0; i < 2; ++i) {
        if (!f->stage[i]) FAB_HIP(f, hipHostMalloc((void**)&f->stage[i], kStageBytes, hipHostMallocDefault));
        if (!f->stage_ev[i]) FAB_HIP(f, hipEventCreateWithFlags(&f->stage_ev[i], hipEventDisableTiming));
    }
    return AW_OK;
}

bool check_range(aw_fabric* f, uint32_t region, uint64_t offset, uint64_t bytes, uint64_t* file_off) {
    uint64_t off = 0, size = 0;
    if (!region_span(f->regions, region, &off, &size) || !f->dev[region]) return false;
    if (offset > size || bytes > size - offset) return false;
    *file_off = off + offset;
    return true;
}

// File -> device, chunk by chunk: the threads read chunk c into one staging
// buffer while the DMA of chunk c - 1 runs from the other.
int upload(aw_fabric* f, uint32_t region, uint64_t offset, uint64_t bytes) {
    uint64_t file_off = 0;
    if (!check_range(f, region, offset, bytes, &file_off))
        return ffail(f, AW_E_INVALID_ARG, "region %u range [%llu, +%llu) is not attached or out of bounds", region,
                     (unsigned long long)offset, (unsigned long long)bytes);
    int rc = ensure_staging(f);
    if (rc) return rc;
    uint8_t* dst = (uint8_t*)f->dev[region] + offset;
    const uint64_t nc = (bytes + kStageBytes - 1) / kStageBytes;
    for (uint64_t c = 0; c < nc; ++c) {
        const int b = (int)(c & 1);
        const uint64_t at = c * kStageBytes, len = std::min(kStageBytes, bytes - at);
        if (c >= 2) FAB_HIP(f, hipEventSynchronize(f->stage_ev[b]));
        map_copy(f->base, f->stage[b], len, file_off + at, false);
        FAB_HIP(f, hipMemcpyAsync(dst + at, f->stage[b], len, hipMemcpyHostToDevice, f->stream));
        FAB_HIP(f, hipEventRecord(f->stage_ev[b], f->stream));
    }
    FAB_HIP(f, hipStreamSynchronize(f->stream));
    return AW_OK;
}

// Device -> file: the DMA of chunk c + 1 runs while the threads write chunk c.
int download(aw_fabric* f, uint32_t region, uint64_t offset, uint64_t bytes) {
    uint64_t file_off = 0;
    if (!check_range(f, region, offset, bytes, &file_off))
        return ffail(f, AW_E_INVALID_ARG, "region %u range [%llu, +%llu) is not attached or out of bounds", region,
                     (unsigned long long)offset, (unsigned long long)bytes);
    int rc = ensure_staging(f);
    if (rc) return rc;
    const uint8_t* src = (const uint8_t*)f->dev[region] + offset;
    const uint64_t nc = (bytes + kStageBytes - 1) / kStageBytes;
    auto issue = [&](uint64_t c) -> int {
        const int b = (int)(c & 1);
        const uint64_t at = c * kStageBytes, len = std::min(kStageBytes, bytes - at);
        FAB_HIP(f, hipMemcpyAsync(f->stage[b], src + at, len, hipMemcpyDeviceToHost, f->stream));
        FAB_HIP(f, hipEventRecord(f->stage_ev[b], f->stream));
        return AW_OK;
    };
    if (nc && (rc = issue(0))) return rc;
    for (uint64_t c = 0; c < nc; ++c) {
        const int b = (int)(c & 1);
        const uint64_t at = c * kStageBytes, len = std::min(kStageBytes, bytes - at);
        if (c + 1 < nc && (rc = issue(c + 1))) return rc;
        FAB_HIP(f, hipEventSynchronize(f->stage_ev[b]));
        map_copy(f->base, f->stage[b], len, file_off + at, true);
    }
    FAB_HIP(f, hipStreamSynchronize(f->stream));
    return AW_OK;
}

uint64_t cold_block_bytes(const aw_fabric* f) { return (uint64_t)f->dims.block_size * f->dims.kv_heads * kCodeBytes; }

int launch_reorder(aw_fabric* f, const void* src, void* dst, uint64_t n_blocks, int to_hb) {
    const uint64_t n = n_blocks * f->dims.block_size * f->dims.kv_heads;
    if (!n) return AW_OK;
    hipLaunchKernelGGL(cold_reorder_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, f->stream,
                       (const u32x4*)src, (u32x4*)dst, n, f->dims.block_size, f->dims.kv_heads, to_hb);
    FAB_HIP(f, hipGetLastError());
    return AW_OK;
}

// The head-blocked device cold pool moves in whole blocks: bytes
// [offset, offset + bytes) of the file's cold region are widened to the blocks
// that hold them.  Upload: the file's blocks go through pinned and device
// staging and are reordered into place.
int upload_cold_hb(aw_fabric* f, uint64_t offset, uint64_t bytes) {
    const uint64_t bb = cold_block_bytes(f), per_chunk = std::max<uint64_t>(1, kStageBytes / bb);
    const uint64_t b0 = offset / bb, b1 = (offset + bytes + bb - 1) / bb;
    uint8_t* pool = (uint8_t*)f->dev[AW_REGION_COLD];
    uint64_t c = 0;
    for (uint64_t blk = b0; blk < b1; blk += per_chunk, ++c) {
        const int b = (int)(c & 1);
        const uint64_t nb = std::min(per_chunk, b1 - blk), len = nb * bb;
        if (c >= 2) FAB_HIP(f, hipEventSynchronize(f->stage_ev[b]));
        map_copy(f->base, f->stage[b], len, f->regions.cold_pool_offset + blk * bb, false);
        FAB_HIP(f, hipMemcpyAsync(f->dstage, f->stage[b], len, hipMemcpyHostToDevice, f->stream));
        FAB_HIP(f, hipEventRecord(f->stage_ev[b], f->stream));
        const int rc = launch_reorder(f, f->dstage, pool + blk * bb, nb, 1);
        if (rc) return rc;
    }
    FAB_HIP(f, hipStreamSynchronize(f->stream));
    return AW_OK;
}

// Download: whole blocks are reordered back into device staging and copied
// out; only the requested bytes are written into the mapping.
int download_cold_hb(aw_fabric* f, uint64_t offset, uint64_t bytes) {
    const uint64_t bb = cold_block_bytes(f), per_chunk = std::max<uint64_t>(1, kStageBytes / bb);
    const uint64_t b0 = offset / bb, b1 = (offset + bytes + bb - 1) / bb;
    const uint8_t* pool = (const uint8_t*)f->dev[AW_REGION_COLD];
    const uint64_t nc = (b1 - b0 + per_chunk - 1) / per_chunk;
    auto issue = [&](uint64_t c) -> int {
        const int b = (int)(c & 1);
        const uint64_t blk = b0 + c * per_chunk, nb = std::min(per_chunk, b1 - blk);
        int rc = launch_reorder(f, pool + blk * bb, f->dstage, nb, 0);
        if (rc) return rc;
        FAB_HIP(f, hipMemcpyAsync(f->stage[b], f->dstage, nb * bb, hipMemcpyDeviceToHost, f->stream));
        FAB_HIP(f, hipEventRecord(f->stage_ev[b], f->stream));
        return AW_OK;
    };
    int rc = AW_OK;
    if (nc && (rc = issue(0))) return rc;
    for (uint64_t c = 0; c < nc; ++c) {
        const int b = (int)(c & 1);
        const uint64_t blk = b0 + c * per_chunk, nb = std::min(per_chunk, b1 - blk);
        if (c + 1 < nc && (rc = issue(c + 1))) return rc;
        FAB_HIP(f, hipEventSynchronize(f->stage_ev[b]));
        // This chunk holds cold-region bytes [blk * bb, (blk + nb) * bb); keep the requested part.
        const uint64_t lo = std::max(offset, blk * bb), hi = std::min(offset + bytes, (blk + nb) * bb);
        map_copy(f->base, f->stage[b] + (lo - blk * bb), hi - lo, f->regions.cold_pool_offset + lo, true);
    }
    FAB_HIP(f, hipStreamSynchronize(f->stream));
    return AW_OK;
}

int ensure_dstage(aw_fabric* f) {
    if (!f->dstage) FAB_HIP(f, hipMalloc((void**)&f->dstage, kStageBytes));
    return AW_OK;
}

// Host -> device / device -> host of a byte range, in the device layout of the region.
int move(aw_fabric* f, uint32_t region, uint64_t offset, uint64_t bytes, bool to_device) {
    if (region == AW_REGION_COLD && f->cold_hb) {
        uint64_t file_off = 0;
        if (!check_range(f, region, offset, bytes, &file_off))
            return ffail(f, AW_E_INVALID_ARG, "region %u range [%llu, +%llu) is not attached or out of bounds",
                         region, (unsigned long long)offset, (unsigned long long)bytes);
        int rc = ensure_staging(f);
        if (!rc) rc = ensure_dstage(f);
        if (rc) return rc;
        if (!bytes) return AW_OK;
        return to_device ? upload_cold_hb(f, offset, bytes) : download_cold_hb(f, offset, bytes);
    }
    return to_device ? upload(f, region, offset, bytes) : download(f, region, offset, bytes);
}

void free_device(aw_fabric* f) {
    if (f->device < 0) return;
    (void)hipSetDevice(f->device);
    if (f->stream) (void)hipStreamSynchronize(f->stream);
    for (auto& p : f->dev) {
        if (p) (void)hipFree(p);
        p = nullptr;
    }
    for (int i = 0; i < 2; ++i) {
        if (f->stage_ev[i]) (void)hipEventDestroy(f->stage_ev[i]);
        if (f->stage[i]) (void)hipHostFree(f->stage[i]);
        f->stage_ev[i] = nullptr;
        f->stage[i] = nullptr;
    }
    if (f->dstage) (void)hipFree(f->dstage);
    f->dstage = nullptr;
    if (f->stream) (void)hipStreamDestroy(f->stream);
    f->stream = nullptr;
    f->device = -1;
}

} // namespace

extern "C" {

int aw_model_dims_preset(const char* name, aw_model_dims* out) {
    if (!name || !out) return AW_E_INVALID_ARG;
    // ModelDims defaults (types.rs:150-164) and the presets' overrides (:166-202).
    aw_model_dims d{32, 32, 8, 128, 32 * 128, 14336, 128256, 16, 4, 512};
    if (!strcmp(name, "llama8b")) {
    } else if (!strcmp(name, "granite2b")) {
        d.layers = 40, d.q_heads = 32, d.kv_heads = 8, d.head_dim = 64;
        d.hidden_size = 2048, d.intermediate_size = 8192, d.vocab_size = 49155;
    } else if (!strcmp(name, "qwen05b")) {
        d.layers = 24, d.q_heads = 14, d.kv_heads = 2, d.head_dim = 64;
        d.hidden_size = 896, d.intermediate_size = 4864, d.vocab_size = 151936;
    } else if (!strcmp(name, "deepseek_r1_1_5b")) {
        d.layers = 28, d.q_heads = 12, d.kv_heads = 2, d.head_dim = 128;
        d.hidden_size = 1536, d.intermediate_size = 8960, d.vocab_size = 151936;
    } else {
        return AW_E_INVALID_ARG;
    }
    *out = d;
    return AW_OK;
}

int aw_fabric_regions_compute(const aw_model_dims* dims, aw_fabric_regions* out) {
    if (!dims || !out) return AW_E_INVALID_ARG;
    return compute_regions(*dims, out) ? AW_OK : AW_E_INVALID_ARG;
}

int aw_weaver_params_from_loom(const aw_model_dims* d, const aw_loom_descriptor* loom, aw_weaver_params* out) {
    if (!d || !loom || !out || !d->kv_heads) return AW_E_INVALID_ARG;
    aw_weaver_params p{};
    p.q_heads = d->q_heads;
    p.kv_heads = d->kv_heads;
    p.head_dim = d->head_dim;
    p.block_size = d->block_size;
    p.gqa_group = d->q_heads / d->kv_heads;
    p.hot_count = loom->hot_count;
    p.cold_count = loom->cold_count;
    p.dict_size = d->dict_size;
    p.sparsity_k = d->sparsity_k;
    *out = p;
    return AW_OK;
}

int aw_fabric_create_genesis(const char* path, const aw_model_dims* dims, char* msg, size_t mlen) {
    if (!path || !dims) return AW_E_INVALID_ARG;
    aw_fabric_regions r{};
    if (!compute_regions(*dims, &r)) {
        put(msg, mlen, "layout mismatch: region sizes overflow");
        return AW_E_INVALID_ARG;
    }
    const int fd = open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) {
        put(msg, mlen, "mmap failed: %s", os_error(errno).c_str());
        return AW_E_IO;
    }
    uint8_t head[AW_FABRIC_MAGIC_LEN + 4];
    memcpy(head, AW_FABRIC_MAGIC, AW_FABRIC_MAGIC_LEN);
    const uint32_t v = AW_FABRIC_VERSION;
    for (int i = 0; i < 4; ++i) head[AW_FABRIC_MAGIC_LEN + i] = (uint8_t)(v >> (8 * i));
    bool ok = ftruncate(fd, (off_t)r.total_size) == 0 && pwrite_all(fd, head, sizeof head, 0);
    for (uint32_t i = 0; ok && i < AW_FABRIC_PERSONAS; ++i) {
        const uint8_t persona = (uint8_t)i;
        ok = pwrite_all(fd, &persona, 1, r.looms_offset + i * kLoomBytes);
    }
    ok = ok && fsync(fd) == 0;
    const int err = errno;
    close(fd);
    if (!ok) {
        put(msg, mlen, "checkpoint flush failed: %s", os_error(err).c_str());
        return AW_E_IO;
    }
    return AW_OK;
}

int aw_fabric_boot(const char* path, const aw_model_dims* dims, const uint8_t* public_key, aw_fabric** out,
                   char* msg, size_t mlen) {
    if (!path || !dims || !out) return AW_E_INVALID_ARG;
    *out = nullptr;
    aw_fabric_regions r{};
    if (!compute_regions(*dims, &r)) {
        put(msg, mlen, "layout mismatch: region sizes overflow");
        return AW_E_INVALID_ARG;
    }
    const int fd = open(path, O_RDWR);
    if (fd < 0) {
        put(msg, mlen, "mmap failed: %s", os_error(errno).c_str());
        return AW_E_IO;
    }
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        put(msg, mlen, "mmap failed: %s", os_error(errno).c_str());
        close(fd);
        return AW_E_IO;
    }
    const uint64_t len = (uint64_t)st.st_size;
    if (len < r.total_size) {
        put(msg, mlen, "file too small: expected at least %llu bytes, got %llu", (unsigned long long)r.total_size,
            (unsigned long long)len);
        close(fd);
        return AW_E_TOO_SMALL;
    }
    void* base = mmap(nullptr, (size_t)len, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    if (base == MAP_FAILED) {
        put(msg, mlen, "mmap failed: %s", os_error(errno).c_str());
        close(fd);
        return AW_E_IO;
    }
    const uint8_t* b = (const uint8_t*)base;
    int rc = AW_OK;
    if (memcmp(b, AW_FABRIC_MAGIC, AW_FABRIC_MAGIC_LEN) != 0) {
        put(msg, mlen, "invalid magic bytes");
        rc = AW_E_BAD_MAGIC;
    } else if (rd_u32(b + AW_FABRIC_MAGIC_LEN) != AW_FABRIC_VERSION) {
        put(msg, mlen, "version mismatch: expected 0x%08x, got 0x%08x", AW_FABRIC_VERSION,
            rd_u32(b + AW_FABRIC_MAGIC_LEN));
        rc = AW_E_VERSION;
    } else if (public_key) {
        put(msg, mlen, "Ed25519 signature verification is not implemented by this library; boot with no key (dev mode)");
        rc = AW_E_UNSUPPORTED;
    }
    if (rc) {
        munmap(base, (size_t)len);
        close(fd);
        return rc;
    }
    aw_fabric* f = new aw_fabric();
    f->fd = fd;
    f->base = (uint8_t*)base;
    f->map_len = len;
    f->dims = *dims;
    f->regions = r;
    parse_looms(f->base + r.looms_offset, f->looms);
    f->last_ckpt = std::chrono::steady_clock::now();
    *out = f;
    return AW_OK;
}

void aw_fabric_close(aw_fabric* f) {
    if (!f) return;
    free_device(f);
    if (f->base) munmap(f->base, (size_t)f->map_len);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

const char* aw_fabric_last_error(const aw_fabric* f) { return f ? f->last_error.c_str() : "null fabric"; }

int aw_fabric_regions_of(const aw_fabric* f, aw_fabric_regions* out) {
    if (!f || !out) return AW_E_INVALID_ARG;
    *out = f->regions;
    return AW_OK;
}

int aw_fabric_looms(const aw_fabric* f, aw_loom_descriptor out[4]) {
    if (!f || !out) return AW_E_INVALID_ARG;
    for (int i = 0; i < 4; ++i) out[i] = f->looms[i];
    return AW_OK;
}

int aw_fabric_region(aw_fabric* f, uint32_t region, int writable, void** ptr, uint64_t* bytes) {
    if (!f || !ptr) return AW_E_INVALID_ARG;
    uint64_t off = 0, size = 0;
    if (!region_span(f->regions, region, &off, &size)) return ffail(f, AW_E_INVALID_ARG, "unknown region %u", region);
    *ptr = f->base + off;
    if (bytes) *bytes = size;
    if (writable && region != AW_REGION_TRACE) f->dirty.store(true, std::memory_order_release);
    return AW_OK;
}

int aw_fabric_checkpoint(aw_fabric* f) {
    if (!f) return AW_E_INVALID_ARG;
    if (!f->dirty.load(std::memory_order_acquire)) return AW_OK;
    std::lock_guard<std::mutex> lock(f->ckpt_mu);
    if (std::chrono::steady_clock::now() - f->last_ckpt < std::chrono::milliseconds(AW_FABRIC_CHECKPOINT_MS))
        return AW_OK;
    if (msync(f->base, (size_t)f->map_len, MS_ASYNC) != 0)
        return ffail(f, AW_E_IO, "checkpoint flush failed: %s", os_error(errno).c_str());
    f->dirty.store(false, std::memory_order_release);
    f->last_ckpt = std::chrono::steady_clock::now();
    return AW_OK;
}

int aw_fabric_force_checkpoint(aw_fabric* f) {
    if (!f) return AW_E_INVALID_ARG;
    std::lock_guard<std::mutex> lock(f->ckpt_mu);
    if (msync(f->base, (size_t)f->map_len, MS_SYNC) != 0)
        return ffail(f, AW_E_IO, "checkpoint flush failed: %s", os_error(errno).c_str());
    f->dirty.store(false, std::memory_order_release);
    f->last_ckpt = std::chrono::steady_clock::now();
    return AW_OK;
}

int aw_fabric_is_dirty(const aw_fabric* f) { return f && f->dirty.load(std::memory_order_acquire) ? 1 : 0; }

int aw_fabric_attach_device(aw_fabric* f, int device, uint32_t mask) {
    if (!f) return AW_E_INVALID_ARG;
    const bool hb = (mask & AW_FABRIC_COLD_HEAD_BLOCKED) != 0;
    mask &= ~AW_FABRIC_COLD_HEAD_BLOCKED;
    if (mask & ~((1u << AW_REGION_COUNT) - 1u)) return ffail(f, AW_E_INVALID_ARG, "unknown region bits 0x%x", mask);
    if (hb && !(mask & AW_REGION_BIT(AW_REGION_COLD)))
        return ffail(f, AW_E_INVALID_ARG, "AW_FABRIC_COLD_HEAD_BLOCKED needs the cold region in the mask");
    if (f->device >= 0 && f->device != device)
        return ffail(f, AW_E_INVALID_ARG, "fabric is attached to device %d", f->device);
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
        return ffail(f, AW_E_HIP, "no HIP device %d", device);
    FAB_HIP(f, hipSetDevice(device));
    if (!f->stream) FAB_HIP(f, hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking));
    f->device = device;
    for (uint32_t r = 0; r < AW_REGION_COUNT; ++r) {
        if (!(mask & (1u << r))) continue;
        uint64_t off = 0, size = 0;
        region_span(f->regions, r, &off, &size);
        if (!f->dev[r]) FAB_HIP(f, hipMalloc(&f->dev[r], (size_t)size));
        if (r == AW_REGION_COLD) f->cold_hb = hb;
        const int rc = move(f, r, 0, size, true);
        if (rc) return rc;
    }
    return AW_OK;
}

int aw_fabric_device_region(const aw_fabric* f, uint32_t region, void** dptr, uint64_t* bytes) {
    if (!f || !dptr || region >= AW_REGION_COUNT || !f->dev[region]) return AW_E_INVALID_ARG;
    uint64_t off = 0, size = 0;
    region_span(f->regions, region, &off, &size);
    *dptr = f->dev[region];
    if (bytes) *bytes = size;
    return AW_OK;
}

uint32_t aw_fabric_device_flags(const aw_fabric* f) {
    return (f && f->dev[AW_REGION_COLD] && f->cold_hb) ? AW_F_COLD_HEAD_BLOCKED : 0u;
}

int aw_fabric_push(aw_fabric* f, uint32_t region, uint64_t offset, uint64_t bytes) {
    if (!f) return AW_E_INVALID_ARG;
    if (f->device < 0) return ffail(f, AW_E_INVALID_ARG, "fabric is not attached to a device");
    FAB_HIP(f, hipSetDevice(f->device));
    return move(f, region, offset, bytes, true);
}

int aw_fabric_pull(aw_fabric* f, uint32_t region, uint64_t offset, uint64_t bytes) {
    if (!f) return AW_E_INVALID_ARG;
    if (f->device < 0) return ffail(f, AW_E_INVALID_ARG, "fabric is not attached to a device");
    FAB_HIP(f, hipSetDevice(f->device));
    const int rc = move(f, region, offset, bytes, false);
    if (rc == AW_OK && bytes && region != AW_REGION_TRACE) f->dirty.store(true, std::memory_order_release);
    return rc;
}

int aw_fabric_detach_device(aw_fabric* f) {
    if (!f) return AW_E_INVALID_ARG;
    free_device(f);
    return AW_OK;
}

int aw_fabric_distill(aw_fabric* f, aw_engine* e, float threshold, float* entropy, uint32_t* n_distilled) {
    if (!f || !e) return AW_E_INVALID_ARG;
    if (n_distilled) *n_distilled = 0;
    if (!f->dev[AW_REGION_HOT] || !f->dev[AW_REGION_COLD] || !f->dev[AW_REGION_DICT])
        return ffail(f, AW_E_INVALID_ARG, "distill needs the hot pool, cold pool and dictionary attached");
    const aw_model_dims& d = f->dims;
    if (d.block_size != 16 || d.sparsity_k != 4)
        return ffail(f, AW_E_UNSUPPORTED, "blocks of %u tokens with %u codes are not supported (16 and 4)",
                     d.block_size, d.sparsity_k);
    const uint64_t block_bytes = (uint64_t)d.block_size * d.kv_heads * d.head_dim * 2;
    const uint64_t code_block_bytes = (uint64_t)d.block_size * d.kv_heads * kCodeBytes;
    // evaluate_entropy: every hot block of the pool, at most 8192 (distiller.rs:101-107).
    const uint32_t n = (uint32_t)std::min<uint64_t>(f->regions.hot_pool_size / block_bytes, 8192);
    if (!n) return AW_OK;
    FAB_HIP(f, hipSetDevice(f->device));
    float* d_ent = nullptr;
    uint32_t* d_list = nullptr;
    FAB_HIP(f, hipMalloc((void**)&d_ent, (size_t)n * 4));
    if (hipMalloc((void**)&d_list, (size_t)n * 4) != hipSuccess) {
        (void)hipFree(d_ent);
        return ffail(f, AW_E_HIP, "hipMalloc of the candidate list failed");
    }
    auto release = [&] {
        (void)hipStreamSynchronize(f->stream);
        (void)hipFree(d_ent);
        (void)hipFree(d_list);
    };
    std::vector<float> ent(n);
    int rc = aw_block_entropy_device(e, (const uint16_t*)f->dev[AW_REGION_HOT], n, d.kv_heads, d.head_dim, nullptr,
                                     n, d_ent, f->stream);
    if (rc) {
        release();
        return ffail(f, rc, "block entropy: %s", aw_engine_last_error(e));
    }
    if (hipMemcpyAsync(ent.data(), d_ent, (size_t)n * 4, hipMemcpyDeviceToHost, f->stream) != hipSuccess ||
        hipStreamSynchronize(f->stream) != hipSuccess) {
        release();
        return ffail(f, AW_E_HIP, "copy of the block proxies failed");
    }
    if (entropy) memcpy(entropy, ent.data(), (size_t)n * 4);
    // Candidates: 0 < proxy < threshold, ascending (distiller.rs:112-115).
    std::vector<uint32_t> cand;
    for (uint32_t b = 0; b < n; ++b)
        if (ent[b] < threshold && ent[b] > 0.0f) cand.push_back(b);
    if (n_distilled) *n_distilled = (uint32_t)cand.size();
    const uint64_t cold_blocks = f->regions.cold_pool_size / code_block_bytes;
    if (!cand.empty() && cand.back() >= cold_blocks) {
        release();
        return ffail(f, AW_E_OOB, "cold pool overflow"); // distill_block, distiller.rs:178-180
    }
    if (!cand.empty()) {
        if (hipMemcpyAsync(d_list, cand.data(), cand.size() * 4, hipMemcpyHostToDevice, f->stream) != hipSuccess) {
            release();
            return ffail(f, AW_E_HIP, "copy of the candidate list failed");
        }
        aw_encode_desc ed{};
        ed.kv_heads = d.kv_heads;
        ed.head_dim = d.head_dim;
        ed.dict_size = d.dict_size;
        ed.dict_heads = d.kv_heads; // one dictionary per kv head (distiller.rs:201-202)
        ed.n_blocks = (uint32_t)cand.size();
        ed.hot_blocks = f->regions.hot_pool_size / block_bytes;
        ed.cold_blocks = cold_blocks;
        ed.hot = (const uint16_t*)f->dev[AW_REGION_HOT];
        ed.dict = (const uint16_t*)f->dev[AW_REGION_DICT];
        ed.src_blocks = d_list;
        ed.dst_blocks = nullptr;
        ed.cold = (aw_sparse_code*)f->dev[AW_REGION_COLD];
        ed.flags = f->cold_hb ? AW_F_COLD_HEAD_BLOCKED : 0u;
        rc = aw_encode_device(e, &ed, f->stream);
        if (rc) {
            release();
            return ffail(f, rc, "encode: %s", aw_engine_last_error(e));
        }
        if (hipStreamSynchronize(f->stream) != hipSuccess) {
            release();
            return ffail(f, AW_E_HIP, "encode failed on the device");
        }
        // Write back each run of consecutive candidate blocks.
        for (size_t i = 0; i < cand.size();) {
            size_t j = i + 1;
            while (j < cand.size() && cand[j] == cand[j - 1] + 1) ++j;
            rc = move(f, AW_REGION_COLD, (uint64_t)cand[i] * code_block_bytes, (uint64_t)(j - i) * code_block_bytes,
                      false);
            if (rc) {
                release();
                return rc;
            }
            i = j;
        }
        f->dirty.store(true, std::memory_order_release);
    }
    release();
    return aw_fabric_checkpoint(f);
}

} // extern "C"
