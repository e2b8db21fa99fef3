// ops.hip — C ABI of the dense transformer ops (include/aether_ops.h).
//
// Replaces the dispatch methods of the reference's Ops engine
// (nexus-core/src/ops.rs:166-462); the kernels are in ops_kernels.hpp.  Every
// entry point validates its arguments on the host, picks the 16-byte vector
// variant of a kernel when the pointers and sizes allow it, and enqueues on the
// caller's stream.  There is no CPU fallback.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../../include/aether_ops.h"
#include "engine_internal.hpp"
#include "ops_kernels.hpp"

namespace {

namespace ei = aw_engine_internal;

uint64_t cdiv64(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

#define OPS_HIP(e, call)                                                                        \
    do {                                                                                        \
        const hipError_t err_ = (call);                                                         \
        if (err_ != hipSuccess) return ei::fail(e, AW_E_HIP, "%s: %s", #call, hipGetErrorString(err_)); \
    } while (0)

int enter(aw_engine* e) {
    if (!e) return AW_E_INVALID_ARG;
    OPS_HIP(e, hipSetDevice(ei::device(e)));
    return AW_OK;
}

// Grid of an HBM-bound grid-strided kernel: enough work-groups for `units`
// threads' worth of work, at most 16 per CU.
uint32_t stream_grid(aw_engine* e, uint64_t units) {
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(cdiv64(units, 256), (uint64_t)ei::compute_units(e) * 16));
}

template <awo::Ew OP>
int launch_ew(aw_engine* e, const awo::EwArgs& p, bool vec, hipStream_t st) {
    if (p.n == 0) return AW_OK;
    const uint32_t grid = stream_grid(e, vec ? std::max<uint64_t>(p.n / 8, 1) : p.n);
    if (vec)
        hipLaunchKernelGGL((awo::ew_kernel<OP, true>), dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL((awo::ew_kernel<OP, false>), dim3(grid), dim3(256), 0, st, p);
    OPS_HIP(e, hipGetLastError());
    return AW_OK;
}

// One weight matrix of a product: B [n][k] (and B2, the up weights of a fused
// SiLU gate), output C [m][n].
struct Product {
    const uint16_t* b;
    const uint16_t* b2;
    void* c;
    uint32_t n;
};

// The products `p[0 .. np)` over the same activations a [m][k], one launch when
// m <= 64 (skinny), one launch each otherwise (tiled).  EPI picks the store;
// F32 the scaled fp32 output of matmul_scaled.
template <awo::Epi EPI, bool F32>
int launch_products(aw_engine* e, const char* what, const uint16_t* a, const Product* p, int np, uint32_t m,
                    uint32_t k, float scale, hipStream_t st) {
    if (m == 0) return AW_OK;
    if (!a) return ei::fail(e, AW_E_INVALID_ARG, "%s: null pointer", what);
    awo::GemmArgs g{};
    g.A = a;
    g.M = m;
    g.K = k;
    g.scale = scale;
    bool vec = k % 8 == 0 && aligned(a, 16);
    uint64_t tiles = 0;
    for (int i = 0; i < np; ++i) {
        if (!p[i].b || !p[i].c || (EPI == awo::Epi::SiluGate && !p[i].b2))
            return ei::fail(e, AW_E_INVALID_ARG, "%s: null pointer", what);
        vec = vec && aligned(p[i].b, 16) && (EPI != awo::Epi::SiluGate || aligned(p[i].b2, 16));
        g.g[g.groups].B = p[i].b;
        g.g[g.groups].B2 = p[i].b2;
        g.g[g.groups].C = p[i].c;
        g.g[g.groups].N = p[i].n;
        g.g[g.groups].tiles = (uint32_t)cdiv64(p[i].n, 16);
        g.g[g.groups].vec_out = p[i].n % 4 == 0 && aligned(p[i].c, F32 ? 16 : 8);
        tiles += cdiv64(p[i].n, 16);
        if (p[i].n) ++g.groups; // empty products drop out
    }
    if (!g.groups) return AW_OK;
    if (m > 64) {
        if (EPI == awo::Epi::SiluGate)
            return ei::fail(e, AW_E_UNSUPPORTED, "%s: m = %u rows (the fused gate takes m <= 64; use matmul and "
                                                 "silu_gate)", what, m);
        // One tiled launch per product, group 0 of its own arguments.
        for (uint32_t i = 0; i < g.groups; ++i) {
            awo::GemmArgs t = g;
            t.g[0] = g.g[i];
            t.groups = 1;
            // 256 x 128 tiles when they fill the CUs at least once (16-byte rows, each
            // operand below 4 GiB - 64 KiB for the buffer loads), else 128 x 128.
            const dim3 wgrid((uint32_t)cdiv64(t.g[0].N, awo::kWideN), (uint32_t)cdiv64(m, awo::kWideM));
            const uint64_t lim = (1ull << 32) - 65536;
            const bool wide = vec && (uint64_t)wgrid.x * wgrid.y >= ei::compute_units(e) &&
                              (uint64_t)t.g[0].N * k * 2 < lim && (uint64_t)m * k * 2 < lim;
            const dim3 grid = wide ? wgrid : dim3((uint32_t)cdiv64(t.g[0].N, awo::kTileN), (uint32_t)cdiv64(m, awo::kTileM));
            if (grid.y > 65535u) return ei::fail(e, AW_E_UNSUPPORTED, "%s: m = %u rows exceed the grid", what, m);
            if constexpr (EPI != awo::Epi::SiluGate) {
                if (wide && k % awo::kWideK != 0)
                    hipLaunchKernelGGL((awo::gemm_wide_kernel<true, F32, EPI>), grid, dim3(awo::kWideThreads), awo::kWideLdsBytes, st, t);
                else if (wide)
                    hipLaunchKernelGGL((awo::gemm_wide_kernel<false, F32, EPI>), grid, dim3(awo::kWideThreads), awo::kWideLdsBytes, st, t);
                else if (vec)
                    hipLaunchKernelGGL((awo::gemm_tiled_kernel<true, F32, EPI>), grid, dim3(256), 0, st, t);
                else
                    hipLaunchKernelGGL((awo::gemm_tiled_kernel<false, F32, EPI>), grid, dim3(256), 0, st, t);
            }
        }
        OPS_HIP(e, hipGetLastError());
        return AW_OK;
    }
    if (tiles > 0x7FFFFFFFull) return ei::fail(e, AW_E_UNSUPPORTED, "%s: grid too large", what);
    const dim3 grid((uint32_t)tiles);
    // Few weight tiles (up to 4 work-groups per CU): 16 waves per tile, so a K of
    // 4096 is in flight at once; many tiles: 8 waves, more work-groups resident
    // (measured at M = 1: 4096 x 4096 10.8 -> 9.6 us, 14336 x 4096 33.1 -> 28.6 us
    // with 16 waves; 128256 x 4096 183 us with 8 waves, 214 with 16).  The wave
    // count does not change the sums.
    const bool wide = tiles <= 4ull * ei::compute_units(e);
#define AW_SKINNY(MT, NW)                                                                                        \
    do {                                                                                                         \
        if (vec)                                                                                                 \
            hipLaunchKernelGGL((awo::gemm_skinny_kernel<MT, NW, true, F32, EPI>), grid, dim3(NW * 64), 0, st, g);  \
        else                                                                                                     \
            hipLaunchKernelGGL((awo::gemm_skinny_kernel<MT, NW, false, F32, EPI>), grid, dim3(NW * 64), 0, st, g); \
    } while (0)
    if (m <= 16 && wide)
        AW_SKINNY(1, 16);
    else if (m <= 16)
        AW_SKINNY(1, 8);
    else if (m <= 32 && wide)
        AW_SKINNY(2, 16);
    else if (m <= 32)
        AW_SKINNY(2, 8);
    else
        AW_SKINNY(4, 8);
#undef AW_SKINNY
    OPS_HIP(e, hipGetLastError());
    return AW_OK;
}

} // namespace

namespace aw_engine_internal {

bool ops_set_lds_limits(size_t max_lds) {
    // <MASK, F32, EPI> of the products that take the wide tiles.
    const void* fns[] = {(const void*)awo::gemm_wide_kernel<true, false, awo::Epi::Store>,
                         (const void*)awo::gemm_wide_kernel<false, false, awo::Epi::Store>,
                         (const void*)awo::gemm_wide_kernel<true, true, awo::Epi::Store>,
                         (const void*)awo::gemm_wide_kernel<false, true, awo::Epi::Store>,
                         (const void*)awo::gemm_wide_kernel<true, false, awo::Epi::Residual>,
                         (const void*)awo::gemm_wide_kernel<false, false, awo::Epi::Residual>};
    bool ok = true;
    for (const void* f : fns)
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds) != hipSuccess) {
            ok = false;
            (void)hipGetLastError();
        }
    return ok && max_lds >= awo::kWideLdsBytes;
}

} // namespace aw_engine_internal

extern "C" {

int aw_ops_copy_buffer(aw_engine* e, const uint16_t* src, uint16_t* dst, uint32_t count, uint32_t src_off,
                       uint32_t dst_off, void* stream) {
    int rc = enter(e);
    if (rc || count == 0) return rc;
    if (!src || !dst) return ei::fail(e, AW_E_INVALID_ARG, "copy_buffer: null pointer");
    awo::EwArgs p{};
    p.a = src + src_off;
    p.out = dst + dst_off;
    p.n = count;
    return launch_ew<awo::Ew::Copy>(e, p, aligned(p.a, 16) && aligned(p.out, 16), (hipStream_t)stream);
}

int aw_ops_embed_lookup(aw_engine* e, const uint32_t* token_ids, const uint16_t* table, uint16_t* out,
                        uint32_t hidden_size, uint32_t seq_len, uint32_t vocab_size, void* stream) {
    int rc = enter(e);
    if (rc || hidden_size == 0 || seq_len == 0) return rc;
    if (!token_ids || !table || !out) return ei::fail(e, AW_E_INVALID_ARG, "embed_lookup: null pointer");
    if (vocab_size == 0) return ei::fail(e, AW_E_INVALID_ARG, "embed_lookup: vocab_size is 0");
    const bool vec = hidden_size % 8 == 0 && aligned(table, 16) && aligned(out, 16);
    const uint32_t cw = (uint32_t)cdiv64(vec ? hidden_size / 8 : hidden_size, 256);
    const uint64_t blocks = (uint64_t)cw * seq_len;
    if (blocks > 0x7FFFFFFFull) return ei::fail(e, AW_E_UNSUPPORTED, "embed_lookup: grid too large");
    hipStream_t st = (hipStream_t)stream;
    if (vec)
        hipLaunchKernelGGL(awo::embed_kernel<true>, dim3((uint32_t)blocks), dim3(256), 0, st, token_ids, table, out,
                           hidden_size, cw, vocab_size, ei::error_word(e));
    else
        hipLaunchKernelGGL(awo::embed_kernel<false>, dim3((uint32_t)blocks), dim3(256), 0, st, token_ids, table, out,
                           hidden_size, cw, vocab_size, ei::error_word(e));
    OPS_HIP(e, hipGetLastError());
    return AW_OK;
}

int aw_ops_rms_norm(aw_engine* e, const uint16_t* input, const uint16_t* weight, uint16_t* output,
                    uint32_t hidden_size, uint32_t num_tokens, float eps, void* stream) {
    int rc = enter(e);
    if (rc || hidden_size == 0 || num_tokens == 0) return rc;
    if (!input || !weight || !output) return ei::fail(e, AW_E_INVALID_ARG, "rms_norm: null pointer");
    if (num_tokens > 0x7FFFFFFFu) return ei::fail(e, AW_E_UNSUPPORTED, "rms_norm: too many tokens");
    const bool vec = hidden_size % 8 == 0 && aligned(input, 16) && aligned(weight, 16) && aligned(output, 16);
    hipStream_t st = (hipStream_t)stream;
    if (vec)
        hipLaunchKernelGGL(awo::rms_norm_kernel<true>, dim3(num_tokens), dim3(256), 0, st, input, weight, output,
                           hidden_size, eps);
    else
        hipLaunchKernelGGL(awo::rms_norm_kernel<false>, dim3(num_tokens), dim3(256), 0, st, input, weight, output,
                           hidden_size, eps);
    OPS_HIP(e, hipGetLastError());
    return AW_OK;
}

int aw_ops_rope(aw_engine* e, uint16_t* q, uint16_t* k, uint32_t num_tokens, uint32_t q_heads, uint32_t kv_heads,
                uint32_t head_dim, uint32_t start_position, float theta, void* stream) {
    int rc = enter(e);
    if (rc || num_tokens == 0 || q_heads + kv_heads == 0) return rc;
    if (head_dim == 0 || head_dim % 2) return ei::fail(e, AW_E_INVALID_ARG, "rope: head_dim %u must be even", head_dim);
    if ((q_heads && !q) || (kv_heads && !k)) return ei::fail(e, AW_E_INVALID_ARG, "rope: null pointer");
    if (!(theta > 0.0f)) return ei::fail(e, AW_E_INVALID_ARG, "rope: theta must be positive");
    const uint64_t threads = (uint64_t)num_tokens * ((uint64_t)q_heads + kv_heads) * (head_dim / 2);
    if (cdiv64(threads, 256) > 0x7FFFFFFFull) return ei::fail(e, AW_E_UNSUPPORTED, "rope: grid too large");
    hipLaunchKernelGGL(awo::rope_kernel, dim3((uint32_t)cdiv64(threads, 256)), dim3(256), 0, (hipStream_t)stream, q, k,
                       num_tokens, q_heads, kv_heads, head_dim, start_position, theta);
    OPS_HIP(e, hipGetLastError());
    return AW_OK;
}

int aw_ops_matmul(aw_engine* e, const uint16_t* a, const uint16_t* b, uint16_t* output, uint32_t m, uint32_t n,
                  uint32_t k, void* stream) {
    int rc = enter(e);
    if (rc) return rc;
    const Product p{b, nullptr, output, n};
    return launch_products<awo::Epi::Store, false>(e, "matmul", a, &p, 1, m, k, 1.0f, (hipStream_t)stream);
}

int aw_ops_matmul_scaled(aw_engine* e, const uint16_t* a, const uint16_t* b, float* output, uint32_t m, uint32_t n,
                         uint32_t k, float scale, void* stream) {
    int rc = enter(e);
    if (rc) return rc;
    const Product p{b, nullptr, output, n};
    return launch_products<awo::Epi::Store, true>(e, "matmul_scaled", a, &p, 1, m, k, scale, (hipStream_t)stream);
}

int aw_ops_matmul_add_residual(aw_engine* e, const uint16_t* a, const uint16_t* b, uint16_t* x, uint32_t m,
                               uint32_t n, uint32_t k, float residual_multiplier, void* stream) {
    int rc = enter(e);
    if (rc) return rc;
    const Product p{b, nullptr, x, n};
    return launch_products<awo::Epi::Residual, false>(e, "matmul_add_residual", a, &p, 1, m, k, residual_multiplier,
                                                      (hipStream_t)stream);
}

int aw_ops_matmul_silu_gate(aw_engine* e, const uint16_t* a, const uint16_t* b_gate, const uint16_t* b_up,
                            uint16_t* output, uint32_t m, uint32_t n, uint32_t k, void* stream) {
    int rc = enter(e);
    if (rc) return rc;
    const Product p{b_gate, b_up, output, n};
    return launch_products<awo::Epi::SiluGate, false>(e, "matmul_silu_gate", a, &p, 1, m, k, 1.0f,
                                                      (hipStream_t)stream);
}

int aw_ops_matmul_qkv(aw_engine* e, const uint16_t* a, const uint16_t* b_q, const uint16_t* b_k, const uint16_t* b_v,
                      uint16_t* q, uint16_t* k_out, uint16_t* v_out, uint32_t m, uint32_t n_q, uint32_t n_kv,
                      uint32_t k, void* stream) {
    int rc = enter(e);
    if (rc) return rc;
    const Product p[3] = {{b_q, nullptr, q, n_q}, {b_k, nullptr, k_out, n_kv}, {b_v, nullptr, v_out, n_kv}};
    return launch_products<awo::Epi::Store, false>(e, "matmul_qkv", a, p, 3, m, k, 1.0f, (hipStream_t)stream);
}

int aw_ops_silu_gate(aw_engine* e, const uint16_t* gate, const uint16_t* up, uint16_t* output, uint32_t size,
                     void* stream) {
    int rc = enter(e);
    if (rc || size == 0) return rc;
    if (!gate || !up || !output) return ei::fail(e, AW_E_INVALID_ARG, "silu_gate: null pointer");
    awo::EwArgs p{};
    p.a = gate;
    p.b = up;
    p.out = output;
    p.n = size;
    const bool vec = aligned(gate, 16) && aligned(up, 16) && aligned(output, 16);
    return launch_ew<awo::Ew::Silu>(e, p, vec, (hipStream_t)stream);
}

int aw_ops_add_residual(aw_engine* e, uint16_t* x, const uint16_t* residual, uint32_t size, void* stream) {
    int rc = enter(e);
    if (rc || size == 0) return rc;
    if (!x || !residual) return ei::fail(e, AW_E_INVALID_ARG, "add_residual: null pointer");
    awo::EwArgs p{};
    p.a = x;
    p.b = residual;
    p.out = x;
    p.n = size;
    return launch_ew<awo::Ew::Add>(e, p, aligned(x, 16) && aligned(residual, 16), (hipStream_t)stream);
}

int aw_ops_add_bias(aw_engine* e, uint16_t* x, const uint16_t* bias, uint32_t hidden_size, uint32_t num_tokens,
                    void* stream) {
    int rc = enter(e);
    if (rc || hidden_size == 0 || num_tokens == 0) return rc;
    if (!x || !bias) return ei::fail(e, AW_E_INVALID_ARG, "add_bias: null pointer");
    awo::EwArgs p{};
    p.a = x;
    p.b = bias;
    p.out = x;
    p.n = (uint64_t)hidden_size * num_tokens;
    p.period = hidden_size;
    const bool vec = hidden_size % 8 == 0 && aligned(x, 16) && aligned(bias, 16);
    return launch_ew<awo::Ew::Bias>(e, p, vec, (hipStream_t)stream);
}

int aw_ops_scale_f16(aw_engine* e, uint16_t* x, uint32_t count, float scale, void* stream) {
    int rc = enter(e);
    if (rc || count == 0) return rc;
    if (!x) return ei::fail(e, AW_E_INVALID_ARG, "scale_f16: null pointer");
    awo::EwArgs p{};
    p.a = x;
    p.out = x;
    p.n = count;
    p.s = scale;
    return launch_ew<awo::Ew::Scale>(e, p, aligned(x, 16), (hipStream_t)stream);
}

int aw_ops_causal_attention(aw_engine* e, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* output,
                            uint32_t kv_len, uint32_t head_dim, uint64_t cache_tokens, void* stream) {
    if (!e) return AW_E_INVALID_ARG;
    return aw_multihead_attention_device(e, q, k, v, output, kv_len, head_dim, 1, 1, 1, cache_tokens, stream);
}

} // extern "C"
