// ops_kernels.hpp — gfx950 kernels of the dense transformer ops
// (nexus-core/src/ops.metal:16-635, dispatched by nexus-core/src/ops.rs:166-462).
//
// f16 tensors are passed as uint16_t bit patterns and converted with the
// hardware's round-to-nearest-even; arithmetic is fp32 as in the reference.
// FMA contraction is off in this file so that every fp32 expression rounds
// per operation, the way the reference writes it (the CPU oracle evaluates the
// same expressions in numpy float32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "engine_internal.hpp"

#pragma clang fp contract(off)

namespace awo {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

// Error bit of an out-of-range token id (embed_lookup) in the engine's device error word.
constexpr uint32_t kErrToken = aw_engine_internal::kErrTokenBit;

__device__ inline float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// f16 of an fp32 value, rounded twice as the reference's half(float expression)
// is: the expression to fp32, then to f16.  The empty asm makes x an fp32 value
// in a register, so the compiler cannot fuse the multiply or add that produced
// it into a mixed-precision instruction (v_fma_mixlo_f16) that rounds the exact
// result once, straight to f16 (measured: 1-ulp differences in ~1 of 20000
// SiLU outputs, between kernels that fused and kernels that did not).
__device__ inline uint16_t f2h(float x) {
    __asm__ volatile("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ inline void flag(uint32_t* err, uint32_t bit) {
    __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------- elementwise ops
//
// copy_buffer (ops.metal:16-26), silu_gate (:325-338), add_residual (:345-353),
// add_bias (:360-371), scale_f16 (:627-635).  One kernel, HBM-bound: 16-byte
// loads and stores of 8 halves (VEC: every pointer 16-byte aligned), grid-
// strided over the n elements, the n % 8 tail element by element.
enum class Ew : int { Copy = 0, Silu = 1, Add = 2, Bias = 3, Scale = 4 };

template <Ew OP>
__device__ inline uint16_t ew_one(uint16_t a, uint16_t b, float s) {
    if constexpr (OP == Ew::Copy) {
        return a;
    } else if constexpr (OP == Ew::Silu) {
        // ops.metal:334-337: g / (1 + exp(-g)) * u
        const float g = h2f(a), u = h2f(b);
        const float silu = g / (1.0f + expf(-g));
        return f2h(silu * u);
    } else if constexpr (OP == Ew::Add || OP == Ew::Bias) {
        return f2h(h2f(a) + h2f(b)); // ops.metal:352, :370
    } else {
        return f2h(h2f(a) * s); // ops.metal:634
    }
}

struct EwArgs {
    const uint16_t* a; // copy: src; silu: gate; add / bias / scale: x
    const uint16_t* b; // silu: up; add: residual; bias: bias [period]
    uint16_t* out;     // copy: dst; silu: output; add / bias / scale: x (in place)
    uint64_t n;        // elements
    uint32_t period;   // bias: hidden_size (b index = i % period)
    float s;           // scale
};

template <Ew OP, bool VEC>
__global__ __launch_bounds__(256) void ew_kernel(EwArgs p) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    constexpr bool TWO = OP == Ew::Silu || OP == Ew::Add || OP == Ew::Bias;
    if constexpr (VEC) {
        const uint64_t n8 = p.n / 8;
        for (uint64_t i = t; i < n8; i += stride) {
            const uint4_t va = ((const uint4_t*)p.a)[i];
            uint4_t vb = (uint4_t)0u;
            if constexpr (OP == Ew::Bias) vb = *(const uint4_t*)(p.b + (i * 8) % p.period); // period % 8 == 0
            else if constexpr (TWO) vb = ((const uint4_t*)p.b)[i];
            uint4_t r;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t lo = ew_one<OP>((uint16_t)(va[w] & 0xFFFFu), (uint16_t)(vb[w] & 0xFFFFu), p.s);
                const uint32_t hi = ew_one<OP>((uint16_t)(va[w] >> 16), (uint16_t)(vb[w] >> 16), p.s);
                r[w] = lo | (hi << 16);
            }
            ((uint4_t*)p.out)[i] = r;
        }
        const uint64_t i = n8 * 8 + t; // tail: fewer than 8 elements
        if (i < p.n) {
            const uint16_t b = OP == Ew::Bias ? p.b[i % p.period] : (TWO ? p.b[i] : (uint16_t)0);
            p.out[i] = ew_one<OP>(p.a[i], b, p.s);
        }
    } else {
        for (uint64_t i = t; i < p.n; i += stride) {
            const uint16_t b = OP == Ew::Bias ? p.b[i % p.period] : (TWO ? p.b[i] : (uint16_t)0);
            p.out[i] = ew_one<OP>(p.a[i], b, p.s);
        }
    }
}

// ------------------------------------------------------- embedding lookup
//
// ops.metal:33-49: output[t][d] = table[ids[t]][d].  `cw` work-groups per
// token row, 8 halves per thread (VEC).  An id >= vocab_size (which the
// reference would read past its table) writes a zero row and sets kErrToken.
template <bool VEC>
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* ids, const uint16_t* table, uint16_t* out,
                                                    uint32_t H, uint32_t cw, uint32_t vocab, uint32_t* err) {
    const uint32_t t = blockIdx.x / cw, chunk = blockIdx.x % cw;
    const uint32_t id = ids[t];
    const bool ok = id < vocab;
    if (!ok && chunk == 0 && threadIdx.x == 0) flag(err, kErrToken);
    const uint16_t* src = table + (uint64_t)(ok ? id : 0u) * H;
    uint16_t* dst = out + (uint64_t)t * H;
    const uint32_t c = chunk * blockDim.x + threadIdx.x;
    if constexpr (VEC) {
        if (c < H / 8) ((uint4_t*)dst)[c] = ok ? ((const uint4_t*)src)[c] : (uint4_t)0u;
    } else {
        if (c < H) dst[c] = ok ? src[c] : (uint16_t)0;
    }
}

// ------------------------------------------------------- RMSNorm
//
// ops.metal:59-99: out = f16(x * rsqrt(mean(x^2) + eps) * w), one work-group
// (256 threads) per token.  Sum of squares in fp32: lane partials over strided
// elements, a wave butterfly, then the four waves' sums in order.
template <bool VEC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* in, const uint16_t* w, uint16_t* out,
                                                       uint32_t H, float eps) {
    __shared__ float s_sum[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint16_t* x = in + (uint64_t)t * H;
    uint16_t* y = out + (uint64_t)t * H;
    float acc = 0.0f;
    if constexpr (VEC) {
        for (uint32_t c = tid; c < H / 8; c += 256) {
            const uint4_t v = ((const uint4_t*)x)[c];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = h2f((uint16_t)(v[e / 2] >> (16 * (e % 2))));
                acc += f * f;
            }
        }
    } else {
        // The VEC path's assignment and order (8 consecutive elements per thread
        // and chunk), so an aligned and an unaligned row give the same bits.
        for (uint32_t c = tid; c < (H + 7) / 8; c += 256) {
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e) {
                const uint32_t i = 8 * c + e;
                const float f = i < H ? h2f(x[i]) : 0.0f;
                acc += f * f;
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if ((tid & 63u) == 0) s_sum[tid >> 6] = acc;
    __syncthreads();
    const float sum = ((s_sum[0] + s_sum[1]) + s_sum[2]) + s_sum[3];
    const float inv = 1.0f / sqrtf(sum / (float)H + eps); // ops.metal:93
    if constexpr (VEC) {
        for (uint32_t c = tid; c < H / 8; c += 256) {
            const uint4_t v = ((const uint4_t*)x)[c], g = ((const uint4_t*)w)[c];
            uint4_t r;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float x0 = h2f((uint16_t)(v[k] & 0xFFFFu)), x1 = h2f((uint16_t)(v[k] >> 16));
                const float g0 = h2f((uint16_t)(g[k] & 0xFFFFu)), g1 = h2f((uint16_t)(g[k] >> 16));
                r[k] = (uint32_t)f2h(x0 * inv * g0) | ((uint32_t)f2h(x1 * inv * g1) << 16);
            }
            ((uint4_t*)y)[c] = r;
        }
    } else {
        for (uint32_t i = tid; i < H; i += 256) y[i] = f2h(h2f(x[i]) * inv * h2f(w[i]));
    }
}

// ------------------------------------------------------- RoPE
//
// ops.metal:107-155, in place on q [T][Hq][hd] and k [T][Hkv][hd]: the pair
// (x[p], x[p + hd/2]) of each head rotates by angle = f32(start + t) * freq_p,
// freq_p = 1 / theta^(2p/hd).  freq_p is the double-precision value rounded
// to fp32; cos and sin of the fp32 angle are taken in double and rounded to
// fp32; the rotation itself is fp32, one rounding per operation.  Thread =
// (pair, head row, token); head rows 0 .. Hq-1 are q, Hq .. Hq+Hkv-1 are k.
__global__ __launch_bounds__(256) void rope_kernel(uint16_t* q, uint16_t* k, uint32_t T, uint32_t Hq, uint32_t Hkv,
                                                   uint32_t hd, uint32_t start, float theta) {
    const uint32_t half_dim = hd / 2;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t per_tok = (uint64_t)(Hq + Hkv) * half_dim;
    if (i >= per_tok * T) return;
    const uint32_t t = (uint32_t)(i / per_tok), rem = (uint32_t)(i % per_tok);
    const uint32_t head = rem / half_dim, pr = rem % half_dim;
    const float freq = (float)(1.0 / pow((double)theta, (double)(2 * pr) / (double)hd));
    const float angle = (float)(start + t) * freq;
    const float c = (float)cos((double)angle), s = (float)sin((double)angle);
    uint16_t* base = head < Hq ? q + ((uint64_t)t * Hq + head) * hd : k + ((uint64_t)t * Hkv + (head - Hq)) * hd;
    const float x0 = h2f(base[pr]), x1 = h2f(base[pr + half_dim]);
    base[pr] = f2h(x0 * c - x1 * s);
    base[pr + half_dim] = f2h(x0 * s + x1 * c);
}

// ------------------------------------------------------- C = A . B^T
//
// matmul_f16 / vecmat_f16 (ops.metal:170-271) and matmul_scaled /
// vecmat_scaled (:279-422): A [M][K] activations, B [N][K] weights, both
// K-contiguous; C [M][N] f16, or f32 times `scale`.  Both products run on
// v_mfma_f32_16x16x32_f16 with the weights as the A operand (16 rows of B x
// 32 k) and the activations as the B operand (16 rows of A x 32 k), so a lane
// ends with 4 consecutive output columns of one row: C[m][n .. n+3].
//
// VEC: K % 8 == 0 and 16-byte aligned rows, every operand piece one 16-byte
// load; otherwise pieces are gathered element by element (same sums).
// Out-of-range rows are clamped for loading and masked at the store; k past K
// reads zeros.

__device__ inline float4_t mfma(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 8 halves of row `row` (already clamped) at k .. k+7; zeros past K.
template <bool VEC>
__device__ inline half8_t piece(const uint16_t* base, uint64_t row, uint32_t K, uint32_t k) {
    if constexpr (VEC) {
        const uint4_t v = k < K ? *(const uint4_t*)(base + row * K + k) : (uint4_t)0u;
        return __builtin_bit_cast(half8_t, v);
    } else {
        half8_t h;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            h[e] = k + e < K ? __builtin_bit_cast(_Float16, base[row * K + k + e]) : (_Float16)0.0f;
        return h;
    }
}

// What a product does with its fp32 result at the store:
//   Store     C = f16(acc), or acc * scale in fp32 (F32);
//   Residual  C (the residual stream x) = f16(x + f16(f16(acc) * scale)): matmul,
//             scale_f16 by the residual multiplier, add_residual (ops.rs:266-296,
//             :350-363, :315-327), the same bits in one pass;
//   SiluGate  C = f16(silu(f16(acc)) * f16(acc2)) with acc2 the product with a second
//             weight matrix: the gate and up matmuls then silu_gate (ops.rs:266-312).
enum class Epi : int { Store = 0, Residual = 1, SiluGate = 2 };

template <Epi EPI, bool F32>
__device__ inline void epi_store(void* C, uint64_t at, float v, float v2, float scale) {
    if constexpr (EPI == Epi::Store) {
        if constexpr (F32) ((float*)C)[at] = v * scale;
        else ((uint16_t*)C)[at] = f2h(v);
    } else if constexpr (EPI == Epi::Residual) {
        uint16_t* x = (uint16_t*)C;
        x[at] = ew_one<Ew::Add>(x[at], ew_one<Ew::Scale>(f2h(v), 0, scale), 0.0f);
    } else {
        ((uint16_t*)C)[at] = ew_one<Ew::Silu>(f2h(v), f2h(v2), 0.0f);
    }
}

// Four results C[m][n .. n+3] of one lane, masked to M x N; `vec_out` (N % 4 == 0,
// C aligned) stores them with one 16- or 8-byte store.
template <Epi EPI, bool F32>
__device__ inline void store4(void* C, uint32_t M, uint32_t N, uint32_t m, uint32_t n, float4_t v, float4_t v2,
                              float scale, bool vec_out) {
    if (m >= M || n >= N) return;
    const uint64_t at = (uint64_t)m * N + n;
    if constexpr (EPI == Epi::Store && F32) {
        if (vec_out && n + 4 <= N) {
            *(float4_t*)((float*)C + at) = v * scale;
            return;
        }
    } else if constexpr (EPI != Epi::Residual) {
        if (vec_out && n + 4 <= N) {
            uint16_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                h[e] = EPI == Epi::Store ? f2h(v[e]) : ew_one<Ew::Silu>(f2h(v[e]), f2h(v2[e]), 0.0f);
            *(uint2_t*)((uint16_t*)C + at) = (uint2_t){(uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                                       (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
            return;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (n + e < N) epi_store<EPI, F32>(C, at + e, v[e], v2[e], scale);
}

// One weight matrix of a product (up to three share the activations A: the q, k
// and v projections in one launch).
struct GemmGroup {
    const uint16_t* B;  // [N][K]
    const uint16_t* B2; // SiluGate: the up weights [N][K]
    void* C;            // [M][N]
    uint32_t N;
    uint32_t tiles;     // skinny: 16-row weight tiles of this group
    bool vec_out;       // N % 4 == 0 and C aligned for 4-element stores
};

struct GemmArgs {
    const uint16_t* A; // [M][K]
    GemmGroup g[3];
    uint32_t groups;
    uint32_t M, K;
    float scale; // f32 output only
};

// Skinny products (M <= 16 * MT: decode and verify steps).  A work-group of
// NW waves owns 16 weight rows; K is cut into 64-wide chunks (a 128-byte line
// per weight row), chunk c summed into partial slot c % 16, and wave w owns the
// slots w, w + NW, ...: each wave streams its rows in whole lines, U chunks in
// flight, and the weights are read once for all MT tiles of 16 activation
// rows.  The slots are added as sum over j < 8 of (slot j + slot j + 8), in
// that order, whatever NW (8: a wave holds both slots of a pair; 16: the pair
// meets in LDS), so the bits depend on neither NW nor the grouping of the
// products.  Bound: HBM, N*K*2 bytes of weights.
constexpr int kSkinnyU = 4;
constexpr int kSkinnySlots = 16;

template <int MT, int NW, bool VEC, bool F32, Epi EPI>
__global__ __launch_bounds__(NW * 64) void gemm_skinny_kernel(GemmArgs a) {
    constexpr bool DUAL = EPI == Epi::SiluGate;
    constexpr int NA = DUAL ? 2 : 1;                 // accumulated products
    constexpr int SPW = kSkinnySlots / NW;           // slots per wave
    static_assert(kSkinnyU % SPW == 0, "chunk u of a batch lands in slot u % SPW");
    __shared__ float4_t s_pair[NA][kSkinnySlots / 2][MT][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    // This work-group's group and tile (uniform selects, no dynamic indexing).
    uint32_t tile = blockIdx.x;
    const bool in0 = tile < a.g[0].tiles;
    if (!in0) tile -= a.g[0].tiles;
    const bool in1 = !in0 && (a.groups < 3 || tile < a.g[1].tiles);
    if (!in0 && !in1) tile -= a.g[1].tiles;
    const GemmGroup& G = in0 ? a.g[0] : (in1 ? a.g[1] : a.g[2]);
    const uint16_t* B = G.B;
    const uint16_t* B2 = G.B2;
    const uint32_t N = G.N;
    const uint32_t n0 = tile * 16u;
    const uint64_t wrow = min(n0 + (uint32_t)li, N - 1u); // this lane's weight row (clamped)
    uint64_t arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) arow[mt] = min((uint32_t)(mt * 16 + li), a.M - 1u);
    float4_t acc[NA][SPW][MT];
#pragma unroll
    for (int x = 0; x < NA; ++x)
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[x][j][mt] = (float4_t)0.0f;
    const uint32_t n_chunks = (a.K + 63u) / 64u;
    for (uint32_t c0 = (uint32_t)wave; c0 < n_chunks; c0 += (uint32_t)(NW * kSkinnyU)) {
        half8_t wv[NA][kSkinnyU][2];
#pragma unroll
        for (int u = 0; u < kSkinnyU; ++u) {
            const uint32_t k = (c0 + (uint32_t)(u * NW)) * 64u + 8u * (uint32_t)lg;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                wv[0][u][h] = piece<VEC>(B, wrow, a.K, k + 32u * h);
                if constexpr (DUAL) wv[NA - 1][u][h] = piece<VEC>(B2, wrow, a.K, k + 32u * h);
            }
        }
#pragma unroll
        for (int u = 0; u < kSkinnyU; ++u) {
            const uint32_t k = (c0 + (uint32_t)(u * NW)) * 64u + 8u * (uint32_t)lg;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const half8_t xo = piece<VEC>(a.A, arow[mt], a.K, k + 32u * h);
#pragma unroll
                    for (int x = 0; x < NA; ++x) acc[x][u % SPW][mt] = mfma(wv[x][u][h], xo, acc[x][u % SPW][mt]);
                }
        }
    }
    // Pairs (slot j, slot j + 8) for j < 8 into LDS.
    if constexpr (SPW == 2) {
#pragma unroll
        for (int x = 0; x < NA; ++x)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) s_pair[x][wave][mt][lane] = acc[x][0][mt] + acc[x][1][mt];
    } else {
        if (wave >= kSkinnySlots / 2)
#pragma unroll
            for (int x = 0; x < NA; ++x)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) s_pair[x][wave - kSkinnySlots / 2][mt][lane] = acc[x][0][mt];
        __syncthreads();
        if (wave < kSkinnySlots / 2)
#pragma unroll
            for (int x = 0; x < NA; ++x)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    s_pair[x][wave][mt][lane] = acc[x][0][mt] + s_pair[x][wave][mt][lane];
    }
    __syncthreads();
    // Wave mt' < MT finishes tile mt': the 8 pairs in order.
    if (wave < MT) {
        float4_t r[NA];
#pragma unroll
        for (int x = 0; x < NA; ++x) {
            r[x] = s_pair[x][0][wave][lane];
#pragma unroll
            for (int j = 1; j < kSkinnySlots / 2; ++j) r[x] += s_pair[x][j][wave][lane];
        }
        store4<EPI, F32>(G.C, a.M, N, (uint32_t)(wave * 16 + li), n0 + 4u * (uint32_t)lg, r[0], r[NA - 1], a.scale,
                         G.vec_out);
    }
}

// General products (prefill-sized M): 128 x 128 output tiles, 4 waves of 64 x 64
// (4 x 4 MFMA tiles each), k-steps of 32 staged in LDS with the next step's
// loads in registers while the current step is multiplied.  One weight matrix
// (group 0).  Bound: the matrix cores for large M, N, K.
constexpr int kTileM = 128, kTileN = 128, kTileK = 32, kTilePitch = kTileK + 8; // halves per staged row

template <bool VEC, bool F32, Epi EPI>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(GemmArgs a) {
    static_assert(EPI != Epi::SiluGate, "one weight matrix");
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][kTileN * kTilePitch]; // weights
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][kTileM * kTilePitch]; // activations
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const int wn = wave & 1, wm = wave >> 1;
    const uint32_t n0 = blockIdx.x * kTileN, m0 = blockIdx.y * kTileM;
    const uint16_t* B = a.g[0].B;
    const uint32_t N = a.g[0].N;
    // Staging: 512 pieces of 8 halves per operand tile, two per thread: piece p =
    // (row p / 4, k 8 * (p % 4)).
    auto load = [&](uint32_t k0, half8_t (&pb)[2], half8_t (&pa)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int p = tid + 256 * j;
            const uint32_t r = (uint32_t)(p >> 2), k = k0 + 8u * (uint32_t)(p & 3);
            pb[j] = piece<VEC>(B, min(n0 + r, N - 1u), a.K, k);
            pa[j] = piece<VEC>(a.A, min(m0 + r, a.M - 1u), a.K, k);
        }
    };
    auto stage = [&](int buf, const half8_t (&pb)[2], const half8_t (&pa)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int p = tid + 256 * j;
            *(half8_t*)(&sB[buf][(p >> 2) * kTilePitch + 8 * (p & 3)]) = pb[j];
            *(half8_t*)(&sA[buf][(p >> 2) * kTilePitch + 8 * (p & 3)]) = pa[j];
        }
    };
    float4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (float4_t)0.0f;
    const uint32_t n_steps = (a.K + kTileK - 1) / kTileK;
    half8_t pb[2], pa[2];
    load(0, pb, pa);
    stage(0, pb, pa);
    __syncthreads();
    for (uint32_t s = 0; s < n_steps; ++s) {
        const int buf = (int)(s & 1u);
        const bool more = s + 1 < n_steps;
        if (more) load((s + 1) * kTileK, pb, pa);
        half8_t bo[4], ao[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) bo[i] = *(const half8_t*)(&sB[buf][(wn * 64 + i * 16 + li) * kTilePitch + 8 * lg]);
#pragma unroll
        for (int j = 0; j < 4; ++j) ao[j] = *(const half8_t*)(&sA[buf][(wm * 64 + j * 16 + li) * kTilePitch + 8 * lg]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma(bo[i], ao[j], acc[i][j]);
        if (more) stage(buf ^ 1, pb, pa); // its last readers (step s - 1) passed the previous barrier
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            store4<EPI, F32>(a.g[0].C, a.M, N, m0 + (uint32_t)(wm * 64 + j * 16 + li),
                             n0 + (uint32_t)(wn * 64 + i * 16 + 4 * lg), acc[i][j], acc[i][j], a.scale,
                             a.g[0].vec_out);
}

// Large products (many 256 x 128 tiles): 256 weight rows x 128 activation rows
// per work-group of 8 waves, each 64 x 64 (4 x 4 MFMA tiles), two waves per
// SIMD (one wave per SIMD does not issue its MFMAs back to back).  The operands
// go from memory straight into LDS (buffer loads with the LDS flag), in LDS
// stages of 64 k: each row of a stage is 128 contiguous bytes, so a wave's load
// instruction (64 lanes x 16 bytes) covers 8 rows x 128 bytes.  Loads of 16
// rows x 64 bytes, the shape of 32-k stages, move about 40 GB/s per CU (also
// measured here); 128-byte runs move more.
//   - Stages rotate through three LDS buffers: stage s + 2's loads are issued
//     during stage s, into the buffer stage s - 1 used, and waited for (s_waitcnt
//     vmcnt, each wave its own) at the end of stage s + 1, before the barrier
//     that publishes them.
//   - A stage's fragments are read at its start; the other wave of the SIMD
//     covers their latency.
// Staged rows are 128 bytes (eight 16-byte chunks) with chunk c of row r stored
// at c ^ (r & 7): the 8 lanes that one 128-byte LDS cycle serves, rows r .. r + 7
// at one chunk, hit 8 distinct 16-byte slots; a load instruction writes 64
// consecutive slots, so each lane fetches the chunk its slot holds.  The 32-k
// MFMA steps are summed in the same order as gemm_tiled_kernel, so both give the
// same bits.
constexpr int kWideN = 256, kWideM = 128, kWideBufs = 3, kWideThreads = 512, kWideK = 64;

__device__ inline uint32_t wide_slot(uint32_t row, uint32_t chunk) { // halves
    return row * 64u + ((chunk ^ (row & 7u)) << 3);
}

// gfx9 buffer resource word 3 (32-bit data format) of the wide kernel's operand loads.
constexpr uint32_t kWideRsrcWord3 = 0x00020000u;
// A buffer offset past any operand (at most 4 GiB - 64 KiB): the load returns zeros.
constexpr uint32_t kWideOutOfRange = 0xFFFFFFF0u;

// The wide kernel's work-group barrier: s_barrier alone, with compiler barriers
// on both sides so no memory access moves across it.  No hardware wait: the
// kernel writes LDS only through its loads, and waits for each wave's own with
// s_waitcnt vmcnt (as many as it needs) before the barrier that publishes them;
// a fence here would wait for every load in flight (vmcnt(0)), also those
// issued for later stages.  LDS reads complete in order, before their registers
// are used, before the barrier after which another load may overwrite them.
__device__ inline void lds_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// MASK: K % 64 != 0, so the last stage's chunks past K load zeros.  Operands:
// 16-byte aligned rows with K % 8 == 0, each below 4 GiB - 64 KiB (buffer loads
// with 32-bit offsets, range-checked).
template <bool MASK, bool F32, Epi EPI>
__global__ __launch_bounds__(kWideThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_wide_kernel(GemmArgs a) {
    static_assert(EPI != Epi::SiluGate, "one weight matrix");
    constexpr uint32_t SB = kWideN * kWideK, SA = kWideM * kWideK; // halves per buffer: weights, activations
    constexpr int LPT = (kWideN + kWideM) * (kWideK / 8) / kWideThreads; // loads per thread and stage: 4 + 2
    extern __shared__ __attribute__((aligned(16))) _Float16 wide_lds[]; // [kWideBufs][SB + SA]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const int wn = wave & 3, wm = wave >> 2; // 4 x 64 weight rows, 2 x 64 activation rows
    const uint32_t n0 = blockIdx.x * kWideN, m0 = blockIdx.y * kWideM;
    const uint32_t N = a.g[0].N, K = a.K;
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)a.g[0].B, (short)0,
                                                                        (int)(uint32_t)((uint64_t)N * K * 2u),
                                                                        (int)kWideRsrcWord3);
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)a.A, (short)0,
                                                                        (int)(uint32_t)((uint64_t)a.M * K * 2u),
                                                                        (int)kWideRsrcWord3);
    // Load instruction j (0-3 weights, 4-5 activations) of this thread fills LDS
    // slot q = tid + 512 * (j % 4) of its region: row q >> 3, chunk (q & 7) ^
    // (row & 7).  off: that chunk's byte offset at k = 0 (rows clamped).
    uint32_t off[LPT];
    bool cin[LPT]; // MASK: the chunk holds k < K in the last stage
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
        const uint32_t q = (uint32_t)tid + (uint32_t)kWideThreads * (uint32_t)(j < 4 ? j : j - 4);
        const uint32_t row = q >> 3, chunk = (q & 7u) ^ (row & 7u);
        const uint32_t r = j < 4 ? min(n0 + row, N - 1u) : min(m0 + row, a.M - 1u);
        off[j] = (r * K + 8u * chunk) * 2u;
        cin[j] = true;
        if constexpr (MASK) cin[j] = 8u * chunk < K % (uint32_t)kWideK;
    }
    const uint32_t n_stages = (K + kWideK - 1u) / kWideK;
    const uint32_t last = n_stages - 1u;
    // Stage `st`'s operands into LDS buffer `buf` (LPT loads per thread, always:
    // the waits below count them).
    auto issue = [&](uint32_t st, uint32_t buf) {
        _Float16* base = wide_lds + buf * (SB + SA);
#pragma unroll
        for (int j = 0; j < LPT; ++j) {
            const uint32_t slot0 = (uint32_t)wave * 64u + (uint32_t)kWideThreads * (uint32_t)(j < 4 ? j : j - 4);
            _Float16* dst = base + (j < 4 ? 0u : SB) + slot0 * 8u; // wave-uniform
            uint32_t v = off[j] + st * (uint32_t)(kWideK * 2);
            if constexpr (MASK) v = (st < last || cin[j]) ? v : kWideOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(j < 4 ? rB : rA, (__attribute__((address_space(3))) void*)dst,
                                                     16, (int)v, 0, 0, 0);
        }
    };
    float4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (float4_t)0.0f;
    // One stage's products: two 32-k MFMA steps, each over the 4 activation and
    // 4 weight fragments of chunks 4 * ks + lg.
    auto products = [&](uint32_t buf) {
        const _Float16* sb = wide_lds + buf * (SB + SA);
#pragma unroll
        for (int ks = 0; ks < kWideK / 32; ++ks) {
            half8_t ao[4], bo[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ao[j] = *(const half8_t*)(sb + SB + wide_slot(wm * 64 + j * 16 + li, 4 * ks + lg));
#pragma unroll
            for (int i = 0; i < 4; ++i) bo[i] = *(const half8_t*)(sb + wide_slot(wn * 64 + i * 16 + li, 4 * ks + lg));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma(bo[i], ao[j], acc[i][j]);
        }
    };
    // Loads allowed still in flight at a stage's end: the next stage's LPT.
    // s_waitcnt immediate (gfx9): vmcnt in bits 3:0 and 15:14, no expcnt (6:4) or
    // lgkmcnt (11:8) wait.
    constexpr uint32_t kInFlight = (uint32_t)LPT;
    constexpr short kWaitLoads = (short)((kInFlight & 15u) | ((kInFlight >> 4) << 14) | 0x0F70u);
    if (K > 0) {
        issue(0, 0);
        issue(min(1u, last), 1);
        __builtin_amdgcn_s_waitcnt(kWaitLoads); // stage 0 is in LDS
        lds_barrier();
        // Stage s (buffer s % 3): stage s + 2's loads into buffer (s + 2) % 3, the
        // one stage s - 1 read before the previous barrier; the products; this
        // wave's stage s + 1 loads waited for; the barrier.  Loads past the last
        // stage re-read it (unconditional, so the wait counts stay exact; nothing
        // reads them).
        uint32_t b = 0;
        for (uint32_t s = 0; s < n_stages; ++s) {
            issue(min(s + 2u, last), b == 0u ? 2u : b - 1u);
            products(b);
            __builtin_amdgcn_s_waitcnt(kWaitLoads);
            lds_barrier();
            b = b == 2u ? 0u : b + 1u;
        }
        __builtin_amdgcn_s_waitcnt(0); // no load still writing LDS when the wave ends
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            store4<EPI, F32>(a.g[0].C, a.M, N, m0 + (uint32_t)(wm * 64 + j * 16 + li),
                             n0 + (uint32_t)(wn * 64 + i * 16 + 4 * lg), acc[i][j], acc[i][j], a.scale,
                             a.g[0].vec_out);
}

// Dynamic LDS of gemm_wide_kernel.
constexpr size_t kWideLdsBytes = (size_t)kWideBufs * (kWideN + kWideM) * kWideK * 2;

} // namespace awo
