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
__device__ inline uint16_t f2h(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
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
        for (uint32_t i = tid; i < H; i += 256) {
            const float f = h2f(x[i]);
            acc += f * f;
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

// Four results C[m][n .. n+3] of one lane, masked to M x N.
template <bool F32>
__device__ inline void store4(void* C, uint32_t M, uint32_t N, uint32_t m, uint32_t n, float4_t v, float scale,
                              bool vec_out) {
    if (m >= M || n >= N) return;
    if constexpr (F32) {
        float* c = (float*)C + (uint64_t)m * N + n;
        const float4_t r = v * scale;
        if (vec_out && n + 4 <= N) {
            *(float4_t*)c = r;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < N) c[e] = r[e];
        }
    } else {
        uint16_t* c = (uint16_t*)C + (uint64_t)m * N + n;
        if (vec_out && n + 4 <= N) {
            const uint2_t r = {(uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16),
                               (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16)};
            *(uint2_t*)c = r;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < N) c[e] = f2h(v[e]);
        }
    }
}

struct GemmArgs {
    const uint16_t* A; // [M][K]
    const uint16_t* B; // [N][K]
    void* C;           // [M][N]
    uint32_t M, N, K;
    float scale;       // f32 output only
    bool vec_out;      // N % 4 == 0: 8- or 16-byte output stores
};

// Skinny products (M <= 16 * MT: decode and verify steps).  A work-group of
// NW waves owns 16 weight rows; its waves split K in 64-wide chunks (wave w
// takes chunks w, w + NW, ...), so each row is streamed in whole 128-byte
// lines, U chunks in flight per wave.  The weights are read once for all MT
// tiles of 16 activation rows.  The waves' partial sums meet in LDS and are
// added in wave order (deterministic).  Bound: HBM, N*K*2 bytes of weights.
constexpr int kSkinnyU = 4;

template <int MT, int NW, bool VEC, bool F32>
__global__ __launch_bounds__(NW * 64) void gemm_skinny_kernel(GemmArgs a) {
    __shared__ float4_t s_part[NW][MT][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const uint32_t n0 = blockIdx.x * 16u;
    const uint64_t wrow = min(n0 + (uint32_t)li, a.N - 1u); // this lane's weight row (clamped)
    uint64_t arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) arow[mt] = min((uint32_t)(mt * 16 + li), a.M - 1u);
    float4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (float4_t)0.0f;
    const uint32_t n_chunks = (a.K + 63u) / 64u;
    for (uint32_t c0 = (uint32_t)wave; c0 < n_chunks; c0 += (uint32_t)(NW * kSkinnyU)) {
        half8_t wv[kSkinnyU][2];
#pragma unroll
        for (int u = 0; u < kSkinnyU; ++u) {
            const uint32_t k = (c0 + (uint32_t)(u * NW)) * 64u + 8u * (uint32_t)lg;
#pragma unroll
            for (int h = 0; h < 2; ++h) wv[u][h] = piece<VEC>(a.B, wrow, a.K, k + 32u * h);
        }
#pragma unroll
        for (int u = 0; u < kSkinnyU; ++u) {
            const uint32_t k = (c0 + (uint32_t)(u * NW)) * 64u + 8u * (uint32_t)lg;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt] = mfma(wv[u][h], piece<VEC>(a.A, arow[mt], a.K, k + 32u * h), acc[mt]);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) s_part[wave][mt][lane] = acc[mt];
    __syncthreads();
    // Wave mt' < MT finishes tile mt'; the sums run over the waves in order.
    if (wave < MT) {
        float4_t s = s_part[0][wave][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += s_part[w][wave][lane];
        store4<F32>(a.C, a.M, a.N, (uint32_t)(wave * 16 + li), n0 + 4u * (uint32_t)lg, s, a.scale, a.vec_out);
    }
}

// General products (prefill-sized M): 128 x 128 output tiles, 4 waves of 64 x 64
// (4 x 4 MFMA tiles each), k-steps of 32 staged in LDS with the next step's
// loads in registers while the current step is multiplied.  Bound: the matrix
// cores for large M, N, K.
constexpr int kTileM = 128, kTileN = 128, kTileK = 32, kTilePitch = kTileK + 8; // halves per staged row

template <bool VEC, bool F32>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][kTileN * kTilePitch]; // weights
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][kTileM * kTilePitch]; // activations
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const int wn = wave & 1, wm = wave >> 1;
    const uint32_t n0 = blockIdx.x * kTileN, m0 = blockIdx.y * kTileM;
    // Staging: 512 pieces of 8 halves per operand tile, two per thread: piece p =
    // (row p / 4, k 8 * (p % 4)).
    auto load = [&](uint32_t k0, half8_t (&pb)[2], half8_t (&pa)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int p = tid + 256 * j;
            const uint32_t r = (uint32_t)(p >> 2), k = k0 + 8u * (uint32_t)(p & 3);
            pb[j] = piece<VEC>(a.B, min(n0 + r, a.N - 1u), a.K, k);
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
            store4<F32>(a.C, a.M, a.N, m0 + (uint32_t)(wm * 64 + j * 16 + li), n0 + (uint32_t)(wn * 64 + i * 16 + 4 * lg),
                        acc[i][j], a.scale, a.vec_out);
}

} // namespace awo
