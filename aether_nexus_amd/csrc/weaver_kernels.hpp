// weaver_kernels.hpp — gfx950 (CDNA4) kernels of the Weaver decode path.
//
// The reference computes Weaver decode in one Metal kernel, one 32-thread
// group per query head, walking every hot token and then every cold token
// serially with an online softmax (nexus-core/src/weaver_kernel.metal:118-240).
// Here the same math is split into stages shaped for MI355X:
//
//   project_kernel  q_latent = q . D^T on MFMA (v_mfma_f32_16x16x32_f16).
//                   The identity the reference assumes for its q_latent input
//                   (weaver_kernel.metal:184-190, docs/YELLOWPAPER.md:84-92).
//   hot_kernel      exact attention over the f16 hot pool, split-K over the
//                   token axis.  One wave owns one (sequence, kv head, token
//                   range) and all G*Q query rows of that kv head, so each K/V
//                   row is read from HBM once for the whole GQA group
//                   (the reference re-reads it per query head).  S^T = K Q^T and
//                   O^T += V^T P^T both run on MFMA; K == V unless a separate V
//                   pool is given (weaver_kernel.metal:162-166).
//   cold_kernel     attention on the SparseCodes without decompression: scores
//                   from the LDS-resident q_latent table (metal:186-190), and
//                   instead of rebuilding V per token (metal:206-219) the
//                   softmax weight times each coefficient is accumulated into a
//                   per-atom bin in LDS.  sum_t p_t V_t = sum_a bin[a] D[a].
//   finish_kernel   bin . D on MFMA (fp32 bins split into two f16 terms),
//                   optionally fused with the log-sum-exp merge.
//   merge_kernel    log-sum-exp merge of hot and cold partials, f16 output
//                   (metal:226-239: zero output when nothing is visible).
//
// Scores are carried in the log2 domain (score * scale * log2(e)) so every
// exponential is one v_exp_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aw {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kBlockTokens = 16;      // tokens per block (ModelDims::BLOCK_SIZE)
constexpr uint32_t kRefMask = 0x7FFFFFFFu; // weaver_kernel.metal:145,174
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kColdThreads = 512;
constexpr int kFinishWaves = 4;
constexpr int kMaxSplits = 64;

// Error bits written to the engine's device error word.
constexpr uint32_t kErrHotRef = 1u, kErrColdRef = 2u, kErrAtom = 4u;

__device__ inline float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ inline half8_t as_h8(uint4_t v) { return __builtin_bit_cast(half8_t, v); }
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float h2f_bits(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ inline void flag_error(uint32_t* err, uint32_t bit) {
    __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wave-wide max / sum with DPP: quad permutes and row rotates reduce each
// 16-lane row, row_bcast15 / row_bcast31 fold the rows into lane 63, which is
// broadcast.  Every lane returns the result.
template <bool MAX>
__device__ inline float wave_reduce(float v) {
    const int id = __builtin_bit_cast(int, MAX ? -INFINITY : 0.0f);
#define AW_DPP_STEP(ctrl, rmask)                                                                               \
    {                                                                                                          \
        const float o = __builtin_bit_cast(                                                                    \
            float, __builtin_amdgcn_update_dpp(id, __builtin_bit_cast(int, v), ctrl, rmask, 0xF, false));     \
        v = MAX ? fmaxf(v, o) : v + o;                                                                         \
    }
    AW_DPP_STEP(0xB1, 0xF)  // quad_perm [1,0,3,2]
    AW_DPP_STEP(0x4E, 0xF)  // quad_perm [2,3,0,1]
    AW_DPP_STEP(0x124, 0xF) // row_ror:4
    AW_DPP_STEP(0x128, 0xF) // row_ror:8
    AW_DPP_STEP(0x142, 0xA) // row_bcast:15 into rows 1 and 3
    AW_DPP_STEP(0x143, 0xC) // row_bcast:31 into rows 2 and 3
#undef AW_DPP_STEP
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ inline float wave_max(float v) { return wave_reduce<true>(v); }
__device__ inline float wave_sum(float v) { return wave_reduce<false>(v); }

// Log-sum-exp combination of one row's splits, one wave, lane = split
// (S <= 64; lanes past S pass l = 0).  Empty splits (l == 0) get factor 0.
// Returns the row maximum M, the combined sum L, and this lane's factor
// 2^(m - M).
__device__ inline void combine_splits(float m, float l, float& M, float& L, float& f) {
    const bool ok = l > 0.0f;
    M = wave_max(ok ? m : -INFINITY);
    f = ok ? fast_exp2(m - M) : 0.0f;
    L = wave_sum(f * l);
}

// ---------------------------------------------------------------- arguments

struct ProjArgs {
    const uint16_t* q;    // [L][B][Q][Hq][HD]
    const uint16_t* dict; // [L][dict_heads][A][HD]
    uint16_t* ql;         // [L][B][Q][Hq][A] f16
    uint32_t batch, queries, q_heads, kv_heads, gqa, rows_r;
    uint32_t dict_size, dict_heads;
    uint32_t rows_per_group; // B*Q*(dict_heads==1 ? Hq : G)
    uint64_t dict_layer;     // elements per layer
};

struct HotArgs {
    const uint16_t* q;
    const uint16_t* hot_k;
    const uint16_t* hot_v; // may be null (K == V)
    const uint32_t* refs;
    const uint32_t* seq_hot;
    float* part_m; // [lbg][S][R]
    float* part_l;
    float* part_o; // [lbg][S][R][HD]
    uint32_t* err;
    uint32_t batch, queries, q_heads, kv_heads, gqa, rows_r;
    uint32_t hot_count, refs_stride, splits, tokens_per_split, causal;
    float scale_log2;
    uint64_t hot_blocks, hot_layer, refs_layer;
};

struct ColdArgs {
    const uint16_t* ql; // q_latent, addressed through the strides below
    const uint4_t* cold;
    const uint32_t* refs;
    const uint32_t* seq_cold;
    float* part_m; // [lbg][S][R]
    float* part_l;
    float* part_w;   // [lbg][S][R][A]
    float* part_amax; // [lbg][S][R]: max_a |bin[a]|
    uint32_t* err;
    uint32_t batch, kv_heads, gqa, rows_r;
    uint32_t hot_count, cold_count, refs_stride, dict_size;
    uint32_t splits, tokens_per_split, n_chunks, n_units;
    float scale_log2;
    uint64_t cold_blocks, cold_layer, refs_layer;
    // q_latent element (lb, g, q, j, a) = ql[lb*s_lb + g*s_g + q*s_q + j*s_j + a*s_a]
    uint64_t s_lb, s_g, s_q, s_j, s_a;
};

struct FinishArgs {
    const uint16_t* dict;
    const float* cold_m;
    const float* cold_l;
    const float* cold_w;
    const float* cold_amax;
    const float* hot_m;
    const float* hot_l;
    const float* hot_o;
    float* ocp; // [lbg*R + r][n_ar][HD] when n_ar > 1
    uint16_t* out;
    uint32_t batch, queries, q_heads, kv_heads, gqa, rows_r;
    uint32_t dict_size, dict_heads, rows_per_group, tiles_per_group;
    uint32_t cold_splits, hot_splits, n_ar, atoms_per_range;
    uint64_t dict_layer;
};

struct MergeArgs {
    const float* cold_m;
    const float* cold_l;
    const float* cold_amax;
    const float* ocp; // [rows][n_ar][HD] or null (no cold)
    const float* hot_m;
    const float* hot_l;
    const float* hot_o;
    uint16_t* out;
    uint32_t batch, queries, q_heads, kv_heads, gqa, rows_r;
    uint32_t cold_splits, hot_splits, n_ar;
    uint64_t total_rows; // L*B*Hkv*R
};

// ------------------------------------------------------------ q . D^T (MFMA)
//
// Computes q_latent^T = D q^T so that each lane ends up with four consecutive
// atoms of one query row and stores them with one 8-byte write into
// q_latent [L][B][Q][Hq][A] (the layout of the reference's q_latent buffer,
// weaver_kernel.metal:111).  One wave computes (16*NA atoms) x (16*MR rows),
// K = HD.  Operand layouts of v_mfma_f32_16x16x32_f16 (lane l, li = l%16,
// lg = l/16):
//   A[i][k]: lane holds row i = li, k = 8*lg .. 8*lg+7  -> 16 bytes of dictionary row (atom li)
//   B[k][j]: lane holds col j = li, k = 8*lg .. 8*lg+7  -> 16 bytes of query row li
//   C[i][j]: lane holds rows i = 4*lg .. 4*lg+3, col j = li -> 4 atoms of query row li
// Rows of one group share one dictionary: group = (layer, dict head); inside a
// group row i enumerates (b, q, head) with head over Hq (shared dictionary) or
// over the G heads of kv head dg (per-kv-head dictionary).
template <int HD, int MR, int NA>
__global__ __launch_bounds__(64) void project_kernel(ProjArgs a) {
    constexpr int KS = HD / 32;
    const int lane = threadIdx.x, li = lane & 15, lg = lane >> 4;
    const uint32_t group = blockIdx.z;
    const uint32_t l = group / a.dict_heads, dg = group % a.dict_heads;
    const uint32_t atom0 = blockIdx.x * 16 * NA, row0 = blockIdx.y * 16 * MR;
    const uint16_t* dict = a.dict + l * a.dict_layer + (uint64_t)dg * a.dict_size * HD;
    const bool shared = a.dict_heads == 1;

    // This lane's query rows (one per row block): global row index into q / q_latent.
    uint64_t qrow[MR];
    bool rok[MR];
#pragma unroll
    for (int mr = 0; mr < MR; ++mr) {
        const uint32_t i = row0 + 16 * mr + li;
        rok[mr] = i < a.rows_per_group;
        if (shared) {
            qrow[mr] = (uint64_t)l * a.rows_per_group + i; // rows of a layer are (b, q, h) in q's order
        } else {                                           // (b, q, head hh of kv head dg)
            const uint32_t bq = i / a.gqa, hh = i % a.gqa;
            qrow[mr] = ((uint64_t)l * a.batch * a.queries + bq) * a.q_heads + dg * a.gqa + hh;
        }
    }
    half8_t bop[MR][KS];
#pragma unroll
    for (int mr = 0; mr < MR; ++mr)
#pragma unroll
        for (int j = 0; j < KS; ++j)
            bop[mr][j] = rok[mr] ? as_h8(*(const uint4_t*)(a.q + qrow[mr] * HD + 32 * j + 8 * lg))
                                 : (half8_t)(_Float16)0;
#pragma unroll
    for (int na = 0; na < NA; ++na) {
        const uint32_t at = atom0 + 16 * na + li;
        half8_t aop[KS];
#pragma unroll
        for (int j = 0; j < KS; ++j)
            aop[j] = at < a.dict_size ? as_h8(*(const uint4_t*)(dict + (uint64_t)at * HD + 32 * j + 8 * lg))
                                      : (half8_t)(_Float16)0;
        const uint32_t ao = atom0 + 16 * na + 4 * lg; // this lane's 4 output atoms
#pragma unroll
        for (int mr = 0; mr < MR; ++mr) {
            float4_t acc = (float4_t)0.0f;
#pragma unroll
            for (int j = 0; j < KS; ++j) acc = mfma16x16x32(aop[j], bop[mr][j], acc);
            if (rok[mr] && ao < a.dict_size) { // dict_size % 16 == 0: all four atoms are in range
                half4_t v;
                v[0] = (_Float16)acc[0];
                v[1] = (_Float16)acc[1];
                v[2] = (_Float16)acc[2];
                v[3] = (_Float16)acc[3];
                *(half4_t*)(a.ql + qrow[mr] * a.dict_size + ao) = v;
            }
        }
    }
}

// ------------------------------------------------- hot pool, split-K (MFMA)
//
// Work item = (lbg, split); one wave; the wave holds all R = G*Q query rows of
// its kv head in RT tiles of 16.  Per chunk of 32 tokens (two 16-token blocks):
//   S^T[token][row] = K Q^T: A = K (lane: token li of block tb, dims 8*lg+32j..)
//                            B = Q^T (lane: row li, same dims), 4 k-steps at HD=128
//   -> lane holds scores of tokens 4*lg+e (e<4) of each block for row li, so
//      the P^T operand of the second product is already in the lane:
//      k-index 8*lg+e' <-> token 4*lg+e' (e'<4) / 16+4*lg+(e'-4) (e'>=4).
//   O^T[dim][row] += V^T P^T: A = V^T (lane: dim 16*nb+li, the 8 tokens above),
//      gathered from the chunk staged in LDS.
// LDS pitch HD+4 halves (66 words at HD=128) puts the four token rows 4*lg+e'
// of one read on disjoint 8-bank groups.
template <int HD, int RT>
__global__ __launch_bounds__(64) void hot_kernel(HotArgs a) {
    constexpr int KS = HD / 32, NB = HD / 16, P = HD + 4;
    __shared__ __attribute__((aligned(16))) _Float16 lds[32 * P];
    const int lane = threadIdx.x, li = lane & 15, lg = lane >> 4;
    const uint32_t s = blockIdx.x % a.splits, lbg = blockIdx.x / a.splits;
    const uint32_t g = lbg % a.kv_heads, lb = lbg / a.kv_heads, l = lb / a.batch;
    uint32_t nh = a.hot_count;
    if (a.seq_hot) nh = min(nh, a.seq_hot[lb]);
    const uint32_t n_tok = nh * kBlockTokens;
    const uint32_t t_begin = s * a.tokens_per_split;
    const uint32_t t_end = min(t_begin + a.tokens_per_split, n_tok);
    const uint32_t R = a.rows_r;

    half8_t qop[RT][KS];
    int lim[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t r = 16 * rt + li;
        if (r < R) {
            const uint32_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
            const uint16_t* p = a.q + (((uint64_t)lb * a.queries + q) * a.q_heads + h) * HD;
#pragma unroll
            for (int j = 0; j < KS; ++j) qop[rt][j] = as_h8(*(const uint4_t*)(p + 32 * j + 8 * lg));
            lim[rt] = a.causal ? (int)n_tok - (int)a.queries + 1 + (int)q : (int)n_tok;
        } else {
#pragma unroll
            for (int j = 0; j < KS; ++j) qop[rt][j] = (half8_t)(_Float16)0;
            lim[rt] = 0;
        }
    }

    float m_run[RT], l_run[RT];
    float4_t oacc[RT][NB];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.0f;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oacc[rt][nb] = (float4_t)0.0f;
    }

    const uint16_t* kbase = a.hot_k + (uint64_t)l * a.hot_layer;
    const uint16_t* vbase = a.hot_v ? a.hot_v + (uint64_t)l * a.hot_layer : nullptr;
    const uint32_t* refs = a.refs + (uint64_t)l * a.refs_layer + (uint64_t)(lb % a.batch) * a.refs_stride;

    // Resolve the two blocks of chunk c0 and load this lane's K pieces.
    auto load_chunk = [&](uint32_t c0, uint4_t (&kr)[2][KS], uint64_t (&rowoff)[2], bool (&ok)[2]) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const bool in = c0 + 16 * tb < t_end;
            const uint32_t ref = in ? (refs[c0 / 16 + tb] & kRefMask) : 0u;
            ok[tb] = in && ref < a.hot_blocks;
            if (in && !ok[tb]) flag_error(a.err, kErrHotRef);
            rowoff[tb] = (((uint64_t)ref * kBlockTokens + li) * a.kv_heads + g) * HD + 8 * lg;
#pragma unroll
            for (int j = 0; j < KS; ++j)
                kr[tb][j] = ok[tb] ? *(const uint4_t*)(kbase + rowoff[tb] + 32 * j) : (uint4_t)0u;
        }
    };

    uint4_t kcur[2][KS];
    uint64_t offcur[2];
    bool okcur[2];
    if (t_begin < t_end) load_chunk(t_begin, kcur, offcur, okcur);

    for (uint32_t c0 = t_begin; c0 < t_end; c0 += 32) {
        uint4_t knext[2][KS];
        uint64_t offnext[2];
        bool oknext[2];
        const bool more = c0 + 32 < t_end;
        if (more) load_chunk(c0 + 32, knext, offnext, oknext);

        // S^T = K Q^T
        float4_t sacc[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                sacc[rt][tb] = (float4_t)0.0f;
#pragma unroll
                for (int j = 0; j < KS; ++j)
                    sacc[rt][tb] = mfma16x16x32(as_h8(kcur[tb][j]), qop[rt][j], sacc[rt][tb]);
            }

        // Stage V (= K unless a V pool is given) in LDS as [token][dim].
        __syncthreads();
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                uint4_t v = kcur[tb][j];
                if (vbase) v = okcur[tb] ? *(const uint4_t*)(vbase + offcur[tb] + 32 * j) : (uint4_t)0u;
                _Float16* dst = lds + (16 * tb + li) * P + 32 * j + 8 * lg;
                *(uint2_t*)dst = (uint2_t){v[0], v[1]};
                *(uint2_t*)(dst + 4) = (uint2_t){v[2], v[3]};
            }
        __syncthreads();

        // Online softmax per query row (row li of each tile).
        half8_t pop[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float sv[8];
            float mx = -INFINITY;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int tok = (int)(c0 + 16 * tb + 4 * lg + e);
                    const bool v = okcur[tb] && tok < lim[rt];
                    sv[4 * tb + e] = v ? sacc[rt][tb][e] * a.scale_log2 : -INFINITY;
                    mx = fmaxf(mx, sv[4 * tb + e]);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mnew = fmaxf(m_run[rt], mx);
            float alpha = 1.0f, psum = 0.0f;
            if (mnew != -INFINITY) {
                alpha = fast_exp2(m_run[rt] - mnew);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float p = fast_exp2(sv[e] - mnew);
                    psum += p;
                    pop[rt][e] = (_Float16)p;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) pop[rt][e] = (_Float16)0;
            }
            l_run[rt] = l_run[rt] * alpha + psum;
            m_run[rt] = mnew;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) oacc[rt][nb] *= alpha;
        }

        // O^T += V^T P^T
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            half8_t vop;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int row = e < 4 ? 4 * lg + e : 16 + 4 * lg + (e - 4);
                vop[e] = lds[row * P + 16 * nb + li];
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) oacc[rt][nb] = mfma16x16x32(vop, pop[rt], oacc[rt][nb]);
        }

        if (more) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                offcur[tb] = offnext[tb];
                okcur[tb] = oknext[tb];
#pragma unroll
                for (int j = 0; j < KS; ++j) kcur[tb][j] = knext[tb][j];
            }
        }
    }

    const uint64_t pbase = ((uint64_t)lbg * a.splits + s) * R;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        float lt = l_run[rt] + __shfl_xor(l_run[rt], 16);
        lt += __shfl_xor(lt, 32);
        const uint32_t r = 16 * rt + li;
        if (r < R) {
            if (lg == 0) {
                a.part_m[pbase + r] = m_run[rt];
                a.part_l[pbase + r] = lt;
            }
            float* po = a.part_o + (pbase + r) * HD;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) *(float4_t*)(po + 16 * nb + 4 * lg) = oacc[rt][nb];
        }
    }
}

// ----------------------------------------------- cold pool, scores + bins
//
// Work item = (layer*batch+seq, chunk of RC query rows, split) x kv head g.
// LDS: q_latent table [A][RC] f16; per atom NP = ceil(RC/2) 64-bit bins,
// each holding two rows' sums as 32-bit fixed point; the split's block refs.
//
// Integer bins: on gfx950 an LDS ds_add_f32 retires about one lane per 3
// cycles per CU whatever the addresses, ds_add_u64 about one lane per 0.3
// cycles (measured).  A row pair (v0, v1) is added as the 64-bit integer
// v1*2^32 + v0 (v0 sign-extended); sums of such words are exact and decode back
// to (sum v0, sum v1) while each row sum stays inside int32.
//
// Values are p*c*2^F with p = 2^(s - ref_r).  ref_r (integral, log2 units) and
// F come from the split's first tile: ref_r = ceil(max score of the tile),
// F sized so that the planned bound on sum |p*c| over the whole split stays
// near 2^28.  The work-group then streams every tile with no further
// synchronisation.  At the end a conservative bound, 4 * max|c| * sum_t sum_r p,
// proves the bins could not have overflowed; when it cannot (scores far above
// the first tile's, or coefficients far larger), the split is recomputed
// exactly: a pass for the per-row maxima, a pass for the exact bound, a pass
// for the bins.  Each contribution is rounded to the nearest unit of 2^-F
// (half away from zero), so bin errors are unbiased, at most half a unit per
// contribution.
//
// The kv heads of one (sequence, chunk, split) run on one XCD (work-groups are
// dealt round-robin over the 8 XCDs), so the 128-byte lines interleaving their
// 16-byte codes come from HBM once per XCD L2.
template <int RC, int CPT, int PD>
__global__ __launch_bounds__(kColdThreads) void cold_kernel(ColdArgs a) {
    constexpr int NT = kColdThreads, NW = NT / 64, NP = (RC + 1) / 2, NRED = 2 * RC + 2;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t x = blockIdx.x % 8u, k = blockIdx.x / 8u;
    const uint32_t g = k % a.kv_heads;
    const uint32_t u = (k / a.kv_heads) * 8u + x;
    if (u >= a.n_units) return;
    const uint32_t s = u % a.splits, uc = u / a.splits;
    const uint32_t c = uc % a.n_chunks, lb = uc / a.n_chunks;
    const uint32_t l = lb / a.batch;
    const uint64_t lbg = (uint64_t)lb * a.kv_heads + g;
    const uint32_t A = a.dict_size, R = a.rows_r;
    uint32_t nc = a.cold_count;
    if (a.seq_cold) nc = min(nc, a.seq_cold[lb]);
    const uint32_t n_tok = nc * kBlockTokens;
    const uint32_t t_begin = s * a.tokens_per_split;
    const uint32_t t_end = min(t_begin + a.tokens_per_split, n_tok);
    const uint64_t pbase = (lbg * a.splits + s) * R;

    if (t_begin >= t_end) {
        if (tid < RC) {
            const uint32_t r = c * RC + tid;
            if (r < R) {
                a.part_m[pbase + r] = -INFINITY;
                a.part_l[pbase + r] = 0.0f;
                a.part_amax[pbase + r] = 0.0f;
            }
        }
        return;
    }

    const uint32_t qtab_bytes = (A * RC * 2 + 15) & ~15u;
    const uint32_t n_blk = (t_end - t_begin + 15) / 16; // t_begin is a multiple of 16
    _Float16* qtab = (_Float16*)smem;
    uint64_t* bins = (uint64_t*)(smem + qtab_bytes);       // [A][NP]
    uint32_t* sref = (uint32_t*)(bins + (uint64_t)A * NP); // [n_blk] physical blocks, ~0 = invalid
    float* red = (float*)(sref + ((n_blk + 3) & ~3u));    // [NW][NRED]

    // q_latent rows of this chunk into LDS; rows past R are zero.
    {
        uint64_t rbase[RC];
        bool rok[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            const uint32_t r = c * RC + rr;
            rok[rr] = r < R;
            rbase[rr] = rok[rr] ? (uint64_t)lb * a.s_lb + g * a.s_g + (uint64_t)(r / a.gqa) * a.s_q +
                                      (uint64_t)(r % a.gqa) * a.s_j
                                : 0;
        }
        // Atom-contiguous rows (s_a == 1, q_latent's layout): 16-byte loads of 8 atoms per
        // row, interleaved into [A][RC] in registers.
        if (a.s_a == 1 && (A % 8) == 0 && ((uintptr_t)a.ql & 15u) == 0) {
            for (uint32_t a8 = tid; a8 < A / 8; a8 += NT) {
                uint4_t w[RC];
#pragma unroll
                for (int rr = 0; rr < RC; ++rr)
                    w[rr] = rok[rr] ? *(const uint4_t*)(a.ql + rbase[rr] + (uint64_t)a8 * 8) : (uint4_t)0u;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    _Float16 hv[RC];
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr)
                        hv[rr] = __builtin_bit_cast(_Float16, (uint16_t)(w[rr][e / 2] >> (16 * (e % 2))));
                    if constexpr (RC == 4) {
                        half4_t v4 = {hv[0], hv[1], hv[2], hv[3]};
                        *(half4_t*)(qtab + (a8 * 8 + e) * 4) = v4;
                    } else {
#pragma unroll
                        for (int rr = 0; rr < RC; ++rr) qtab[(a8 * 8 + e) * RC + rr] = hv[rr];
                    }
                }
            }
        } else {
            for (uint32_t at = tid; at < A; at += NT)
#pragma unroll
                for (int rr = 0; rr < RC; ++rr)
                    qtab[at * RC + rr] =
                        __builtin_bit_cast(_Float16, rok[rr] ? a.ql[rbase[rr] + (uint64_t)at * a.s_a] : (uint16_t)0);
        }
    }
    // The split's block refs, resolved once, so code addresses come from LDS.
    {
        const uint32_t* refs = a.refs + (uint64_t)l * a.refs_layer + (uint64_t)(lb % a.batch) * a.refs_stride +
                               a.hot_count + t_begin / 16;
        for (uint32_t i = tid; i < n_blk; i += NT) {
            uint32_t ref = refs[i] & kRefMask;
            if (ref >= a.cold_blocks) {
                flag_error(a.err, kErrColdRef);
                ref = ~0u;
            }
            sref[i] = ref;
        }
    }

    const uint4_t* cold = a.cold + (uint64_t)l * a.cold_layer;
    const uint32_t tile_tokens = NT * CPT;
    const uint32_t n_tiles = (t_end - t_begin + tile_tokens - 1) / tile_tokens;
    const float sl = a.scale_log2;

    auto load_tile = [&](uint32_t t0, uint4_t (&buf)[CPT], bool (&ok)[CPT]) {
#pragma unroll
        for (int kk = 0; kk < CPT; ++kk) {
            const uint32_t t = t0 + kk * NT + tid;
            bool v = t < t_end;
            buf[kk] = (uint4_t)0u; // a token past the split or behind a bad ref scores as a zero code
            if (v) {
                const uint32_t ref = sref[(t - t_begin) >> 4];
                v = ref != ~0u;
                if (v) buf[kk] = cold[((uint64_t)ref * kBlockTokens + (t & 15u)) * a.kv_heads + g];
            }
            ok[kk] = v;
        }
    };
    // Unscaled score sums of one code for the RC rows: sum_k c_k * q_latent[idx_k][r].
    auto score = [&](const uint4_t cw, float (&sc)[RC], uint32_t (&ia)[4], float (&cf)[4]) {
        ia[0] = cw[0] & 0xFFFFu;
        ia[1] = cw[0] >> 16;
        ia[2] = cw[1] & 0xFFFFu;
        ia[3] = cw[1] >> 16;
        cf[0] = h2f_bits(cw[2] & 0xFFFFu);
        cf[1] = h2f_bits(cw[2] >> 16);
        cf[2] = h2f_bits(cw[3] & 0xFFFFu);
        cf[3] = h2f_bits(cw[3] >> 16);
        if (max(max(ia[0], ia[1]), max(ia[2], ia[3])) >= A) { // out-of-range atoms: skip those terms
            flag_error(a.err, kErrAtom);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (ia[j] >= A) {
                    ia[j] = 0;
                    cf[j] = 0.0f;
                }
        }
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) sc[rr] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const _Float16* qp = qtab + ia[j] * RC;
            if constexpr (RC == 4) {
                const half4_t qv = *(const half4_t*)qp;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) sc[rr] += cf[j] * (float)qv[rr];
            } else {
#pragma unroll
                for (int rr = 0; rr < RC; ++rr) sc[rr] += cf[j] * (float)qp[rr];
            }
        }
    };
    auto cmax4 = [](const float (&cf)[4]) { return fmaxf(fmaxf(fabsf(cf[0]), fabsf(cf[1])), fmaxf(fabsf(cf[2]), fabsf(cf[3]))); };

    // Work-group sums/maxima of up to NRED per-lane values (one barrier pair).
    auto wg_reduce = [&](float (&v)[NRED], const bool (&is_max)[NRED]) {
        __syncthreads(); // previous readers of `red` are done
#pragma unroll
        for (int i = 0; i < NRED; ++i) {
            const float w = is_max[i] ? wave_max(v[i]) : wave_sum(v[i]);
            if (lane == 0) red[wave * NRED + i] = w;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NRED; ++i) {
            float acc = is_max[i] ? -INFINITY : 0.0f;
            for (int w = 0; w < NW; ++w) acc = is_max[i] ? fmaxf(acc, red[w * NRED + i]) : acc + red[w * NRED + i];
            v[i] = acc;
        }
    };

    float ref[RC];
    int F = 0;
    float lpart[RC], cmx = 0.0f;
    uint4_t cur[CPT];
    bool curv[CPT];
    bool exact = false;
    for (int attempt = 0; attempt < 2; ++attempt) {
        for (uint32_t i = tid; i < A * NP; i += NT) bins[i] = 0ull;
        __syncthreads();
        load_tile(t_begin, cur, curv);
        if (!exact) {
            // Reference and scale from the first tile.
            float v[NRED];
            bool is_max[NRED];
#pragma unroll
            for (int i = 0; i < NRED; ++i) {
                v[i] = i < RC ? -INFINITY : 0.0f;
                is_max[i] = i < RC;
            }
            float scs[CPT][RC];
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk) {
                uint32_t ia[4];
                float cf[4];
                score(cur[kk], scs[kk], ia, cf);
                if (curv[kk]) {
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) v[rr] = fmaxf(v[rr], scs[kk][rr] * sl);
                    v[2 * RC] = fmaxf(v[2 * RC], cmax4(cf)); // summed below: only a plan
                }
            }
            wg_reduce(v, is_max);
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) ref[rr] = v[rr] == -INFINITY ? 0.0f : ceilf(v[rr]);
            float w[NRED];
#pragma unroll
            for (int i = 0; i < NRED; ++i) {
                w[i] = 0.0f;
                is_max[i] = false;
            }
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk)
                if (curv[kk]) {
                    float ps = 0.0f;
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) ps += fast_exp2(scs[kk][rr] * sl - ref[rr]);
                    uint32_t ia[4];
                    float cf[4], dummy[RC];
                    score(cur[kk], dummy, ia, cf);
                    w[0] += 4.0f * cmax4(cf) * ps;
                }
            wg_reduce(w, is_max);
            const float plan = w[0] * (float)n_tiles; // bound on sum |p*c| over the split, if tiles are alike
            F = plan > 0.0f ? min(100, max(-100, 28 - (ilogbf(plan) + 1))) : 0;
        }
        // Stream every tile into the bins; PD tiles of code loads stay in flight
        // (a ring of registers, refilled as each slot is consumed).
        const float Ff = (float)F;
        float rf[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            lpart[rr] = 0.0f;
            rf[rr] = Ff - ref[rr];
        }
        cmx = 0.0f;
        uint4_t ring[PD][CPT];
        bool rv[PD][CPT];
#pragma unroll
        for (int kk = 0; kk < CPT; ++kk) {
            ring[0][kk] = cur[kk];
            rv[0][kk] = curv[kk];
        }
#pragma unroll
        for (int d = 1; d < PD; ++d) load_tile(t_begin + d * tile_tokens, ring[d], rv[d]);
        for (uint32_t t0 = t_begin; t0 < t_end; t0 += PD * tile_tokens) {
#pragma unroll
            for (int d = 0; d < PD; ++d) {
#pragma unroll
                for (int kk = 0; kk < CPT; ++kk) {
                    if (!rv[d][kk]) continue;
                    const uint4_t cw = ring[d][kk];
                    float sc[RC];
                    uint32_t ia[4];
                    float cf[4];
                    score(cw, sc, ia, cf);
                    cmx = fmaxf(cmx, cmax4(cf));
                    float ps[RC]; // p * 2^F
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) {
                        ps[rr] = fast_exp2(fmaf(sc[rr], sl, rf[rr]));
                        lpart[rr] += ps[rr];
                    }
                    // Round half away from zero (p > 0, so the sign is c's): the
                    // +-0.5 rides in the FMA and the conversion truncates.
                    const uint32_t cbits[4] = {cw[2] << 16, cw[2], cw[3] << 16, cw[3]};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint64_t* bp = bins + ia[j] * NP;
                        const float hc = __builtin_bit_cast(float, (cbits[j] & 0x80000000u) | 0x3F000000u);
#pragma unroll
                        for (int pp = 0; pp < NP; ++pp) {
                            const int32_t v0 = (int32_t)fmaf(ps[2 * pp], cf[j], hc);
                            const int32_t v1 =
                                (2 * pp + 1 < RC) ? (int32_t)fmaf(ps[min(2 * pp + 1, RC - 1)], cf[j], hc) : 0;
                            const uint64_t wv = ((uint64_t)(uint32_t)v1 << 32) + (uint64_t)(int64_t)v0;
                            __hip_atomic_fetch_add(bp + pp, wv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        }
                    }
                }
                // Refill this slot with the tile PD ahead.
                load_tile(t0 + (d + PD) * tile_tokens, ring[d], rv[d]);
            }
        }
        // Overflow proof: every |bin| <= sum over contributions |p*c|*2^F <= 4*max|c|*sum_r sum_t p*2^F.
        float v[NRED];
        bool is_max[NRED];
#pragma unroll
        for (int i = 0; i < NRED; ++i) {
            v[i] = 0.0f;
            is_max[i] = false;
        }
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) v[rr] = lpart[rr];
        v[2 * RC] = cmx;
        is_max[2 * RC] = true;
        wg_reduce(v, is_max);
        float psum = 0.0f;
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            lpart[rr] = v[rr];
            psum += v[rr];
        }
        const float bound = 4.0f * v[2 * RC] * psum; // already in units of 2^-F
        if (exact || (bound < 2147483648.0f && bound == bound)) break;

        // Exact path: per-row maxima, then the exact bound, then the bins.
        exact = true;
        float mx[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) mx[rr] = -INFINITY;
        for (uint32_t t0 = t_begin; t0 < t_end; t0 += tile_tokens) {
            load_tile(t0, cur, curv);
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk)
                if (curv[kk]) {
                    float sc[RC];
                    uint32_t ia[4];
                    float cf[4];
                    score(cur[kk], sc, ia, cf);
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) mx[rr] = fmaxf(mx[rr], sc[rr] * sl);
                }
        }
        float m2[NRED];
        bool im2[NRED];
#pragma unroll
        for (int i = 0; i < NRED; ++i) {
            m2[i] = i < RC ? mx[i] : 0.0f;
            im2[i] = i < RC;
        }
        wg_reduce(m2, im2);
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) ref[rr] = m2[rr] == -INFINITY ? 0.0f : ceilf(m2[rr]);
        float eb = 0.0f; // exact sum over contributions of |p*c|, maximised over rows below
        float ebr[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) ebr[rr] = 0.0f;
        for (uint32_t t0 = t_begin; t0 < t_end; t0 += tile_tokens) {
            load_tile(t0, cur, curv);
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk)
                if (curv[kk]) {
                    float sc[RC];
                    uint32_t ia[4];
                    float cf[4];
                    score(cur[kk], sc, ia, cf);
                    const float ca = fabsf(cf[0]) + fabsf(cf[1]) + fabsf(cf[2]) + fabsf(cf[3]);
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) ebr[rr] += fast_exp2(sc[rr] * sl - ref[rr]) * ca;
                }
        }
#pragma unroll
        for (int i = 0; i < NRED; ++i) {
            m2[i] = i < RC ? ebr[i] : 0.0f;
            im2[i] = false;
        }
        wg_reduce(m2, im2);
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) eb = fmaxf(eb, m2[rr]);
        F = eb > 0.0f ? min(100, max(-100, 29 - (ilogbf(eb) + 1))) : 0;
        __syncthreads();
    }

    // Bins out as float rows [r][A]; track max |bin| per row for the f16 split of the finish.
    const float inv = ldexpf(1.0f, -F);
    float amax[RC];
#pragma unroll
    for (int rr = 0; rr < RC; ++rr) amax[rr] = 0.0f;
    for (uint32_t at = tid; at < A; at += NT) {
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) {
            const uint64_t wv = bins[at * NP + pp];
            const int32_t v0 = (int32_t)(uint32_t)wv;
            const int32_t v1 = (int32_t)((uint32_t)(wv >> 32) + (v0 < 0 ? 1u : 0u));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int rr = 2 * pp + h;
                if (rr >= RC) continue;
                const float v = (float)(h ? v1 : v0) * inv;
                amax[rr] = fmaxf(amax[rr], fabsf(v));
                const uint32_t r = c * RC + rr;
                if (r < R) a.part_w[(pbase + r) * A + at] = v;
            }
        }
    }
    float v[NRED];
    bool is_max[NRED];
#pragma unroll
    for (int i = 0; i < NRED; ++i) {
        v[i] = i < RC ? amax[i] : 0.0f;
        is_max[i] = true;
    }
    wg_reduce(v, is_max);
    if (tid < RC) {
        const uint32_t r = c * RC + tid;
        if (r < R) {
            a.part_m[pbase + r] = ref[tid];
            a.part_l[pbase + r] = lpart[tid] * inv; // sum of p, back from units of 2^-F
            a.part_amax[pbase + r] = v[tid];
        }
    }
}

// Shared-memory bytes of cold_kernel<RC> for a dictionary of A atoms and
// splits of `tokens_per_split` tokens.
inline size_t cold_smem_bytes(uint32_t A, int RC, uint32_t tokens_per_split) {
    const size_t qtab = ((size_t)A * RC * 2 + 15) & ~(size_t)15;
    const int NW = kColdThreads / 64, NP = (RC + 1) / 2;
    const size_t n_blk = ((size_t)(tokens_per_split + 15) / 16 + 3) & ~(size_t)3;
    return qtab + (size_t)A * NP * 8 + n_blk * 4 + (size_t)NW * (2 * RC + 2) * 4;
}

// ----------------------------------------------- per-row merge factors
//
// For one row (lbg, r): cold splits combine to max Mc and sum Lc; the bins are
// pre-multiplied by 2^(m_s - Mc) / Lc * scl with scl a power of two that keeps
// the largest combined bin below 2^14, so the hi/lo f16 split of each bin keeps
// ~22 significant bits.  Hot splits combine to Mh, Lh with factors 2^(m_s - Mh).
// Computed by one wave per row, lane = split.
struct RowFactors {
    float Mc, Lc, inv_scl, Mh, Lh;
};

__device__ inline float bin_scale(float bound, float Lc) {
    float scl = 1.0f;
    if (Lc > 0.0f && bound > 0.0f) {
        int e = ilogbf(bound / Lc) + 1;
        e = max(-100, min(100, e));
        scl = ldexpf(1.0f, 14 - e);
    }
    return scl;
}

// out = (wh*Oh + wc*Lc*Oc) / (wh*Lh + wc*Lc); zero when nothing was visible.
__device__ inline float merge_value(float oh, float Mh, float Lh, float oc, float Mc, float Lc) {
    const float M = fmaxf(Lh > 0.0f ? Mh : -INFINITY, Lc > 0.0f ? Mc : -INFINITY);
    if (M == -INFINITY) return 0.0f;
    const float wh = Lh > 0.0f ? fast_exp2(Mh - M) : 0.0f;
    const float wc = Lc > 0.0f ? fast_exp2(Mc - M) : 0.0f;
    const float den = wh * Lh + wc * Lc;
    return den > 0.0f ? (wh * oh + wc * Lc * oc) / den : 0.0f;
}

// ------------------------------------------------------ bins . D (MFMA)
//
// Work-group = 64 rows sharing one dictionary (4 waves x 16 rows) x one atom
// range.  All four waves walk the same 32-atom dictionary chunks, staged once
// per work-group in LDS (double-buffered, the next chunk's loads in flight
// during the current chunk's MFMAs).  Per wave: O^T[dim][row] += D^T W^T with
//   B = W^T (lane: row li, atoms a0+4*lg+{0..3} and a0+16+4*lg+{0..3}: two
//       16-byte loads per cold split, combined with the split factors),
//       split into hi + lo f16 terms -> two MFMAs,
//   A = D^T (lane: dim 16*nb+li, the same 8 atoms) gathered from the LDS chunk
//       (pitch HD+4 halves: the four atom rows 4*lg+e of one read fall on
//       disjoint 8-bank groups).
// With one atom range the log-sum-exp merge runs here too; otherwise the
// partial cold outputs go to `ocp` for merge_kernel.
template <int HD>
__global__ __launch_bounds__(256) void finish_kernel(FinishArgs a) {
    constexpr int NB = HD / 16, P = HD + 4, ROWS = 64;
    constexpr int PIECES = 32 * HD / 8; // 16-byte pieces per dictionary chunk
    constexpr int PPT = PIECES / 256;   // pieces per thread (2 at HD=128, 1 at HD=64)
    __shared__ __attribute__((aligned(16))) _Float16 sd[2][32 * P];
    __shared__ float s_cfac[ROWS][kMaxSplits];
    __shared__ float s_hfac[ROWS][kMaxSplits];
    __shared__ RowFactors s_rf[ROWS];
    __shared__ uint64_t s_row[ROWS]; // lbg*R + r, or ~0 for padding rows
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const uint32_t group = blockIdx.x / a.tiles_per_group, tile = blockIdx.x % a.tiles_per_group;
    const uint32_t ar = blockIdx.y;
    const uint32_t l = group / a.dict_heads, dg = group % a.dict_heads;
    const uint32_t R = a.rows_r, A = a.dict_size;
    const uint32_t hg = a.dict_heads == 1 ? a.kv_heads : 1;
    const bool fused = a.n_ar == 1 && a.hot_splits > 0;

    // Split factors: wave w combines rows 16w..16w+15, lane = split; all loads first.
    {
        constexpr int RPW = ROWS / 4;
        uint64_t rid[RPW];
        float cm[RPW], cl[RPW], ca[RPW], hm[RPW], hl[RPW];
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const uint32_t row = tile * ROWS + wave * RPW + i;
            rid[i] = ~0ull;
            cm[i] = hm[i] = -INFINITY;
            cl[i] = ca[i] = hl[i] = 0.0f;
            if (row < a.rows_per_group) {
                const uint32_t b = row / (hg * R), rem = row % (hg * R);
                const uint32_t g = a.dict_heads == 1 ? rem / R : dg, r = rem % R;
                const uint64_t lbg = ((uint64_t)l * a.batch + b) * a.kv_heads + g;
                rid[i] = lbg * R + r;
                if ((uint32_t)lane < a.cold_splits) {
                    const uint64_t cb = (lbg * a.cold_splits + lane) * R + r;
                    cm[i] = a.cold_m[cb];
                    cl[i] = a.cold_l[cb];
                    ca[i] = a.cold_amax[cb];
                }
                if (fused && (uint32_t)lane < a.hot_splits) {
                    const uint64_t hb = (lbg * a.hot_splits + lane) * R + r;
                    hm[i] = a.hot_m[hb];
                    hl[i] = a.hot_l[hb];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = wave * RPW + i;
            RowFactors rf;
            float f;
            combine_splits(cm[i], cl[i], rf.Mc, rf.Lc, f);
            const float scl = bin_scale(wave_sum(f * ca[i]), rf.Lc);
            rf.inv_scl = 1.0f / scl;
            if (lane < kMaxSplits) s_cfac[row][lane] = rf.Lc > 0.0f ? f / rf.Lc * scl : 0.0f;
            rf.Mh = -INFINITY;
            rf.Lh = 0.0f;
            if (fused) {
                float fh;
                combine_splits(hm[i], hl[i], rf.Mh, rf.Lh, fh);
                if (lane < kMaxSplits) s_hfac[row][lane] = fh;
            }
            if (lane == 0) {
                s_rf[row] = rf;
                s_row[row] = rid[i];
            }
        }
    }

    const uint16_t* dict = a.dict + (uint64_t)l * a.dict_layer + (uint64_t)dg * A * HD;
    const uint32_t a_begin = ar * a.atoms_per_range;
    const uint32_t a_end = min(a_begin + a.atoms_per_range, A);
    const uint32_t n_ch = (a_end - a_begin + 31) / 32;

    uint4_t dreg[PPT];
    auto load_d = [&](uint32_t a0) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int pc = tid + 256 * q, at = pc / (HD / 8), col = (pc % (HD / 8)) * 8;
            dreg[q] = (a0 + at < a_end) ? *(const uint4_t*)(dict + (uint64_t)(a0 + at) * HD + col) : (uint4_t)0u;
        }
    };
    auto store_d = [&](int buf) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int pc = tid + 256 * q, at = pc / (HD / 8), col = (pc % (HD / 8)) * 8;
            _Float16* dst = &sd[buf][at * P + col];
            *(uint2_t*)dst = (uint2_t){dreg[q][0], dreg[q][1]};
            *(uint2_t*)(dst + 4) = (uint2_t){dreg[q][2], dreg[q][3]};
        }
    };
    if (n_ch) {
        load_d(a_begin);
        store_d(0);
    }
    __syncthreads();

    const int myr = 16 * wave + li; // this lane's B-operand row
    const uint64_t myrow = s_row[myr];
    const bool rowok = myrow != ~0ull;
    const uint64_t lbg_me = rowok ? myrow / R : 0, r_me = rowok ? myrow % R : 0;
    const float* wbase = a.cold_w + ((lbg_me * a.cold_splits) * R + r_me) * A;
    const uint64_t wsplit = (uint64_t)R * A;

    float4_t acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = (float4_t)0.0f;

    // With one cold split (large batches) the next chunk's W values are
    // prefetched with the next dictionary chunk.
    const bool single = a.cold_splits == 1;
    const float f0 = rowok ? s_cfac[myr][0] : 0.0f;
    const bool wok = rowok && f0 != 0.0f; // an empty split wrote no bins: never read them
    float4_t wn0 = (float4_t)0.0f, wn1 = (float4_t)0.0f;
    auto load_w = [&](uint32_t a0) {
        const uint32_t at0 = a0 + 4 * lg, at1 = a0 + 16 + 4 * lg;
        wn0 = (wok && at0 < a_end) ? *(const float4_t*)(wbase + at0) : (float4_t)0.0f;
        wn1 = (wok && at1 < a_end) ? *(const float4_t*)(wbase + at1) : (float4_t)0.0f;
    };
    if (single && n_ch) load_w(a_begin);

    for (uint32_t ch = 0; ch < n_ch; ++ch) {
        const int buf = ch & 1;
        const uint32_t a0 = a_begin + ch * 32;
        const bool more = ch + 1 < n_ch;
        const float4_t wc0 = wn0, wc1 = wn1;
        if (more) {
            load_d(a0 + 32);
            if (single) load_w(a0 + 32);
        }
        float w8[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w8[e] = f0 * wc0[e];
            w8[4 + e] = f0 * wc1[e];
        }
        if (rowok && !single) {
#pragma unroll
            for (int e = 0; e < 8; ++e) w8[e] = 0.0f;
            const uint32_t at0 = a0 + 4 * lg, at1 = a0 + 16 + 4 * lg;
            // Four splits' loads in flight at a time; empty splits are never read.
            for (uint32_t s0 = 0; s0 < a.cold_splits; s0 += 4) {
                float4_t v0[4], v1[4];
                float fs[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t sp = s0 + j;
                    fs[j] = sp < a.cold_splits ? s_cfac[myr][sp] : 0.0f;
                    const float* wrow = wbase + sp * wsplit;
                    v0[j] = (fs[j] != 0.0f && at0 < a_end) ? *(const float4_t*)(wrow + at0) : (float4_t)0.0f;
                    v1[j] = (fs[j] != 0.0f && at1 < a_end) ? *(const float4_t*)(wrow + at1) : (float4_t)0.0f;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        w8[e] += fs[j] * v0[j][e];
                        w8[4 + e] += fs[j] * v1[j][e];
                    }
            }
        }
        half8_t hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            hi[e] = (_Float16)w8[e];
            lo[e] = (_Float16)(w8[e] - (float)hi[e]);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            half8_t dop;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int row = e < 4 ? 4 * lg + e : 16 + 4 * lg + (e - 4);
                dop[e] = sd[buf][row * P + 16 * nb + li];
            }
            acc[nb] = mfma16x16x32(dop, hi, acc[nb]);
            acc[nb] = mfma16x16x32(dop, lo, acc[nb]);
        }
        if (more) store_d(buf ^ 1);
        __syncthreads();
    }

    if (!rowok) return;
    // Lane holds O^T[dims 16*nb + 4*lg + e][row li of this wave].
    const RowFactors rf = s_rf[myr];
    const uint64_t rowid = myrow;
    if (!fused && a.n_ar > 1) {
        float* dst = a.ocp + (rowid * a.n_ar + ar) * HD;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) *(float4_t*)(dst + 16 * nb + 4 * lg) = acc[nb] * rf.inv_scl;
        return;
    }
    // Fused merge with the hot partials of this row.
    const uint64_t lbg = rowid / R, r = rowid % R;
    float4_t oh[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oh[nb] = (float4_t)0.0f;
    for (uint32_t s = 0; s < a.hot_splits; ++s) {
        const float f = s_hfac[myr][s];
        if (f == 0.0f) continue;
        const float* src = a.hot_o + ((lbg * a.hot_splits + s) * R + r) * HD;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) oh[nb] += f * *(const float4_t*)(src + 16 * nb + 4 * lg);
    }
    const uint64_t lb = lbg / a.kv_heads, g = lbg % a.kv_heads;
    const uint64_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
    uint16_t* o = a.out + ((lb * a.queries + q) * a.q_heads + h) * HD;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        half4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[e] = (_Float16)merge_value(oh[nb][e], rf.Mh, rf.Lh, acc[nb][e] * rf.inv_scl, rf.Mc, rf.Lc);
        *(half4_t*)(o + 16 * nb + 4 * lg) = v;
    }
}

// --------------------------------------------------- log-sum-exp merge
//
// One wave per row (row id lbg*R + r), four rows per work-group: lanes first
// combine the row's splits (lane = split), then each lane merges HD/64 dims.
// Used when there is no cold pool or when the cold output was split over
// several atom ranges.
template <int HD>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
    constexpr int DPT = HD / 64;
    __shared__ float s_hfac[4][kMaxSplits];
    const int tid = threadIdx.x, row = tid / 64, lane = tid % 64;
    const uint64_t rowid = (uint64_t)blockIdx.x * 4 + row;
    if (rowid >= a.total_rows) return; // whole wave: no barrier follows
    const uint32_t R = a.rows_r;
    const uint64_t lbg = rowid / R, r = rowid % R;
    float Mc = -INFINITY, Lc = 0.0f, Mh = -INFINITY, Lh = 0.0f;
    {
        float cm = -INFINITY, cl = 0.0f, hm = -INFINITY, hl = 0.0f;
        if (a.ocp && (uint32_t)lane < a.cold_splits) {
            const uint64_t cb = (lbg * a.cold_splits + lane) * R + r;
            cm = a.cold_m[cb];
            cl = a.cold_l[cb];
        }
        if ((uint32_t)lane < a.hot_splits) {
            const uint64_t hb = (lbg * a.hot_splits + lane) * R + r;
            hm = a.hot_m[hb];
            hl = a.hot_l[hb];
        }
        float f;
        combine_splits(cm, cl, Mc, Lc, f);
        combine_splits(hm, hl, Mh, Lh, f);
        if (lane < kMaxSplits) s_hfac[row][lane] = f;
    }
    __builtin_amdgcn_wave_barrier();
    const int d0 = lane * DPT;
    float oc[DPT], oh[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
        oc[e] = 0.0f;
        oh[e] = 0.0f;
    }
    if (a.ocp) {
        const float* src = a.ocp + rowid * a.n_ar * HD + d0;
        uint32_t ar = 0;
        for (; ar + 4 <= a.n_ar; ar += 4) {
            float v[4][DPT];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < DPT; ++e) v[j][e] = src[(ar + j) * HD + e];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < DPT; ++e) oc[e] += v[j][e];
        }
        for (; ar < a.n_ar; ++ar)
#pragma unroll
            for (int e = 0; e < DPT; ++e) oc[e] += src[ar * HD + e];
    }
    const float* hsrc = a.hot_o + (lbg * a.hot_splits * R + r) * HD + d0;
    for (uint32_t s0 = 0; s0 < a.hot_splits; s0 += 4) {
        float v[4][DPT], fs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t sp = s0 + j;
            fs[j] = sp < a.hot_splits ? s_hfac[row][sp] : 0.0f;
#pragma unroll
            for (int e = 0; e < DPT; ++e) v[j][e] = fs[j] != 0.0f ? hsrc[(uint64_t)sp * R * HD + e] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < DPT; ++e) oh[e] += fs[j] * v[j][e];
    }
    const uint64_t lb = lbg / a.kv_heads, g = lbg % a.kv_heads;
    const uint64_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
    uint16_t* o = a.out + ((lb * a.queries + q) * a.q_heads + h) * HD + d0;
#pragma unroll
    for (int e = 0; e < DPT; ++e)
        o[e] = __builtin_bit_cast(uint16_t, (_Float16)merge_value(oh[e], Mh, Lh, oc[e], Mc, Lc));
}

// ------------------------------------------------ codec check (bit-exact)
__global__ void gather_codes_kernel(const uint4_t* codes, uint64_t n, const uint16_t* dict, uint32_t A,
                                    uint32_t HD, uint32_t* idx, float* coef, uint16_t* atoms, uint32_t* err) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * 4) return;
    const uint64_t i = t / 4;
    const uint32_t k = t % 4;
    const uint4_t cw = codes[i];
    const uint32_t word = k < 2 ? cw[0] : cw[1];
    const uint32_t at = (k & 1) ? word >> 16 : word & 0xFFFFu;
    const uint32_t cword = k < 2 ? cw[2] : cw[3];
    const uint32_t cbits = (k & 1) ? cword >> 16 : cword & 0xFFFFu;
    idx[t] = at;
    coef[t] = h2f_bits(cbits);
    if (at >= A) flag_error(err, kErrAtom);
    for (uint32_t j = 0; j < HD; ++j) atoms[t * HD + j] = at < A ? dict[(uint64_t)at * HD + j] : (uint16_t)0xFFFFu;
}

} // namespace aw
