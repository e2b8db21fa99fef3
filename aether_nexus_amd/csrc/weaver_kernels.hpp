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

#include <type_traits>

namespace aw {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kBlockTokens = 16;      // tokens per block (ModelDims::BLOCK_SIZE)
constexpr uint32_t kRefMask = 0x7FFFFFFFu; // weaver_kernel.metal:145,174
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kColdThreads = 512;
constexpr int kMaxSplits = 64;              // splits per row: the merges combine them lane = split
constexpr uint32_t kMaxHotSplitBlocks = 4096; // hot blocks per split (16 KiB of LDS refs): 4 Mi tokens per sequence


// Error bits written to the engine's device error word.
constexpr uint32_t kErrHotRef = 1u, kErrColdRef = 2u, kErrAtom = 4u;

__device__ inline float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ inline half8_t as_h8(uint4_t v) { return __builtin_bit_cast(half8_t, v); }

typedef short short4_t __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (gfx950): in each group of 16 lanes, lane 4*r + c supplies the
// LDS address of 4 consecutive halves (row r, columns 4c..4c+3 of a 4 x 16 block);
// lane j of the group receives column j, rows 0..3.  p must be 8-byte aligned.
__device__ __forceinline__ short4_t lds_read_tr16(const _Float16* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)p);
}
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// e with 2^(e-1) <= x < 2^e for finite x > 0 (v_frexp_exp_i32_f32), and x * 2^e (v_ldexp_f32).
__device__ inline int exp_of(float x) { return __builtin_amdgcn_frexp_expf(x); }
__device__ inline float pow2f(int e) { return __builtin_amdgcn_ldexpf(1.0f, e); }
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
    uint16_t* ql;         // [L][B][Q][Hq][A] f16, or null
    float* qlf;           // [L][B][Q][Hq][A] fp32, or null (both null: transpose only)
    uint16_t* dt;         // [L][dict_heads][HD][dt_pitch] f16: D^T for the finish (or tiled, below); null: none
    uint32_t dt_pitch;    // A + padding: rows of D^T do not alias one L2 channel
    uint32_t dt_tiled;    // D^T as [group][A/32][HD/16][64 lanes][8 atoms] (finish_rows_kernel's A operand)
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
    uint32_t part_splits; // S of the partial arrays: splits, plus the cold splits when they write values here
    uint32_t refs_cap;   // block refs the launch's LDS holds per split (>= tokens_per_split / 16)
    uint32_t refs_identity; // refs[i] == i for every sequence (a contiguous cache): refs are not read
    uint32_t n_tok_max;  // hot tokens of a sequence (hot_count * 16 unless the request gives fewer)
    uint32_t seq_tokens; // seq_hot counts tokens rather than blocks
    float scale_log2;
    uint64_t hot_blocks, hot_layer, refs_layer;
};

struct ColdArgs {
    const uint16_t* ql;  // q_latent (f16), addressed through the strides below
    const float* qlf;    // or q_latent in fp32 (computed on the device), same strides
    const uint4_t* cold;
    const uint32_t* refs;
    const uint32_t* seq_cold;
    float* part_m; // [lbg][S][R]
    float* part_l;
    float* part_w;   // [lbg][S][R][w_pitch]
    uint32_t w_pitch; // A + padding (rows 16 KiB apart would share L2 channels)
    float* part_amax; // [lbg][S][R]: max_a |bin[a]|
    uint32_t* err;
    uint32_t batch, kv_heads, gqa, rows_r;
    uint32_t hot_count, cold_count, refs_stride, dict_size;
    uint32_t s_tok, s_head; // code (block b, token j, kv head g) = cold[b*16*kv_heads + j*s_tok + g*s_head]
    uint32_t splits, tokens_per_split, n_chunks, n_units;
    uint32_t n_wg; // work items (8 XCD slots x kv heads x unit groups)
    // Which items share an XCD: 0 = the kv heads of one (sequence, chunk, split)
    // (the reference order interleaves their codes in one line); 1 = the row
    // chunks of one (sequence, split, kv head) (head-blocked order: they read the
    // same lines).
    uint32_t chunk_xcd;
    // Bins tiled for finish_rows_kernel: [group][row tile of 16][A/32][2][64 lanes][4],
    // group and group row as the finish numbers them (one split only).
    uint32_t w_tiled, w_rows_per_group, w_dict_heads;
    float scale_log2;
    uint64_t cold_blocks, cold_layer, refs_layer;
    // q_latent element (lb, g, q, j, a) = ql[lb*s_lb + g*s_g + q*s_q + j*s_j + a*s_a]
    uint64_t s_lb, s_g, s_q, s_j, s_a;
    // Value partials instead of bins (OUT, dictionaries of at most 64 Ki elements
    // per head, A % 32 == 0): each split's sum_a bin[a][r] * D[a] goes out with its
    // m and l in the hot kernel's partial layout, as split out_split0 + s of
    // out_splits, for the merge.  D^T comes from the projection in the row-tile
    // finish's order ([L][dict_heads] groups of [A/32][head_dim/16][64 lanes][8
    // atoms]); the bins' f16 hi + lo terms are staged in LDS at byte w_lds_off.
    const uint16_t* dt;
    uint32_t dict_heads, head_dim, out_splits, out_split0, w_lds_off;
    float* out_m;
    float* out_l;
    float* out_o;
};

struct FinishArgs {
    const uint16_t* dt; // D^T [L][dict_heads][HD][dt_pitch]
    uint32_t dt_pitch, w_pitch;
    const float* cold_m;
    const float* cold_l;
    const float* cold_w;
    const float* cold_amax;
    const float* hot_m;
    const float* hot_l;
    const float* hot_o;
    float* ocp; // [lbg*R + r][n_ar][HD] when n_ar > 1 or sep_merge
    uint16_t* out;
    uint32_t batch, queries, q_heads, kv_heads, gqa, rows_r;
    uint32_t dict_size, dict_heads, rows_per_group, tiles_per_group;
    uint32_t cold_splits, hot_splits, n_ar, atoms_per_range;
    // 1: the cold output goes to `ocp` for merge_kernel even with one atom range
    // (the finish then does not wait for the hot kernel).
    uint32_t sep_merge;
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
// q_latent[row][atom] = q[row] . D[atom] over K = HD, written f16 into
// q_latent [L][B][Q][Hq][A] (the layout of the reference's q_latent buffer,
// weaver_kernel.metal:111).  Rows of one group share one dictionary: group =
// (layer, dict head); inside a group row i enumerates (b, q, head) with head
// over Hq (shared dictionary) or over the G heads of kv head dg (per-kv-head
// dictionary).
//
// Work-group = TR rows x TA atoms, 8 waves.  The q rows and dictionary atoms
// of the tile are staged once in LDS (16-byte coalesced loads, all issued
// before any is stored), so the dictionary is read from L2 once per TR rows and
// q once per TA atoms.  Waves form a WR x WA grid; each computes MT x NT tiles
// of 16 x 16 with v_mfma_f32_16x16x32_f16 (lane l, li = l%16, lg = l/16):
//   A[i][k]: atom li of the tile, k = 8*lg .. 8*lg+7  (one 16-byte LDS read)
//   B[k][j]: row li of the tile, the same k               (one 16-byte LDS read)
//   C[i][j]: atoms 4*lg .. 4*lg+3, row li.
// The f16 results go through LDS (the staging area, free once every wave has
// its operands) so q_latent is written in 16-byte pieces of whole rows.
// Every work-group also writes D^T ([HD][dt_pitch], f16) for its atoms and a
// share of the dims (the row blocks split HD) from the staged tile: the finish
// contracts over atoms, and MFMA operands want the contracted index contiguous
// in each lane.
constexpr int kProjThreads = 512;
constexpr int kProjPitch(int HD) { return HD + 8; } // halves per staged row: 16 rows of a read hit distinct banks

// Staged q and dictionary tiles, reused afterwards for the f16 output tile.
inline size_t project_smem_bytes(int HD, int TR, int TA) {
    const size_t in = (size_t)(TR + TA) * kProjPitch(HD) * 2, out = (size_t)TR * (TA + 8) * 2;
    return in > out ? in : out;
}

// D^T of a staged tile of TA atoms (rows of `sd`, pitch P halves), the dims
// split over the grid's row blocks: pieces of 8 atoms, piece p = (atom group
// p / nd, dim d0 + p % nd), written [HD][dt_pitch] or in the row-tile finish's
// lane order.
template <int HD, int TA, int NTH>
__device__ __forceinline__ void write_dt(const ProjArgs& a, const _Float16* sd, int P, uint32_t group, uint32_t atom0) {
    const uint32_t A = a.dict_size;
    if (a.dt == nullptr) return; // no finish reads D^T (the cold kernel writes value partials)
    const uint32_t nrb = gridDim.y, y = blockIdx.y;
    const int d0 = (int)((y * (uint32_t)HD) / nrb), nd = (int)(((y + 1) * (uint32_t)HD) / nrb) - d0;
    const int TP = nd * (TA / 8);
    uint16_t* dt = a.dt + (uint64_t)group * HD * (a.dt_tiled ? A : a.dt_pitch);
    for (int p = (int)threadIdx.x; p < TP; p += NTH) {
        const int d = d0 + p % nd, ag = p / nd;
        const uint32_t at = atom0 + 8 * ag;
        if (at >= A) continue;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = (uint32_t)__builtin_bit_cast(uint16_t, sd[(8 * ag + 2 * e) * P + d]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, sd[(8 * ag + 2 * e + 1) * P + d]) << 16);
        // Tiled: the piece of lane (li = d % 16, lg = (at % 32) / 8) of k-step at / 32, dim block d / 16.
        const uint64_t off = a.dt_tiled ? (((uint64_t)(at / 32) * (HD / 16) + (uint32_t)d / 16) * 64 +
                                           ((at % 32) / 8) * 16 + (uint32_t)d % 16) * 8
                                        : (uint64_t)d * a.dt_pitch + at;
        *(uint4_t*)(dt + off) = (uint4_t){w[0], w[1], w[2], w[3]};
    }
}

template <int HD, int TR, int TA, int WR>
__global__ __launch_bounds__(kProjThreads) void project_kernel(ProjArgs a) {
    constexpr int NW = kProjThreads / 64, P = kProjPitch(HD), KS = HD / 32, PR = HD / 8; // 16-byte pieces per row
    constexpr int WA = NW / WR;
    constexpr int MT = TR / WR / 16, NT = TA / WA / 16;
    static_assert(MT >= 1 && NT >= 1 && MT * WR * 16 == TR && NT * WA * 16 == TA, "tile shape");
    constexpr int PIECES = (TR + TA) * PR, PT = (PIECES + kProjThreads - 1) / kProjThreads;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    _Float16* sq = (_Float16*)smem; // [TR][P] query rows
    _Float16* sd = sq + TR * P;     // [TA][P] dictionary atoms
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const uint32_t group = blockIdx.z;
    const uint32_t l = group / a.dict_heads, dg = group % a.dict_heads;
    const uint32_t atom0 = blockIdx.x * TA, row0 = blockIdx.y * TR;
    const uint32_t A = a.dict_size;
    const uint16_t* dict = a.dict + l * a.dict_layer + (uint64_t)dg * A * HD;
    const bool shared = a.dict_heads == 1;
    // Global q / q_latent row of group row i (clamped into the group).
    auto qrow_of = [&](uint32_t i) -> uint64_t {
        i = min(i, a.rows_per_group - 1u);
        if (shared) return (uint64_t)l * a.rows_per_group + i; // rows of a layer are (b, q, h) in q's order
        const uint32_t bq = i / a.gqa, hh = i % a.gqa;         // (b, q, head hh of kv head dg)
        return ((uint64_t)l * a.batch * a.queries + bq) * a.q_heads + dg * a.gqa + hh;
    };

    // Stage the tile: every load first (clamped rows and atoms), then every store.
    {
        uint4_t v[PT];
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int p = min(tid + k * kProjThreads, PIECES - 1);
            const int r = p / PR, c = p % PR;
            const uint16_t* src = r < TR ? a.q + qrow_of(row0 + r) * HD : dict + (uint64_t)min(atom0 + (uint32_t)(r - TR), A - 1u) * HD;
            v[k] = *(const uint4_t*)(src + 8 * c);
        }
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int p = tid + k * kProjThreads;
            if (p < PIECES) *(uint4_t*)(sq + (p / PR) * P + 8 * (p % PR)) = v[k]; // sd follows sq
        }
    }
    __syncthreads();

    const int wr = wave / WA, wa = wave % WA;
    float4_t acc[MT][NT];
    const bool want = a.ql != nullptr || a.qlf != nullptr;
    if (want) {
        half8_t aop[NT][KS];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < KS; ++j)
                aop[nt][j] = *(const half8_t*)(sd + (wa * (TA / WA) + nt * 16 + li) * P + 32 * j + 8 * lg);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            half8_t bop[KS];
#pragma unroll
            for (int j = 0; j < KS; ++j) bop[j] = *(const half8_t*)(sq + (wr * (TR / WR) + mt * 16 + li) * P + 32 * j + 8 * lg);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                acc[mt][nt] = (float4_t)0.0f;
#pragma unroll
                for (int j = 0; j < KS; ++j) acc[mt][nt] = mfma16x16x32(aop[nt][j], bop[j], acc[mt][nt]);
            }
        }
    }
    write_dt<HD, TA, kProjThreads>(a, sd, P, group, atom0);
    if (a.qlf != nullptr) {
        // fp32 rows straight from the accumulators: a lane holds atoms 4*lg .. +3
        // of row li of each tile (16 contiguous bytes; A % 16 == 0).
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t i = row0 + wr * (TR / WR) + mt * 16 + li;
                const uint32_t at = atom0 + wa * (TA / WA) + nt * 16 + 4 * lg;
                if (i < a.rows_per_group && at < A) *(float4_t*)(a.qlf + qrow_of(i) * A + at) = acc[mt][nt];
            }
    } else if (a.ql != nullptr) {
        constexpr int OP = TA + 8; // halves per staged output row
        __syncthreads(); // every wave is done with the staged q and dictionary
        _Float16* so = sq;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                half4_t h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = (_Float16)acc[mt][nt][e];
                *(half4_t*)(so + (wr * (TR / WR) + mt * 16 + li) * OP + wa * (TA / WA) + nt * 16 + 4 * lg) = h;
            }
        __syncthreads();
        constexpr int OPR = TA / 8, OPIECES = TR * OPR; // 16-byte pieces per row / tile
        for (int p = tid; p < OPIECES; p += kProjThreads) {
            const int r = p / OPR, c = p % OPR;
            const uint32_t i = row0 + r, ao = atom0 + 8 * c;
            if (i < a.rows_per_group && ao < A)
                *(uint4_t*)(a.ql + qrow_of(i) * A + ao) = *(const uint4_t*)(so + r * OP + 8 * c);
        }
    }
}

// ------------------------------------------------------ q . D^T (VALU)
//
// The same projection on the vector ALUs, for few rows per dictionary group.
// Work-group = TA atoms (one per thread) x RB rows: the atoms' dictionary
// rows and the RB q rows are staged in LDS (the same loads-then-stores
// pattern), then each thread forms its atom's RB dot products with
// v_dot2_f32_f16 (two f16 products per instruction, fp32 sums in dim order)
// and writes one value per row: consecutive threads, consecutive atoms, so the
// stores of a row are contiguous.  D^T is written as by project_kernel.
inline size_t project_valu_smem_bytes(int HD, int TA, int RB) {
    return ((size_t)TA * kProjPitch(HD) + (size_t)RB * HD) * 2;
}

template <int HD, int TA, int RB>
__global__ __launch_bounds__(TA) void project_valu_kernel(ProjArgs a) {
    constexpr int P = kProjPitch(HD), PR = HD / 8;
    constexpr int PIECES = (TA + RB) * PR, PT = (PIECES + TA - 1) / TA;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    _Float16* sd = (_Float16*)smem; // [TA][P] dictionary atoms
    _Float16* sq = sd + TA * P;     // [RB][HD] query rows
    const int tid = threadIdx.x;
    const uint32_t group = blockIdx.z;
    const uint32_t l = group / a.dict_heads, dg = group % a.dict_heads;
    const uint32_t atom0 = blockIdx.x * TA, row0 = blockIdx.y * RB;
    const uint32_t A = a.dict_size;
    const uint16_t* dict = a.dict + l * a.dict_layer + (uint64_t)dg * A * HD;
    const bool shared = a.dict_heads == 1;
    auto qrow_of = [&](uint32_t i) -> uint64_t {
        i = min(i, a.rows_per_group - 1u);
        if (shared) return (uint64_t)l * a.rows_per_group + i;
        const uint32_t bq = i / a.gqa, hh = i % a.gqa;
        return ((uint64_t)l * a.batch * a.queries + bq) * a.q_heads + dg * a.gqa + hh;
    };
    {
        uint4_t v[PT];
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int p = min(tid + k * TA, PIECES - 1);
            const int r = p / PR, c = p % PR;
            const uint16_t* src = r < TA ? dict + (uint64_t)min(atom0 + (uint32_t)r, A - 1u) * HD
                                         : a.q + qrow_of(row0 + (uint32_t)(r - TA)) * HD;
            v[k] = *(const uint4_t*)(src + 8 * c);
        }
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int p = tid + k * TA;
            if (p >= PIECES) continue;
            const int r = p / PR, c = p % PR;
            *(uint4_t*)(r < TA ? sd + r * P + 8 * c : sq + (r - TA) * HD + 8 * c) = v[k];
        }
    }
    __syncthreads();
    const bool want = a.ql != nullptr || a.qlf != nullptr;
    if (want) {
        float acc[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r] = 0.0f;
#pragma unroll 4
        for (int c = 0; c < PR; ++c) {
            const half8_t dv = *(const half8_t*)(sd + tid * P + 8 * c);
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const half8_t qv = *(const half8_t*)(sq + r * HD + 8 * c); // one address: a broadcast
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[r] = __builtin_amdgcn_fdot2((half2_t){dv[2 * e], dv[2 * e + 1]},
                                                    (half2_t){qv[2 * e], qv[2 * e + 1]}, acc[r], false);
            }
        }
        const uint32_t at = atom0 + (uint32_t)tid;
        if (at < A) {
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const uint32_t i = row0 + (uint32_t)r;
                if (i >= a.rows_per_group) break;
                if (a.qlf != nullptr) a.qlf[qrow_of(i) * A + at] = acc[r];
                else a.ql[qrow_of(i) * A + at] = __builtin_bit_cast(uint16_t, (_Float16)acc[r]);
            }
        }
    }
    write_dt<HD, TA, TA>(a, sd, P, group, atom0);
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
//      read from the chunk staged in LDS as [token][dim] by transposing loads:
//      ds_read_b64_tr_b16 gives lane li of each 16-lane group one column (dim
//      16*nb+li) of the 4 x 16 block whose rows (tokens 4*lg..4*lg+3, then
//      16+4*lg..) its lanes address, 8 bytes each: 2 loads per 16 dims.
// LDS pitch HD+16 halves (72 words at HD=128, 40 at 64): 16-byte aligned rows for
// the staging stores, and the 16 token rows of one transposing load start on
// 8-word bank groups that cover the 64 banks twice.
//
// A split holds at most kMaxHotSplitBlocks blocks; their refs are staged in
// (dynamic) LDS once.  Every global load of the loop is unconditional (a bad
// ref reads block 0 and the chunk's registers are zeroed before use), so the
// next chunk's loads really stay in flight while the current chunk is computed.
template <int HD, int RT, bool SEPV>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu((RT == 1 && !SEPV) ? 3 : 1))) void hot_kernel(HotArgs a) {
    constexpr int KS = HD / 32, NB = HD / 16, P = HD + 16;
    __shared__ __attribute__((aligned(16))) _Float16 lds[32 * P];
    const int lane = threadIdx.x, li = lane & 15, lg = lane >> 4;
    const uint32_t s = blockIdx.x % a.splits, lbg = blockIdx.x / a.splits;
    const uint32_t g = lbg % a.kv_heads, lb = lbg / a.kv_heads, l = lb / a.batch;
    uint32_t n_tok = a.n_tok_max;
    if (a.seq_hot) {
        const uint32_t sh = a.seq_hot[lb];
        n_tok = min(n_tok, a.seq_tokens ? sh : min(sh, a.hot_count) * kBlockTokens);
    }
    const uint32_t t_begin = s * a.tokens_per_split;
    const uint32_t t_end = min(t_begin + a.tokens_per_split, n_tok);
    const uint32_t R = a.rows_r;

    // The query rows first: their loads then overlap the block refs' below.
    half8_t qop[RT][KS];
    int lim[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const uint32_t r = min(16u * rt + li, R - 1u);
        const uint32_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
        const uint16_t* p = a.q + (((uint64_t)lb * a.queries + q) * a.q_heads + h) * HD;
#pragma unroll
        for (int j = 0; j < KS; ++j) qop[rt][j] = as_h8(*(const uint4_t*)(p + 32 * j + 8 * lg));
        lim[rt] = 16u * rt + li < R ? (a.causal ? (int)n_tok - (int)a.queries + 1 + (int)q : (int)n_tok) : 0;
    }

    // Block refs of this split (at most refs_cap = tokens_per_split / 16 blocks,
    // dynamic LDS sized by the launch), staged once: the loop reads them with LDS
    // loads, which never wait behind the K loads.  An identity table (a
    // contiguous cache) is not read at all: block i of the sequence is block i.
    extern __shared__ uint32_t s_refs[];
    const uint32_t blk0 = t_begin / kBlockTokens;
    const uint32_t n_blk = t_end > t_begin ? (t_end - t_begin + kBlockTokens - 1) / kBlockTokens : 0u;
    if (!a.refs_identity) {
        const uint32_t* refs = a.refs + (uint64_t)l * a.refs_layer + (uint64_t)(lb % a.batch) * a.refs_stride;
        for (uint32_t i = (uint32_t)lane; i < n_blk; i += 64u) s_refs[i] = refs[blk0 + i] & kRefMask;
        __syncthreads();
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
    const uint16_t* vbase = SEPV ? a.hot_v + (uint64_t)l * a.hot_layer : nullptr;
    bool bad = false;

    // The two blocks of chunk c0: this lane's K (and V) pieces, and whether each block is usable.
    auto load_chunk = [&](uint32_t c0, uint4_t (&kr)[2][KS], uint4_t (&vr)[2][KS], bool (&ok)[2]) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const uint32_t bi = (c0 - t_begin) / kBlockTokens + tb;
            const bool in = c0 + 16 * tb < t_end;
            // entries past n_blk: `in` is false
            const uint32_t ref = a.refs_identity ? blk0 + bi : s_refs[min(bi, a.refs_cap - 1u)];
            ok[tb] = in && ref < a.hot_blocks;
            bad |= in && !ok[tb];
            const uint32_t pr = ok[tb] ? ref : 0u;
            const uint64_t rowoff = (((uint64_t)pr * kBlockTokens + li) * a.kv_heads + g) * HD + 8 * lg;
#pragma unroll
            for (int j = 0; j < KS; ++j) kr[tb][j] = *(const uint4_t*)(kbase + rowoff + 32 * j);
            if constexpr (SEPV) {
#pragma unroll
                for (int j = 0; j < KS; ++j) vr[tb][j] = *(const uint4_t*)(vbase + rowoff + 32 * j);
            }
        }
    };

    // Two chunk buffers used in turn (no register copies between iterations, so
    // the wait for a chunk's loads sits right before its first use).
    uint4_t kb[2][2][KS], vb[2][2][KS];
    bool okb[2][2] = {{false, false}, {false, false}};
    const uint32_t last = t_end > t_begin ? t_begin + ((t_end - t_begin - 1) / 32) * 32 : t_begin;
    if (t_begin < t_end) load_chunk(t_begin, kb[0], vb[0], okb[0]);
    // Rows past R: zero query (their lim is 0, so their output is never written).
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        if (16u * rt + li >= R)
#pragma unroll
            for (int j = 0; j < KS; ++j) qop[rt][j] = (half8_t)(_Float16)0;

    auto process = [&](uint32_t c0, uint4_t (&kcur)[2][KS], uint4_t (&vcur)[2][KS], const bool (&okcur)[2]) {
        // Unusable blocks (past the split or a bad ref) become zeros, and so do the
        // lane's token rows past the sequence's end inside its last block: masked
        // scores give p = 0, but 0 * (a stale NaN or inf) would not vanish.
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
            if (!okcur[tb] || c0 + 16u * tb + (uint32_t)li >= n_tok) {
#pragma unroll
                for (int j = 0; j < KS; ++j) {
                    kcur[tb][j] = (uint4_t)0u;
                    vcur[tb][j] = (uint4_t)0u;
                }
            }

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
                *(uint4_t*)(lds + (16 * tb + li) * P + 32 * j + 8 * lg) = SEPV ? vcur[tb][j] : kcur[tb][j];
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

        // O^T += V^T P^T; lane li + 16*lg addresses token 4*lg + li/4, dims 4*(li%4)..+3
        // of each 16-dim block, and receives tokens 4*lg..+3 (then 16+4*lg..+3) of dim 16*nb+li.
        const _Float16* vrow = lds + (4 * lg + (li >> 2)) * P + 4 * (li & 3);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const half8_t vop = __builtin_bit_cast(
                half8_t, __builtin_shufflevector(lds_read_tr16(vrow + 16 * nb), lds_read_tr16(vrow + 16 * P + 16 * nb),
                                                 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) oacc[rt][nb] = mfma16x16x32(vop, pop[rt], oacc[rt][nb]);
        }
    };

    for (uint32_t c0 = t_begin; c0 < t_end; c0 += 64) {
        load_chunk(min(c0 + 32, last), kb[1], vb[1], okb[1]); // the last chunk reloads itself
        process(c0, kb[0], vb[0], okb[0]);
        if (c0 + 32 >= t_end) break;
        // No reload of the last chunk here: with a split of two chunks (one-sequence
        // attention) it was a third of the split's loads (10.77 -> 10.53 us per layer).
        if (c0 + 64 < t_end) load_chunk(c0 + 64, kb[0], vb[0], okb[0]);
        process(c0 + 32, kb[1], vb[1], okb[1]);
    }
    if (bad) flag_error(a.err, kErrHotRef);

    const uint64_t pbase = ((uint64_t)lbg * a.part_splits + s) * R;
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
// LDS: the q_latent table of the RC rows and NP = ceil(RC/2) 64-bit bins per
// atom, each bin holding two rows' sums as 32-bit fixed point; the split's
// block refs.
//   RC = 4, f16 table: one 24-byte record per atom, [bin rows 0-1][bin rows
//     2-3][q_latent rows 0-3], so one address (atom * 24) serves the table read
//     and both bins.  6 * atom mod 64 takes every even bank, so a wave's 64
//     random atoms spread over the bank pairs as they do in separate planes.
//   otherwise: table [A][RC], then planes [NP][A] of bins.  Planes rather than
//     [A][NP]: a wave's 64 random atoms then spread over every bank pair of the
//     LDS (measured on gfx950: ds_add_u64 at random atoms 0.21 cycles per lane
//     and CU in planes, 0.28 with the 16-byte atom stride of [A][2], 0.11 with
//     no bank conflicts).
//
// Integer bins: on gfx950 an LDS ds_add_f32 retires about one lane per 3
// cycles per CU whatever the addresses, ds_add_u64 about one lane per 0.3
// cycles (measured).  A row pair (v0, v1) is added as the 64-bit integer
// v1*2^32 + v0 (v0 sign-extended); sums of such words are exact and decode back
// to (sum v0, sum v1) while each row sum stays inside int32.
//
// Each row r has its own scale 2^F_r, so a peaked row is not quantised on the
// scale of a flat row in the same chunk.  A contribution x = p*c*2^F_r is
// rounded to an integer in one of two ways, chosen per split:
//   narrow (every row's largest planned contribution below 2^18): one FMA with
//     1.5*2^23 rounds to nearest even; for |x| < 2^22 the sum's bit pattern is
//     0x4B400000 + round(x), and the two patterns of a row pair, read as one
//     64-bit word, minus 0x4B4000004B400000 give exactly v1*2^32 + v0;
//   wide (a peaked row, whose largest contributions would otherwise be capped
//     near 2^18, about 18 significant bits): floor(x + 1/2) by
//     v_cvt_flr_i32_f32, exact for any |x| < 2^31, and the word v1*2^32 + v0
//     from the sign of v0; three more VALU operations per row pair.
//
// p = 2^(s - ref_r).  ref_r (integral, log2 units) and F_r come from the
// split's first tile: ref_r = ceil(max score of the tile); F_r keeps the
// planned bound on row r's sum |p*c| over the whole split near 2^28 and the
// tile's largest contribution below 2^18 (narrow) or 2^26 (wide).  The
// work-group then streams every tile with no further synchronisation.  At the
// end, per row, 4 * max|c| * sum_t p + 2 * tokens < 2^31 - 2^27 (the last term
// covers the rounding of each contribution) bounds every bin and every single
// contribution, and a narrow split also needs max p * max|c| < 2^22; together
// they prove the bins exact.  When they fail (scores far above the first
// tile's, coefficients far larger), the split is recomputed exactly and wide:
// a pass for the per-row maxima, a pass for the exact bounds, a pass for the bins.
//
// Code loads.  BUF (a layer's pool of at most kColdWindow bytes): buffer loads
// through a resource whose base is the item's kv head in the layer's pool; the
// staged block refs are byte offsets (ref * block bytes) and a bad ref or a
// token past the split becomes kBadCodeOff, which lies past the resource's
// range, so the load returns the all-zero code.  Otherwise 64-bit addresses,
// bad refs reading g_zero_code.  Every load of the streaming loop is
// unconditional (prefetches past the split re-read its last tile), so the
// compiler can count loads in flight and the PD-deep ring really prefetches.
// Tiles wholly inside the split, in a split without bad refs, are consumed
// without per-token masks; the split's last partial tile masks p to zero for
// tokens that read the zero code.
//
// Items that read the same lines run on one XCD (work-groups are dealt
// round-robin over the 8 XCDs), so each line comes from HBM once per XCD L2: in
// the reference order the kv heads of one (sequence, chunk, split), whose
// 16-byte codes interleave in 128-byte lines; in the head-blocked order the row
// chunks of one (sequence, split, kv head), which read the same codes.
// All-zero code read by tokens behind a bad ref on the 64-bit address path;
// global (not constant) memory, so every code load stays a global load.
__device__ __attribute__((aligned(16))) uint4_t g_zero_code = {0u, 0u, 0u, 0u};

constexpr uint32_t kBadCodeOff = 0xFFFF0000u;         // staged offset of a token without a code
constexpr uint64_t kColdWindow = kBadCodeOff;         // largest layer pool (bytes) the buffer loads cover
constexpr uint32_t kColdRefPad = 16;                  // staged refs are padded to whole wave tiles
constexpr uint32_t kBufferWord3 = 0x00020000u;        // gfx9 buffer resource word 3 (32-bit data format)
constexpr uint32_t kColdRec = 24;                     // bytes of an RC = 4 f16 atom record
constexpr uint32_t kNoHot = ~0u;                      // no atom hot enough for private bins
constexpr uint32_t kHotMin = 64;                      // plan samples (of 4096) that make an atom hot

// LDS of the plan histogram / the hot atom's private bins, and its offset after
// the tables (tab bytes), the staged refs (n_ref) and the reduction slots (nred floats).
__host__ __device__ constexpr size_t cold_hp_bytes(uint32_t A, int NP) {
    return (((size_t)A * 2 > (size_t)kColdThreads * NP * 8 ? (size_t)A * 2 : (size_t)kColdThreads * NP * 8) + 15) &
           ~(size_t)15;
}
__host__ __device__ constexpr size_t cold_hp_offset(size_t tab, uint32_t n_ref, uint32_t nred) {
    return (tab + (((size_t)n_ref + 3) & ~(size_t)3) * 4 + (size_t)nred * 4 + 15) & ~(size_t)15;
}

typedef uint16_t ushort2_t __attribute__((ext_vector_type(2)));
typedef int16_t short2_t __attribute__((ext_vector_type(2)));

constexpr float kMagic = 12582912.0f;                 // 1.5 * 2^23
constexpr uint64_t kMagic2 = 0x4B4000004B400000ull;   // two magic patterns

// floor(x) as an int32 in one instruction (the compiler emits v_floor_f32 +
// v_cvt_i32_f32 for the same expression).  Saturates outside int32.
__device__ __forceinline__ int32_t cvt_flr_i32(float x) {
    int32_t r;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
// The bins' bound: no bin of a row may reach it (2^31 - 2^27, slack for the
// float arithmetic of the bound itself).
constexpr float kBinLimit = 2013265920.0f;

// One work item `wg` (its index in the full grid of work items; the kernel below
// walks them persistently, one work-group per CU slot).
//
// Tokens are dealt to waves in wave tiles of 64*CPT consecutive tokens: wave w
// takes tiles w, w + NW, w + 2*NW, ... (so the first NW tiles, the planning
// sample, cover the split's first NT*CPT tokens).  The assignment is static, so
// every float sum runs in the same order on every call.  OUT: value partials
// (a.out_*) instead of bins.
template <int RC, int CPT, int PD, bool POW2, bool QF32, bool BUF, bool OUT>
__device__ __forceinline__ void cold_unit(const ColdArgs& a, uint32_t wg) {
    using QT = std::conditional_t<QF32, float, _Float16>; // q_latent table element
    constexpr int NT = kColdThreads, NW = NT / 64, NP = (RC + 1) / 2;
    constexpr int NB = RC + 2;      // values of the end-of-split reductions
    constexpr int NR = 2 * RC + 4;  // LDS slots per wave: the plan's (max, sum) pairs, max|c|, bad refs, hot key
    constexpr uint32_t WT = 64u * CPT; // tokens of one wave tile
    constexpr uint32_t RPT = WT / 16;  // block refs of one wave tile
    static_assert(kColdRefPad % RPT == 0, "ref padding");
    constexpr bool REC = RC == 4 && !QF32;
    constexpr uint32_t kBad = BUF ? kBadCodeOff : ~0u;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // uniform, so tile branches stay scalar
    // Work-groups are dealt round-robin over the 8 XCDs (x = wg % 8); the items
    // that read the same code lines get one x and consecutive slots k, so they run
    // on one XCD at about the same time and its L2 fetches each line once.
    const uint32_t x = wg % 8u, k = wg / 8u;
    uint32_t g, s, c, lb;
    if (a.chunk_xcd) {
        // p = (sequence, split, kv head): its n_chunks row chunks share XCD p % 8.
        c = k % a.n_chunks;
        const uint32_t p = (k / a.n_chunks) * 8u + x;
        if (p >= a.n_units) return; // n_units counts (sequence, split, kv head) here
        g = p % a.kv_heads;
        const uint32_t ls = p / a.kv_heads;
        s = ls % a.splits;
        lb = ls / a.splits;
    } else {
        g = k % a.kv_heads;
        const uint32_t u = (k / a.kv_heads) * 8u + x;
        if (u >= a.n_units) return;
        s = u % a.splits;
        const uint32_t uc = u / a.splits;
        c = uc % a.n_chunks;
        lb = uc / a.n_chunks;
    }
    const uint32_t l = lb / a.batch;
    const uint64_t lbg = (uint64_t)lb * a.kv_heads + g;
    const uint32_t A = a.dict_size, R = a.rows_r;
    uint32_t nc = a.cold_count;
    if (a.seq_cold) nc = min(nc, a.seq_cold[lb]);
    const uint32_t n_tok = nc * kBlockTokens;
    const uint32_t t_begin = s * a.tokens_per_split;
    const uint32_t t_end = min(t_begin + a.tokens_per_split, n_tok);
    const uint64_t pbase = (lbg * a.splits + s) * R;

    // Value partials: split out_split0 + s of the merge's partial arrays.
    const uint64_t obase = (lbg * a.out_splits + a.out_split0 + s) * R;
    if (t_begin >= t_end) {
        if (tid < RC) {
            const uint32_t r = c * RC + tid;
            if (r < R) {
                if constexpr (OUT) {
                    a.out_m[obase + r] = -INFINITY;
                    a.out_l[obase + r] = 0.0f;
                } else {
                    a.part_m[pbase + r] = -INFINITY;
                    a.part_l[pbase + r] = 0.0f;
                    a.part_amax[pbase + r] = 0.0f;
                }
            }
        }
        return;
    }

    const uint32_t qtab_bytes = (A * RC * (uint32_t)sizeof(QT) + 15) & ~15u;
    const uint32_t tab_bytes = REC ? A * kColdRec : qtab_bytes + A * NP * 8u;
    const uint32_t n_blk = (t_end - t_begin + 15) / 16; // t_begin is a multiple of 16
    const uint32_t n_wt = (t_end - t_begin + WT - 1) / WT;
    const uint32_t n_ref = n_wt * RPT;                   // staged refs, padded to whole wave tiles
    QT* qtab = (QT*)smem;                                  // [A][RC] (not REC)
    uint64_t* bins = (uint64_t*)(smem + qtab_bytes);       // [NP][A] (not REC)
    uint32_t* sref = (uint32_t*)(smem + tab_bytes);        // [n_ref]: staged block refs, kBad = none
    float* red = (float*)(sref + ((n_ref + 3) & ~3u));    // [NW][NR]
    // Plan histogram of atom indices (two 16-bit counters per word), then each
    // lane's private bins of the split's hottest atom ([lane][NP] u64).
    uint32_t* hp = (uint32_t*)(smem + cold_hp_offset(tab_bytes, n_ref, NW * NR));
    const uint32_t hp_words = cold_hp_bytes(A, NP) / 4;
    // q_latent values of atom `at` (RC of them) and its bin of row pair pp.
    auto qrow = [&](uint32_t at) -> const QT* {
        if constexpr (REC) return (const QT*)(smem + at * kColdRec + 16u);
        else return qtab + at * RC;
    };
    auto binp = [&](uint32_t at, int pp) -> uint64_t* {
        if constexpr (REC) return (uint64_t*)(smem + at * kColdRec + 8u * (uint32_t)pp);
        else return bins + (uint32_t)pp * A + at;
    };

    const uint4_t* cold = a.cold + (uint64_t)l * a.cold_layer;
    const uint64_t blk_codes = (uint64_t)kBlockTokens * a.kv_heads;
    const uint32_t* grefs = a.refs + (uint64_t)l * a.refs_layer + (uint64_t)(lb % a.batch) * a.refs_stride +
                            a.hot_count + t_begin / 16;
    const float sl = a.scale_log2;
    // Token slot of this lane inside its block: wave tiles start on block boundaries.
    const uint32_t lane_tok = (uint32_t)lane & 15u;
    const uint32_t lane_off = BUF ? lane_tok * a.s_tok * 16u : 0u;
    __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)0, (short)0, 0, (int)kBufferWord3);
    if constexpr (BUF) {
        const uint64_t head0 = (uint64_t)g * a.s_head; // codes before this kv head's first code
        const uint64_t span = a.cold_blocks * blk_codes * 16u - head0 * 16u;
        rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)(cold + head0), (short)0, (int)(uint32_t)min(span, kColdWindow),
                                                 (int)kBufferWord3);
    }
    // Staged entry of block ref `ref` (kBad when outside the pool).
    auto stage_ref = [&](uint32_t ref) -> uint32_t {
        ref &= kRefMask;
        if (ref >= a.cold_blocks) return kBad;
        return BUF ? ref * (uint32_t)(blk_codes * 16u) : ref;
    };
    // The code of this lane's token in the block of staged entry e.
    auto code_at = [&](uint32_t e) -> uint4_t {
        if constexpr (BUF) {
            return __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(e + lane_off), 0, 0);
        } else {
            const uint4_t* p = e != ~0u ? cold + (uint64_t)e * blk_codes + lane_tok * a.s_tok + (uint64_t)g * a.s_head
                                        : &g_zero_code;
            return *p;
        }
    };
    // Staged entries of wave tile `tile` (< n_wt) from LDS, and their codes.
    auto tile_refs = [&](uint32_t tile, uint32_t (&rb)[CPT]) {
        const uint32_t* sp = sref + tile * RPT + ((uint32_t)lane >> 4);
#pragma unroll
        for (int kk = 0; kk < CPT; ++kk) rb[kk] = sp[4 * kk];
    };
    auto tile_codes = [&](const uint32_t (&rb)[CPT], uint4_t (&buf)[CPT]) {
#pragma unroll
        for (int kk = 0; kk < CPT; ++kk) buf[kk] = code_at(rb[kk]);
    };
    auto load_tile = [&](uint32_t tile, uint4_t (&buf)[CPT], bool (&ok)[CPT]) {
        uint32_t rb[CPT];
        tile_refs(min(tile, n_wt - 1u), rb);
        tile_codes(rb, buf);
#pragma unroll
        for (int kk = 0; kk < CPT; ++kk) ok[kk] = tile < n_wt && rb[kk] != kBad;
    };
    // Atom indices of a code word, always inside the tables: a power-of-two
    // dictionary masks them (any bit outside the mask is recorded in `oob`),
    // others are clamped (recorded when clamping changed them).
    auto atoms = [&](const uint4_t cw, uint32_t (&ia)[4], uint32_t& oob) {
        if constexpr (POW2) {
            const uint32_t am = (A - 1u) & 0xFFFFu; // A <= 65536: indices stay 16-bit (24-bit products)
            ia[0] = cw[0] & am;
            ia[1] = (cw[0] >> 16) & am;
            ia[2] = cw[1] & am;
            ia[3] = (cw[1] >> 16) & am;
            oob |= cw[0] | cw[1];
        } else {
            const uint32_t r0 = cw[0] & 0xFFFFu, r1 = cw[0] >> 16, r2 = cw[1] & 0xFFFFu, r3 = cw[1] >> 16;
            oob = max(oob, max(max(r0, r1), max(r2, r3)));
            ia[0] = min(r0, A - 1u);
            ia[1] = min(r1, A - 1u);
            ia[2] = min(r2, A - 1u);
            ia[3] = min(r3, A - 1u);
        }
    };
    auto coef = [](const uint4_t cw, int j) -> _Float16 {
        return __builtin_bit_cast(_Float16, (uint16_t)(cw[2 + j / 2] >> (16 * (j % 2))));
    };
    // Unscaled score sums of one code for the RC rows: sum_k c_k * q_latent[idx_k][r].
    auto score = [&](const uint4_t cw, const uint32_t (&ia)[4], float (&sc)[RC]) {
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) sc[rr] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float cj = (float)coef(cw, j);
            const QT* qp = qrow(ia[j]);
            if constexpr (RC == 4 && QF32) {
                const float4_t qv = *(const float4_t*)qp;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) sc[rr] = fmaf(cj, qv[rr], sc[rr]);
            } else if constexpr (RC == 4) {
                const half4_t qv = *(const half4_t*)qp;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) sc[rr] = fmaf(cj, (float)qv[rr], sc[rr]);
            } else {
#pragma unroll
                for (int rr = 0; rr < RC; ++rr) sc[rr] = fmaf(cj, (float)qp[rr], sc[rr]);
            }
        }
    };
    // max |c| of a code, as packed f16 magnitudes (monotone as integers).
    auto cmax_bits = [](const uint4_t cw) -> uint32_t {
        const uint32_t m0 = cw[2] & 0x7FFF7FFFu, m1 = cw[3] & 0x7FFF7FFFu;
        const uint32_t lo = max(m0 & 0xFFFFu, m1 & 0xFFFFu), hi = max(m0 >> 16, m1 >> 16);
        return max(lo, hi);
    };
    auto cmax_f = [&](const uint4_t cw) { return (float)__builtin_bit_cast(_Float16, (uint16_t)cmax_bits(cw)); };

    // Work-group sums/maxima of NB per-lane values (one barrier pair).
    auto wg_reduce = [&](float (&v)[NB], const bool (&is_max)[NB]) {
        __syncthreads(); // previous readers of `red` are done
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float w = is_max[i] ? wave_max(v[i]) : wave_sum(v[i]);
            if (lane == 0) red[wave * NR + i] = w;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            float acc = is_max[i] ? -INFINITY : 0.0f;
            for (int w = 0; w < NW; ++w) acc = is_max[i] ? fmaxf(acc, red[w * NR + i]) : acc + red[w * NR + i];
            v[i] = acc;
        }
    };

    // Set-up loads, oldest first, so that waiting for one never waits for the
    // code loads behind it: the first SR block refs and the first q_latent chunk
    // of each thread, then the refs of the ring's first tiles, then their codes.
    constexpr int SR = 4; // block refs per thread loaded up front (splits of <= 64*NT blocks)
    uint32_t srg[SR];
#pragma unroll
    for (int j = 0; j < SR; ++j) srg[j] = grefs[min(tid + (uint32_t)j * NT, n_blk - 1)];
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
    // Atom-contiguous rows (s_a == 1, q_latent's layout) load as 16-byte pieces of
    // 8 f16 (or 4 fp32) atoms per row, interleaved into the table in registers.
    const bool qvec = QF32 || (a.s_a == 1 && (A % 8) == 0 && ((uintptr_t)a.ql & 15u) == 0);
    constexpr uint32_t QPA = QF32 ? 4u : 8u; // atoms per 16-byte piece
    uint4_t qw[RC];
    if (qvec) {
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            const uint64_t at = rbase[rr] + (uint64_t)min((uint32_t)tid, A / QPA - 1) * QPA;
            qw[rr] = QF32 ? *(const uint4_t*)(a.qlf + at) : *(const uint4_t*)(a.ql + at);
        }
    }
    // fp32 table: piece a4 of every row (4 atoms) into [A][RC].
    auto put_qf = [&](uint32_t a4, uint4_t (&w)[RC]) {
        uint4_t v[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) v[rr] = rok[rr] ? w[rr] : (uint4_t)0u;
        if constexpr (RC == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) *(uint4_t*)(qtab + (a4 * 4 + e) * 4) = (uint4_t){v[0][e], v[1][e], v[2][e], v[3][e]};
        } else if constexpr (RC == 2) {
            // atoms 4*a4 .. +3 x rows 0, 1: two 16-byte stores
            *(uint4_t*)(qtab + a4 * 8) = (uint4_t){v[0].x, v[1].x, v[0].y, v[1].y};
            *(uint4_t*)(qtab + a4 * 8 + 4) = (uint4_t){v[0].z, v[1].z, v[0].w, v[1].w};
        } else {
            *(uint4_t*)(qtab + a4 * 4) = v[0]; // one row: the piece as it is
        }
    };
    auto put_q = [&](uint32_t a8, uint4_t (&w)[RC]) {
#pragma unroll
        for (int rr = 0; rr < RC; ++rr)
            if (!rok[rr]) w[rr] = (uint4_t)0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            _Float16 hv[RC];
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) hv[rr] = __builtin_bit_cast(_Float16, (uint16_t)(w[rr][e / 2] >> (16 * (e % 2))));
            if constexpr (QF32) {
                (void)hv; // the f16 table only
            } else if constexpr (RC == 4) {
                half4_t v4 = {hv[0], hv[1], hv[2], hv[3]};
                *(half4_t*)qrow(a8 * 8 + e) = v4;
            } else {
#pragma unroll
                for (int rr = 0; rr < RC; ++rr) qtab[(a8 * 8 + e) * RC + rr] = hv[rr];
            }
        }
    };

    // Ring of PD wave tiles of codes in flight per wave; slot d holds tile tl[d].
    // The first fill takes its refs from global memory (the LDS copy is staged
    // below); slot 0's validity feeds the plan.
    uint4_t ring[PD][CPT];
    bool rv0[CPT];
    uint32_t tl[PD];
    {
        uint32_t rg[PD][CPT];
#pragma unroll
        for (int d = 0; d < PD; ++d) {
            tl[d] = (uint32_t)(wave + d * NW);
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk) {
                const uint32_t t = t_begin + tl[d] * WT + (uint32_t)kk * 64u + (uint32_t)lane;
                rg[d][kk] = grefs[min((t - t_begin) >> 4, n_blk - 1)];
            }
        }
#pragma unroll
        for (int d = 0; d < PD; ++d) {
            uint32_t rb[CPT];
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk) {
                const uint32_t t = t_begin + tl[d] * WT + (uint32_t)kk * 64u + (uint32_t)lane;
                rb[kk] = t < t_end ? stage_ref(rg[d][kk]) : kBad;
                if (d == 0) rv0[kk] = rb[kk] != kBad;
            }
            tile_codes(rb, ring[d]);
        }
    }
    // Tables into LDS: q_latent rows of this chunk (rows past R are zero) and the
    // split's block refs, resolved once so code addresses come from LDS.
    if constexpr (QF32) {
        if ((uint32_t)tid < A / 4) put_qf(tid, qw);
        for (uint32_t a4 = tid + NT; a4 < A / 4; a4 += NT) {
            uint4_t w[RC];
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) w[rr] = *(const uint4_t*)(a.qlf + rbase[rr] + (uint64_t)a4 * 4);
            put_qf(a4, w);
        }
    } else if (qvec) {
        if ((uint32_t)tid < A / 8) put_q(tid, qw);
        for (uint32_t a8 = tid + NT; a8 < A / 8; a8 += NT) {
            uint4_t w[RC];
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) w[rr] = *(const uint4_t*)(a.ql + rbase[rr] + (uint64_t)a8 * 8);
            put_q(a8, w);
        }
    } else {
        for (uint32_t at = tid; at < A; at += NT) {
            _Float16 hv[RC];
#pragma unroll
            for (int rr = 0; rr < RC; ++rr)
                hv[rr] = __builtin_bit_cast(_Float16, rok[rr] ? a.ql[rbase[rr] + (uint64_t)at * a.s_a] : (uint16_t)0);
            if constexpr (REC) {
                *(half4_t*)qrow(at) = (half4_t){hv[0], hv[1], hv[2], hv[3]};
            } else {
#pragma unroll
                for (int rr = 0; rr < RC; ++rr) qtab[at * RC + rr] = hv[rr];
            }
        }
    }
    bool bad = false; // a bad ref in the split (recorded, and its tokens masked)
    auto put_ref = [&](uint32_t i, uint32_t ref) {
        uint32_t e = kBad;
        if (i < n_blk) {
            e = stage_ref(ref);
            if (e == kBad) {
                flag_error(a.err, kErrColdRef);
                bad = true;
            }
        }
        sref[i] = e;
    };
#pragma unroll
    for (int j = 0; j < SR; ++j)
        if (tid + (uint32_t)j * NT < n_ref) put_ref(tid + j * NT, srg[j]);
    for (uint32_t i = tid + SR * NT; i < n_ref; i += NT) put_ref(i, i < n_blk ? grefs[i] : 0u);
    for (uint32_t at = tid; at < A; at += NT)
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) *binp(at, pp) = 0ull;
    for (uint32_t i = tid; i < hp_words; i += NT) hp[i] = 0u;
    __syncthreads(); // tables, refs, bins and the histogram ready

    // Plan from the first NW tiles (the ring's slot 0 of every wave): per row the
    // pair (max scaled score m, sum over tokens of 4*max|c|*2^(s - m)), combined
    // over lanes and waves like log-sum-exp partials, plus max |c|.
    float ref[RC];
    int F[RC]; // per-row fixed-point scale 2^F_r
    bool wide = false; // contributions rounded by v_cvt_flr_i32_f32 instead of the 2^22-range FMA
    bool any_bad = false;
    // The split's hottest atom (REC layout only): its adds go to per-lane private
    // bins instead of one LDS address, then one add per wave.  Integer sums, so
    // the bins are the same bits either way.
    uint32_t hot = kNoHot;
    {
        const uint32_t n_tiles = (t_end - t_begin + NT * CPT - 1) / (NT * CPT); // plan tiles of NT*CPT tokens
        float scs[CPT][RC], cm[CPT];
        float m[RC], w[RC], cmw = 0.0f;
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) m[rr] = -INFINITY;
        uint32_t hkey = 0; // (largest plan count of an atom) << 16 | that atom
#pragma unroll
        for (int kk = 0; kk < CPT; ++kk) {
            uint32_t ia[4];
            uint32_t dummy = 0;
            atoms(ring[0][kk], ia, dummy);
            score(ring[0][kk], ia, scs[kk]);
            if (rv0[kk])
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // The last add to an atom returns its final count - 1.
                    const uint32_t sh = 16u * (ia[j] & 1u);
                    const uint32_t old = __hip_atomic_fetch_add(hp + (ia[j] >> 1), 1u << sh, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_WORKGROUP);
                    hkey = max(hkey, ((((old >> sh) & 0xFFFFu) + 1u) << 16) | ia[j]);
                }
            cm[kk] = rv0[kk] ? cmax_f(ring[0][kk]) : 0.0f;
            cmw = fmaxf(cmw, cm[kk]);
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) {
                scs[kk][rr] *= sl;
                if (rv0[kk]) m[rr] = fmaxf(m[rr], scs[kk][rr]);
            }
        }
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            float acc = 0.0f;
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk) acc += cm[kk] * fast_exp2(scs[kk][rr] - (rv0[kk] ? m[rr] : scs[kk][rr]));
            // Onto the wave's maximum.
            const float mw = wave_max(m[rr]);
            w[rr] = wave_sum(m[rr] == -INFINITY ? 0.0f : 4.0f * acc * fast_exp2(m[rr] - mw));
            m[rr] = mw;
        }
        cmw = wave_max(cmw);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) hkey = max(hkey, (uint32_t)__shfl_xor((int)hkey, o));
        const bool wave_bad = __builtin_amdgcn_ballot_w64(bad) != 0ull;
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) {
                red[wave * NR + 2 * rr] = m[rr];
                red[wave * NR + 2 * rr + 1] = w[rr];
            }
            red[wave * NR + 2 * RC] = cmw;
            red[wave * NR + 2 * RC + 1] = wave_bad ? 1.0f : 0.0f;
            ((uint32_t*)red)[wave * NR + 2 * RC + 2] = hkey;
        }
        __syncthreads();
        float plan[RC], cmax0 = 0.0f;
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            float M = -INFINITY;
            for (int v = 0; v < NW; ++v) M = fmaxf(M, red[v * NR + 2 * rr]);
            ref[rr] = M == -INFINITY ? 0.0f : ceilf(M);
            float L = 0.0f;
            for (int v = 0; v < NW; ++v) {
                const float mv = red[v * NR + 2 * rr];
                L += mv == -INFINITY ? 0.0f : red[v * NR + 2 * rr + 1] * fast_exp2(mv - ref[rr]);
            }
            plan[rr] = L;
        }
        uint32_t hk = 0;
        for (int v = 0; v < NW; ++v) {
            cmax0 = fmaxf(cmax0, red[v * NR + 2 * RC]);
            any_bad |= red[v * NR + 2 * RC + 1] != 0.0f;
            hk = max(hk, ((const uint32_t*)red)[v * NR + 2 * RC + 2]);
        }
        if (REC && (hk >> 16) >= kHotMin) hot = hk & 0xFFFFu;
        // p <= 1 in the first tile: its contributions stay below 2^18 (narrow) or 2^26 (wide).
        const int Fm = cmax0 > 0.0f ? 18 - exp_of(cmax0) : 100;
        int Fs[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            // Bound on row rr's sum |p*c| over the split, if tiles are alike.
            const float pl = plan[rr] * (float)n_tiles;
            Fs[rr] = pl > 0.0f ? 28 - exp_of(pl) : 100;
            wide |= Fs[rr] > Fm;
        }
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) F[rr] = min(100, max(-100, min(Fs[rr], wide ? Fm + 8 : Fm)));
    }
    // Wave tiles below n_full hold only tokens with codes.
    const uint32_t n_full = any_bad ? 0u : (t_end - t_begin) / WT;

    float lpart[RC];
    uint32_t oob = 0;
    bool exact = false;
    // Attempt 0 streams narrow with the prefetching ring, unless the plan found a
    // peaked row (wide), which goes straight to attempt 1: the exact recompute,
    // streamed wide.  Unrolled, so each attempt holds one streaming loop and the
    // ring's registers are dead in attempt 1.
#pragma unroll
    for (int attempt = 0; attempt < 2; ++attempt) {
        if (attempt) {
            for (uint32_t at = tid; at < A; at += NT)
#pragma unroll
                for (int pp = 0; pp < NP; ++pp) *binp(at, pp) = 0ull;
            __syncthreads(); // bins zeroed before any wave adds
        }
        if (attempt > 0 || !wide) {
        // Stream the split into the bins.  Each slot, once consumed, is refilled
        // with the wave's tile PD*NW further on; slot 0 always holds the wave's
        // earliest tile, so once it is past the end the wave is done.
        float rf[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            lpart[rr] = 0.0f;
            rf[rr] = (float)F[rr] - ref[rr];
        }
        // max |c| as two packed accumulators of f16 bit patterns: the unsigned
        // maximum holds the largest negative pattern if any (else the largest
        // positive), the signed maximum the largest positive (else the largest
        // negative); their magnitudes' maximum is max |c|.
        ushort2_t cmu = (ushort2_t)(uint16_t)0;
        short2_t cmi = (short2_t)(int16_t)0x8000;
        float pmx = 0.0f; // largest p * 2^F_r (narrow splits)
        const bool wide_run = attempt > 0;
        // This lane's private bins of the hot atom (its own [NP] u64; only it touches them).
        uint64_t* priv_me = (uint64_t*)hp + (uint32_t)tid * NP;
        if (hot != kNoHot)
#pragma unroll
            for (int pp = 0; pp < NP; ++pp) priv_me[pp] = 0ull;
        // One code: scores, p (zero for a token without a code when MASKED), bins
        // (the hot atom's go to this lane's private bins; kNoHot matches no atom).
        auto consume = [&](const uint4_t cw, const bool ok, auto masked, auto wide_t) {
            constexpr bool MASKED = decltype(masked)::value;
            constexpr bool WIDE = decltype(wide_t)::value;
            uint32_t ia[4];
            atoms(cw, ia, oob);
            float sc[RC];
            score(cw, ia, sc);
            // Coefficient words copied out first: this compiler's __builtin_bit_cast
            // of a vector element reads element 0.
            const uint32_t w2 = cw[2], w3 = cw[3];
            cmu = __builtin_elementwise_max(cmu, __builtin_elementwise_max(__builtin_bit_cast(ushort2_t, w2),
                                                                           __builtin_bit_cast(ushort2_t, w3)));
            cmi = __builtin_elementwise_max(cmi, __builtin_elementwise_max(__builtin_bit_cast(short2_t, w2),
                                                                           __builtin_bit_cast(short2_t, w3)));
            float ps[RC]; // p * 2^F_r
#pragma unroll
            for (int rr = 0; rr < RC; ++rr) {
                const float p = fast_exp2(fmaf(sc[rr], sl, rf[rr]));
                ps[rr] = (!MASKED || ok) ? p : 0.0f;
                lpart[rr] += ps[rr];
            }
            if constexpr (!WIDE) {
                if constexpr (RC == 4) pmx = fmaxf(pmx, fmaxf(fmaxf(ps[0], ps[1]), fmaxf(ps[2], ps[3])));
                else if constexpr (RC == 2) pmx = fmaxf(pmx, fmaxf(ps[0], ps[1]));
                else pmx = fmaxf(pmx, ps[0]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float cj = (float)coef(cw, j);
                uint64_t* bb = binp(ia[j], 0); // plane pp at bb + pp (REC) in both cases
                if constexpr (REC) bb = ia[j] == hot ? priv_me : bb;
#pragma unroll
                for (int pp = 0; pp < NP; ++pp) {
                    uint64_t wv;
                    if constexpr (WIDE) {
                        const int32_t v0 = cvt_flr_i32(fmaf(ps[2 * pp], cj, 0.5f));
                        const int32_t v1 =
                            (2 * pp + 1 < RC) ? cvt_flr_i32(fmaf(ps[min(2 * pp + 1, RC - 1)], cj, 0.5f)) : 0;
                        wv = ((uint64_t)(uint32_t)(v1 + (v0 >> 31)) << 32) | (uint32_t)v0;
                    } else {
                        const uint32_t b0 = __builtin_bit_cast(uint32_t, fmaf(ps[2 * pp], cj, kMagic));
                        const uint32_t b1 = (2 * pp + 1 < RC)
                                                ? __builtin_bit_cast(uint32_t, fmaf(ps[min(2 * pp + 1, RC - 1)], cj, kMagic))
                                                : 0x4B400000u;
                        wv = (((uint64_t)b1 << 32) | b0) - kMagic2;
                    }
                    __hip_atomic_fetch_add(REC ? bb + pp : binp(ia[j], pp), wv, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        };
        if (!wide_run) {
            while (tl[0] < n_wt) {
#pragma unroll
                for (int d = 0; d < PD; ++d) {
                    const uint32_t nt = tl[d] + (uint32_t)(PD * NW);
                    uint32_t rnext[CPT]; // refs of the slot's next tile, read before this slot's atomics
                    tile_refs(min(nt, n_wt - 1u), rnext);
                    if (tl[d] < n_full) { // uniform; no global loads inside
#pragma unroll
                        for (int kk = 0; kk < CPT; ++kk)
                            consume(ring[d][kk], true, std::false_type{}, std::false_type{});
                    } else if (tl[d] < n_wt) {
                        uint32_t rcur[CPT];
                        tile_refs(tl[d], rcur);
#pragma unroll
                        for (int kk = 0; kk < CPT; ++kk)
                            consume(ring[d][kk], rcur[kk] != kBad, std::true_type{}, std::false_type{});
                    }
                    tile_codes(rnext, ring[d]); // unconditional: past the end they re-read the last tile
                    tl[d] = nt;
                }
            }
        } else {
            // Wide splits (peaked rows, or the exact recompute): a plain tile loop
            // with one tile in flight, so that its registers stay within those of
            // the prefetching loop above.
            for (uint32_t tile = wave; tile < n_wt; tile += NW) {
                uint4_t cur[CPT];
                bool curv[CPT];
                load_tile(tile, cur, curv);
#pragma unroll
                for (int kk = 0; kk < CPT; ++kk) consume(cur[kk], curv[kk], std::true_type{}, std::true_type{});
            }
        }
        if (REC && hot != kNoHot) {
            // The private bins into the hot atom's bins: one add per wave.
#pragma unroll
            for (int pp = 0; pp < NP; ++pp) {
                uint64_t s = priv_me[pp];
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
                if (lane == 0) __hip_atomic_fetch_add(binp(hot, pp), s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        uint32_t cmx_bits;
        {
            const uint32_t mi = max((uint32_t)(uint16_t)cmi.x & 0x7FFFu, (uint32_t)(uint16_t)cmi.y & 0x7FFFu);
            const uint32_t mu = max((uint32_t)cmu.x & 0x7FFFu, (uint32_t)cmu.y & 0x7FFFu);
            cmx_bits = max(mu, mi);
        }
        const float cmx = (float)__builtin_bit_cast(_Float16, (uint16_t)cmx_bits);
        // Overflow proof, per row: every |bin| <= sum over its contributions (|p*c|*2^F_r + 1/2)
        // <= 4*max|c|*sum_t p*2^F_r + 2*tokens, and so is every single contribution; a narrow
        // split's contributions |p*c|*2^F_r <= max p*2^F_r * max|c| stay inside the FMA's 2^22.
        float v[NB];
        bool is_max[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            v[i] = 0.0f;
            is_max[i] = false;
        }
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) v[rr] = lpart[rr];
        v[RC] = cmx;
        is_max[RC] = true;
        v[RC + 1] = pmx;
        is_max[RC + 1] = true;
        wg_reduce(v, is_max);
        float lmax = 0.0f;
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) {
            lpart[rr] = v[rr];
            lmax = fmaxf(lmax, v[rr]);
        }
        const float bound = 4.0f * v[RC] * lmax + 2.0f * (float)(t_end - t_begin); // units of 2^-F_r
        if (exact || (bound < kBinLimit && v[RC + 1] * v[RC] < 4194304.0f)) break;
        }

        // Exact path: per-row maxima, then the exact bound, then the bins.
        exact = true;
        float mx[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) mx[rr] = -INFINITY;
        for (uint32_t tile = wave; tile < n_wt; tile += NW) {
            uint4_t cur[CPT];
            bool curv[CPT];
            load_tile(tile, cur, curv);
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk)
                if (curv[kk]) {
                    uint32_t ia[4];
                    uint32_t dummy = 0;
                    atoms(cur[kk], ia, dummy);
                    float sc[RC];
                    score(cur[kk], ia, sc);
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) mx[rr] = fmaxf(mx[rr], sc[rr] * sl);
                }
        }
        float m2[NB];
        bool im2[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            m2[i] = i < RC ? mx[i] : 0.0f;
            im2[i] = i < RC;
        }
        wg_reduce(m2, im2);
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) ref[rr] = m2[rr] == -INFINITY ? 0.0f : ceilf(m2[rr]);
        float ebr[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) ebr[rr] = 0.0f;
        for (uint32_t tile = wave; tile < n_wt; tile += NW) {
            uint4_t cur[CPT];
            bool curv[CPT];
            load_tile(tile, cur, curv);
#pragma unroll
            for (int kk = 0; kk < CPT; ++kk)
                if (curv[kk]) {
                    uint32_t ia[4];
                    uint32_t dummy = 0;
                    atoms(cur[kk], ia, dummy);
                    float sc[RC];
                    score(cur[kk], ia, sc);
                    float ca = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) ca += fabsf((float)coef(cur[kk], j));
#pragma unroll
                    for (int rr = 0; rr < RC; ++rr) ebr[rr] += fast_exp2(sc[rr] * sl - ref[rr]) * ca;
                }
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            m2[i] = i < RC ? ebr[i] : 0.0f;
            im2[i] = false;
        }
        wg_reduce(m2, im2);
        // Row rr's exact sum over contributions of |p*c|: its bins stay within
        // 2^29 * (1 + float rounding) + 2 * tokens.
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) F[rr] = m2[rr] > 0.0f ? min(100, max(-100, 29 - exp_of(m2[rr]))) : 100;
        __syncthreads(); // every wave is done with the bins
    }
    // Atom indices outside the dictionary: recorded (their terms went to a clamped atom).
    {
        bool badat;
        if constexpr (POW2) badat = (oob & ~((A - 1u) | ((A - 1u) << 16))) != 0u;
        else badat = oob >= A;
        if (badat) flag_error(a.err, kErrAtom);
    }
    // Bins out as float rows [r][A] (or tiled); track max |bin| per row for the f16 split of the finish.
    float inv[RC];
#pragma unroll
    for (int rr = 0; rr < RC; ++rr) inv[rr] = pow2f(-F[rr]);
    if constexpr (OUT) {
        // Value partials: O^T[d][r] = sum_a D^T[d][a] * W[a][r] on MFMA, so no bins
        // leave the work-group and no finish runs.  W = bins * 2^-16 as f16 hi + lo
        // (|bin| < 2^31, so both terms stay inside f16: ~22 significant bits, the
        // finish's split), staged in LDS as [A/32 k-steps][4 lg][RC rows][8 atoms],
        // hi then lo: the MFMA B operand of lane (row li, lg) is one 16-byte read.
        // The A operand, D^T, is the projection's tiled copy: a wave's 16-byte loads
        // cover 1 KiB.  Wave w takes dim block w (16 dims) over every atom; lanes
        // with li >= RC carry zero rows.  Output: lane (li, lg) holds dims
        // 16 w + 4 lg .. +3 of row li, scaled back by 2^(16 - F_li).
        const uint32_t HD = a.head_dim, nkb = A / 32u, ndb = HD / 16u;
        _Float16* wl = (_Float16*)(smem + a.w_lds_off);
        const uint32_t wlo = nkb * 4u * RC * 8u; // halves of the hi plane
        for (uint32_t i = tid; i < (A / 8u) * RC; i += NT) {
            const uint32_t rr = i % RC, a8 = i / RC; // atoms 8 a8 .. +7 of row rr: k-step a8 / 4, lg a8 % 4
            half8_t hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint64_t wv = *binp(a8 * 8u + (uint32_t)e, (int)(rr >> 1));
                const int32_t v0 = (int32_t)(uint32_t)wv;
                const int32_t v1 = (int32_t)((uint32_t)(wv >> 32) + (v0 < 0 ? 1u : 0u));
                const float x = (float)((rr & 1u) ? v1 : v0) * 1.52587890625e-05f; // 2^-16
                hi[e] = (_Float16)x;
                lo[e] = (_Float16)(x - (float)hi[e]);
            }
            *(half8_t*)(wl + (a8 * RC + rr) * 8u) = hi;
            *(half8_t*)(wl + wlo + (a8 * RC + rr) * 8u) = lo;
        }
        __syncthreads(); // W staged
        const uint32_t li = (uint32_t)lane & 15u, lg = (uint32_t)lane >> 4;
        if ((uint32_t)wave < ndb) {
            const uint32_t grp = a.dict_heads == 1 ? l : l * a.kv_heads + g;
            const uint4_t* dtp = (const uint4_t*)(a.dt + (uint64_t)grp * HD * A) + (uint32_t)wave * 64u + (uint32_t)lane;
            const bool rowl = li < (uint32_t)RC;
            const _Float16* wrow = wl + (lg * RC + (rowl ? li : 0u)) * 8u;
            float4_t acc = (float4_t)0.0f;
            constexpr int KB = 8; // k-steps of D^T loads in flight
            for (uint32_t k0 = 0; k0 < nkb; k0 += KB) {
                uint4_t av[KB];
#pragma unroll
                for (int j = 0; j < KB; ++j) av[j] = dtp[(uint64_t)min(k0 + (uint32_t)j, nkb - 1u) * ndb * 64u];
#pragma unroll
                for (int j = 0; j < KB; ++j) {
                    if (k0 + (uint32_t)j >= nkb) break;
                    const uint32_t ko = (k0 + (uint32_t)j) * 4u * RC * 8u;
                    const half8_t bh = rowl ? *(const half8_t*)(wrow + ko) : (half8_t)(_Float16)0.0f;
                    const half8_t bl = rowl ? *(const half8_t*)(wrow + wlo + ko) : (half8_t)(_Float16)0.0f;
                    acc = mfma16x16x32(as_h8(av[j]), bh, acc);
                    acc = mfma16x16x32(as_h8(av[j]), bl, acc);
                }
            }
            const uint32_t r = c * RC + li;
            if (rowl && r < R) {
                int f = 0; // F of row li, by arithmetic (no register array indexed at run time)
#pragma unroll
                for (int k = 0; k < RC; ++k) f += F[k] * (int)(li == (uint32_t)k);
                const float sc = pow2f(16 - f);
                *(float4_t*)(a.out_o + (obase + r) * HD + 16u * (uint32_t)wave + 4u * lg) = acc * sc;
            }
        }
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) // static indices: no register array indexed at run time
            if (tid == rr) {
                const uint32_t r = c * RC + rr;
                if (r < R) {
                    a.out_m[obase + r] = ref[rr];
                    a.out_l[obase + r] = lpart[rr] * inv[rr];
                }
            }
    } else {
        // 2^-F_rr for a row index known only at run time, by arithmetic: selects over
        // the array would be folded into an indexed load from scratch memory.
        auto inv_of = [&](int rr) -> float {
            int f = 0;
#pragma unroll
            for (int k = 0; k < RC; ++k) f += F[k] * (int)(rr == k);
            return pow2f(-f);
        };
        float amax[RC];
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) amax[rr] = 0.0f;
        // The bin of row rr at atom `at` as a float.
        auto bin_value = [&](uint32_t at, int rr) -> float {
            const uint64_t wv = *binp(at, rr / 2);
            const int32_t v0 = (int32_t)(uint32_t)wv;
            const int32_t v1 = (int32_t)((uint32_t)(wv >> 32) + (v0 < 0 ? 1u : 0u));
            return (float)((rr & 1) ? v1 : v0) * inv_of(rr);
        };
        if (a.w_tiled) {
            // Thread -> (group of 4 atoms, row): 16-byte pieces, the rows of one piece
            // position adjacent in the tile (64-byte runs for 4 rows).
            const uint32_t l_in = lb / a.batch, b_in = lb % a.batch;
            const uint32_t grp = a.w_dict_heads == 1 ? l_in : l_in * a.kv_heads + g;
            const uint32_t tiles = (a.w_rows_per_group + 15) / 16, nk = A / 32;
            for (uint32_t i = tid; i < (A / 4) * RC; i += NT) {
                const int rr = (int)(i % RC);
                const uint32_t a4 = i / RC, r = c * RC + (uint32_t)rr;
                float4_t v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = bin_value(4 * a4 + e, rr);
                amax[rr] = fmaxf(amax[rr], fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
                if (r >= R) continue;
                const uint32_t grow = a.w_dict_heads == 1 ? (b_in * a.kv_heads + g) * R + r : b_in * R + r;
                const uint32_t at = 4 * a4, kk = at / 32, lgv = (at % 32) / 8, h = (at % 8) / 4;
                const uint64_t off = ((((uint64_t)grp * tiles + grow / 16) * nk + kk) * 2 + h) * 64 + lgv * 16 + grow % 16;
                *(float4_t*)(a.part_w + off * 4) = v;
            }
        } else
        for (uint32_t at = tid; at < A; at += NT) {
#pragma unroll
            for (int pp = 0; pp < NP; ++pp) {
                const uint64_t wv = *binp(at, pp);
                const int32_t v0 = (int32_t)(uint32_t)wv;
                const int32_t v1 = (int32_t)((uint32_t)(wv >> 32) + (v0 < 0 ? 1u : 0u));
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int rr = 2 * pp + h;
                    if (rr >= RC) continue;
                    const float v = (float)(h ? v1 : v0) * inv[rr];
                    amax[rr] = fmaxf(amax[rr], fabsf(v));
                    const uint32_t r = c * RC + rr;
                    if (r < R) a.part_w[(pbase + r) * a.w_pitch + at] = v;
                }
            }
        }
        float v[NB];
        bool is_max[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            v[i] = i < RC ? amax[i] : 0.0f;
            is_max[i] = true;
        }
        wg_reduce(v, is_max);
#pragma unroll
        for (int rr = 0; rr < RC; ++rr) // static indices: no register array indexed at run time
            if (tid == rr) {
                const uint32_t r = c * RC + rr;
                if (r < R) {
                    a.part_m[pbase + r] = ref[rr];
                    a.part_l[pbase + r] = lpart[rr] * inv[rr]; // sum of p, back from units of 2^-F_r
                    a.part_amax[pbase + r] = v[rr];
                }
            }
    }
}

// Persistent: work-group i takes work items i, i + gridDim.x, ... (gridDim.x a
// multiple of 8, so each keeps its XCD), so the grid is one resident round and
// the hot kernel can run beside it in the resources it leaves free.
template <int RC, int CPT, int PD, bool POW2, bool QF32, bool BUF, bool OUT>
__global__ __launch_bounds__(kColdThreads) void cold_kernel(ColdArgs a) {
    for (uint32_t wg = blockIdx.x; wg < a.n_wg; wg += gridDim.x) {
        cold_unit<RC, CPT, PD, POW2, QF32, BUF, OUT>(a, wg);
        __syncthreads(); // the next item rewrites the LDS tables
    }
}

// Shared-memory bytes of cold_kernel<RC> for a dictionary of A atoms, splits of
// `tokens_per_split` tokens and a q_latent table of `qbytes` (2 or 4) per entry.
inline size_t cold_smem_bytes(uint32_t A, int RC, uint32_t tokens_per_split, uint32_t qbytes) {
    const size_t qtab = ((size_t)A * RC * qbytes + 15) & ~(size_t)15;
    const int NW = kColdThreads / 64, NP = (RC + 1) / 2;
    const size_t tables = (RC == 4 && qbytes == 2) ? (size_t)A * kColdRec : qtab + (size_t)A * NP * 8;
    const size_t n_ref = ((size_t)(tokens_per_split + 15) / 16 + kColdRefPad - 1) / kColdRefPad * kColdRefPad;
    return cold_hp_offset(tables, (uint32_t)n_ref, (uint32_t)(NW * (2 * RC + 4))) + cold_hp_bytes(A, NP);
}

// ----------------------------------------------- per-row merge factors
//
// For one row (lbg, r): cold splits combine to max Mc and sum Lc; the bins are
// pre-multiplied by 2^(m_s - Mc) / Lc * scl with scl a power of two that keeps
// the largest combined bin below 2^14, so the hi/lo f16 split of each bin keeps
// ~22 significant bits.  Hot splits combine to Mh, Lh with factors 2^(m_s - Mh).
// Computed by lanes = splits (a wave per row, or segments of a wave).
__device__ inline float bin_scale(float bound, float Lc) {
    float scl = 1.0f;
    if (Lc > 0.0f && bound > 0.0f) {
        const int e = max(-100, min(100, exp_of(bound / Lc)));
        scl = pow2f(14 - e);
    }
    return scl;
}

// Segmented wave reductions over groups of `lpr` lanes (a power of two <= 64).
template <bool MAX>
__device__ inline float seg_reduce(float v, uint32_t lpr) {
    for (uint32_t o = lpr >> 1; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, (int)o);
        v = MAX ? fmaxf(v, w) : v + w;
    }
    return v;
}
// combine_splits over a segment of lanes (lane = split).
__device__ inline void combine_seg(float m, float l, uint32_t lpr, float& M, float& L, float& f) {
    const bool ok = l > 0.0f;
    M = seg_reduce<true>(ok ? m : -INFINITY, lpr);
    f = ok ? fast_exp2(m - M) : 0.0f;
    L = seg_reduce<false>(f * l, lpr);
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
// Work-group = 128 rows sharing one dictionary (8 waves x 16 rows) x one atom
// range, walked in super-chunks of 64 atoms.  A super-chunk's D^T (64 atoms x
// HD dims, written by the projection as [HD][A]) is staged once in LDS and
// shared by the 8 waves, so D^T is read from L2 once per 128 rows.  Per wave:
// O^T[dim][row] += D^T W^T in sub-chunks of 32 atoms,
//   A = D^T (lane: dim 16*nb+li, atoms 8*lg .. +7: one 16-byte LDS read),
//   B = W^T (lane: row li, the same 8 atoms), split into hi + lo f16 terms ->
//       two MFMAs per dim block.
// Pipelining, one barrier per super-chunk: the bins W of super-chunk s+1 load
// into the second of two register sets while s is computed (SINGLE: one cold
// split; with several splits each super-chunk's splits are loaded and combined
// at its start), and the D^T pieces of s+1, loaded one super-chunk ahead into
// registers, go to the other LDS buffer after s's MFMAs.  The first loads are
// issued before the per-row split factors are worked out.  Each wave finishes
// its own rows: with one atom range the log-sum-exp merge runs here, otherwise
// the partial cold outputs go to `ocp` for merge_kernel.
constexpr int kFinishWaves = 8;
constexpr int kFinishRows = 16 * kFinishWaves;
constexpr int kFinishSC = 64;                  // atoms per super-chunk
constexpr int kFinishPitch = kFinishSC + 8;    // halves per staged D^T row

// Dynamic LDS of finish_kernel: D^T double buffer, per-row split factors for
// `sf` splits (cold and, when fused, hot), row factors.
inline size_t finish_smem_bytes(int HD, uint32_t sf) {
    return (size_t)2 * HD * kFinishPitch * 2 + (size_t)2 * kFinishRows * sf * 4 + (size_t)kFinishRows * 5 * 4;
}

template <int HD, bool SINGLE>
__global__ __launch_bounds__(kFinishWaves * 64) void finish_kernel(FinishArgs a) {
    constexpr int NB = HD / 16, DP = kFinishPitch, NS = kFinishSC / 32; // sub-chunks per super-chunk
    constexpr int GP = kFinishSC / 8, PIECES = HD * GP, PPT = PIECES / (kFinishWaves * 64); // 16-byte D^T pieces
    static_assert(PIECES % (kFinishWaves * 64) == 0, "D^T pieces per thread");
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const uint32_t group = blockIdx.x / a.tiles_per_group, tile = blockIdx.x % a.tiles_per_group;
    const uint32_t ar = blockIdx.y;
    const uint32_t l = group / a.dict_heads, dg = group % a.dict_heads;
    const uint32_t R = a.rows_r, A = a.dict_size;
    const bool fused = a.n_ar == 1 && a.hot_splits > 0 && !a.sep_merge;
    const uint32_t sneed = max(a.cold_splits, fused ? a.hot_splits : 1u);
    const uint32_t lpr = sneed <= 1 ? 1u : 1u << (32 - __builtin_clz(sneed - 1u)); // factors per row
    _Float16* sd = (_Float16*)smem;                           // [2][HD][DP]
    float* s_cfac = (float*)(smem + (size_t)2 * HD * DP * 2); // [ROWS][lpr]
    float* s_hfac = s_cfac + (size_t)kFinishRows * lpr;       // [ROWS][lpr]
    float* s_rf = s_hfac + (size_t)kFinishRows * lpr;         // [ROWS][5]: Mc, Lc, inv_scl, Mh, Lh

    // Row (lbg, r) of group row `row` (clamped into the group).
    auto row_id = [&](uint32_t row, uint64_t& lbg, uint32_t& r) {
        row = min(row, a.rows_per_group - 1u);
        if (a.dict_heads == 1) lbg = (uint64_t)l * a.batch * a.kv_heads + row / R; // row = (b*Hkv + g)*R + r
        else lbg = ((uint64_t)l * a.batch + row / R) * a.kv_heads + dg;            // row = b*R + r
        r = row % R;
    };
    // This lane's B-operand row.
    const uint32_t my_raw = tile * kFinishRows + wave * 16 + li;
    const bool rowok = my_raw < a.rows_per_group;
    uint64_t lbg_me;
    uint32_t r_me;
    row_id(my_raw, lbg_me, r_me);
    const int myr = wave * 16 + li;
    const float* wbase = a.cold_w + ((lbg_me * a.cold_splits) * R + r_me) * a.w_pitch;
    const uint64_t wsplit = (uint64_t)R * a.w_pitch;

    const uint16_t* dt = a.dt + (uint64_t)group * HD * a.dt_pitch;
    const uint32_t a_begin = ar * a.atoms_per_range;
    const uint32_t a_end = min(a_begin + a.atoms_per_range, A);
    const uint32_t n_sc = (a_end - a_begin + kFinishSC - 1) / kFinishSC;

    // Loads past the range (the prefetch beyond the last super-chunk, the tail of a
    // partial one) are clamped to its last 8 atoms: lines already read, never the
    // next range's bins.
    const uint32_t a_last = a_end - 8u;
    // D^T pieces of super-chunk s: piece p = (dim p / GP, atoms 8*(p%GP) .. +7).
    auto load_dt = [&](uint32_t s, uint4_t (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kFinishWaves * 64;
            const uint32_t at = min(a_begin + kFinishSC * s + 8 * (p % GP), a_last);
            v[q] = *(const uint4_t*)(dt + (uint64_t)(p / GP) * a.dt_pitch + at);
        }
    };
    auto store_dt = [&](int buf, const uint4_t (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kFinishWaves * 64;
            *(uint4_t*)(sd + ((size_t)buf * HD + p / GP) * DP + 8 * (p % GP)) = v[q];
        }
    };
    // Single-split W of super-chunk s: this lane's row, atoms 32*k + 8*lg .. +7 of each sub-chunk k.
    auto load_w = [&](uint32_t s, float4_t (&w)[2 * NS]) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const uint32_t at = min(a_begin + kFinishSC * s + 32 * k + 8 * lg, a_last);
            w[2 * k] = *(const float4_t*)(wbase + at);
            w[2 * k + 1] = *(const float4_t*)(wbase + at + 4);
        }
    };

    // First loads, oldest first: D^T of super-chunk 0, its W (SINGLE), then D^T of 1 and W of 1.
    uint4_t dpre[PPT];
    float4_t wA[2 * NS], wB[2 * NS];
    load_dt(0, dpre);
    if constexpr (SINGLE) load_w(0, wA);
    uint4_t d1[PPT];
    load_dt(1, d1);
    if constexpr (SINGLE) load_w(1, wB);

    // Split factors of this wave's 16 rows: lanes form segments of lpr lanes (lane
    // in segment = split), one row per segment, 64/lpr rows per pass; all loads of
    // a pass are unconditional (clamped).
    {
        const uint32_t seg = (uint32_t)lane / lpr, sp = (uint32_t)lane % lpr;
        const uint32_t per_pass = 64u / lpr;
        const float* hmp = fused ? a.hot_m : a.cold_m; // any valid array when the hot side is absent
        const float* hlp = fused ? a.hot_l : a.cold_l;
        for (uint32_t i0 = 0; i0 < 16u; i0 += per_pass) {
            const uint32_t i = i0 + seg; // row of this wave handled by this segment
            const uint32_t row_raw = tile * kFinishRows + wave * 16 + i;
            const bool rv = i < 16u && row_raw < a.rows_per_group;
            uint64_t lbg;
            uint32_t r;
            row_id(row_raw, lbg, r);
            const uint32_t cs = min(sp, a.cold_splits - 1u);
            const uint64_t cb = (lbg * a.cold_splits + cs) * R + r;
            float cm = a.cold_m[cb], cl = a.cold_l[cb], ca = a.cold_amax[cb];
            const uint32_t hs = min(sp, a.hot_splits > 0 ? a.hot_splits - 1u : 0u);
            const uint64_t hb = fused ? (lbg * a.hot_splits + hs) * R + r : cb;
            float hm = hmp[hb], hl = hlp[hb];
            const bool cv = rv && sp < a.cold_splits, hv = rv && fused && sp < a.hot_splits;
            cm = cv ? cm : -INFINITY;
            cl = cv ? cl : 0.0f;
            ca = cv ? ca : 0.0f;
            hm = hv ? hm : -INFINITY;
            hl = hv ? hl : 0.0f;
            float Mc, Lc, f;
            combine_seg(cm, cl, lpr, Mc, Lc, f);
            const float scl = bin_scale(seg_reduce<false>(f * ca, lpr), Lc);
            float Mh = -INFINITY, Lh = 0.0f, fh = 0.0f;
            if (fused) combine_seg(hm, hl, lpr, Mh, Lh, fh);
            const uint32_t srow = wave * 16 + min(i, 15u);
            if (i < 16u) {
                s_cfac[srow * lpr + sp] = Lc > 0.0f ? f / Lc * scl : 0.0f;
                s_hfac[srow * lpr + sp] = fh;
                if (sp == 0) {
                    float* rf = s_rf + srow * 5;
                    rf[0] = Mc;
                    rf[1] = Lc;
                    rf[2] = 1.0f / scl;
                    rf[3] = Mh;
                    rf[4] = Lh;
                }
            }
        }
    }
    store_dt(0, dpre);
    __syncthreads(); // factors and D^T of super-chunk 0 visible

    const float f0 = rowok ? s_cfac[myr * lpr] : 0.0f;
    const bool wok = rowok && f0 != 0.0f; // an empty split wrote no bins: never read them
    float4_t acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = (float4_t)0.0f;

    // One super-chunk: MFMAs from LDS buffer s&1 and W (SINGLE: registers w, then refilled
    // with super-chunk s+2); D^T of s+1 (registers dn) into the other buffer, then the
    // loads of D^T s+2 into dn; one barrier.
    auto step = [&](uint32_t s, float4_t (&w)[2 * NS], uint4_t (&dn)[PPT], auto last) {
        const int buf = (int)(s & 1u);
        const uint32_t a0 = a_begin + kFinishSC * s;
        // B operands of the NS sub-chunks, hi + lo f16 terms; atoms past the range
        // (and rows without bins) are zero.
        half8_t his[NS], los[NS];
        auto split = [&](int k, const float (&x8)[8], bool rows_ok) {
            const bool in = a0 + 32 * k + 8 * lg < a_end && rows_ok; // this lane's 8 atoms count
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = in ? x8[e] : 0.0f;
                his[k][e] = (_Float16)x;
                los[k][e] = (_Float16)(x - (float)his[k][e]);
            }
        };
        if constexpr (SINGLE) {
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                float x8[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x8[e] = f0 * w[2 * k][e];
                    x8[4 + e] = f0 * w[2 * k + 1][e];
                }
                split(k, x8, wok);
            }
            // Refill two super-chunks ahead (clamped), below every read of w: loads
            // hoisted above them would need fresh registers and a copy, which waits.
            __builtin_amdgcn_sched_barrier(0);
            load_w(s + 2, w);
        } else {
            float w8s[NS][8];
#pragma unroll
            for (int k = 0; k < NS; ++k)
#pragma unroll
                for (int e = 0; e < 8; ++e) w8s[k][e] = 0.0f;
            // Four splits' loads in flight at a time (clamped split index); splits with
            // factor 0 (empty) are masked at use.
            for (uint32_t s0 = 0; s0 < a.cold_splits; s0 += 4) {
                float fs[4];
                float4_t v[4][2 * NS];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t sp = min(s0 + j, a.cold_splits - 1u);
                    const float* wrow = wbase + sp * wsplit;
#pragma unroll
                    for (int k = 0; k < NS; ++k) {
                        const uint32_t at = min(a0 + 32 * k + 8 * lg, a_last);
                        v[j][2 * k] = *(const float4_t*)(wrow + at);
                        v[j][2 * k + 1] = *(const float4_t*)(wrow + at + 4);
                    }
                    fs[j] = rowok && s0 + j < a.cold_splits ? s_cfac[myr * lpr + s0 + j] : 0.0f;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int k = 0; k < NS; ++k)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            w8s[k][e] += fs[j] != 0.0f ? fs[j] * v[j][2 * k][e] : 0.0f;
                            w8s[k][4 + e] += fs[j] != 0.0f ? fs[j] * v[j][2 * k + 1][e] : 0.0f;
                        }
            }
#pragma unroll
            for (int k = 0; k < NS; ++k) split(k, w8s[k], rowok);
        }
        // Sub-chunks past the range run with zero operands: no branch here, so nothing
        // above sinks below the refill.
#pragma unroll
        for (int k = 0; k < NS; ++k) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const uint4_t dv = *(const uint4_t*)(sd + ((size_t)buf * HD + 16 * nb + li) * DP + 32 * k + 8 * lg);
                acc[nb] = mfma16x16x32(as_h8(dv), his[k], acc[nb]);
                acc[nb] = mfma16x16x32(as_h8(dv), los[k], acc[nb]);
            }
        }
        if constexpr (!decltype(last)::value) {
            // D^T of s+1 into the other buffer: its last readers (s-1) passed the previous barrier.
            store_dt(buf ^ 1, dn);
            load_dt(s + 2, dn);
            __syncthreads();
        }
    };
    // The last super-chunk stores and prefetches nothing, so it waits for nothing.
    using more_t = std::integral_constant<bool, false>;
    using last_t = std::integral_constant<bool, true>;
    uint32_t s = 0;
    for (; s + 2 < n_sc; s += 2) {
        step(s, wA, d1, more_t{});
        step(s + 1, wB, d1, more_t{});
    }
    if (s + 1 < n_sc) {
        step(s, wA, d1, more_t{});
        step(s + 1, wB, d1, last_t{});
    } else {
        step(s, wA, d1, last_t{});
    }

    if (!rowok) return;
    // Lane holds O^T[dims 16*nb + 4*lg + e][row li of this wave].
    const float* rf = s_rf + myr * 5;
    const float Mc = rf[0], Lc = rf[1], inv_scl = rf[2], Mh = rf[3], Lh = rf[4];
    const uint64_t rowid = lbg_me * R + r_me;
    if (!fused && (a.n_ar > 1 || a.sep_merge)) {
        float* dst = a.ocp + (rowid * a.n_ar + ar) * HD;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) *(float4_t*)(dst + 16 * nb + 4 * lg) = acc[nb] * inv_scl;
        return;
    }
    // Fused merge with the hot partials of this row.
    const uint64_t lbg = lbg_me, r = r_me;
    float4_t oh[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oh[nb] = (float4_t)0.0f;
    for (uint32_t s = 0; s < a.hot_splits; ++s) {
        const float f = s_hfac[myr * lpr + s];
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
            v[e] = (_Float16)merge_value(oh[nb][e], Mh, Lh, acc[nb][e] * inv_scl, Mc, Lc);
        *(half4_t*)(o + 16 * nb + 4 * lg) = v;
    }
}

// ---------------------------------------- bins . D by row tiles (MFMA)
//
// For many rows with one cold split each.  Work-group = 16 rows sharing one
// dictionary x one atom range; its 8 waves split the range into 8 stretches of
// whole 32-atom k-steps and each streams its stretch of D^T and of the rows'
// bins straight from memory, kFinRowsPD k-steps of loads ahead, with no LDS
// staging and no barrier: per k-step
//   A = D^T (lane: dim 16*nb + li, atoms 8*lg .. +7: one 16-byte load per dim block)
//   B = W^T (lane: row li, the same 8 atoms) times the row's cold factor, split
//       into hi + lo f16 terms -> two MFMAs per dim block.
// The projection writes D^T and the cold kernel the bins in these lane orders
// (ProjArgs::dt_tiled, ColdArgs::w_tiled), so every load instruction reads 1 KB
// contiguous: on gfx950 a CU reads L2-resident data at ~135 GB/s that way and at
// ~37 GB/s when a load spans 16 rows of 64 bytes (measured).
// Every wave reads a different stretch of D^T, so no operand is shared through
// LDS; the 16 rows fill the MFMA's 16 columns.  The 8 waves' O^T partials are
// then summed in LDS in wave order, and each thread finishes 4 dims of one row:
// with one atom range the row is merged with its hot partials and written as
// f16, otherwise the range partial goes to `ocp` for merge_kernel.
constexpr int kFinRowsWaves = 8;
// k-steps of loads in flight per wave: 2 measured faster than 3 or 4 (B = 64 finish 15.0 against
// 16.9 and 16.8 us: deeper rings issue more than the CU's memory pipeline drains).
constexpr int kFinRowsPD = 2;

// The waves' partials, then (Mc, Lc, 1/scale) of the tile's 16 rows.
inline size_t finish_rows_smem_bytes(int HD) { return (size_t)kFinRowsWaves * (HD / 16) * 64 * 16 + 16 * 16; }

template <int HD>
__global__ __launch_bounds__(kFinRowsWaves * 64) void finish_rows_kernel(FinishArgs a) {
    constexpr int NB = HD / 16;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    float4_t* s_part = (float4_t*)smem; // [wave][nb][lane]
    const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tiles = (a.rows_per_group + 15) / 16;
    const uint32_t group = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const uint32_t ar = blockIdx.y;
    const uint32_t l = group / a.dict_heads, dg = group % a.dict_heads;
    const uint32_t R = a.rows_r, A = a.dict_size;

    // Row (lbg, r) of group row `row` (clamped into the group).
    auto row_id = [&](uint32_t row, uint64_t& lbg, uint32_t& r) {
        row = min(row, a.rows_per_group - 1u);
        if (a.dict_heads == 1) lbg = (uint64_t)l * a.batch * a.kv_heads + row / R; // row = (b*Hkv + g)*R + r
        else lbg = ((uint64_t)l * a.batch + row / R) * a.kv_heads + dg;            // row = b*R + r
        r = row % R;
    };

    // This lane's B-operand row and its cold factor (one split: the bins' own scale).
    const uint32_t my_raw = tile * 16 + li;
    uint64_t lbg_b;
    uint32_t r_b;
    row_id(my_raw, lbg_b, r_b);
    const uint64_t cb_b = lbg_b * R + r_b;
    const float mc_b = a.cold_m[cb_b], lc_b = a.cold_l[cb_b], ca_b = a.cold_amax[cb_b];
    const float f_b = my_raw < a.rows_per_group && lc_b > 0.0f ? bin_scale(ca_b, lc_b) / lc_b : 0.0f;
    // The row's factors for the end, kept in LDS so that no thread reloads them
    // from memory after the wave reduction (published by its barrier).
    float4_t* s_rowf = (float4_t*)(smem + (size_t)kFinRowsWaves * NB * 64 * 16); // [16]
    if (wave == 0 && lg == 0) {
        float4_t rf;
        rf[0] = mc_b;
        rf[1] = lc_b;
        rf[2] = lc_b > 0.0f ? 1.0f / bin_scale(ca_b, lc_b) : 1.0f;
        rf[3] = 0.0f;
        s_rowf[li] = rf;
    }

    // This wave's stretch of the range, in k-steps of 32 atoms.
    const uint32_t a_begin = ar * a.atoms_per_range;
    const uint32_t a_end = min(a_begin + a.atoms_per_range, A);
    const uint32_t n_k = (a_end - a_begin + 31) / 32;
    const uint32_t k_per = (n_k + kFinRowsWaves - 1) / kFinRowsWaves;
    const uint32_t k0 = min(n_k, (uint32_t)wave * k_per), k1 = min(n_k, k0 + k_per);
    // Both operands tiled so that each load instruction reads 1 KB contiguous (64
    // lanes x 16 bytes): D^T as [A/32][NB][lane][8 atoms], the bins of this row
    // tile as [A/32][2][lane][4].
    const uint32_t kbase = a_begin / 32;
    const uint16_t* dt = a.dt + (uint64_t)group * HD * A + (uint64_t)lane * 8;
    const float* wt = a.cold_w + ((uint64_t)blockIdx.x * (A / 32) * 2 * 64 + (uint64_t)lane) * 4;

    struct KLoads {
        uint4_t d[NB];
        float4_t w[2];
    };
    auto load_k = [&](uint32_t k, KLoads& v) {
        const uint64_t kk = kbase + k;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) v.d[nb] = *(const uint4_t*)(dt + (kk * NB + nb) * 64 * 8);
        v.w[0] = *(const float4_t*)(wt + kk * 2 * 64 * 4);
        v.w[1] = *(const float4_t*)(wt + (kk * 2 + 1) * 64 * 4);
    };
    float4_t acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = (float4_t)0.0f;
    auto compute_k = [&](uint32_t k, const KLoads& v) {
        // This lane's 8 atoms count (inside the wave's stretch and the range); a row
        // without cold tokens has no bins (never read).
        const bool in = k < k1 && a_begin + 32u * k + 8u * (uint32_t)lg < a_end && f_b != 0.0f;
        half8_t hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = in ? f_b * v.w[e / 4][e % 4] : 0.0f;
            hi[e] = (_Float16)x;
            lo[e] = (_Float16)(x - (float)hi[e]);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            acc[nb] = mfma16x16x32(as_h8(v.d[nb]), hi, acc[nb]);
            acc[nb] = mfma16x16x32(as_h8(v.d[nb]), lo, acc[nb]);
        }
    };
    // Ring of kFinRowsPD k-steps in flight; its first loads are clamped into the
    // range (a stretch may be shorter than the ring), its refills stay inside the stretch.
    KLoads ring[kFinRowsPD];
#pragma unroll
    for (int j = 0; j < kFinRowsPD; ++j) {
        // Issued in ring order (oldest first), as the loop below refills it.
        load_k(min(k0 + (uint32_t)j, n_k - 1u), ring[j]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Whole rounds of kFinRowsPD k-steps (k-steps past the stretch are masked to
    // zero); a slot is refilled only with a k-step of the stretch (re-reading
    // clamped ones cost B = 64 a microsecond: 15.7 -> 14.8 us).
    for (uint32_t k = k0; k < k1; k += kFinRowsPD) {
#pragma unroll
        for (int j = 0; j < kFinRowsPD; ++j) {
            compute_k(k + j, ring[j]);
            // The refill stays below this k-step's MFMAs: hoisted above them it would
            // take fresh registers and make the MFMAs wait for every load in flight.
            __builtin_amdgcn_sched_barrier(0);
            if (k + j + kFinRowsPD < k1) load_k(k + j + kFinRowsPD, ring[j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Sum the waves' partials in wave order.
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) s_part[(wave * NB + nb) * 64 + lane] = acc[nb];
    __syncthreads();
    // Thread t: dim block nb = t / 64, lane position p = t % 64 -> row p % 16,
    // dims 16*nb + 4*(p / 16) .. +3.
    static_assert(NB * 64 <= kFinRowsWaves * 64, "one float4 of O^T per thread");
    if (tid >= NB * 64) return;
    const int nb = tid / 64, p = tid % 64, pr = p & 15, pd = 16 * nb + 4 * (p >> 4);
    float4_t o = s_part[nb * 64 + p];
#pragma unroll
    for (int w = 1; w < kFinRowsWaves; ++w) o += s_part[(w * NB + nb) * 64 + p];
    const uint32_t row_raw = tile * 16 + pr;
    if (row_raw >= a.rows_per_group) return;
    uint64_t lbg;
    uint32_t r;
    row_id(row_raw, lbg, r);
    const float4_t rf = s_rowf[pr];
    const float Mc = rf[0], Lc = rf[1], inv_scl = rf[2];
    const uint64_t rowid = lbg * R + r;
    if (a.n_ar > 1 || a.sep_merge) {
        *(float4_t*)(a.ocp + (rowid * a.n_ar + ar) * HD + pd) = o * inv_scl;
        return;
    }
    // Merge with the row's hot splits (log-sum-exp over splits, then over hot / cold).
    float Mh = -INFINITY;
    for (uint32_t s = 0; s < a.hot_splits; ++s) {
        const uint64_t hb = (lbg * a.hot_splits + s) * R + r;
        if (a.hot_l[hb] > 0.0f) Mh = fmaxf(Mh, a.hot_m[hb]);
    }
    float Lh = 0.0f;
    float4_t oh = (float4_t)0.0f;
    for (uint32_t s = 0; s < a.hot_splits; ++s) {
        const uint64_t hb = (lbg * a.hot_splits + s) * R + r;
        const float hl = a.hot_l[hb];
        if (!(hl > 0.0f)) continue;
        const float f = fast_exp2(a.hot_m[hb] - Mh);
        Lh += f * hl;
        oh += f * *(const float4_t*)(a.hot_o + hb * HD + pd);
    }
    const uint64_t lb = lbg / a.kv_heads, g = lbg % a.kv_heads;
    const uint64_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
    uint16_t* dst = a.out + ((lb * a.queries + q) * a.q_heads + h) * HD + pd;
    half4_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (_Float16)merge_value(oh[e], Mh, Lh, o[e] * inv_scl, Mc, Lc);
    *(half4_t*)dst = v;
}

// --------------------------------------------------- log-sum-exp merge
//
// One wave per row (row id lbg*R + r), four rows per work-group: lanes first
// combine the row's splits (lane = split), then the partial outputs are summed.
// Used when there is no cold pool or when the cold output was split over
// several atom ranges.  A partial's HD floats are read as float4 pieces by
// LP = HD/4 lanes, so one load instruction covers PG = 64/LP partials (two at
// HD = 128) and a batch of U instructions U*PG of them; the PG lane groups'
// sums are added by shuffles at the end.  Rows with many partials (small
// batches: 64 atom ranges, 64 hot splits) want deep batches, rows with few
// shallow ones (no clamped duplicate loads).  Every load is unconditional
// (clamped indices, masked at use), and the first batch of hot partials is
// issued before the split factors are worked out.
template <int HD, int U>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
    constexpr int LP = HD / 4, PG = 64 / LP;
    __shared__ float s_hfac[4][kMaxSplits];
    const int tid = threadIdx.x, row = tid / 64, lane = tid % 64;
    const uint64_t rowid = (uint64_t)blockIdx.x * 4 + row;
    if (rowid >= a.total_rows) return; // whole wave: no barrier follows
    const uint32_t R = a.rows_r;
    const uint64_t lbg = rowid / R, r = rowid % R;
    const bool has_c = a.ocp != nullptr, has_h = a.hot_splits > 0;
    const float* zero = (const float*)&g_zero_code;
    const uint32_t cs = has_c ? min((uint32_t)lane, a.cold_splits - 1u) : 0u;
    const uint32_t hs = has_h ? min((uint32_t)lane, a.hot_splits - 1u) : 0u;
    const uint64_t cb = has_c ? (lbg * a.cold_splits + cs) * R + r : 0;
    const uint64_t hb = has_h ? (lbg * a.hot_splits + hs) * R + r : 0;
    float cm = (has_c ? a.cold_m : zero)[cb];
    float cl = (has_c ? a.cold_l : zero)[cb];
    float hm = (has_h ? a.hot_m : zero)[hb];
    float hl = (has_h ? a.hot_l : zero)[hb];
    const uint32_t sub = (uint32_t)lane / LP, d0 = 4u * ((uint32_t)lane % LP);
    // Cold atom-range partials: plain sum (every range carries the row's factors).
    float4_t oc = (float4_t)0.0f;
    const uint32_t n_ar = has_c ? a.n_ar : 0u;
    const float* csrc = has_c ? a.ocp + rowid * a.n_ar * HD + d0 : zero;
    for (uint32_t a0 = 0; a0 < n_ar; a0 += U * PG) {
        float4_t v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = *(const float4_t*)(csrc + (uint64_t)min(a0 + j * PG + sub, n_ar - 1u) * HD);
#pragma unroll
        for (int j = 0; j < U; ++j) oc += a0 + j * PG + sub < n_ar ? v[j] : (float4_t)0.0f;
    }
    // First batch of hot partials, before the factors (S = 0: the zero code, unused).
    const uint32_t S = a.hot_splits;
    const float* hsrc = has_h ? a.hot_o + (lbg * S * R + r) * HD + d0 : zero;
    auto load_hot = [&](uint32_t s0, float4_t (&v)[U]) {
#pragma unroll
        for (int j = 0; j < U; ++j)
            v[j] = *(const float4_t*)(hsrc + (has_h ? (uint64_t)min(s0 + j * PG + sub, S - 1u) * R * HD : 0));
    };
    float4_t vh[U];
    load_hot(0, vh);
    float Mc = -INFINITY, Lc = 0.0f, Mh = -INFINITY, Lh = 0.0f;
    {
        const bool cv = has_c && (uint32_t)lane < a.cold_splits;
        const bool hv = has_h && (uint32_t)lane < a.hot_splits;
        cm = cv ? cm : -INFINITY;
        cl = cv ? cl : 0.0f;
        hm = hv ? hm : -INFINITY;
        hl = hv ? hl : 0.0f;
        float f;
        combine_splits(cm, cl, Mc, Lc, f);
        combine_splits(hm, hl, Mh, Lh, f);
        if (lane < kMaxSplits) s_hfac[row][lane] = f;
    }
    __builtin_amdgcn_wave_barrier();
    float4_t oh = (float4_t)0.0f;
    for (uint32_t s0 = 0; s0 < S; s0 += U * PG) {
        if (s0) load_hot(s0, vh);
        float fs[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint32_t sp = s0 + j * PG + sub;
            fs[j] = sp < S ? s_hfac[row][min(sp, S - 1u)] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < U; ++j) oh += fs[j] != 0.0f ? fs[j] * vh[j] : (float4_t)0.0f;
    }
#pragma unroll
    for (int o = LP; o < 64; o *= 2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            oc[e] += __shfl_xor(oc[e], o);
            oh[e] += __shfl_xor(oh[e], o);
        }
    if (sub != 0) return;
    const uint64_t lb = lbg / a.kv_heads, g = lbg % a.kv_heads;
    const uint64_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
    half4_t hv;
#pragma unroll
    for (int e = 0; e < 4; ++e) hv[e] = (_Float16)merge_value(oh[e], Mh, Lh, oc[e], Mc, Lc);
    *(half4_t*)(a.out + ((lb * a.queries + q) * a.q_heads + h) * HD + d0) = hv;
}

// Merge for few rows (fewer than CUs: small batches, one sequence's attention):
// one 4-wave work-group per row, the row's partials dealt over the 4 waves (wave
// w takes partial groups w, w + 4, ...), so each wave needs a quarter of the load
// batches; the waves' sums meet in LDS and are added in wave order.  Split
// factors: every wave combines the statistics itself (lane = split) and reads a
// split's factor from its lane with a shuffle.
template <int HD, int U>
__global__ __launch_bounds__(256) void merge_row_kernel(MergeArgs a) {
    constexpr int LP = HD / 4, PG = 64 / LP, NWV = 4;
    __shared__ float4_t s_part[2][NWV][LP];
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const uint64_t rowid = blockIdx.x;
    const uint32_t R = a.rows_r;
    const uint64_t lbg = rowid / R, r = rowid % R;
    const bool has_c = a.ocp != nullptr, has_h = a.hot_splits > 0;
    const float* zero = (const float*)&g_zero_code;
    const uint32_t cs = has_c ? min((uint32_t)lane, a.cold_splits - 1u) : 0u;
    const uint32_t hs = has_h ? min((uint32_t)lane, a.hot_splits - 1u) : 0u;
    const uint64_t cb = has_c ? (lbg * a.cold_splits + cs) * R + r : 0;
    const uint64_t hb = has_h ? (lbg * a.hot_splits + hs) * R + r : 0;
    float cm = (has_c ? a.cold_m : zero)[cb];
    float cl = (has_c ? a.cold_l : zero)[cb];
    float hm = (has_h ? a.hot_m : zero)[hb];
    float hl = (has_h ? a.hot_l : zero)[hb];
    const uint32_t sub = (uint32_t)lane / LP, d0 = 4u * ((uint32_t)lane % LP);
    // Partial index of this lane for slot j of the batch starting at p0.
    auto pidx = [&](uint32_t p0, int j) { return p0 + (uint32_t)(j * NWV + wave) * PG + sub; };
    constexpr uint32_t STEP = (uint32_t)(U * NWV * PG);
    float4_t oc = (float4_t)0.0f;
    const uint32_t n_ar = has_c ? a.n_ar : 0u;
    const float* csrc = has_c ? a.ocp + rowid * a.n_ar * HD + d0 : zero;
    for (uint32_t a0 = 0; a0 < n_ar; a0 += STEP) {
        float4_t v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = *(const float4_t*)(csrc + (uint64_t)min(pidx(a0, j), n_ar - 1u) * HD);
#pragma unroll
        for (int j = 0; j < U; ++j) oc += pidx(a0, j) < n_ar ? v[j] : (float4_t)0.0f;
    }
    const uint32_t S = a.hot_splits;
    const float* hsrc = has_h ? a.hot_o + (lbg * S * R + r) * HD + d0 : zero;
    auto load_hot = [&](uint32_t s0, float4_t (&v)[U]) {
#pragma unroll
        for (int j = 0; j < U; ++j)
            v[j] = *(const float4_t*)(hsrc + (has_h ? (uint64_t)min(pidx(s0, j), S - 1u) * R * HD : 0));
    };
    float4_t vh[U];
    load_hot(0, vh); // before the factors are known
    float Mc = -INFINITY, Lc = 0.0f, Mh = -INFINITY, Lh = 0.0f, fh = 0.0f;
    {
        const bool cv = has_c && (uint32_t)lane < a.cold_splits;
        const bool hv = has_h && (uint32_t)lane < a.hot_splits;
        cm = cv ? cm : -INFINITY;
        cl = cv ? cl : 0.0f;
        hm = hv ? hm : -INFINITY;
        hl = hv ? hl : 0.0f;
        float f;
        combine_splits(cm, cl, Mc, Lc, f);
        combine_splits(hm, hl, Mh, Lh, fh); // fh: factor of hot split `lane`
    }
    float4_t oh = (float4_t)0.0f;
    for (uint32_t s0 = 0; s0 < S; s0 += STEP) {
        if (s0) load_hot(s0, vh);
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint32_t sp = pidx(s0, j);
            const float fs = __shfl(fh, (int)min(sp, S - 1u)); // splits <= kMaxSplits <= 64 lanes
            oh += (sp < S && fs != 0.0f) ? fs * vh[j] : (float4_t)0.0f;
        }
    }
#pragma unroll
    for (int o = LP; o < 64; o *= 2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            oc[e] += __shfl_xor(oc[e], o);
            oh[e] += __shfl_xor(oh[e], o);
        }
    if (sub == 0) {
        s_part[0][wave][lane] = oc;
        s_part[1][wave][lane] = oh;
    }
    __syncthreads();
    if (wave != 0 || sub != 0) return;
    float4_t c4 = s_part[0][0][lane], h4 = s_part[1][0][lane];
#pragma unroll
    for (int w = 1; w < NWV; ++w) {
        c4 += s_part[0][w][lane];
        h4 += s_part[1][w][lane];
    }
    const uint64_t lb = lbg / a.kv_heads, g = lbg % a.kv_heads;
    const uint64_t q = r / a.gqa, h = g * a.gqa + r % a.gqa;
    half4_t hv;
#pragma unroll
    for (int e = 0; e < 4; ++e) hv[e] = (_Float16)merge_value(h4[e], Mh, Lh, c4[e], Mc, Lc);
    *(half4_t*)(a.out + ((lb * a.queries + q) * a.q_heads + h) * HD + d0) = hv;
}

// ------------------------------------------------ read-only HBM stream
//
// Attainable read bandwidth: every lane issues U 16-byte loads (grid-strided,
// so a wave's load covers 1 KiB of consecutive bytes) before folding them.  A
// wave writes its XOR fold (64 words, one per lane) only when it equals
// kReadSinkMagic, so nothing is written in practice but the loads cannot be
// elided.
constexpr uint32_t kReadSinkMagic = 0xA5A5A5A5u;

template <int U>
__global__ __launch_bounds__(256) void read_stream_kernel(const uint4_t* p, uint64_t n16, uint32_t* sink) {
    const uint64_t nth = (uint64_t)gridDim.x * 256u;
    uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    uint4_t acc = (uint4_t)0u;
    for (; i + (uint64_t)(U - 1) * nth < n16; i += (uint64_t)U * nth) {
        uint4_t v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = p[i + (uint64_t)j * nth];
#pragma unroll
        for (int j = 0; j < U; ++j) acc ^= v[j];
    }
    for (; i < n16; i += nth) acc ^= p[i];
    uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o);
    if (x == kReadSinkMagic) sink[threadIdx.x & 63u] = x; // lane-indexed: a vector store
}

// ------------------------------------------------ pool gather (read only)
//
// The attainable rate of the decode's own pool reads: every hot K (and V) row
// and every cold code of a request, through its block table, in the pools'
// layouts, with nothing computed and (almost) nothing written.  One wave per
// unit: a (layer, sequence, kv head) and a stretch of kGatherHotBlocks hot
// blocks (16 rows of HD halves each) or kGatherColdBlocks cold blocks (16
// codes each); the unit's block refs are staged in LDS first (as the decode
// kernels stage theirs), then every lane keeps U 16-byte loads in flight.
// A wave's XOR fold is written to `sink` only when it equals kReadSinkMagic.
constexpr uint32_t kGatherHotBlocks = 32;   // 512 tokens: the hot kernel's split at B = 64
constexpr uint32_t kGatherColdBlocks = 256; // 4096 tokens

struct GatherArgs {
    const uint4_t* hot_k;
    const uint4_t* hot_v; // may be null
    const uint4_t* cold;
    const uint32_t* refs;
    uint32_t* sink;
    uint32_t batch, kv_heads, hd16; // hd16: 16-byte pieces per row (HD / 8)
    uint32_t hot_count, cold_count, refs_stride, cold_head_blocked;
    uint32_t hot_units, cold_units; // per (layer, sequence, kv head)
    uint64_t hot_blocks, cold_blocks, hot_layer16, cold_layer16, refs_layer;
};

template <int U>
__global__ __launch_bounds__(64) void gather_read_kernel(GatherArgs a) {
    __shared__ uint32_t s_ref[kGatherColdBlocks];
    const uint32_t lane = threadIdx.x;
    const uint32_t per = a.hot_units + a.cold_units;
    const uint32_t unit = blockIdx.x % per, lbg = blockIdx.x / per;
    const uint32_t g = lbg % a.kv_heads, lb = lbg / a.kv_heads, l = lb / a.batch;
    const uint32_t* refs = a.refs + (uint64_t)l * a.refs_layer + (uint64_t)(lb % a.batch) * a.refs_stride;
    const bool hot = unit < a.hot_units;
    const uint32_t nblk_all = hot ? a.hot_count : a.cold_count;
    const uint32_t per_unit = hot ? kGatherHotBlocks : kGatherColdBlocks;
    const uint32_t b0 = (hot ? unit : unit - a.hot_units) * per_unit;
    const uint32_t nb = b0 < nblk_all ? min(per_unit, nblk_all - b0) : 0u;
    const uint64_t cap = hot ? a.hot_blocks : a.cold_blocks;
    for (uint32_t i = lane; i < nb; i += 64u) {
        const uint32_t r = refs[(hot ? 0u : a.hot_count) + b0 + i] & 0x7FFFFFFFu;
        s_ref[i] = r < cap ? r : 0u;
    }
    __syncthreads();
    uint4_t acc = (uint4_t)0u;
    if (hot) {
        // Row (block i, token t): hd16 pieces; a load instruction covers 64 / hd16 rows.
        const uint32_t rows = nb * 16u, pieces = rows * a.hd16;
        const uint4_t* kb = a.hot_k + (uint64_t)l * a.hot_layer16;
        const uint4_t* vb = a.hot_v ? a.hot_v + (uint64_t)l * a.hot_layer16 : nullptr;
        auto addr = [&](uint32_t pc) -> uint64_t {
            const uint32_t row = pc / a.hd16, q = pc % a.hd16;
            return (((uint64_t)s_ref[row / 16u] * 16u + row % 16u) * a.kv_heads + g) * a.hd16 + q;
        };
        for (uint32_t p0 = 0; p0 < pieces; p0 += 64u * U) {
            uint4_t v[U], w[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const uint32_t pc = min(p0 + (uint32_t)j * 64u + lane, pieces - 1u);
                v[j] = kb[addr(pc)];
                if (vb) w[j] = vb[addr(pc)];
            }
#pragma unroll
            for (int j = 0; j < U; ++j) {
                acc ^= v[j];
                if (vb) acc ^= w[j];
            }
        }
    } else {
        const uint32_t codes = nb * 16u;
        const uint4_t* cb = a.cold + (uint64_t)l * a.cold_layer16;
        for (uint32_t c0 = 0; c0 < codes; c0 += 64u * U) {
            uint4_t v[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const uint32_t c = min(c0 + (uint32_t)j * 64u + lane, codes - 1u);
                const uint64_t blk = s_ref[c / 16u], t = c % 16u;
                v[j] = cb[a.cold_head_blocked ? (blk * a.kv_heads + g) * 16u + t : (blk * 16u + t) * a.kv_heads + g];
            }
#pragma unroll
            for (int j = 0; j < U; ++j) acc ^= v[j];
        }
    }
    uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o);
    if (x == kReadSinkMagic) a.sink[lane] = x; // lane-indexed: a vector store
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

// --------------------------------------------- SparseCode encoder (distiller)
//
// Replaces Distiller::distill_block (distiller.rs:171-246).  Lane = one token of
// one kv head: it keeps the token's HD values in registers and walks every atom
// of the head's dictionary in index order, each dot product summed in head-dim
// order from -0.0 with one FMA per term (f16 x f16 products are exact in f32, so
// the FMA rounds exactly like the reference's product-then-add,
// distiller.rs:212-216).  A wave holds 64 tokens of one kv head, so it reads one
// dictionary row at a time: 16-atom chunks are staged in LDS by the work-group
// (double-buffered, the next chunk's loads in flight while the current one is
// used) and read back as broadcasts.  The running top 4 keeps (score desc,
// atom asc): an atom enters only with a strictly larger score, and atoms come in
// index order, so equal scores keep the lower index first (the reference test at
// distiller.rs:299-307 expects 0,1,2,3 for equal scores).  NaN and -inf never
// enter; an unfilled slot keeps the zero code's index 0 and coefficient 0.
struct EncodeArgs {
    const uint16_t* hot;  // [hot_blocks][16][kv_heads][HD]
    const uint16_t* dict; // [dict_heads][A][HD]
    const uint32_t* src;  // hot block per encoded block
    const uint32_t* dst;  // cold block per encoded block, or null: the source index
    uint4_t* cold;        // code (block, token, head) = cold[block*16*kv_heads + token*s_tok + head*s_head]
    float* entropy;       // [n_blocks] or null
    uint32_t* err;
    uint32_t kv_heads, dict_size, dict_heads, n_blocks;
    uint32_t s_tok, s_head;
    uint64_t hot_blocks, cold_blocks;
};
constexpr int kEncThreads = 256;
constexpr int kEncAtoms = 16; // atoms per staged dictionary chunk (dict_size % 16 == 0)

template <int HD>
__global__ __launch_bounds__(kEncThreads) void encode_kernel(EncodeArgs a) {
    constexpr int PR = HD / 8, NPC = kEncAtoms * PR; // 16-byte pieces per row / per chunk
    __shared__ __attribute__((aligned(16))) uint4_t sd[2][NPC];
    const int tid = threadIdx.x;
    const uint32_t g = blockIdx.y;
    const uint32_t n_tok = a.n_blocks * kBlockTokens;
    const uint32_t T = blockIdx.x * kEncThreads + tid; // token of the request
    const bool live = T < n_tok;
    const uint32_t Tc = live ? T : n_tok - 1u;
    const uint32_t bi = Tc / kBlockTokens, tt = Tc % kBlockTokens;
    const uint32_t b = a.src[bi] & kRefMask;
    const uint32_t c = a.dst ? (a.dst[bi] & kRefMask) : b;
    const bool ok = live && b < a.hot_blocks && c < a.cold_blocks;
    if (live && g == 0 && tt == 0) { // one report per block
        if (b >= a.hot_blocks) flag_error(a.err, kErrHotRef);
        if (c >= a.cold_blocks) flag_error(a.err, kErrColdRef);
    }
    const uint32_t A = a.dict_size, n_ch = A / kEncAtoms;
    const uint4_t* D = (const uint4_t*)(a.dict + (uint64_t)(a.dict_heads == 1 ? 0u : g) * A * HD);
    // Dictionary chunk ch: piece p of it (threads beyond NPC idle; loads clamped into the dictionary).
    auto load_chunk = [&](uint32_t ch) -> uint4_t { return D[(uint64_t)min(ch, n_ch - 1u) * NPC + min(tid, NPC - 1)]; };
    uint4_t pre = load_chunk(0);
    // This lane's token (a valid block when the request's is out of range: its code is not written).
    const uint4_t* xp = (const uint4_t*)(a.hot + (((uint64_t)(b < a.hot_blocks ? b : 0u) * kBlockTokens + tt) * a.kv_heads + g) * HD);
    half8_t x[PR];
#pragma unroll
    for (int j = 0; j < PR; ++j) x[j] = as_h8(xp[j]);
    if (tid < NPC) sd[0][tid] = pre;
    pre = load_chunk(1);
    __syncthreads();

    float v[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    uint32_t ix[4] = {0u, 0u, 0u, 0u};
    for (uint32_t ch = 0; ch < n_ch; ++ch) {
        const uint4_t* row = sd[ch & 1u];
#pragma unroll 2
        for (int at = 0; at < kEncAtoms; ++at) {
            float s = -0.0f;
#pragma unroll
            for (int j = 0; j < PR; ++j) {
                const half8_t d8 = as_h8(row[at * PR + j]); // same address in every lane: a broadcast
#pragma unroll
                for (int e = 0; e < 8; ++e) s = fmaf((float)x[j][e], (float)d8[e], s);
            }
            if (s > v[3]) { // NaN and -inf never enter
                const uint32_t ai = ch * kEncAtoms + (uint32_t)at;
                const bool g0 = s > v[0], g1 = s > v[1], g2 = s > v[2];
                v[3] = g2 ? v[2] : s;
                ix[3] = g2 ? ix[2] : ai;
                v[2] = g1 ? v[1] : (g2 ? s : v[2]);
                ix[2] = g1 ? ix[1] : (g2 ? ai : ix[2]);
                v[1] = g0 ? v[0] : (g1 ? s : v[1]);
                ix[1] = g0 ? ix[0] : (g1 ? ai : ix[1]);
                v[0] = g0 ? s : v[0];
                ix[0] = g0 ? ai : ix[0];
            }
        }
        // The next chunk into the other buffer (its last readers passed the previous barrier).
        if (tid < NPC) sd[(ch + 1u) & 1u][tid] = pre;
        pre = load_chunk(ch + 2u);
        __syncthreads();
    }
    if (!ok) return;
    uint32_t cb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const bool filled = v[k] != -INFINITY;
        cb[k] = filled ? (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[k]) : 0u;
        ix[k] = filled ? ix[k] : 0u;
    }
    const uint4_t code = {ix[0] | (ix[1] << 16), ix[2] | (ix[3] << 16), cb[0] | (cb[1] << 16), cb[2] | (cb[3] << 16)};
    a.cold[(uint64_t)c * kBlockTokens * a.kv_heads + tt * a.s_tok + g * a.s_head] = code;
}

// ------------------------------------- encoder: MFMA prefilter, exact rescoring
//
// The same codes as encode_kernel (bit for bit) at a fraction of the exact FMAs.
// For token x and atom d_a let S_a be the reference's score (f32, sequential in
// head-dim order) and M_a the MFMA score of the same exact f16 x f16 products
// summed in another order.  Both are sums of the HD products p_k with one
// rounding per addition, so |M_a - S_a| <= 2*HD*u*sum|p_k| <= 2*HD*u*|x|*|d_a|
// (u = 2^-24; Cauchy-Schwarz); the kernel uses E_a = 8*HD*u*|x|*|d_a|, four
// times that, with the norms rounded up.  Subnormal components may be flushed by
// the matrix unit: an atom with some gets E_a += |x|_1 * 2^-14, a token with some
// E_a += |d_a|_1 * 2^-14 (a flushed term is below 2^-14 times its partner).  Then:
//   T   = the 4th largest of M_a - E_a          (four atoms have S >= T, so
//                                                 the exact 4th score is >= T);
//   C   = { a : M_a + E_a >= T }                (holds every atom whose exact
//                                                 score can reach the top 4);
//   the exact S_a of the atoms of C, in ascending atom order, through the
//   same strict-greater insertion as the full scan: the same four atoms in the
//   same order, hence the same code.
// Tokens with an inf or NaN component, and tokens whose candidate list
// overflows, take the full exact scan; atoms with an inf or NaN component are
// always candidates.
//
// Work-group = 4 waves x 64 tokens of one kv head (4 tiles of 16 tokens per
// wave).  The dictionary streams through LDS in chunks of 64 atoms, twice:
// pass 1 finds T, pass 2 collects C.  MFMA orientation M^T = D X^T with
// v_mfma_f32_16x16x32_f16 (lane l, li = l%16, lg = l/16): A = atoms (row li of
// the atom tile, dims 32*ks + 8*lg ..), B = the token tile (token li, the same
// dims, held in registers), C: lane l holds token li and atoms 4*lg .. 4*lg+3.
// Pass 2 keeps each lane's candidates of a token in its own sub-list (no
// atomics; ascending, as the lane meets its atoms in order); pass 3: one thread
// per token merges its 4 sub-lists and rescores the candidates exactly.
constexpr int kEncMThreads = 256;
constexpr int kEncMTokens = 256;  // tokens per work-group
constexpr int kEncMChunk = 64;    // atoms per staged dictionary chunk
constexpr int kEncMCap = 32;      // candidates kept per token
constexpr int kEncMSub = kEncMCap / 4; // per token and lane: each of 4 lanes sees a quarter of the atoms
constexpr uint32_t kDictBad = 1u, kDictSubnormal = 2u;

typedef float float2_t __attribute__((ext_vector_type(2)));

// |d_a|_2 and |d_a|_1 (rounded up) and flags (kDictBad: inf or NaN component;
// kDictSubnormal) for every atom of every dictionary head, as {l2, l1, flags}.
struct __attribute__((aligned(16))) AtomNorm {
    float l2, l1;
    uint32_t flags, pad;
};
template <int HD>
__global__ __launch_bounds__(256) void dict_norm_kernel(const uint16_t* dict, uint64_t n_atoms, AtomNorm* out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_atoms) return;
    const uint4_t* row = (const uint4_t*)(dict + i * HD);
    float ss = 0.0f, s1 = 0.0f;
    uint32_t fl = 0;
#pragma unroll 4
    for (int j = 0; j < HD / 8; ++j) {
        const uint4_t w = row[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t bits = (w[e / 2] >> (16 * (e % 2))) & 0xFFFFu;
            const uint32_t ex = (bits >> 10) & 31u, man = bits & 1023u;
            fl |= ex == 31u ? kDictBad : 0u;
            fl |= (ex == 0u && man != 0u) ? kDictSubnormal : 0u;
            const float f = h2f_bits(bits);
            ss = fmaf(f, f, ss);
            s1 += fabsf(f);
        }
    }
    out[i] = AtomNorm{sqrtf(ss) * 1.001f, s1 * 1.001f, fl, 0u};
}

template <int HD>
__global__ __launch_bounds__(kEncMThreads) void encode_mfma_kernel(EncodeArgs a, const AtomNorm* dnorm) {
    constexpr int KS = HD / 32, P = HD + 8, PR = HD / 8, NTT = 4, CH = kEncMChunk, CAP = kEncMCap;
    constexpr int CPIECES = CH * PR, CPT = CPIECES / kEncMThreads; // 16-byte pieces per chunk / thread
    static_assert(CPT * kEncMThreads == CPIECES, "chunk staging");
    __shared__ __attribute__((aligned(16))) _Float16 sd[2][CH * P];
    __shared__ uint4_t s_gs[2][CH / 4]; // per group of 4 atoms: max l2, max l1 (good atoms; float bits), sub flag, bad mask
    __shared__ __attribute__((aligned(16))) unsigned char s_lists[kEncMTokens * CAP * 2]; // pass-1 tops, then candidates
    __shared__ float s_T[kEncMTokens];
    __shared__ uint32_t s_cnt[kEncMTokens * 4];
    __shared__ uint32_t s_xfl[kEncMTokens];
    static_assert(kEncMTokens * 16 * 4 <= (int)sizeof(s_lists), "pass-1 tops fit the candidate lists");
    float* s_top = (float*)s_lists;
    uint16_t* s_cand = (uint16_t*)s_lists;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    const uint32_t g = blockIdx.y;
    const uint32_t n_tok = a.n_blocks * kBlockTokens;
    const uint32_t tok0 = blockIdx.x * kEncMTokens;
    const uint32_t A = a.dict_size, n_ch = (A + CH - 1) / CH;
    const uint32_t dh = a.dict_heads == 1 ? 0u : g;
    const uint16_t* Dg = a.dict + (uint64_t)dh * A * HD;
    const AtomNorm* dn = dnorm + (uint64_t)dh * A;
    constexpr float kBound = 8.0f * HD * 5.9604645e-8f; // 8 * HD * 2^-24
    constexpr float kSub = 6.1035156e-5f;               // 2^-14: bound of a subnormal f16

    // The lane's tokens (B operands) and their norms; xsub: the token has a
    // subnormal component (its bound then takes |d_a|_1 * 2^-14 more).
    half8_t xb[NTT][KS];
    float kx[NTT], sx[NTT], xsub[NTT];
    {
        float ss[NTT], s1[NTT];
        uint32_t fl[NTT];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
            const uint32_t T = min(tok0 + (uint32_t)(wave * 64 + tt * 16 + li), n_tok - 1u);
            const uint32_t bi = T / kBlockTokens, ti = T % kBlockTokens;
            uint32_t b = a.src[bi] & kRefMask;
            b = b < a.hot_blocks ? b : 0u; // such a token is not written
            const uint16_t* xp = a.hot + (((uint64_t)b * kBlockTokens + ti) * a.kv_heads + g) * HD;
            ss[tt] = 0.0f;
            s1[tt] = 0.0f;
            fl[tt] = 0u;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4_t w = *(const uint4_t*)(xp + 32 * ks + 8 * lg);
                xb[tt][ks] = as_h8(w);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t bits = (w[e / 2] >> (16 * (e % 2))) & 0xFFFFu;
                    const uint32_t ex = (bits >> 10) & 31u, man = bits & 1023u;
                    fl[tt] |= ex == 31u ? 1u : 0u;                      // inf or NaN: full scan
                    fl[tt] |= (ex == 0u && man != 0u) ? 2u : 0u;         // subnormal: wider bound
                    const float f = h2f_bits(bits);
                    ss[tt] = fmaf(f, f, ss[tt]);
                    s1[tt] += fabsf(f);
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
            ss[tt] += __shfl_xor(ss[tt], 16);
            ss[tt] += __shfl_xor(ss[tt], 32);
            s1[tt] += __shfl_xor(s1[tt], 16);
            s1[tt] += __shfl_xor(s1[tt], 32);
            fl[tt] |= __shfl_xor(fl[tt], 16);
            fl[tt] |= __shfl_xor(fl[tt], 32);
            kx[tt] = kBound * (sqrtf(ss[tt]) * 1.001f);
            sx[tt] = kSub * (s1[tt] * 1.001f);
            xsub[tt] = (fl[tt] & 2u) ? kSub : 0.0f;
            if (lg == 0) s_xfl[wave * 64 + tt * 16 + li] = fl[tt] & 1u;
        }
    }

    // Dictionary chunk staging: every thread loads CPT pieces (clamped into the
    // dictionary), threads < CH also the atoms' norms.
    uint4_t creg[CPT];
    AtomNorm nreg{};
    auto load_chunk = [&](uint32_t ch) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int p = tid + k * kEncMThreads;
            const uint32_t at = min(ch * CH + (uint32_t)(p / PR), A - 1u);
            creg[k] = *(const uint4_t*)(Dg + (uint64_t)at * HD + 8 * (p % PR));
        }
        if (tid < CH) nreg = dn[min(ch * CH + (uint32_t)tid, A - 1u)];
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int p = tid + k * kEncMThreads;
            *(uint4_t*)(&sd[buf][(p / PR) * P + 8 * (p % PR)]) = creg[k];
        }
        if (tid < CH) { // wave 0: lane = atom; quads of lanes = the groups of 4 atoms of a tile row
            const bool bad = (nreg.flags & kDictBad) != 0u;
            float l2 = bad ? 0.0f : nreg.l2, l1 = bad ? 0.0f : nreg.l1;
            uint32_t sub = bad ? 0u : (nreg.flags & kDictSubnormal), badm = bad ? (1u << (tid & 3)) : 0u;
#pragma unroll
            for (int o = 1; o < 4; o *= 2) {
                l2 = fmaxf(l2, __shfl_xor(l2, o));
                l1 = fmaxf(l1, __shfl_xor(l1, o));
                sub |= (uint32_t)__shfl_xor((int)sub, o);
                badm |= (uint32_t)__shfl_xor((int)badm, o);
            }
            if ((tid & 3) == 0)
                s_gs[buf][tid / 4] = (uint4_t){__builtin_bit_cast(uint32_t, l2), __builtin_bit_cast(uint32_t, l1), sub, badm};
        }
    };
    // One pass over the dictionary.  Per atom tile, fn(acc, E, badm, atom0) gets the
    // MFMA scores acc[tt][e] of the lane's tokens (tt) and atoms atom0 + e, one bound
    // E[tt] for the lane's 4 atoms (from their largest norms, so >= each atom's own
    // bound), and the mask of those atoms with an inf or NaN component.
    auto stream = [&](auto fn) {
        load_chunk(0);
        store_chunk(0);
        __syncthreads();
        for (uint32_t ch = 0; ch < n_ch; ++ch) {
            const int cur = (int)(ch & 1u);
            const bool more = ch + 1 < n_ch;
            if (more) load_chunk(ch + 1);
            const uint32_t tiles = min((uint32_t)(CH / 16), (A - ch * CH) / 16u);
            for (uint32_t at = 0; at < tiles; ++at) {
                half8_t ad[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) ad[ks] = *(const half8_t*)(&sd[cur][(at * 16 + li) * P + 32 * ks + 8 * lg]);
                // The lane's 4 atoms: bad atoms (always candidates) stay out of the bound.
                const uint4_t gs = s_gs[cur][at * 4 + lg];
                // Words copied out first: __builtin_bit_cast of a vector element reads element 0 here.
                const uint32_t g0 = gs[0], g1 = gs[1];
                const float l2m = __builtin_bit_cast(float, g0), l1m = __builtin_bit_cast(float, g1);
                const uint32_t sub = gs[2], badm = gs[3];
                float4_t acc[NTT];
                float E[NTT];
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt) {
                    acc[tt] = (float4_t)0.0f;
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) acc[tt] = mfma16x16x32(ad[ks], xb[tt][ks], acc[tt]);
                    E[tt] = fmaf(kx[tt], l2m, fmaf(xsub[tt], l1m, sub ? sx[tt] : 0.0f));
                }
                fn(acc, E, badm, ch * CH + at * 16 + 4 * lg);
            }
            if (more) store_chunk(cur ^ 1);
            __syncthreads();
        }
    };

    // Inserting y into the descending top[0..3]: max, then three medians of three.
    auto insert4 = [](float (&t)[4], float y) {
        const float t0 = fmaxf(t[0], y);
        const float t1 = __builtin_amdgcn_fmed3f(t[0], t[1], y);
        const float t2 = __builtin_amdgcn_fmed3f(t[1], t[2], y);
        const float t3 = __builtin_amdgcn_fmed3f(t[2], t[3], y);
        t[0] = t0;
        t[1] = t1;
        t[2] = t2;
        t[3] = t3;
    };
    // Pass 1: per lane and token, the 4 largest of max_e(M) - E over its atom
    // tiles: each is a lower bound of the exact score of a distinct atom, so the
    // 4th largest over all lanes is <= the exact 4th score.
    float top[NTT][4];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
        for (int k = 0; k < 4; ++k) top[tt][k] = -INFINITY;
    stream([&](const float4_t (&acc)[NTT], const float (&E)[NTT], uint32_t badm, uint32_t) {
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
            float m = -INFINITY;
#pragma unroll
            for (int e = 0; e < 4; ++e) m = fmaxf(m, (badm >> e) & 1u ? -INFINITY : acc[tt][e]);
            insert4(top[tt], m - E[tt]);
        }
    });
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
        for (int k = 0; k < 4; ++k) s_top[(wave * 64 + tt * 16 + li) * 16 + lg * 4 + k] = top[tt][k];
    if (tid < kEncMTokens) {
#pragma unroll
        for (int q = 0; q < 4; ++q) s_cnt[tid * 4 + q] = 0u;
    }
    __syncthreads();
    {
        // Thread tid = token tid: T = the 4th largest of its 16 values (the 4 lanes' top 4s).
        float t4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        for (int k = 0; k < 16; ++k) insert4(t4, s_top[tid * 16 + k]);
        s_T[tid] = t4[3];
    }
    __syncthreads();
    float T[NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) T[tt] = s_T[wave * 64 + tt * 16 + li];
    // Pass 2: the candidates, M >= T - E (M + E >= T up to a rounding the bound's
    // slack covers) and every atom with an inf or NaN component, into sub-list
    // (token, lg) of kEncMSub entries; counts in s_cnt (each owned by one lane).
    stream([&](const float4_t (&acc)[NTT], const float (&E)[NTT], uint32_t badm, uint32_t atom0) {
        uint32_t mask = 0u;
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
            const float thr = T[tt] - E[tt];
#pragma unroll
            for (int e = 0; e < 4; ++e) mask |= (acc[tt][e] >= thr || ((badm >> e) & 1u)) ? (1u << (tt * 4 + e)) : 0u;
        }
        while (mask) {
            const uint32_t bit = __builtin_ctz(mask);
            mask &= mask - 1u;
            const uint32_t ci = (wave * 64 + (bit >> 2) * 16 + li) * 4 + lg;
            const uint32_t k = s_cnt[ci];
            if (k < (uint32_t)kEncMSub) s_cand[ci * kEncMSub + k] = (uint16_t)(atom0 + (bit & 3u));
            s_cnt[ci] = k + 1u;
        }
    });

    // Pass 3: thread = token; exact scores of the candidates in ascending atom order.
    const uint32_t T3 = tok0 + tid;
    const bool live = T3 < n_tok;
    const uint32_t Tc = live ? T3 : n_tok - 1u;
    const uint32_t bi = Tc / kBlockTokens, tt3 = Tc % kBlockTokens;
    const uint32_t b = a.src[bi] & kRefMask;
    const uint32_t c = a.dst ? (a.dst[bi] & kRefMask) : b;
    const bool ok = live && b < a.hot_blocks && c < a.cold_blocks;
    if (live && g == 0 && tt3 == 0) { // one report per block
        if (b >= a.hot_blocks) flag_error(a.err, kErrHotRef);
        if (c >= a.cold_blocks) flag_error(a.err, kErrColdRef);
    }
    if (!ok) return; // no barrier follows
    const uint4_t* xp = (const uint4_t*)(a.hot + (((uint64_t)b * kBlockTokens + tt3) * a.kv_heads + g) * HD);
    half8_t x[PR];
#pragma unroll
    for (int j = 0; j < PR; ++j) x[j] = as_h8(xp[j]);
    float v[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    uint32_t ix[4] = {0u, 0u, 0u, 0u};
    auto score = [&](uint32_t ai) {
        const uint4_t* dr = (const uint4_t*)(Dg + (uint64_t)ai * HD);
        float s = -0.0f;
#pragma unroll
        for (int j = 0; j < PR; ++j) {
            const half8_t d8 = as_h8(dr[j]);
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf((float)x[j][e], (float)d8[e], s);
        }
        if (s > v[3]) { // NaN and -inf never enter
            const bool g0 = s > v[0], g1 = s > v[1], g2 = s > v[2];
            v[3] = g2 ? v[2] : s;
            ix[3] = g2 ? ix[2] : ai;
            v[2] = g1 ? v[1] : (g2 ? s : v[2]);
            ix[2] = g1 ? ix[1] : (g2 ? ai : ix[2]);
            v[1] = g0 ? v[0] : (g1 ? s : v[1]);
            ix[1] = g0 ? ix[0] : (g1 ? ai : ix[1]);
            v[0] = g0 ? s : v[0];
            ix[0] = g0 ? ai : ix[0];
        }
    };
    uint32_t n = 0;
    bool full = s_xfl[tid] != 0u;
    uint16_t* lst = s_cand + tid * CAP; // the token's 4 sub-lists, compacted in place
    for (int q = 0; q < 4; ++q) {
        const uint32_t m = s_cnt[tid * 4 + q];
        full = full || m > (uint32_t)kEncMSub;
        for (uint32_t k = 0; !full && k < m; ++k) lst[n++] = lst[q * kEncMSub + k];
    }
    if (full) {
        for (uint32_t ai = 0; ai < A; ++ai) score(ai);
    } else {
        for (uint32_t i = 1; i < n; ++i) { // ascending atom order (the list is the thread's own)
            const uint16_t key = lst[i];
            uint32_t j = i;
            while (j > 0 && lst[j - 1] > key) {
                lst[j] = lst[j - 1];
                --j;
            }
            lst[j] = key;
        }
        for (uint32_t i = 0; i < n; ++i) score(lst[i]);
    }
    uint32_t cb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const bool filled = v[k] != -INFINITY;
        cb[k] = filled ? (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[k]) : 0u;
        ix[k] = filled ? ix[k] : 0u;
    }
    const uint4_t code = {ix[0] | (ix[1] << 16), ix[2] | (ix[3] << 16), cb[0] | (cb[1] << 16), cb[2] | (cb[3] << 16)};
    a.cold[(uint64_t)c * kBlockTokens * a.kv_heads + tt3 * a.s_tok + g * a.s_head] = code;
}

// Variance proxy of each listed block (distiller.rs:126-159), bit-exact: one
// lane per block runs the reference's loops in memory order, in f64, with no
// fused multiply-add (the reference squares, then adds), and returns f32; an
// all-zero block gives 0.  Without a block list (src null) lane i takes block i.
//
// The f64 sums are sequential chains, so a block cannot be split across lanes;
// what is parallel is the data supply.  One wave owns kEntBlocks blocks and
// streams them in chunks of kEntChunk values: the wave loads a chunk of all its
// blocks with coalesced 16-byte loads (16 lanes per 256-byte block chunk) into
// one of two LDS tiles while each block's lane runs its chain over the other
// tile.  Rows are padded by 16 bytes so the lanes' row reads spread over the
// banks.
constexpr int kEntChunk = 128;                   // f16 values per block and chunk (256 bytes)
constexpr int kEntCols = kEntChunk / 8;          // 16-byte words per row
constexpr int kEntPitch = kEntCols + 1;          // padded row, in 16-byte words

// The sum of a block's values needs no particular order when it is exact:
// f16 values are multiples of 2^-24, so when sum|v| < 2^29 every partial sum of
// any subset is a multiple of 2^-24 below 2^53 of them, exactly representable
// in f64, and the reference's sequential sum from -0.0 equals any other order
// (a zero total is +0.0 both ways unless every value is a zero, and then the
// proxy is 0 anyway).  Pass 0 sums in four independent chains and records
// sum|v| and whether an inf or NaN occurred; a wave with a block outside the
// exact case repeats the sum sequentially (pass 2).
constexpr int kEntChains = 4;
struct EntSum {
    double s[kEntChains], m[kEntChains];
    bool all_zero, nonfinite;
};

// One 16-byte word (8 values) of a block, in memory order: pass 0 adds the
// values in kEntChains chains (and their magnitudes), pass 1 adds the squared
// deviations, pass 2 adds the values sequentially.
template <int PASS>
__device__ inline void entropy_word(const uint4_t w, EntSum& st, double& acc, double mean) {
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t bits = (w[e / 2] >> (16 * (e % 2))) & 0xFFFFu;
        const float f = h2f_bits(bits);
        if constexpr (PASS == 0) {
            st.all_zero = st.all_zero && f == 0.0f;
            st.nonfinite = st.nonfinite || ((bits >> 10) & 31u) == 31u;
            st.s[e % kEntChains] = st.s[e % kEntChains] + (double)f;
            st.m[e % kEntChains] = st.m[e % kEntChains] + (double)fabsf(f);
        } else if constexpr (PASS == 1) {
            const double diff = (double)f - mean;
            const double sq = diff * diff;
            acc = acc + sq;
        } else {
            acc = acc + (double)f;
        }
    }
}

// Blocks per wave.  A wave's 64 lanes all load (the stream is latency-bound:
// more waves keep more chunks in flight) and all sum the values for the mean,
// four lanes per block; the first kEntBlocks lanes run the sequential chains
// (the variance, and the mean when its sums are not exact).  At 16 blocks a
// wave, 8192 blocks make 512 waves.
constexpr int kEntBlocks = 16;

__global__ __launch_bounds__(64) void entropy_kernel(EncodeArgs a, uint32_t head_dim) {
    constexpr int NB = kEntBlocks, PL = NB * kEntCols / 64; // 16-byte loads per lane and chunk
    static_assert(PL * 64 == NB * kEntCols, "chunk loads");
    static_assert(NB * 4 == 64 && kEntCols % 4 == 0, "four lanes per block in the mean pass");
    __shared__ uint4_t tile[2][NB][kEntPitch];
    __shared__ uint32_t s_blk[NB];
    const uint32_t lane = threadIdx.x;
    const bool chain = lane < (uint32_t)NB; // this lane owns a block
    const uint32_t i = blockIdx.x * NB + lane;
    uint32_t b = 0;
    bool ok = false;
    if (chain && i < a.n_blocks) {
        b = a.src ? (a.src[i] & kRefMask) : i;
        ok = b < a.hot_blocks;
        if (!ok) flag_error(a.err, kErrHotRef);
    }
    if (chain) s_blk[lane] = ok ? b : 0xFFFFFFFFu;
    __syncthreads();
    const uint64_t n = (uint64_t)kBlockTokens * a.kv_heads * head_dim; // values per block
    const uint64_t words = n / 8;                                        // 16-byte words per block
    const uint64_t n_chunks = (words + kEntCols - 1) / kEntCols;
    const uint4_t* hot = (const uint4_t*)a.hot;
    // Lane l loads words (k * 64 + l) of the chunk: row r = that / kEntCols, column c.
    uint4_t reg[PL];
    auto load = [&](uint64_t ch) {
#pragma unroll
        for (int k = 0; k < PL; ++k) {
            const uint32_t idx = k * 64 + lane, r = idx / kEntCols, c = idx % kEntCols;
            const uint32_t rb = s_blk[r];
            const uint64_t w = ch * kEntCols + c;
            reg[k] = (rb != 0xFFFFFFFFu && w < words) ? hot[(uint64_t)rb * words + w] : uint4_t{0, 0, 0, 0};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int k = 0; k < PL; ++k) {
            const uint32_t idx = k * 64 + lane;
            tile[buf][idx / kEntCols][idx % kEntCols] = reg[k];
        }
    };
    EntSum st;
#pragma unroll
    for (int k = 0; k < kEntChains; ++k) st.s[k] = st.m[k] = -0.0;
    st.all_zero = true;
    st.nonfinite = false;
    double mean = 0.0;
    // Streams the whole block once per pass; the pass is a compile-time constant
    // so the inner loops carry no branch.
    auto stream = [&](auto pass, double acc) {
        constexpr int P = decltype(pass)::value;
        load(0);
        store(0);
        __syncthreads();
        for (uint64_t ch = 0; ch < n_chunks; ++ch) {
            const int cur = (int)(ch & 1);
            const bool more = ch + 1 < n_chunks;
            if (more) load(ch + 1);
            if constexpr (P == 0) {
                // Every lane: a quarter of the words of block lane / 4 (exact sums
                // are the same in any order; the quarters are added after the pass).
                constexpr uint32_t QW = kEntCols / 4;
                const uint4_t* row = tile[cur][lane / 4];
                const uint32_t cols = (ch + 1) * kEntCols <= words ? (uint32_t)kEntCols : (uint32_t)(words - ch * kEntCols);
                const uint32_t c0 = (lane % 4) * QW;
#pragma unroll
                for (uint32_t c = 0; c < QW; ++c)
                    if (c0 + c < cols) entropy_word<0>(row[c0 + c], st, acc, mean);
            } else if (chain) {
                const uint4_t* row = tile[cur][lane];
                if ((ch + 1) * kEntCols <= words) {
                    uint4_t w[kEntCols];
#pragma unroll
                    for (int c = 0; c < kEntCols; ++c) w[c] = row[c];
#pragma unroll
                    for (int c = 0; c < kEntCols; ++c) entropy_word<P>(w[c], st, acc, mean);
                } else {
                    const uint32_t cols = (uint32_t)(words - ch * kEntCols);
                    for (uint32_t c = 0; c < cols; ++c) entropy_word<P>(row[c], st, acc, mean);
                }
            }
            if (more) store(cur ^ 1);
            __syncthreads();
        }
        return acc;
    };
    (void)stream(std::integral_constant<int, 0>{}, -0.0);
    // Lanes 4r .. 4r+3 hold block r's quarter sums: added (exact whenever the
    // test below passes) and handed to lane r, the block's owner.
    double s4 = (st.s[0] + st.s[1]) + (st.s[2] + st.s[3]);
    double m4 = (st.m[0] + st.m[1]) + (st.m[2] + st.m[3]);
    uint32_t az = st.all_zero ? 1u : 0u, nf = st.nonfinite ? 1u : 0u;
#pragma unroll
    for (int o = 1; o < 4; o *= 2) {
        s4 += __shfl_xor(s4, o);
        m4 += __shfl_xor(m4, o);
        az &= (uint32_t)__shfl_xor((int)az, o);
        nf |= (uint32_t)__shfl_xor((int)nf, o);
    }
    const int src = (int)(chain ? lane * 4u : 0u);
    double sum = __shfl(s4, src);
    const double mag = __shfl(m4, src);
    st.all_zero = __shfl((int)az, src) != 0;
    st.nonfinite = __shfl((int)nf, src) != 0;
    const bool exact = !chain || (!st.nonfinite && mag < 536870912.0); // 2^29
    if (__any(!exact)) { // wave-uniform: the sequential sum for the blocks that need it
        const double seq = stream(std::integral_constant<int, 2>{}, -0.0);
        sum = exact ? sum : seq;
    }
    mean = sum / (double)n;
    const double var = stream(std::integral_constant<int, 1>{}, -0.0);
    if (chain && i < a.n_blocks) a.entropy[i] = (!ok || st.all_zero) ? 0.0f : (float)(var / (double)n);
}

} // namespace aw
