/*
 * weaver_oracle.c — CPU oracle for the Weaver decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only to check the
 * product's results (or, for the baseline, as the CPU port being timed).  The product library
 * (aether_nexus_amd/libaether_weaver.so) never calls it and has no CPU fallback.
 *
 * The reference has no CPU Weaver implementation (WeaverEngine::decode only
 * dispatches Metal, nexus-core/src/weaver.rs:139-237) and cannot be built here
 * (Rust + Metal, no cargo/xcrun).  This file restates its math:
 *
 *   or_decode_ref32   fp32 restatement of weaver_kernel.metal:118-240 in the
 *                     kernel's own order: per query head, hot pass then cold
 *                     pass, one online softmax (metal:69-96), 32-lane strided
 *                     partial dot products summed by the xor butterfly of
 *                     metal:58-66, K == V, f16 output (metal:226-239).
 *                     Generalised to runtime head_dim / dict_size / batch /
 *                     queries / layers / scale / shared dictionary / causal
 *                     drafts.  Multi-threaded over rows: the CPU baseline.
 *   or_decode_f64     brute force in double: decompress every cold code into a
 *                     dense row sum_k c_k D[idx_k] and run textbook two-pass
 *                     softmax attention.  Independent of the q_latent identity.
 *   or_qlatent_f64    q . D^T in double (the identity of docs/YELLOWPAPER.md:84-92).
 *   or_gather_codes   SparseCode decode + atom gather (metal:182-216), bit-exact.
 *   or_h2f / or_f2h   IEEE-754 binary16 <-> binary32, round to nearest even.
 *   or_encode_blocks  SparseCode encoder, distiller.rs:171-246: per token and kv
 *                     head, f32 dot products with every atom summed in head-dim
 *                     order from -0.0 (Rust >= 1.82 f32 sums; rust-version 1.85),
 *                     a full sort by (score desc, atom index asc) with NaN last,
 *                     the first 4 kept, coefficients f16(score).
 *   or_block_entropy  variance proxy of distiller.rs:126-159: f64 mean and
 *                     variance of a block's f16 values in memory order, as f32.
 *
 * Parity pins (all in tests/): the f16 conversions are checked against numpy
 * exhaustively; or_decode_f64 against closed forms (one token, equal scores,
 * unit codes, zero codes, empty pools) and the reference-derived known answers
 * (weaver.rs:369-396 inputs give 1.0 everywhere; bench.rs:113-120 inputs give
 * 0x201B); or_decode_ref32 against or_decode_f64; or_gather_codes against the
 * SparseCode byte known answer of types.rs:546-557; or_encode_blocks against
 * the reference test distiller.rs:286-310 (zero dictionary -> indices 0,1,2,3),
 * a one-hot dictionary (top-4 = the four largest components, coefficients their
 * f16 values), a brute-force numpy restatement on small inputs and planted
 * mistakes; or_block_entropy against distiller.rs:261-283 (zero block -> 0,
 * uniform block -> 0) and numpy's f64 variance.  Parity unpinned: the order of
 * NaN or -inf scores (the reference sorts them with partial_cmp -> Equal,
 * leaving their order to sort_unstable_by; here they are never chosen and an
 * unfilled slot is the zero code's).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/aether_weaver.h"

#define OR_BLOCK 16u
#define OR_REF_MASK 0x7FFFFFFFu
#define OR_MAX_HEAD_DIM 256u

/* ---------------------------------------------------------------- binary16 */

float or_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    float f;
    if (ex == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        f = (float)man * 5.9604644775390625e-08f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu)); /* NaN, quiet */
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 (or inf) -> inf */
    if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal/zero */
        float v;
        memcpy(&v, &ax, 4);
        float s = v * 16777216.0f; /* exact: power-of-two scaling */
        uint32_t m = (uint32_t)nearbyintf(s); /* ties to even in the default mode */
        return (uint16_t)(sign | m);          /* m == 0x400 encodes 2^-14 correctly */
    }
    uint32_t e = (ax >> 23) - 112u, m = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13), rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach inf: correct */
    return (uint16_t)(sign | h);
}

void or_h2f_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_h2f(in[i]);
}
void or_f2h_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f2h(in[i]);
}

/* ---------------------------------------------------------------- geometry */

typedef struct {
    const aw_decode_desc* d;
    uint32_t G, R;
    uint64_t hot_layer, cold_layer, dict_layer, refs_layer;
} geom_t;

static int geom_init(const aw_decode_desc* d, geom_t* g) {
    if (!d || d->kv_heads == 0 || d->q_heads == 0 || d->q_heads % d->kv_heads) return AW_E_INVALID_ARG;
    if (d->head_dim == 0 || d->head_dim % 32 || d->head_dim > OR_MAX_HEAD_DIM) return AW_E_INVALID_ARG;
    if (d->layers == 0 || d->batch == 0 || d->queries == 0) return AW_E_INVALID_ARG;
    if (d->dict_heads != 1 && d->dict_heads != d->kv_heads) return AW_E_INVALID_ARG;
    if (d->refs_stride < d->hot_count + d->cold_count) return AW_E_INVALID_ARG;
    g->d = d;
    g->G = d->q_heads / d->kv_heads;
    g->R = g->G * d->queries;
    g->hot_layer = d->hot_blocks * OR_BLOCK * d->kv_heads * d->head_dim;
    g->cold_layer = d->cold_blocks * OR_BLOCK * d->kv_heads;
    g->dict_layer = (uint64_t)d->dict_heads * d->dict_size * d->head_dim;
    g->refs_layer = (uint64_t)d->batch * d->refs_stride;
    return AW_OK;
}

/* row id = ((l*B + b)*Q + q)*Hq + h, the layout of q and out */
static void row_split(const geom_t* g, uint64_t row, uint32_t* l, uint32_t* b, uint32_t* q, uint32_t* h) {
    const aw_decode_desc* d = g->d;
    *h = (uint32_t)(row % d->q_heads);
    row /= d->q_heads;
    *q = (uint32_t)(row % d->queries);
    row /= d->queries;
    *b = (uint32_t)(row % d->batch);
    *l = (uint32_t)(row / d->batch);
}

static uint32_t seq_count(const uint32_t* per_seq, uint32_t maxv, uint32_t l, uint32_t b, uint32_t B) {
    if (!per_seq) return maxv;
    uint32_t v = per_seq[(uint64_t)l * B + b];
    return v < maxv ? v : maxv;
}

/* Hot tokens visible to query q: all nh*16, or with AW_F_CAUSAL the rule of
 * ops.metal:549, valid = total - num_queries + 1 + q_idx (clamped at 0). */
static uint64_t hot_limit(const aw_decode_desc* d, uint32_t nh, uint32_t q) {
    int64_t n = (int64_t)nh * OR_BLOCK;
    if (!(d->flags & AW_F_CAUSAL)) return (uint64_t)n;
    int64_t lim = n - (int64_t)d->queries + 1 + (int64_t)q;
    return lim > 0 ? (uint64_t)lim : 0;
}

/* ------------------------------------------- fp32 restatement of the kernel */

/* One (l, b, q, h) row, weaver_kernel.metal:129-239 with runtime sizes. */
static int ref32_row(const geom_t* g, uint64_t row, uint16_t* out_row, float* ql_scratch) {
    const aw_decode_desc* d = g->d;
    uint32_t l, b, q, h;
    row_split(g, row, &l, &b, &q, &h);
    const uint32_t D = d->head_dim, Hkv = d->kv_heads, A = d->dict_size;
    const uint32_t kvh = h / g->G;
    const uint16_t* qrow = d->q + row * D;
    const uint32_t* refs = d->refs + l * g->refs_layer + (uint64_t)b * d->refs_stride;
    const uint16_t* hot_k = d->hot_k ? d->hot_k + l * g->hot_layer : NULL; /* no offset on an absent pool */
    const uint16_t* hot_v = d->hot_v ? d->hot_v + l * g->hot_layer : hot_k;
    const aw_sparse_code* cold = d->cold ? d->cold + l * g->cold_layer : NULL;
    const uint16_t* dict =
        d->dict ? d->dict + l * g->dict_layer + (d->dict_heads == 1 ? 0 : (uint64_t)kvh * A * D) : NULL;
    const uint32_t nh = seq_count(d->seq_hot, d->hot_count, l, b, d->batch);
    const uint32_t nc = seq_count(d->seq_cold, d->cold_count, l, b, d->batch);
    const uint64_t limit = hot_limit(d, nh, q);

    float m = -INFINITY, lsum = 0.0f;
    float acc[OR_MAX_HEAD_DIM];
    float part[32], tmp[32];
    for (uint32_t i = 0; i < D; ++i) acc[i] = 0.0f;

    /* hot pass, metal:143-168 */
    for (uint32_t blk = 0; blk < nh; ++blk) {
        uint32_t phys = refs[blk] & OR_REF_MASK;
        if (phys >= d->hot_blocks) return AW_E_OOB;
        for (uint32_t t = 0; t < OR_BLOCK; ++t) {
            if ((uint64_t)blk * OR_BLOCK + t >= limit) continue;
            uint64_t off = (((uint64_t)phys * OR_BLOCK + t) * Hkv + kvh) * D;
            for (uint32_t lane = 0; lane < 32; ++lane) {
                float s = 0.0f;
                for (uint32_t i = lane; i < D; i += 32) s += or_h2f(qrow[i]) * or_h2f(hot_k[off + i]);
                part[lane] = s;
            }
            for (uint32_t mask = 16; mask; mask >>= 1) { /* simd_reduce_add, metal:58-66 */
                for (uint32_t lane = 0; lane < 32; ++lane) tmp[lane] = part[lane] + part[lane ^ mask];
                memcpy(part, tmp, sizeof part);
            }
            float score = part[0] * d->scale;
            float new_m = fmaxf(m, score); /* online_softmax_update, metal:69-96 */
            float eo = expf(m - new_m), en = expf(score - new_m);
            for (uint32_t i = 0; i < D; ++i) acc[i] *= eo;
            lsum = lsum * eo + en;
            m = new_m;
            for (uint32_t i = 0; i < D; ++i) acc[i] += en * or_h2f(hot_v[off + i]);
        }
    }

    /* cold pass, metal:172-222 */
    if (nc > 0) {
        const float* qlf;
        if (d->q_latent) {
            const uint16_t* qlr = d->q_latent + row * A;
            for (uint32_t a = 0; a < A; ++a) ql_scratch[a] = or_h2f(qlr[a]);
        } else { /* q . D^T in fp32, stored as f16 like the reference's q_latent buffer */
            for (uint32_t a = 0; a < A; ++a) {
                float s = 0.0f;
                for (uint32_t i = 0; i < D; ++i) s += or_h2f(qrow[i]) * or_h2f(dict[(uint64_t)a * D + i]);
                ql_scratch[a] = or_h2f(or_f2h(s));
            }
        }
        qlf = ql_scratch;
        for (uint32_t blk = 0; blk < nc; ++blk) {
            uint32_t phys = refs[d->hot_count + blk] & OR_REF_MASK;
            if (phys >= d->cold_blocks) return AW_E_OOB;
            for (uint32_t t = 0; t < OR_BLOCK; ++t) {
                const aw_sparse_code* c = &cold[((uint64_t)phys * OR_BLOCK + t) * Hkv + kvh];
                float score = 0.0f;
                for (int k = 0; k < 4; ++k) {
                    if (c->indices[k] >= A) return AW_E_OOB;
                    score += qlf[c->indices[k]] * or_h2f(c->coeffs[k]);
                }
                score *= d->scale;
                float new_m = fmaxf(m, score);
                float eo = expf(m - new_m), en = expf(score - new_m);
                for (uint32_t i = 0; i < D; ++i) acc[i] *= eo;
                lsum = lsum * eo + en;
                m = new_m;
                for (uint32_t i = 0; i < D; ++i) {
                    float v = 0.0f;
                    for (int k = 0; k < 4; ++k)
                        v += or_h2f(c->coeffs[k]) * or_h2f(dict[(uint64_t)c->indices[k] * D + i]);
                    acc[i] += en * v;
                }
            }
        }
    }

    /* finalize, metal:226-239 */
    if (lsum > 0.0f)
        for (uint32_t i = 0; i < D; ++i) acc[i] /= lsum;
    for (uint32_t i = 0; i < D; ++i) out_row[i] = or_f2h(acc[i]);
    return AW_OK;
}

/* ------------------------------------------------ fp64 brute force (dense) */

static int f64_row(const geom_t* g, uint64_t row, double* out_row, double* scores, double* qld) {
    const aw_decode_desc* d = g->d;
    uint32_t l, b, q, h;
    row_split(g, row, &l, &b, &q, &h);
    const uint32_t D = d->head_dim, Hkv = d->kv_heads, A = d->dict_size;
    const uint32_t kvh = h / g->G;
    const uint16_t* qrow = d->q + row * D;
    const uint32_t* refs = d->refs + l * g->refs_layer + (uint64_t)b * d->refs_stride;
    const uint16_t* hot_k = d->hot_k ? d->hot_k + l * g->hot_layer : NULL; /* no offset on an absent pool */
    const uint16_t* hot_v = d->hot_v ? d->hot_v + l * g->hot_layer : hot_k;
    const aw_sparse_code* cold = d->cold ? d->cold + l * g->cold_layer : NULL;
    const uint16_t* dict =
        d->dict ? d->dict + l * g->dict_layer + (d->dict_heads == 1 ? 0 : (uint64_t)kvh * A * D) : NULL;
    const uint32_t nh = seq_count(d->seq_hot, d->hot_count, l, b, d->batch);
    const uint32_t nc = seq_count(d->seq_cold, d->cold_count, l, b, d->batch);
    const uint64_t limit = hot_limit(d, nh, q);
    double qd[OR_MAX_HEAD_DIM], kd[OR_MAX_HEAD_DIM];
    for (uint32_t i = 0; i < D; ++i) qd[i] = or_h2f(qrow[i]);
    if (nc > 0 && d->q_latent)
        for (uint32_t a = 0; a < A; ++a) qld[a] = or_h2f(d->q_latent[row * A + a]);

    uint64_t n = 0;
    double mx = -INFINITY;
    /* pass 1: scores */
    for (uint32_t blk = 0; blk < nh; ++blk) {
        uint32_t phys = refs[blk] & OR_REF_MASK;
        if (phys >= d->hot_blocks) return AW_E_OOB;
        for (uint32_t t = 0; t < OR_BLOCK; ++t, ++n) {
            if ((uint64_t)blk * OR_BLOCK + t >= limit) { scores[n] = -INFINITY; continue; }
            uint64_t off = (((uint64_t)phys * OR_BLOCK + t) * Hkv + kvh) * D;
            double s = 0.0;
            for (uint32_t i = 0; i < D; ++i) s += qd[i] * (double)or_h2f(hot_k[off + i]);
            scores[n] = s * (double)d->scale;
            if (scores[n] > mx) mx = scores[n];
        }
    }
    for (uint32_t blk = 0; blk < nc; ++blk) {
        uint32_t phys = refs[d->hot_count + blk] & OR_REF_MASK;
        if (phys >= d->cold_blocks) return AW_E_OOB;
        for (uint32_t t = 0; t < OR_BLOCK; ++t, ++n) {
            const aw_sparse_code* c = &cold[((uint64_t)phys * OR_BLOCK + t) * Hkv + kvh];
            double s = 0.0;
            for (int k = 0; k < 4; ++k)
                if (c->indices[k] >= A) return AW_E_OOB;
            if (d->q_latent) {
                for (int k = 0; k < 4; ++k) s += (double)or_h2f(c->coeffs[k]) * qld[c->indices[k]];
            } else { /* dense decompressed key, then q . k */
                for (uint32_t i = 0; i < D; ++i) kd[i] = 0.0;
                for (int k = 0; k < 4; ++k) {
                    double ck = or_h2f(c->coeffs[k]);
                    const uint16_t* at = dict + (uint64_t)c->indices[k] * D;
                    for (uint32_t i = 0; i < D; ++i) kd[i] += ck * (double)or_h2f(at[i]);
                }
                for (uint32_t i = 0; i < D; ++i) s += qd[i] * kd[i];
            }
            scores[n] = s * (double)d->scale;
            if (scores[n] > mx) mx = scores[n];
        }
    }
    for (uint32_t i = 0; i < D; ++i) out_row[i] = 0.0;
    if (n == 0 || mx == -INFINITY) return AW_OK; /* no visible token: zeros, metal:227 */
    /* pass 2: weights and values */
    double den = 0.0;
    n = 0;
    for (uint32_t blk = 0; blk < nh; ++blk) {
        uint32_t phys = refs[blk] & OR_REF_MASK;
        for (uint32_t t = 0; t < OR_BLOCK; ++t, ++n) {
            if (scores[n] == -INFINITY) continue;
            double w = exp(scores[n] - mx);
            den += w;
            uint64_t off = (((uint64_t)phys * OR_BLOCK + t) * Hkv + kvh) * D;
            for (uint32_t i = 0; i < D; ++i) out_row[i] += w * (double)or_h2f(hot_v[off + i]);
        }
    }
    for (uint32_t blk = 0; blk < nc; ++blk) {
        uint32_t phys = refs[d->hot_count + blk] & OR_REF_MASK;
        for (uint32_t t = 0; t < OR_BLOCK; ++t, ++n) {
            const aw_sparse_code* c = &cold[((uint64_t)phys * OR_BLOCK + t) * Hkv + kvh];
            double w = exp(scores[n] - mx);
            den += w;
            for (int k = 0; k < 4; ++k) {
                double ck = w * (double)or_h2f(c->coeffs[k]);
                const uint16_t* at = dict + (uint64_t)c->indices[k] * D;
                for (uint32_t i = 0; i < D; ++i) out_row[i] += ck * (double)or_h2f(at[i]);
            }
        }
    }
    for (uint32_t i = 0; i < D; ++i) out_row[i] /= den;
    return AW_OK;
}

/* ----------------------------------------------------------- row threading */

typedef struct {
    const geom_t* g;
    const uint64_t* rows; /* NULL = all rows */
    uint64_t n_rows;
    uint32_t thread, n_threads;
    int mode; /* 0 = ref32, 1 = f64 */
    uint16_t* out16;
    double* out64;
    int status;
} job_t;

static void* run_job(void* p) {
    job_t* j = (job_t*)p;
    const geom_t* g = j->g;
    const aw_decode_desc* d = g->d;
    uint64_t ntok = ((uint64_t)d->hot_count + d->cold_count) * OR_BLOCK;
    float* qlf = (float*)malloc(sizeof(float) * (d->dict_size ? d->dict_size : 1));
    double* scores = (double*)malloc(sizeof(double) * (ntok ? ntok : 1));
    double* qld = (double*)malloc(sizeof(double) * (d->dict_size ? d->dict_size : 1));
    j->status = (qlf && scores && qld) ? AW_OK : AW_E_INVALID_ARG;
    for (uint64_t i = j->thread; i < j->n_rows && j->status == AW_OK; i += j->n_threads) {
        uint64_t row = j->rows ? j->rows[i] : i;
        if (j->mode == 0)
            j->status = ref32_row(g, row, j->out16 + i * d->head_dim, qlf);
        else
            j->status = f64_row(g, row, j->out64 + i * d->head_dim, scores, qld);
    }
    free(qlf);
    free(scores);
    free(qld);
    return NULL;
}

static int run_rows(const aw_decode_desc* d, const uint64_t* rows, uint64_t n_rows, int threads,
                    int mode, uint16_t* out16, double* out64) {
    geom_t g;
    int st = geom_init(d, &g);
    if (st) return st;
    uint64_t total = (uint64_t)d->layers * d->batch * d->queries * d->q_heads;
    if (!rows) n_rows = total;
    for (uint64_t i = 0; rows && i < n_rows; ++i)
        if (rows[i] >= total) return AW_E_INVALID_ARG;
    if (threads < 1) threads = 1;
    if ((uint64_t)threads > n_rows) threads = n_rows ? (int)n_rows : 1;
    job_t* jobs = (job_t*)calloc((size_t)threads, sizeof(job_t));
    pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    if (!jobs || !tids) { free(jobs); free(tids); return AW_E_INVALID_ARG; }
    for (int t = 0; t < threads; ++t) {
        jobs[t] = (job_t){&g, rows, n_rows, (uint32_t)t, (uint32_t)threads, mode, out16, out64, AW_OK};
        if (t > 0) pthread_create(&tids[t], NULL, run_job, &jobs[t]);
    }
    run_job(&jobs[0]);
    for (int t = 1; t < threads; ++t) pthread_join(tids[t], NULL);
    st = AW_OK;
    for (int t = 0; t < threads; ++t)
        if (jobs[t].status != AW_OK) st = jobs[t].status;
    free(jobs);
    free(tids);
    return st;
}

/* All rows of the fp32 restatement -> out f16 [L][B][Q][Hq][d]. */
int or_decode_ref32(const aw_decode_desc* d, int threads) {
    if (!d || !d->out) return AW_E_INVALID_ARG;
    return run_rows(d, NULL, 0, threads, 0, d->out, NULL);
}

/* Selected rows of the fp32 restatement -> out16 [n_rows][d]. */
int or_decode_ref32_rows(const aw_decode_desc* d, const uint64_t* rows, uint64_t n_rows,
                         uint16_t* out16, int threads) {
    return run_rows(d, rows, n_rows, threads, 0, out16, NULL);
}

/* fp64 brute force for selected rows (rows == NULL: all) -> out64 [n][d]. */
int or_decode_f64(const aw_decode_desc* d, const uint64_t* rows, uint64_t n_rows, double* out64,
                  int threads) {
    return run_rows(d, rows, n_rows, threads, 1, NULL, out64);
}

/* q . D^T in double -> out [L][B][Q][Hq][A]. */
int or_qlatent_f64(const aw_decode_desc* d, double* out) {
    geom_t g;
    int st = geom_init(d, &g);
    if (st) return st;
    const uint32_t D = d->head_dim, A = d->dict_size;
    uint64_t total = (uint64_t)d->layers * d->batch * d->queries * d->q_heads;
    for (uint64_t row = 0; row < total; ++row) {
        uint32_t l, b, q, h;
        row_split(&g, row, &l, &b, &q, &h);
        uint32_t kvh = h / g.G;
        const uint16_t* dict =
            d->dict ? d->dict + l * g.dict_layer + (d->dict_heads == 1 ? 0 : (uint64_t)kvh * A * D) : NULL;
        for (uint32_t a = 0; a < A; ++a) {
            double s = 0.0;
            for (uint32_t i = 0; i < D; ++i)
                s += (double)or_h2f(d->q[row * D + i]) * (double)or_h2f(dict[(uint64_t)a * D + i]);
            out[row * A + a] = s;
        }
    }
    return AW_OK;
}

/* SparseCode decode + atom gather, bit-exact (metal:182-216). */
int or_gather_codes(const aw_sparse_code* codes, uint64_t n, const uint16_t* dict, uint32_t dict_size,
                    uint32_t head_dim, uint32_t* idx, float* coef, uint16_t* atoms) {
    for (uint64_t i = 0; i < n; ++i)
        for (int k = 0; k < 4; ++k) {
            uint32_t a = codes[i].indices[k];
            idx[4 * i + k] = a;
            coef[4 * i + k] = or_h2f(codes[i].coeffs[k]);
            for (uint32_t j = 0; j < head_dim; ++j)
                atoms[(4 * i + k) * head_dim + j] = a < dict_size ? dict[(uint64_t)a * head_dim + j] : 0xFFFFu;
        }
    return AW_OK;
}

/* ------------------------------------------------------ SparseCode encoder */

typedef struct {
    float s;
    uint32_t a;
} or_scored;

/* score descending, index ascending; NaN after every number */
static int or_scored_cmp(const void* x, const void* y) {
    const or_scored* p = (const or_scored*)x;
    const or_scored* q = (const or_scored*)y;
    const int pn = isnan(p->s), qn = isnan(q->s);
    if (pn != qn) return pn - qn;
    if (!pn && p->s != q->s) return p->s > q->s ? -1 : 1;
    return p->a < q->a ? -1 : (p->a > q->a ? 1 : 0);
}

/* distiller.rs:126-159 */
float or_block_entropy(const uint16_t* vals, uint64_t n) {
    if (n == 0) return 0.0f;
    int all_zero = 1;
    for (uint64_t i = 0; i < n; ++i)
        if (or_h2f(vals[i]) != 0.0f) {
            all_zero = 0;
            break;
        }
    if (all_zero) return 0.0f;
    double sum = -0.0;
    for (uint64_t i = 0; i < n; ++i) sum += (double)or_h2f(vals[i]);
    const double mean = sum / (double)n;
    double var = -0.0;
    for (uint64_t i = 0; i < n; ++i) {
        const double diff = (double)or_h2f(vals[i]) - mean;
        var += diff * diff;
    }
    return (float)(var / (double)n);
}

/* distiller.rs:171-246 over a list of blocks: hot block src[i] -> cold block
 * dst[i] (dst NULL: the same index).  cold is [cold_blocks][16][kv_heads], or
 * [cold_blocks][kv_heads][16] when head_blocked. */
int or_encode_blocks(const uint16_t* hot, uint64_t hot_blocks, uint32_t kv_heads, uint32_t head_dim,
                     const uint16_t* dict, uint32_t dict_size, uint32_t dict_heads, const uint32_t* src,
                     const uint32_t* dst, uint32_t n_blocks, aw_sparse_code* cold, uint64_t cold_blocks,
                     int head_blocked, float* entropy) {
    if (!kv_heads || !head_dim || !dict_size || (dict_heads != 1 && dict_heads != kv_heads)) return AW_E_INVALID_ARG;
    or_scored* sc = (or_scored*)malloc(sizeof(or_scored) * dict_size);
    float* x = (float*)malloc(sizeof(float) * head_dim);
    if (!sc || !x) {
        free(sc);
        free(x);
        return AW_E_INVALID_ARG;
    }
    const uint64_t per_block = (uint64_t)OR_BLOCK * kv_heads * head_dim;
    for (uint32_t i = 0; i < n_blocks; ++i) {
        const uint32_t b = src[i] & OR_REF_MASK, c = dst ? (dst[i] & OR_REF_MASK) : b;
        if (b >= hot_blocks || c >= cold_blocks) {
            free(sc);
            free(x);
            return AW_E_OOB;
        }
        const uint16_t* blk = hot + (uint64_t)b * per_block;
        if (entropy) entropy[i] = or_block_entropy(blk, per_block);
        for (uint32_t t = 0; t < OR_BLOCK; ++t)
            for (uint32_t g = 0; g < kv_heads; ++g) {
                const uint16_t* xv = blk + ((uint64_t)t * kv_heads + g) * head_dim;
                for (uint32_t j = 0; j < head_dim; ++j) x[j] = or_h2f(xv[j]);
                const uint16_t* D = dict + (uint64_t)(dict_heads == 1 ? 0 : g) * dict_size * head_dim;
                for (uint32_t a = 0; a < dict_size; ++a) {
                    float acc = -0.0f; /* compiled without FMA contraction: product, then sum */
                    for (uint32_t j = 0; j < head_dim; ++j) acc = acc + x[j] * or_h2f(D[(uint64_t)a * head_dim + j]);
                    sc[a].s = acc;
                    sc[a].a = a;
                }
                qsort(sc, dict_size, sizeof(or_scored), or_scored_cmp);
                aw_sparse_code code;
                memset(&code, 0, sizeof code);
                for (int k = 0; k < 4 && (uint32_t)k < dict_size; ++k) {
                    if (isnan(sc[k].s) || sc[k].s == -INFINITY) break; /* never chosen: the zero code's slot */
                    code.indices[k] = (uint16_t)sc[k].a;
                    code.coeffs[k] = or_f2h(sc[k].s);
                }
                const uint64_t o = head_blocked ? ((uint64_t)c * kv_heads + g) * OR_BLOCK + t
                                                : ((uint64_t)c * OR_BLOCK + t) * kv_heads + g;
                cold[o] = code;
            }
    }
    free(sc);
    free(x);
    return AW_OK;
}
