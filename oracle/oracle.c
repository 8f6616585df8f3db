/*
 * CPU oracle for the FLAT-ATTENTION hot path — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates the reference crate's scalar Rust oracles in C. Compile with -ffp-contract=off:
 * Rust never fuses a*b+c, so neither may this file. f32::exp/ln/powf/sin/cos map to glibc
 * expf/logf/powf/sinf/cosf, f32::max to fmaxf, f32::recip to 1.0f/x.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "../include/flat_hip.h"

/* ------------------------------------------------------------------ helpers ---------- */

static int mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
    if (a != 0 && b > UINT64_MAX / a) return 0;
    *out = a * b;
    return 1;
}

int ora_resolved_scale(int has_scale, float scale, uint64_t head_dim, float* out) {
    /* src/lib.rs:257-272 */
    if (head_dim == 0) return FA_ERR_ZERO_DIMENSION;
    float s = has_scale ? scale : 1.0f / sqrtf((float)head_dim);
    if (!isfinite(s) || s <= 0.0f) return FA_ERR_INVALID_SCALE;
    *out = s;
    return FA_OK;
}

/* rotated_pair src/rotary_grouped.rs:37-50 (identical in src/projection_asymmetric.rs:70-83). */
static inline void rotated_pair(float even, float odd, uint64_t pair, uint64_t head_dim,
                                uint64_t position, float theta, float* re, float* ro) {
    float exponent = -2.0f * (float)pair / (float)head_dim;
    float frequency = powf(theta, exponent);
    float angle = (float)position * frequency;
    float s = sinf(angle);
    float c = cosf(angle);
    *re = even * c - odd * s;
    *ro = even * s + odd * c;
}

/* One online-softmax step, src/lib.rs:491-507. */
static inline void online_update(float score, float* running_max, float* running_sum,
                                 float* out_row, const float* v_row, uint64_t dim) {
    float new_max = fmaxf(*running_max, score);
    float alpha = isinf(*running_max) ? 0.0f : expf(*running_max - new_max);
    float p = expf(score - new_max);
    for (uint64_t d = 0; d < dim; ++d) out_row[d] = out_row[d] * alpha + p * v_row[d];
    *running_sum = *running_sum * alpha + p;
    *running_max = new_max;
}

static inline void finish_row(float* out_row, uint64_t dim, float running_max,
                              float running_sum, float* lse) {
    float inv_sum = 1.0f / running_sum; /* f32::recip */
    for (uint64_t d = 0; d < dim; ++d) out_row[d] *= inv_sum;
    *lse = running_max + logf(running_sum);
}

/* ------------------------------------------------------------------ unit threading --- */

typedef void (*unit_fn)(void* args, uint64_t unit);

typedef struct {
    unit_fn fn;
    void* args;
    uint64_t begin, end;
} worker_t;

static void* worker_main(void* p) {
    worker_t* w = (worker_t*)p;
    for (uint64_t u = w->begin; u < w->end; ++u) w->fn(w->args, u);
    return NULL;
}

static void run_units(unit_fn fn, void* args, uint64_t total, uint64_t begin, uint64_t end,
                      int threads) {
    if (end > total) end = total;
    if (begin >= end) return;
    uint64_t n = end - begin;
    if (threads <= 1 || n == 1) {
        for (uint64_t u = begin; u < end; ++u) fn(args, u);
        return;
    }
    if ((uint64_t)threads > n) threads = (int)n;
    pthread_t* tid = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    worker_t* ws = (worker_t*)calloc((size_t)threads, sizeof(worker_t));
    uint64_t per = n / (uint64_t)threads, rem = n % (uint64_t)threads, cur = begin;
    for (int t = 0; t < threads; ++t) {
        uint64_t cnt = per + ((uint64_t)t < rem ? 1 : 0);
        ws[t].fn = fn;
        ws[t].args = args;
        ws[t].begin = cur;
        ws[t].end = cur + cnt;
        cur += cnt;
        pthread_create(&tid[t], NULL, worker_main, &ws[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(tid);
    free(ws);
}

/* ------------------------------------------------------------------ grouped core ------ */
/* forward_reference (src/lib.rs:454) is forward_reference_grouped with q_heads == kv_heads;
 * forward_reference_grouped (src/grouped.rs:81) and forward_reference_grouped_rope
 * (src/rotary_grouped.rs:57) share the loop nest and differ only in the dot product. */

typedef struct {
    const float *q, *k, *v;
    uint64_t q_heads, kv_heads, seq, dim;
    int causal, rope;
    float scale, theta;
    uint64_t position_offset;
    float *out, *lse;
} grouped_args;

static void grouped_unit(void* p, uint64_t unit) {
    const grouped_args* a = (const grouped_args*)p;
    uint64_t batch = unit / a->q_heads, q_head = unit % a->q_heads;
    uint64_t group_size = a->q_heads / a->kv_heads;
    uint64_t kv_head = q_head / group_size;
    uint64_t q_bh = batch * a->q_heads + q_head;
    uint64_t kv_bh = batch * a->kv_heads + kv_head;
    uint64_t head_stride = a->seq * a->dim;
    uint64_t q_head_base = q_bh * head_stride, kv_head_base = kv_bh * head_stride;
    uint64_t lse_base = q_bh * a->seq;
    for (uint64_t qp = 0; qp < a->seq; ++qp) {
        uint64_t q_base = q_head_base + qp * a->dim;
        float* orow = a->out + q_base;
        float running_max = -INFINITY, running_sum = 0.0f;
        for (uint64_t kp = 0; kp < a->seq; ++kp) {
            if (a->causal && kp > qp) break;
            uint64_t kv_base = kv_head_base + kp * a->dim;
            float dot = 0.0f;
            if (a->rope) {
                for (uint64_t pair = 0; pair < a->dim / 2; ++pair) {
                    uint64_t d = 2 * pair;
                    float qe, qo, ke, ko;
                    rotated_pair(a->q[q_base + d], a->q[q_base + d + 1], pair, a->dim,
                                 a->position_offset + qp, a->theta, &qe, &qo);
                    rotated_pair(a->k[kv_base + d], a->k[kv_base + d + 1], pair, a->dim,
                                 a->position_offset + kp, a->theta, &ke, &ko);
                    dot += qe * ke;
                    dot += qo * ko;
                }
            } else {
                for (uint64_t d = 0; d < a->dim; ++d) dot += a->q[q_base + d] * a->k[kv_base + d];
            }
            float score = dot * a->scale;
            online_update(score, &running_max, &running_sum, orow, a->v + kv_base, a->dim);
        }
        finish_row(orow, a->dim, running_max, running_sum, &a->lse[lse_base + qp]);
    }
}

static int grouped_common(const float* q, const float* k, const float* v, uint64_t batch,
                          uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                          int causal, float scale, int rope, float theta, uint64_t offset,
                          float* out, float* lse, uint64_t ub, uint64_t ue, int threads) {
    if (!batch || !q_heads || !kv_heads || !seq || !dim) return FA_ERR_ZERO_DIMENSION;
    if (q_heads % kv_heads) return FA_ERR_INVALID_HEAD_GROUPING;
    if (rope) {
        if (dim % 2) return FA_ERR_INVALID_ROTARY_HEAD_DIM;
        if (!isfinite(theta) || theta <= 0.0f) return FA_ERR_INVALID_ROTARY_THETA;
        if (offset > UINT64_MAX - (seq - 1)) return FA_ERR_POSITION_OVERFLOW;
    }
    if (!isfinite(scale) || scale <= 0.0f) return FA_ERR_INVALID_SCALE;
    uint64_t units, qlen;
    if (!mul_ok(batch, q_heads, &units) || !mul_ok(units, seq, &qlen) ||
        !mul_ok(qlen, dim, &qlen))
        return FA_ERR_SHAPE_OVERFLOW;
    grouped_args a = {q, k, v, q_heads, kv_heads, seq, dim, causal, rope, scale, theta,
                      offset, out, lse};
    /* outputs start zeroed (vec![0.0; len]) */
    uint64_t e = ue > units ? units : ue;
    if (ub < e) {
        memset(out + ub * seq * dim, 0, (size_t)((e - ub) * seq * dim) * sizeof(float));
    }
    run_units(grouped_unit, &a, units, ub, ue, threads);
    return FA_OK;
}

int ora_forward(const float* q, const float* k, const float* v, uint64_t batch, uint64_t heads,
                uint64_t seq, uint64_t dim, int causal, float scale, float* out, float* lse,
                uint64_t ub, uint64_t ue, int threads) {
    return grouped_common(q, k, v, batch, heads, heads, seq, dim, causal, scale, 0, 0.0f, 0, out,
                          lse, ub, ue, threads);
}

int ora_forward_grouped(const float* q, const float* k, const float* v, uint64_t batch,
                        uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                        int causal, float scale, float* out, float* lse, uint64_t ub,
                        uint64_t ue, int threads) {
    return grouped_common(q, k, v, batch, q_heads, kv_heads, seq, dim, causal, scale, 0, 0.0f, 0,
                          out, lse, ub, ue, threads);
}

int ora_forward_grouped_rope(const float* q, const float* k, const float* v, uint64_t batch,
                             uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                             int causal, float scale, float theta, uint64_t position_offset,
                             float* out, float* lse, uint64_t ub, uint64_t ue, int threads) {
    return grouped_common(q, k, v, batch, q_heads, kv_heads, seq, dim, causal, scale, 1, theta,
                          position_offset, out, lse, ub, ue, threads);
}

/* ------------------------------------------------------------------ asymmetric -------- */
/* src/projection_asymmetric.rs:97-238. projection_index (:45-67) =
 * ((batch*seq_len + position) * heads + head) * head_dim + dim. */

typedef struct {
    const float *q, *k, *v;
    uint64_t q_heads, kv_heads, query_len, kv_len, dim, qpos_off;
    int causal, use_rope, rotate_k;
    float scale, theta;
    uint64_t q_rope_off, kv_rope_off;
    float *out, *lse;
} asym_args;

static void asym_unit(void* p, uint64_t unit) {
    const asym_args* a = (const asym_args*)p;
    uint64_t batch = unit / a->q_heads, q_head = unit % a->q_heads;
    uint64_t group_size = a->q_heads / a->kv_heads;
    uint64_t kv_head = q_head / group_size;
    uint64_t lse_base = (batch * a->q_heads + q_head) * a->query_len;
    uint64_t qw = a->q_heads * a->dim, kw = a->kv_heads * a->dim;
    for (uint64_t qp = 0; qp < a->query_len; ++qp) {
        uint64_t causal_pos = a->qpos_off + qp;
        uint64_t q_rot_pos = a->q_rope_off + qp;
        uint64_t q_base = (batch * a->query_len + qp) * qw + q_head * a->dim;
        float* orow = a->out + q_base;
        float running_max = -INFINITY, running_sum = 0.0f;
        for (uint64_t kp = 0; kp < a->kv_len; ++kp) {
            if (a->causal && kp > causal_pos) break;
            uint64_t k_rot_pos = a->kv_rope_off + kp;
            uint64_t k_base = (batch * a->kv_len + kp) * kw + kv_head * a->dim;
            float dot = 0.0f;
            if (a->use_rope) {
                for (uint64_t pair = 0; pair < a->dim / 2; ++pair) {
                    uint64_t d = 2 * pair;
                    float qe, qo, ke, ko;
                    rotated_pair(a->q[q_base + d], a->q[q_base + d + 1], pair, a->dim, q_rot_pos,
                                 a->theta, &qe, &qo);
                    if (a->rotate_k) {
                        rotated_pair(a->k[k_base + d], a->k[k_base + d + 1], pair, a->dim,
                                     k_rot_pos, a->theta, &ke, &ko);
                    } else {
                        ke = a->k[k_base + d];
                        ko = a->k[k_base + d + 1];
                    }
                    dot += qe * ke;
                    dot += qo * ko;
                }
            } else {
                for (uint64_t d = 0; d < a->dim; ++d) dot += a->q[q_base + d] * a->k[k_base + d];
            }
            float score = dot * a->scale;
            online_update(score, &running_max, &running_sum, orow, a->v + k_base, a->dim);
        }
        finish_row(orow, a->dim, running_max, running_sum, &a->lse[lse_base + qp]);
    }
}

int ora_forward_projection_asymmetric(const float* q, const float* k, const float* v,
                                      uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                                      uint64_t query_len, uint64_t kv_len, uint64_t dim,
                                      uint64_t qpos_off, int causal, float scale, int use_rope,
                                      float theta, uint64_t q_rope_offset,
                                      uint64_t kv_rope_offset, int rotate_k, float* out,
                                      float* lse, uint64_t ub, uint64_t ue, int threads) {
    if (!batch || !q_heads || !kv_heads || !query_len || !kv_len || !dim)
        return FA_ERR_ZERO_DIMENSION;
    if (q_heads % kv_heads) return FA_ERR_INVALID_HEAD_GROUPING;
    if (use_rope) {
        if (dim % 2) return FA_ERR_INVALID_ROTARY_HEAD_DIM;
        if (!isfinite(theta) || theta <= 0.0f) return FA_ERR_INVALID_ROTARY_THETA;
        if (q_rope_offset > UINT64_MAX - (query_len - 1) ||
            kv_rope_offset > UINT64_MAX - (kv_len - 1))
            return FA_ERR_POSITION_OVERFLOW;
    }
    if (qpos_off > UINT64_MAX - (query_len - 1)) return FA_ERR_POSITION_OVERFLOW;
    if (!isfinite(scale) || scale <= 0.0f) return FA_ERR_INVALID_SCALE;
    uint64_t units = batch * q_heads;
    asym_args a = {q, k, v, q_heads, kv_heads, query_len, kv_len, dim, qpos_off, causal,
                   use_rope, rotate_k, scale, theta, q_rope_offset, kv_rope_offset, out, lse};
    /* zero the output rows of the selected units */
    uint64_t e = ue > units ? units : ue;
    for (uint64_t u = ub; u < e; ++u) {
        uint64_t b = u / q_heads, h = u % q_heads;
        for (uint64_t qp = 0; qp < query_len; ++qp)
            memset(out + (b * query_len + qp) * q_heads * dim + h * dim, 0, dim * sizeof(float));
    }
    run_units(asym_unit, &a, units, ub, ue, threads);
    return FA_OK;
}

/* ------------------------------------------------------------------ chunked ----------- */
/* src/chunked_projection_prefill.rs:63-169: per chunk, copy the Q rows of every batch,
 * run the asymmetric oracle with query_len = chunk, kv_len = seq, causal offset = start,
 * q-RoPE offset = offset + start, kv-RoPE offset = offset, then scatter O and LSE back. */
int ora_chunked_prefill(const float* q, const float* k, const float* v, uint64_t batch,
                        uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                        int causal, float scale, float theta, uint64_t position_offset,
                        uint64_t chunk, float* out, float* lse) {
    if (chunk == 0) return FA_ERR_ZERO_QUERY_CHUNK_SIZE;
    if (!batch || !q_heads || !kv_heads || !seq || !dim) return FA_ERR_ZERO_DIMENSION;
    if (q_heads % kv_heads) return FA_ERR_INVALID_HEAD_GROUPING;
    uint64_t qw = q_heads * dim;
    float* cq = (float*)malloc(sizeof(float) * batch * chunk * qw);
    float* co = (float*)malloc(sizeof(float) * batch * chunk * qw);
    float* cl = (float*)malloc(sizeof(float) * batch * q_heads * chunk);
    int rc = FA_OK;
    for (uint64_t start = 0; start < seq; ) {
        uint64_t len = chunk < seq - start ? chunk : seq - start;
        for (uint64_t b = 0; b < batch; ++b)
            memcpy(cq + b * len * qw, q + (b * seq + start) * qw, sizeof(float) * len * qw);
        rc = ora_forward_projection_asymmetric(cq, k, v, batch, q_heads, kv_heads, len, seq, dim,
                                               start, causal, scale, 1, theta,
                                               position_offset + start, position_offset, 1, co,
                                               cl, 0, UINT64_MAX, 1);
        if (rc) break;
        for (uint64_t b = 0; b < batch; ++b) {
            memcpy(out + (b * seq + start) * qw, co + b * len * qw, sizeof(float) * len * qw);
            for (uint64_t h = 0; h < q_heads; ++h)
                memcpy(lse + (b * q_heads + h) * seq + start, cl + (b * q_heads + h) * len,
                       sizeof(float) * len);
        }
        start += len;
    }
    free(cq);
    free(co);
    free(cl);
    return rc;
}

/* ------------------------------------------------------------------ RoPE rows --------- */
int ora_rope_rotate_rows(const float* in, float* out, uint64_t rows, uint64_t heads,
                         uint64_t dim, float theta, uint64_t position_offset,
                         const int64_t* positions) {
    if (dim % 2) return FA_ERR_INVALID_ROTARY_HEAD_DIM;
    uint64_t w = heads * dim;
    for (uint64_t r = 0; r < rows; ++r) {
        uint64_t pos = positions ? (uint64_t)positions[r] : position_offset + r;
        for (uint64_t h = 0; h < heads; ++h) {
            uint64_t base = r * w + h * dim;
            for (uint64_t pair = 0; pair < dim / 2; ++pair) {
                float re, ro;
                rotated_pair(in[base + 2 * pair], in[base + 2 * pair + 1], pair, dim, pos, theta,
                             &re, &ro);
                out[base + 2 * pair] = re;
                out[base + 2 * pair + 1] = ro;
            }
        }
    }
    return FA_OK;
}

/* ------------------------------------------------------------------ paged ------------- */

static void gather_rows(const float* pool, uint64_t page_size, const int32_t* table,
                        uint64_t n_tokens, uint64_t width, float* dst) {
    for (uint64_t key = 0; key < n_tokens; ++key) {
        uint64_t lp = key / page_size, off = key % page_size;
        uint64_t row = (uint64_t)table[lp] * page_size + off;
        memcpy(dst + key * width, pool + row * width, sizeof(float) * width);
    }
}

typedef struct {
    const float *q, *kp, *vp;
    uint64_t physical_pages, page_size, max_pages;
    const int32_t *bt, *ctx, *qpos;
    uint64_t q_heads, kv_heads, dim;
    int causal;
    float scale, theta;
    float *out, *lse;
    int rc;
} pdec_args;

static void pdec_unit(void* p, uint64_t s) {
    pdec_args* a = (pdec_args*)p;
    uint64_t n = (uint64_t)a->ctx[s], w = a->kv_heads * a->dim;
    uint64_t qp = a->qpos ? (uint64_t)a->qpos[s] : n - 1;
    float* kc = (float*)malloc(sizeof(float) * n * w);
    float* vc = (float*)malloc(sizeof(float) * n * w);
    gather_rows(a->kp, a->page_size, a->bt + s * a->max_pages, n, w, kc);
    gather_rows(a->vp, a->page_size, a->bt + s * a->max_pages, n, w, vc);
    int rc = ora_forward_projection_asymmetric(
        a->q + s * a->q_heads * a->dim, kc, vc, 1, a->q_heads, a->kv_heads, 1, n, a->dim, qp,
        a->causal, a->scale, 1, a->theta, qp, 0, 0, a->out + s * a->q_heads * a->dim,
        a->lse + s * a->q_heads, 0, UINT64_MAX, 1);
    if (rc) a->rc = rc;
    free(kc);
    free(vc);
}

int ora_paged_decode(const float* q, const float* k_pool, const float* v_pool,
                     uint64_t physical_pages, uint64_t page_size, const int32_t* block_tables,
                     uint64_t max_pages, const int32_t* ctx_lens, const int32_t* q_positions,
                     uint64_t n_seqs, uint64_t q_heads, uint64_t kv_heads, uint64_t dim,
                     int causal, float scale, float theta, float* out, float* lse,
                     uint64_t sb, uint64_t se, int threads) {
    if (!page_size || !n_seqs || !q_heads || !kv_heads || !dim) return FA_ERR_ZERO_DIMENSION;
    for (uint64_t s = 0; s < n_seqs; ++s) {
        if (ctx_lens[s] <= 0) return FA_ERR_EMPTY_TABLE;
        uint64_t pages = ((uint64_t)ctx_lens[s] + page_size - 1) / page_size;
        if (pages > max_pages) return FA_ERR_INDEX_SPACE_EXCEEDED;
        for (uint64_t p = 0; p < pages; ++p) {
            int32_t id = block_tables[s * max_pages + p];
            if (id < 0 || (uint64_t)id >= physical_pages) return FA_ERR_INVALID_PAGE;
        }
    }
    pdec_args a = {q, k_pool, v_pool, physical_pages, page_size, max_pages, block_tables,
                   ctx_lens, q_positions, q_heads, kv_heads, dim, causal, scale, theta, out,
                   lse, 0};
    run_units(pdec_unit, &a, n_seqs, sb, se, threads);
    return a.rc;
}

typedef struct {
    const float *q, *kp, *vp;
    uint64_t page_size, max_pages;
    const int32_t* bt;
    uint64_t q_heads, kv_heads, query_len, kv_len, dim, qoff;
    int causal;
    float scale, theta;
    uint64_t q_rope_off;
    float *out, *lse;
    int rc;
} ppre_args;

static void ppre_unit(void* p, uint64_t s) {
    ppre_args* a = (ppre_args*)p;
    uint64_t w = a->kv_heads * a->dim, qw = a->q_heads * a->dim;
    float* kc = (float*)malloc(sizeof(float) * a->kv_len * w);
    float* vc = (float*)malloc(sizeof(float) * a->kv_len * w);
    gather_rows(a->kp, a->page_size, a->bt + s * a->max_pages, a->kv_len, w, kc);
    gather_rows(a->vp, a->page_size, a->bt + s * a->max_pages, a->kv_len, w, vc);
    int rc = ora_forward_projection_asymmetric(
        a->q + s * a->query_len * qw, kc, vc, 1, a->q_heads, a->kv_heads, a->query_len,
        a->kv_len, a->dim, a->qoff, a->causal, a->scale, 1, a->theta, a->q_rope_off, 0, 0,
        a->out + s * a->query_len * qw, a->lse + s * a->q_heads * a->query_len, 0, UINT64_MAX,
        1);
    if (rc) a->rc = rc;
    free(kc);
    free(vc);
}

int ora_paged_prefill(const float* q, const float* k_pool, const float* v_pool,
                      uint64_t physical_pages, uint64_t page_size, const int32_t* block_tables,
                      uint64_t max_pages, uint64_t n_seqs, uint64_t q_heads, uint64_t kv_heads,
                      uint64_t query_len, uint64_t kv_len, uint64_t dim, uint64_t qoff,
                      int causal, float scale, float theta, uint64_t q_rope_offset, float* out,
                      float* lse, uint64_t sb, uint64_t se, int threads) {
    if (!page_size || !n_seqs || !q_heads || !kv_heads || !dim || !query_len || !kv_len)
        return FA_ERR_ZERO_DIMENSION;
    uint64_t pages = (kv_len + page_size - 1) / page_size;
    if (pages > max_pages) return FA_ERR_INDEX_SPACE_EXCEEDED;
    for (uint64_t s = 0; s < n_seqs; ++s)
        for (uint64_t p = 0; p < pages; ++p) {
            int32_t id = block_tables[s * max_pages + p];
            if (id < 0 || (uint64_t)id >= physical_pages) return FA_ERR_INVALID_PAGE;
        }
    ppre_args a = {q, k_pool, v_pool, page_size, max_pages, block_tables, q_heads, kv_heads,
                   query_len, kv_len, dim, qoff, causal, scale, theta, q_rope_offset, out, lse,
                   0};
    run_units(ppre_unit, &a, n_seqs, sb, se, threads);
    return a.rc;
}

/* ------------------------------------------------------------------ 16-bit formats ---- */

/* F16::from_f32 src/f16.rs:26-80 */
/* ------------------------------------------------------------------ recompute backward */
/* backward_reference_grouped src/backward_grouped.rs:17-95 (backward_reference
 * src/backward.rs:27 is its q_heads == kv_heads case). One unit is one (batch, kv head): its
 * query heads run in ascending order inside the unit, so the dK/dV accumulation order of every
 * element is the reference's (batch, q_head, query, key) order. */
typedef struct {
    const float *q, *k, *v, *d_out, *out, *lse;
    uint64_t q_heads, kv_heads, seq, dim;
    int causal;
    float scale;
    float *dq, *dk, *dv;
} bwd_args;

static void bwd_unit(void* p, uint64_t unit) {
    const bwd_args* a = (const bwd_args*)p;
    uint64_t batch = unit / a->kv_heads, kv_head = unit % a->kv_heads;
    uint64_t group_size = a->q_heads / a->kv_heads;
    uint64_t head_stride = a->seq * a->dim;
    uint64_t kv_bh = batch * a->kv_heads + kv_head;
    uint64_t kv_head_base = kv_bh * head_stride;
    for (uint64_t q_head = kv_head * group_size; q_head < (kv_head + 1) * group_size; ++q_head) {
        uint64_t q_bh = batch * a->q_heads + q_head;
        uint64_t q_head_base = q_bh * head_stride, lse_base = q_bh * a->seq;
        for (uint64_t qp = 0; qp < a->seq; ++qp) {
            uint64_t q_base = q_head_base + qp * a->dim;
            float lse = a->lse[lse_base + qp];
            float delta = 0.0f;
            for (uint64_t d = 0; d < a->dim; ++d) delta += a->d_out[q_base + d] * a->out[q_base + d];
            uint64_t key_limit = a->causal ? qp + 1 : a->seq;
            for (uint64_t kp = 0; kp < key_limit; ++kp) {
                uint64_t kv_base = kv_head_base + kp * a->dim;
                float dot_qk = 0.0f, d_probability = 0.0f;
                for (uint64_t d = 0; d < a->dim; ++d) {
                    dot_qk += a->q[q_base + d] * a->k[kv_base + d];
                    d_probability += a->d_out[q_base + d] * a->v[kv_base + d];
                }
                float score = dot_qk * a->scale;
                float probability = expf(score - lse);
                float d_score = probability * (d_probability - delta);
                float d_dot = d_score * a->scale;
                for (uint64_t d = 0; d < a->dim; ++d) {
                    a->dq[q_base + d] += d_dot * a->k[kv_base + d];
                    a->dk[kv_base + d] += d_dot * a->q[q_base + d];
                    a->dv[kv_base + d] += probability * a->d_out[q_base + d];
                }
            }
        }
    }
}

int ora_backward_grouped(const float* q, const float* k, const float* v, const float* d_out,
                         const float* out, const float* lse, uint64_t batch, uint64_t q_heads,
                         uint64_t kv_heads, uint64_t seq, uint64_t dim, int causal, float scale,
                         float* dq, float* dk, float* dv, int threads) {
    /* GroupedAttentionShape::validate src/grouped.rs:24 */
    if (!batch || !q_heads || !kv_heads || !seq || !dim) return FA_ERR_ZERO_DIMENSION;
    if (q_heads % kv_heads) return FA_ERR_INVALID_HEAD_GROUPING;
    if (!isfinite(scale) || scale <= 0.0f) return FA_ERR_INVALID_SCALE;
    uint64_t qn, kvn, units;
    if (!mul_ok(batch, q_heads, &qn) || !mul_ok(qn, seq, &qn) || !mul_ok(qn, dim, &qn) ||
        !mul_ok(batch, kv_heads, &units) || !mul_ok(units, seq, &kvn) || !mul_ok(kvn, dim, &kvn))
        return FA_ERR_SHAPE_OVERFLOW;
    memset(dq, 0, (size_t)qn * sizeof(float));
    memset(dk, 0, (size_t)kvn * sizeof(float));
    memset(dv, 0, (size_t)kvn * sizeof(float));
    bwd_args a = {q, k, v, d_out, out, lse, q_heads, kv_heads, seq, dim, causal, scale,
                  dq, dk, dv};
    run_units(bwd_unit, &a, units, 0, units, threads);
    return FA_OK;
}

uint16_t ora_f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exponent = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mantissa = bits & 0x007fffffu;
    if (exponent == 0xff) {
        if (mantissa == 0) return sign | 0x7c00u;
        uint16_t payload = (uint16_t)(mantissa >> 13);
        if (payload == 0) payload = 1;
        return sign | 0x7c00u | payload;
    }
    int32_t he = exponent - 127 + 15;
    if (he >= 31) return sign | 0x7c00u;
    if (he <= 0) {
        if (he < -10) return sign;
        uint32_t m = mantissa | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - he);
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm += 1;
        return sign | (uint16_t)hm;
    }
    uint32_t hm = mantissa >> 13;
    uint32_t rem = mantissa & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) {
        hm += 1;
        if (hm == 0x400u) {
            hm = 0;
            he += 1;
            if (he >= 31) return sign | 0x7c00u;
        }
    }
    return sign | (uint16_t)((uint32_t)he << 10) | (uint16_t)hm;
}

/* F16::to_f32 src/f16.rs:82-109 */
float ora_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)(bits & 0x8000u)) << 16;
    uint32_t exponent = (bits >> 10) & 0x1fu;
    uint32_t mantissa = bits & 0x03ffu;
    uint32_t outb;
    if (exponent == 0) {
        if (mantissa == 0) {
            outb = sign;
        } else {
            uint32_t normalized = mantissa;
            int32_t e32 = 127 - 14;
            while ((normalized & 0x400u) == 0) {
                normalized <<= 1;
                e32 -= 1;
            }
            normalized &= 0x03ffu;
            outb = sign | ((uint32_t)e32 << 23) | (normalized << 13);
        }
    } else if (exponent == 0x1f) {
        outb = sign | 0x7f800000u | (mantissa << 13);
    } else {
        outb = sign | ((exponent + (127 - 15)) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &outb, 4);
    return f;
}

/* bfloat16: same round-to-nearest-even convention; NaN keeps a quiet payload. */
uint16_t ora_f32_to_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu)) {
        return (uint16_t)((bits >> 16) | 0x0040u);
    }
    uint32_t lsb = (bits >> 16) & 1u;
    bits += 0x7fffu + lsb;
    return (uint16_t)(bits >> 16);
}

float ora_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

void ora_f32_to_bf16_array(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ora_f32_to_bf16(in[i]);
}
void ora_bf16_to_f32_array(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ora_bf16_to_f32(in[i]);
}
void ora_f32_to_f16_array(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ora_f32_to_f16(in[i]);
}
void ora_f16_to_f32_array(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ora_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------ inputs ------------ */

void ora_fill_normal(float* out, uint64_t n, uint64_t seed) {
    uint64_t state = seed;
    for (uint64_t i = 0; i < n; i += 2) {
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        uint32_t a = (uint32_t)(state >> 32);
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        uint32_t b = (uint32_t)(state >> 32);
        double u1 = ((double)a + 1.0) / 4294967296.0; /* (0, 1] */
        double u2 = (double)b / 4294967296.0;         /* [0, 1) */
        double r = sqrt(-2.0 * log(u1));
        double t = 6.283185307179586 * u2;
        out[i] = (float)(r * cos(t));
        if (i + 1 < n) out[i + 1] = (float)(r * sin(t));
    }
}
