/*
 * CPU oracle for the attention path: test infrastructure only (see attn_oracle.h for the reference lines each
 * function follows). Double precision throughout; rows are independent and spread over pthreads.
 *
 * ORACLE_MUTANT (a build flag used only by the oracle's own tests) plants one known mistake, so the tests can
 * show that their checks catch it:
 *   1 mask off by one (j < pos)          2 GQA map h % kv_heads           3 lse without the maximum
 *   4 k and v swapped in the scores      5 cube_topk ties to the larger   6 sparse dense rows ignore valid
 *   7 heads: the second value of a rotated pair takes v c - u s          8 heads: the norm divides by the sum
 *   9 gathered lists read entries up to stride, not count[t]            10 probabilities not rounded to half
 *  11 proj: x not rounded to bf16 before the product                    12 proj: the weight read as w[k][n]
 *  13 kda_scan: the read of S k before the decay                          14 kda_scan: beta not applied
 */
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#ifndef ORACLE_MUTANT
#define ORACLE_MUTANT 0
#endif

/* ---- element types ---------------------------------------------------------------------------------------- */

float oracle_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * (1.0f / 16777216.0f);
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
        return (uint16_t)((u >> 16) | 0x40);
    const uint32_t lsb = (u >> 16) & 1;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

uint16_t oracle_f32_to_f16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) /* inf or NaN */
        return (uint16_t)(sign | 0x7c00 | (a > 0x7f800000u ? 0x200 : 0));
    if (a >= 0x477ff000u) /* rounds to >= 65520: overflow to inf */
        return (uint16_t)(sign | 0x7c00);
    if (a < 0x38800000u) { /* below the smallest normal half (2^-14): subnormal or zero */
        /* value = a_float; half subnormal unit = 2^-24; round(value / 2^-24) to nearest even */
        float af;
        memcpy(&af, &a, 4);
        const double q = (double)af * 16777216.0;
        double r = floor(q);
        const double frac = q - r;
        if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) != 0.0))
            r += 1.0;
        return (uint16_t)(sign | (uint16_t)r); /* r == 1024 becomes the smallest normal, as it should */
    }
    /* normal: rebias the exponent, round the 23-bit mantissa to 10 bits (nearest even) */
    const uint32_t lsb = (a >> 13) & 1;
    const uint32_t r = (a + 0xfffu + lsb) >> 13; /* carries into the exponent correctly */
    return (uint16_t)(sign | (uint16_t)(r - ((uint32_t)112 << 10)));
}

double oracle_load(const void* p, int dtype, size_t i)
{
    if (dtype == ORACLE_F32)
        return (double)((const float*)p)[i];
    const uint16_t b = ((const uint16_t*)p)[i];
    if (dtype == ORACLE_F16)
        return (double)oracle_f16_to_f32(b);
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

/* ---- a pool of threads over independent items --------------------------------------------------------------- */

typedef void (*item_fn)(void* ctx, size_t item, double* scratch);

typedef struct {
    item_fn fn;
    void* ctx;
    size_t n, scratch_len;
    size_t next;
    pthread_mutex_t mu;
} pool_t;

static void* pool_worker(void* arg)
{
    pool_t* p = (pool_t*)arg;
    double* scratch = (double*)malloc((p->scratch_len ? p->scratch_len : 1) * sizeof(double));
    for (;;) {
        pthread_mutex_lock(&p->mu);
        const size_t i0 = p->next;
        const size_t chunk = 4;
        p->next = i0 + chunk;
        pthread_mutex_unlock(&p->mu);
        if (i0 >= p->n)
            break;
        const size_t i1 = i0 + chunk < p->n ? i0 + chunk : p->n;
        for (size_t i = i0; i < i1; ++i)
            p->fn(p->ctx, i, scratch);
    }
    free(scratch);
    return NULL;
}

static void run_pool(item_fn fn, void* ctx, size_t n, size_t scratch_len, int nthreads)
{
    if (nthreads <= 0) {
        const long c = sysconf(_SC_NPROCESSORS_ONLN);
        nthreads = c > 0 ? (int)c : 1;
    }
    if ((size_t)nthreads > n)
        nthreads = n ? (int)n : 1;
    pool_t p = {fn, ctx, n, scratch_len, 0, PTHREAD_MUTEX_INITIALIZER};
    if (nthreads == 1) {
        pool_worker(&p);
        return;
    }
    pthread_t* t = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
    for (int i = 0; i < nthreads; ++i)
        pthread_create(&t[i], NULL, pool_worker, &p);
    for (int i = 0; i < nthreads; ++i)
        pthread_join(t[i], NULL);
    free(t);
}

/* ---- one row over an explicit key list (tests/sparse_attn_test.cpp:156-173) ------------------------------------ */

/* keys: n_keys indices into the kv head's rows (duplicates count twice, as a pass visited twice does). */
static void softmax_row(const void* q, const void* k, const void* v, int dtype, size_t q_off, size_t kv_off,
                        uint32_t dim, double scale, const uint32_t* keys, size_t n_keys, double* w, double* out,
                        double* lse)
{
    for (uint32_t d = 0; d < dim; ++d)
        out[d] = 0.0;
    if (n_keys == 0) { /* a fully masked row is zero (ops.metal:355) */
        if (lse)
            *lse = -INFINITY;
        return;
    }
    double mx = -INFINITY;
    for (size_t i = 0; i < n_keys; ++i) {
        const size_t kr = kv_off + (size_t)keys[i] * dim;
        double s = 0.0;
        for (uint32_t d = 0; d < dim; ++d)
#if ORACLE_MUTANT == 4
            s += oracle_load(q, dtype, q_off + d) * oracle_load(k == v ? k : v, dtype, kr + d);
#else
            s += oracle_load(q, dtype, q_off + d) * oracle_load(k, dtype, kr + d);
#endif
        w[i] = s * scale;
        if (w[i] > mx)
            mx = w[i];
    }
    double sum = 0.0;
    for (size_t i = 0; i < n_keys; ++i) {
        w[i] = exp(w[i] - mx);
        sum += w[i];
    }
    for (size_t i = 0; i < n_keys; ++i) {
        const double p = w[i] / sum;
        const size_t vr = kv_off + (size_t)keys[i] * dim;
        for (uint32_t d = 0; d < dim; ++d)
            out[d] += p * oracle_load(v, dtype, vr + d);
    }
    if (lse)
#if ORACLE_MUTANT == 3
        *lse = log(sum);
#else
        *lse = mx + log(sum);
#endif
}

static uint32_t kv_head_of(uint32_t h, uint32_t heads, uint32_t kv_heads)
{
#if ORACLE_MUTANT == 2
    (void)heads;
    return h % kv_heads;
#else
    return h / (heads / kv_heads);
#endif
}

/* ---- dense ------------------------------------------------------------------------------------------------------ */

typedef struct {
    const oracle_attn_args* a;
    uint32_t dim;
    int dtype;
    const void *q, *k, *v;
    const uint32_t* head_row; /* NULL: item = h * n_q + r over all rows */
    double *o, *lse;          /* full layout, or per item when head_row is set */
} dense_ctx;

/* The visible keys of query position pos (ops.metal:289). */
static size_t dense_keys(const oracle_attn_args* a, uint32_t pos, uint32_t* keys)
{
    size_t n = 0;
    for (uint32_t j = 0; j < a->n_k; ++j) {
#if ORACLE_MUTANT == 1
        const int seen = j < pos || (pos >= a->block && j >= a->block);
#else
        const int seen = j <= pos || (pos >= a->block && j >= a->block);
#endif
        if (seen)
            keys[n++] = j;
    }
    return n;
}

static void dense_item(void* vctx, size_t item, double* scratch)
{
    const dense_ctx* c = (const dense_ctx*)vctx;
    const oracle_attn_args* a = c->a;
    uint32_t h, r;
    if (c->head_row) {
        h = c->head_row[2 * item];
        r = c->head_row[2 * item + 1];
    } else {
        h = (uint32_t)(item / a->n_q);
        r = (uint32_t)(item % a->n_q);
    }
    const uint32_t dim = c->dim, kvh = kv_head_of(h, a->heads, a->kv_heads);
    uint32_t* keys = (uint32_t*)(scratch + a->n_k);
    const size_t n_keys = dense_keys(a, a->q_pos0 + r, keys);
    double* out;
    double* lse;
    if (c->head_row) {
        out = c->o + item * dim;
        lse = c->lse ? c->lse + item : NULL;
    } else {
        out = c->o + (size_t)r * a->width + (size_t)h * dim;
        lse = c->lse ? c->lse + (size_t)h * a->n_q + r : NULL;
    }
    softmax_row(c->q, c->k, c->v, c->dtype, ((size_t)h * a->q_pad + r) * dim, (size_t)kvh * a->k_pad * dim, dim,
                (double)a->scale, keys, n_keys, scratch, out, lse);
}

static int dense_ok(const oracle_attn_args* a, uint32_t dim)
{
    return dim && a->heads && a->kv_heads && a->heads % a->kv_heads == 0 && a->n_q <= a->q_pad &&
           a->n_k <= a->k_pad && a->width >= a->heads * dim;
}

int oracle_attn_dense(const oracle_attn_args* a, uint32_t dim, int dtype, const void* q, const void* k,
                      const void* v, double* o, double* lse, int nthreads)
{
    if (!dense_ok(a, dim))
        return -1;
    dense_ctx c = {a, dim, dtype, q, k, v, NULL, o, lse};
    /* scratch: n_k weights, then n_k key indices (as u32 in the doubles' room) */
    run_pool(dense_item, &c, (size_t)a->heads * a->n_q, 2 * (size_t)a->n_k + 1, nthreads);
    return 0;
}

int oracle_attn_dense_rows(const oracle_attn_args* a, uint32_t dim, int dtype, const void* q, const void* k,
                           const void* v, const uint32_t* head_row, size_t n, double* o_rows, double* lse_rows,
                           int nthreads)
{
    if (!dense_ok(a, dim))
        return -1;
    for (size_t i = 0; i < n; ++i)
        if (head_row[2 * i] >= a->heads || head_row[2 * i + 1] >= a->n_q)
            return -1;
    dense_ctx c = {a, dim, dtype, q, k, v, head_row, o_rows, lse_rows};
    run_pool(dense_item, &c, n, 2 * (size_t)a->n_k + 1, nthreads);
    return 0;
}

/* ---- block-sparse (ops.metal:1079-1113, 1173-1184) --------------------------------------------------------------- */

enum { SPARSE_D = 128, SPARSE_TILE = 64 };

typedef struct {
    const oracle_sparse_args* a;
    int dtype;
    const void *q, *k, *v;
    const uint16_t *sel, *nsel;
    const uint8_t* valid;
    const int32_t* map;
    const uint32_t* head_row;
    double *o, *lse;
    uint32_t o_rows;
} sparse_ctx;

static int sparse_seen(const oracle_sparse_args* a, const uint8_t* valid, uint32_t j, uint32_t row)
{
    if (!valid[j])
        return 0;
    if (a->causal && j > row)
        return 0;
    return 1;
}

/* The keys tile row `row` of head h visits, pass by pass. */
static size_t sparse_keys(const sparse_ctx* c, uint32_t h, uint32_t row, uint32_t* keys)
{
    const oracle_sparse_args* a = c->a;
    const uint32_t qt = row / SPARSE_TILE;
    size_t n = 0;
    if (qt < a->n_cubes) {
        const uint32_t sh = a->sel_heads == a->heads ? h : kv_head_of(h, a->heads, a->kv_heads);
        const uint32_t ns = c->nsel[(size_t)sh * a->n_cubes + qt];
        const uint16_t* my = c->sel + ((size_t)sh * a->n_cubes + qt) * a->max_sel;
        for (uint32_t i = 0; i < ns; ++i)
            for (uint32_t j = (uint32_t)my[i] * SPARSE_TILE; j < (uint32_t)my[i] * SPARSE_TILE + SPARSE_TILE; ++j)
                if (sparse_seen(a, c->valid, j, row))
                    keys[n++] = j;
        for (uint32_t j = a->dense0; j < a->dense1; ++j)
#if ORACLE_MUTANT == 6
            if (!a->causal || j <= row)
#else
            if (sparse_seen(a, c->valid, j, row))
#endif
                keys[n++] = j;
    } else {
        for (uint32_t j = 0; j < a->n_k; ++j)
            if (sparse_seen(a, c->valid, j, row))
                keys[n++] = j;
    }
    return n;
}

static void sparse_item(void* vctx, size_t item, double* scratch)
{
    const sparse_ctx* c = (const sparse_ctx*)vctx;
    const oracle_sparse_args* a = c->a;
    uint32_t h, r;
    if (c->head_row) {
        h = c->head_row[2 * item];
        r = c->head_row[2 * item + 1];
    } else {
        h = (uint32_t)(item / a->n_q);
        r = (uint32_t)(item % a->n_q);
        if (c->map[r] < 0 || (uint32_t)c->map[r] >= c->o_rows)
            return;
    }
    const size_t cap = (size_t)a->max_sel * SPARSE_TILE + a->k_pad;
    uint32_t* keys = (uint32_t*)(scratch + cap);
    const size_t n_keys = sparse_keys(c, h, r, keys);
    const uint32_t kvh = kv_head_of(h, a->heads, a->kv_heads);
    double* out;
    double* lse;
    if (c->head_row) {
        out = c->o + item * SPARSE_D;
        lse = c->lse ? c->lse + item : NULL;
    } else {
        out = c->o + (size_t)c->map[r] * a->width + (size_t)h * SPARSE_D;
        lse = c->lse ? c->lse + (size_t)h * a->q_pad + r : NULL;
    }
    softmax_row(c->q, c->k, c->v, c->dtype, ((size_t)h * a->q_pad + r) * SPARSE_D,
                (size_t)kvh * a->k_pad * SPARSE_D, SPARSE_D, (double)a->scale, keys, n_keys, scratch, out, lse);
}

static int sparse_ok(const oracle_sparse_args* a)
{
    if (!a->heads || !a->kv_heads || a->heads % a->kv_heads || a->n_q > a->q_pad || a->n_k > a->k_pad ||
        a->dense0 > a->dense1 || a->dense1 > a->k_pad || a->width < a->heads * SPARSE_D)
        return 0;
    if (a->sel_heads != a->heads && a->sel_heads != a->kv_heads)
        return 0;
    return (size_t)a->n_cubes * SPARSE_TILE <= a->k_pad;
}

int oracle_attn_sparse(const oracle_sparse_args* a, int dtype, const void* q, const void* k, const void* v,
                       const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid, const int32_t* map,
                       double* o, uint32_t o_rows, double* lse, int nthreads)
{
    if (!sparse_ok(a))
        return -1;
    sparse_ctx c = {a, dtype, q, k, v, sel, nsel, valid, map, NULL, o, lse, o_rows};
    const size_t cap = (size_t)a->max_sel * SPARSE_TILE + a->k_pad;
    run_pool(sparse_item, &c, (size_t)a->heads * a->n_q, 2 * cap + 1, nthreads);
    return 0;
}

int oracle_attn_sparse_rows(const oracle_sparse_args* a, int dtype, const void* q, const void* k, const void* v,
                            const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                            const uint32_t* head_row, size_t n, double* o_rows, double* lse_rows, int nthreads)
{
    if (!sparse_ok(a))
        return -1;
    for (size_t i = 0; i < n; ++i)
        if (head_row[2 * i] >= a->heads || head_row[2 * i + 1] >= a->n_q)
            return -1;
    sparse_ctx c = {a, dtype, q, k, v, sel, nsel, valid, NULL, head_row, o_rows, lse_rows, 0};
    const size_t cap = (size_t)a->max_sel * SPARSE_TILE + a->k_pad;
    run_pool(sparse_item, &c, n, 2 * cap + 1, nthreads);
    return 0;
}

/* ---- cube_select (ops.metal:926-1027) ----------------------------------------------------------------------------- */

int oracle_cube_select(uint32_t heads, uint32_t dim, int dtype, const void* q, uint32_t q_pad, const void* k,
                       uint32_t k_pad, uint32_t n_cubes, const uint32_t* cnt, uint32_t topk, uint32_t local,
                       uint32_t stride, uint16_t* sel, uint16_t* nsel, double* qp_out, double* kp_out,
                       double* sc_out)
{
    if (n_cubes > 4096 || !topk || (local != 0 && local != 1 && local != 3))
        return -1;
    if ((size_t)n_cubes * SPARSE_TILE > q_pad || (size_t)n_cubes * SPARSE_TILE > k_pad)
        return -1;
    const uint32_t n = n_cubes, kk = topk < n ? topk : n;
    double* qp = (double*)malloc(sizeof(double) * ((size_t)n * dim + 1));
    double* kp = (double*)malloc(sizeof(double) * ((size_t)n * dim + 1));
    double* sc = (double*)malloc(sizeof(double) * ((size_t)n + 1));
    for (uint32_t h = 0; h < heads; ++h) {
        /* pool: the sum of the cube's 64 rows over cnt (0 when cnt is 0) */
        for (uint32_t cb = 0; cb < n; ++cb)
            for (uint32_t d = 0; d < dim; ++d) {
                double sq = 0.0, sk = 0.0;
                for (uint32_t r = 0; r < SPARSE_TILE; ++r) {
                    sq += oracle_load(q, dtype, ((size_t)h * q_pad + (size_t)cb * SPARSE_TILE + r) * dim + d);
                    sk += oracle_load(k, dtype, ((size_t)h * k_pad + (size_t)cb * SPARSE_TILE + r) * dim + d);
                }
                qp[(size_t)cb * dim + d] = cnt[cb] ? sq / cnt[cb] : 0.0;
                kp[(size_t)cb * dim + d] = cnt[cb] ? sk / cnt[cb] : 0.0;
            }
        if (qp_out)
            memcpy(qp_out + (size_t)h * n * dim, qp, sizeof(double) * (size_t)n * dim);
        if (kp_out)
            memcpy(kp_out + (size_t)h * n * dim, kp, sizeof(double) * (size_t)n * dim);
        for (uint32_t qc = 0; qc < n; ++qc) {
            for (uint32_t kc = 0; kc < n; ++kc) {
                double s = 0.0;
                for (uint32_t d = 0; d < dim; ++d)
                    s += qp[(size_t)qc * dim + d] * kp[(size_t)kc * dim + d];
                sc[kc] = s;
            }
            if (sc_out)
                memcpy(sc_out + ((size_t)h * n + qc) * n, sc, sizeof(double) * n);
            uint16_t* out = sel + ((size_t)h * n + qc) * kk;
            uint32_t it = 0;
            if (local) { /* the local cubes first, their scores taken out of the running */
                const uint32_t picks[3] = {qc, qc >= stride ? qc - stride : n, qc + stride < n ? qc + stride : n};
                for (uint32_t j = 0; j < local && it < kk; ++j)
                    if (picks[j] < n) {
                        out[it++] = (uint16_t)picks[j];
                        sc[picks[j]] = -INFINITY;
                    }
            }
            for (; it < kk; ++it) { /* repeated argmax: the larger score, the smaller index on ties */
                double best = -INFINITY;
                uint32_t idx = 0;
                for (uint32_t i = 0; i < n; ++i)
#if ORACLE_MUTANT == 5
                    if (sc[i] >= best && sc[i] != -INFINITY) {
#else
                    if (sc[i] > best) {
#endif
                        best = sc[i];
                        idx = i;
                    }
                out[it] = (uint16_t)idx;
                sc[idx] = -INFINITY;
            }
            nsel[(size_t)h * n + qc] = (uint16_t)kk;
        }
    }
    free(qp);
    free(kp);
    free(sc);
    return 0;
}

/* ---- batched decode ------------------------------------------------------------------------------------------- */

typedef struct {
    uint32_t batch, heads, kv_heads, dim, cap;
    double scale;
    int dtype;
    const void *q, *k, *v;
    const uint32_t* ctx;
    const uint32_t* seq_head;
    double *o, *lse;
} decode_ctx;

static void decode_item(void* vctx, size_t item, double* scratch)
{
    const decode_ctx* c = (const decode_ctx*)vctx;
    uint32_t b, h;
    if (c->seq_head) {
        b = c->seq_head[2 * item];
        h = c->seq_head[2 * item + 1];
    } else {
        b = (uint32_t)(item / c->heads);
        h = (uint32_t)(item % c->heads);
    }
    /* one query at position ctx - 1, causal: it sees keys [0, ctx) (ops.metal:289 with n_q = 1) */
    oracle_attn_args a = {1, 1, c->ctx[b], c->cap, c->heads, c->kv_heads, c->ctx[b] ? c->ctx[b] - 1 : 0,
                          0xffffffffu, c->heads * c->dim, (float)c->scale};
    uint32_t* keys = (uint32_t*)(scratch + c->cap);
    const size_t n_keys = c->ctx[b] ? dense_keys(&a, a.q_pos0, keys) : 0;
    const uint32_t kvh = kv_head_of(h, c->heads, c->kv_heads);
    double* out = c->seq_head ? c->o + item * c->dim : c->o + ((size_t)b * c->heads + h) * c->dim;
    double* lse = c->lse ? (c->seq_head ? c->lse + item : c->lse + (size_t)b * c->heads + h) : NULL;
    softmax_row(c->q, c->k, c->v, c->dtype, ((size_t)b * c->heads + h) * c->dim,
                ((size_t)b * c->kv_heads + kvh) * c->cap * c->dim, c->dim, c->scale, keys, n_keys, scratch, out,
                lse);
}

int oracle_attn_decode(uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t dim, uint32_t cap, float scale,
                       int dtype, const void* q, const void* k, const void* v, const uint32_t* ctx, double* o,
                       double* lse, int nthreads)
{
    if (!heads || !kv_heads || heads % kv_heads || !dim)
        return -1;
    for (uint32_t b = 0; b < batch; ++b)
        if (ctx[b] > cap)
            return -1;
    decode_ctx c = {batch, heads, kv_heads, dim, cap, (double)scale, dtype, q, k, v, ctx, NULL, o, lse};
    run_pool(decode_item, &c, (size_t)batch * heads, 2 * (size_t)cap + 1, nthreads);
    return 0;
}

int oracle_attn_decode_rows(uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t dim, uint32_t cap,
                            float scale, int dtype, const void* q, const void* k, const void* v,
                            const uint32_t* ctx, const uint32_t* seq_head, size_t n, double* o_rows,
                            double* lse_rows, int nthreads)
{
    if (!heads || !kv_heads || heads % kv_heads || !dim)
        return -1;
    for (size_t i = 0; i < n; ++i)
        if (seq_head[2 * i] >= batch || seq_head[2 * i + 1] >= heads || ctx[seq_head[2 * i]] > cap)
            return -1;
    decode_ctx c = {batch, heads, kv_heads, dim, cap, (double)scale, dtype, q, k, v, ctx, seq_head, o_rows,
                    lse_rows};
    run_pool(decode_item, &c, n, 2 * (size_t)cap + 1, nthreads);
    return 0;
}

/* ---- split-K merge ------------------------------------------------------------------------------------------------ */

void oracle_lse_merge(uint32_t n, uint32_t dim, const double* o_i, const double* lse_i, double* o, double* lse)
{
    double mx = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        if (lse_i[i] > mx)
            mx = lse_i[i];
    for (uint32_t d = 0; d < dim; ++d)
        o[d] = 0.0;
    if (mx == -INFINITY) {
        *lse = -INFINITY;
        return;
    }
    double sum = 0.0;
    for (uint32_t i = 0; i < n; ++i)
        sum += exp(lse_i[i] - mx);
    for (uint32_t i = 0; i < n; ++i) {
        const double w = exp(lse_i[i] - mx) / sum;
        for (uint32_t d = 0; d < dim; ++d)
            o[d] += w * o_i[(size_t)i * dim + d];
    }
    *lse = mx + log(sum);
}

/* ---- head tiles ------------------------------------------------------------------------------------------- */

static uint16_t round_to(int out_dtype, double v)
{
    return out_dtype == ORACLE_BF16 ? oracle_f32_to_bf16((float)v) : oracle_f32_to_f16((float)v);
}

int oracle_heads(const oracle_heads_args* a, int out_dtype, const float* x, const float* cs, const float* w,
                 const int32_t* map, uint16_t* y)
{
    if (a->dim == 0 || a->dim > 256 || a->rot % 2 || a->rot > a->dim || a->row0 + a->rows > a->n_pad)
        return 1;
    double v[256], r[256];
    const uint32_t half = a->rot / 2;
    for (uint32_t h = 0; h < a->heads; ++h) {
        for (uint32_t t = 0; t < a->rows; ++t) {
            uint16_t* yr = y + ((size_t)h * a->n_pad + a->row0 + t) * a->dim;
            const int32_t src = map ? map[t] : (int32_t)t;
            if (src < 0) { /* heads_partial: a zero row (ops.metal:598-601) */
                for (uint32_t i = 0; i < a->dim; ++i)
                    yr[i] = 0;
                continue;
            }
            const float* xr = x + (size_t)src * a->ld + a->col0 + (size_t)h * a->stride;
            for (uint32_t i = 0; i < a->dim; ++i)
                v[i] = xr[i];
            if (a->eps > 0.0f) { /* ops.metal:389-396, 602-611 */
                double ss = 0.0;
                for (uint32_t i = 0; i < a->dim; ++i)
                    ss += v[i] * v[i];
#if ORACLE_MUTANT == 8
                const double inv = 1.0 / sqrt(ss + a->eps);
#else
                const double inv = 1.0 / sqrt(ss / a->dim + a->eps);
#endif
                for (uint32_t i = 0; i < a->dim; ++i)
                    v[i] *= inv * w[i];
            }
            for (uint32_t i = 0; i < a->dim; ++i)
                r[i] = v[i];
            if (a->rope) { /* ops.metal:33-38, 398-403, 614-617 */
                for (uint32_t i = 0; i < a->rot; ++i) {
                    const int first = a->rope == 1 ? i < half : (i % 2) == 0;
                    const uint32_t j = a->rope == 1 ? (first ? i + half : i - half) : (i ^ 1u);
                    const uint32_t p = a->rope == 1 ? (first ? i : i - half) : i / 2;
                    const double c = cs[((size_t)src * half + p) * 2], s = cs[((size_t)src * half + p) * 2 + 1];
#if ORACLE_MUTANT == 7
                    r[i] = first ? v[i] * c - v[j] * s : v[i] * c - v[j] * s;
#else
                    r[i] = first ? v[i] * c - v[j] * s : v[i] * c + v[j] * s;
#endif
                }
            }
            for (uint32_t i = 0; i < a->dim; ++i)
                yr[i] = round_to(out_dtype, r[i]);
        }
        if (a->clear) /* heads_clear (ops.metal:44-52) */
            for (uint32_t t = a->row0 + a->rows; t < a->n_pad; ++t)
                for (uint32_t i = 0; i < a->dim; ++i)
                    y[((size_t)h * a->n_pad + t) * a->dim + i] = 0;
    }
    return 0;
}

/* ---- split-K and gathered latent-cache primitives ----------------------------------------------------------- */

static double p_half(float p)
{
#if ORACLE_MUTANT == 10
    return p;
#else
    return oracle_f16_to_f32(oracle_f32_to_f16(p)); /* half(p[...]) (gemm.metal:711, 822-827) */
#endif
}

int oracle_attn_pv(uint32_t heads, uint32_t dim, uint32_t n_kv, uint32_t kps, const float* p, const uint16_t* kv,
                   double* partial)
{
    if (!kps)
        return 1;
    const uint32_t splits = (n_kv + kps - 1) / kps;
    for (uint32_t z = 0; z < splits; ++z)
        for (uint32_t h = 0; h < heads; ++h) {
            double* o = partial + ((size_t)z * heads + h) * dim;
            for (uint32_t d = 0; d < dim; ++d)
                o[d] = 0.0;
            const uint32_t t_end = (z + 1) * kps < n_kv ? (z + 1) * kps : n_kv;
            for (uint32_t t = z * kps; t < t_end; ++t) {
                const double w = p_half(p[(size_t)h * n_kv + t]);
                for (uint32_t d = 0; d < dim; ++d)
                    o[d] += w * oracle_f16_to_f32(kv[(size_t)t * dim + d]);
            }
        }
    return 0;
}

static uint32_t used(uint32_t cnt, uint32_t stride)
{
#if ORACLE_MUTANT == 9
    (void)cnt;
    return stride;
#else
    return cnt < stride ? cnt : stride;
#endif
}

int oracle_gather_scores(uint32_t heads, uint32_t dim, uint32_t stride, uint32_t tokens, const uint16_t* q,
                         const uint16_t* kv, const uint32_t* list, const uint32_t* count, double* scores)
{
    for (uint32_t t = 0; t < tokens; ++t) {
        const uint32_t n = used(count[t], stride);
        for (uint32_t h = 0; h < heads; ++h) {
            const uint16_t* qr = q + ((size_t)t * heads + h) * dim;
            double* o = scores + ((size_t)t * heads + h) * stride;
            for (uint32_t s = 0; s < stride; ++s) {
                double acc = 0.0;
                if (s < n) {
                    const uint16_t* kr = kv + (size_t)list[(size_t)t * stride + s] * dim;
                    for (uint32_t d = 0; d < dim; ++d)
                        acc += (double)oracle_f16_to_f32(qr[d]) * oracle_f16_to_f32(kr[d]);
                }
                o[s] = acc;
            }
        }
    }
    return 0;
}

int oracle_gather_pv(uint32_t heads, uint32_t dim, uint32_t stride, uint32_t splits, uint32_t tokens,
                     const float* p, const uint16_t* kv, const uint32_t* list, const uint32_t* count,
                     double* partial)
{
    if (!splits)
        return 1;
    const uint32_t per = (stride + splits * 64 - 1) / (splits * 64) * 64; /* gemm.metal:811 */
    for (uint32_t z = 0; z < splits; ++z)
        for (uint32_t t = 0; t < tokens; ++t) {
            const uint32_t n = used(count[t], stride), s0 = z * per, s1 = s0 + per < n ? s0 + per : n;
            for (uint32_t h = 0; h < heads; ++h) {
                double* o = partial + (((size_t)z * tokens + t) * heads + h) * dim;
                for (uint32_t d = 0; d < dim; ++d)
                    o[d] = 0.0;
                for (uint32_t s = s0; s < s1; ++s) {
                    const double w = p_half(p[((size_t)t * heads + h) * stride + s]);
                    const uint16_t* kr = kv + (size_t)list[(size_t)t * stride + s] * dim;
                    for (uint32_t d = 0; d < dim; ++d)
                        o[d] += w * oracle_f16_to_f32(kr[d]);
                }
            }
        }
    return 0;
}

int oracle_idx_dots(uint32_t heads, uint32_t dim, uint32_t pools, uint32_t stride, uint32_t tokens, const float* q,
                    const float* pooled, double* dots)
{
    for (uint32_t t = 0; t < tokens; ++t)
        for (uint32_t h = 0; h < heads; ++h)
            for (uint32_t pl = 0; pl < pools; ++pl) {
                double acc = 0.0;
                for (uint32_t d = 0; d < dim; ++d)
                    acc += (double)q[((size_t)t * heads + h) * dim + d] * pooled[(size_t)pl * dim + d];
                dots[((size_t)t * heads + h) * stride + pl] = acc;
            }
    return 0;
}

/* ---- the output projection (Runtime::proj, BF16 weights) --------------------------------------------------------- */

static double bf16_bits_to_double(uint16_t b)
{
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int oracle_proj_bf16(uint32_t t, uint32_t k, uint32_t n, uint32_t ldx, uint32_t ldy, int x_dtype, int split,
                     const uint16_t* w, const void* x, double* y)
{
    if (x_dtype != ORACLE_F32 && x_dtype != ORACLE_BF16)
        return 1;
    double* hi = malloc(sizeof(double) * k);
    double* lo = malloc(sizeof(double) * k);
    if (!hi || !lo) {
        free(hi);
        free(lo);
        return 2;
    }
    for (uint32_t r = 0; r < t; ++r) {
        for (uint32_t j = 0; j < k; ++j) {
            lo[j] = 0.0;
            if (x_dtype == ORACLE_BF16) {
                hi[j] = bf16_bits_to_double(((const uint16_t*)x)[(size_t)r * ldx + j]);
                continue;
            }
            const float f = ((const float*)x)[(size_t)r * ldx + j];
#if ORACLE_MUTANT == 11
            hi[j] = f;
            (void)split;
#else
            const uint16_t hb = oracle_f32_to_bf16(f); /* to_bf16 (gemm.metal:680) */
            hi[j] = bf16_bits_to_double(hb);
            if (split) /* bf16_lo: bfloat(x - float(hi)) (ops.metal:428) */
                lo[j] = bf16_bits_to_double(oracle_f32_to_bf16(f - (float)hi[j]));
#endif
        }
        for (uint32_t c = 0; c < n; ++c) {
            double acc = 0.0;
            for (uint32_t j = 0; j < k; ++j) {
#if ORACLE_MUTANT == 12
                const double wv = bf16_bits_to_double(w[((size_t)j * n + c) % ((size_t)n * k)]);
#else
                const double wv = bf16_bits_to_double(w[(size_t)c * k + j]);
#endif
                acc += wv * (hi[j] + lo[j]);
            }
            y[(size_t)r * ldy + c] = acc;
        }
    }
    free(hi);
    free(lo);
    return 0;
}

/* ---- the gated delta rule (kda_scan) ---------------------------------------------------------------------------- */

int oracle_kda_scan(uint32_t head_dim, uint32_t tokens, uint32_t qkv_stride, uint32_t inner, uint32_t heads,
                    uint32_t snap, const float* q, const float* k, const float* v, const float* g, const float* beta,
                    double* state, double* o, double* snap_state)
{
    const uint32_t D = head_dim;
    if (!D || (snap && !snap_state) || snap > tokens)
        return 1;
    double* eg = malloc(sizeof(double) * D);
    if (!eg)
        return 2;
    const double scale = 1.0 / sqrt((double)D);
    for (uint32_t h = 0; h < heads; ++h) {
        double* M = state + (size_t)h * D * D; /* M[j][i] = S[i][j] */
        for (uint32_t t = 0; t < tokens; ++t) {
            const float* qt = q + (size_t)t * qkv_stride + (size_t)h * D;
            const float* kt = k + (size_t)t * qkv_stride + (size_t)h * D;
            const float* vt = v + (size_t)t * qkv_stride + (size_t)h * D;
            const float* gt = g + (size_t)t * inner + (size_t)h * D;
#if ORACLE_MUTANT == 14
            const double b = 1.0;
            (void)beta;
#else
            const double b = beta[(size_t)t * heads + h];
#endif
            for (uint32_t i = 0; i < D; ++i)
                eg[i] = exp((double)gt[i]);
            for (uint32_t j = 0; j < D; ++j) {
                double* Mj = M + (size_t)j * D;
                double sum = 0.0;
#if ORACLE_MUTANT == 13
                for (uint32_t i = 0; i < D; ++i)
                    sum += Mj[i] * kt[i];
                for (uint32_t i = 0; i < D; ++i)
                    Mj[i] *= eg[i];
#else
                for (uint32_t i = 0; i < D; ++i) {
                    Mj[i] *= eg[i];             /* S[i][:] *= exp(g[i]) (ops.metal:496) */
                    sum += Mj[i] * kt[i];       /* sum_i S[i][j] k[i] (:497) */
                }
#endif
                const double delta = ((double)vt[j] - sum) * b; /* (:501) */
                double out = 0.0;
                for (uint32_t i = 0; i < D; ++i) {
                    Mj[i] += kt[i] * delta;     /* (:504) */
                    out += Mj[i] * qt[i];       /* (:505) */
                }
                o[(size_t)t * inner + (size_t)h * D + j] = out * scale;
            }
            if (t + 1 == snap)
                memcpy(snap_state + (size_t)h * D * D, M, sizeof(double) * D * D);
        }
    }
    free(eg);
    return 0;
}
