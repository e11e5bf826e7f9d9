/*
 * CPU oracle for the attention path: test infrastructure only.
 *
 * A double-precision restatement of the reference's attention semantics, used to check the HIP kernels and
 * timed as the CPU baseline. Nothing in the product library links or calls it.
 *
 * Followed, function by function (reference file:line):
 *   oracle_attn_dense   - tests/sparse_attn_test.cpp:143-173 (double softmax over an explicit key list),
 *                         generalised with the mask rule of src/kernels/ops.metal:289 (j < n_k && (j <= pos ||
 *                         (pos >= block && j >= block)), pos = q_pos0 + row), the GQA head map of ops.metal:242
 *                         (kv head = h / (heads / kv_heads)), fully masked rows -> 0 (ops.metal:355), rows >= n_q
 *                         not stored (ops.metal:359-362), and lse = max + log(sum) (natural log).
 *   oracle_attn_sparse  - the pass list of ops.metal:1079-1098 (selected 64-row cubes, then dense rows
 *                         [dense0, dense1); tiles past n_cubes see [0, n_k)), the validity mask of ops.metal:1109,
 *                         and the row map of ops.metal:1173-1184; plus a causal flag (j <= row) that the
 *                         reference does not have.
 *   oracle_cube_select  - cube_pool / cube_scores / cube_topk (ops.metal:926-1027): mean of the 64 rows over
 *                         cnt[c], dot products, local picks first, then repeated argmax, ties to the smaller index;
 *                         the CPU form of tests/sparse_attn_test.cpp:103-128.
 *   oracle_attn_decode  - one query row per sequence at position ctx - 1 against keys [0, ctx): the dense rule
 *                         with n_q = 1, q_pos0 = ctx - 1 (ops.metal:289), batched.
 *   oracle_lse_merge    - the split-K merge: o = sum_i exp(lse_i - lse) o_i, lse = log sum_i exp(lse_i).
 *   oracle_attn_pv, oracle_gather_scores, oracle_gather_pv, oracle_idx_dots
 *                       - attn_pv, attn_gather_scores, attn_gather_pv and idx_dots (src/kernels/gemm.metal:683-870):
 *                         probabilities rounded to half before the product (gemm.metal:711, 822-827), gathered rows
 *                         past count[t] as zeros (:767-774, :830-837), the split ranges of :700 and :811-812.
 *   oracle_proj_bf16    - Runtime::proj with BF16 weights (src/gpu/runtime.cpp:164-205): to_bf16 of the activations
 *                         (src/kernels/gemm.metal:676-681), gemm_dense's y[t][n] = sum_k W[n][k] x[t][k]
 *                         (gemm.metal:251-280), and with bf16_split_ the remainder bf16(x - bf16(x)) through the same
 *                         product, added (src/kernels/ops.metal:421-437; runtime.cpp:184-203).
 *   oracle_kda_scan     - the gated delta rule with a decay per channel (src/kernels/ops.metal:459-519): per head,
 *                         S[i][:] *= exp(g[i]); delta[j] = (v[j] - sum_i S[i][j] k[i]) beta; S[i][j] += k[i] delta[j];
 *                         o[j] = sum_i S[i][j] q[i] / sqrt(head_dim), token after token.
 *   oracle_heads        - the tile producers heads_half, heads_clear, heads_norm_half and heads_partial
 *                         (src/kernels/ops.metal:21-52, 376-407, 587-620): slice, RMS norm times w
 *                         (x / sqrt(mean(x^2) + eps)), rotation of pairs (u, v) -> (u c - v s, v c + u s),
 *                         row map (a zero row where map[t] < 0), padding rows zeroed.
 *
 * Inputs are raw element arrays of a stated type (f32, f16 or bf16 bits), widened exactly to double.
 */
#ifndef MAKO_ATTN_ORACLE_H
#define MAKO_ATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_BF16 = 2 };

/* The reference's AttnArgs (src/kernels/ops.metal:54-64), field for field. */
typedef struct oracle_attn_args {
    uint32_t n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, width;
    float scale;
} oracle_attn_args;

/* The reference's SparseAttnArgs (src/kernels/ops.metal:1029-1034) plus causal and sel_heads. */
typedef struct oracle_sparse_args {
    uint32_t n_q, q_pad, n_k, k_pad, heads, kv_heads, width;
    float scale;
    uint32_t n_cubes, max_sel, dense0, dense1;
    uint32_t causal;    /* 1: key j is seen by tile row r only when j <= r */
    uint32_t sel_heads; /* rows of sel / nsel: heads (one list per query head) or kv_heads (shared by a group) */
} oracle_sparse_args;

/* Element i of a raw array of type `dtype`, widened exactly. */
double oracle_load(const void* p, int dtype, size_t i);
/* f32 -> f16 / bf16 bits, round to nearest even (NaN stays NaN). */
uint16_t oracle_f32_to_f16(float f);
uint16_t oracle_f32_to_bf16(float f);
float oracle_f16_to_f32(uint16_t h);

/*
 * Dense attention (causal / bidirectional / prefix-causal by `block`). q [heads][q_pad][dim], k and v
 * [kv_heads][k_pad][dim]; o [n_q][width] (head h at column h * dim), lse [heads][n_q] (may be NULL).
 * nthreads 0: all online cores. Returns 0, or -1 on a shape it cannot take.
 */
int oracle_attn_dense(const oracle_attn_args* a, uint32_t dim, int dtype, const void* q, const void* k,
                      const void* v, double* o, double* lse, int nthreads);

/*
 * The same for a list of (head, row) pairs only: o_rows [n][dim], lse_rows [n]. For sampled checks and the
 * CPU baseline's bounded sample.
 */
int oracle_attn_dense_rows(const oracle_attn_args* a, uint32_t dim, int dtype, const void* q, const void* k,
                           const void* v, const uint32_t* head_row, size_t n, double* o_rows, double* lse_rows,
                           int nthreads);

/*
 * Block-sparse attention, D = 128 (64-row tiles and cubes). sel u16 [sel_heads][n_cubes][max_sel], nsel u16
 * [sel_heads][n_cubes], valid u8 [k_pad], map i32 [q_pad]; o has o_rows rows of width (rows with map < 0 or
 * row >= n_q are not written), lse [heads][q_pad] indexed by tile row (may be NULL; written where o is).
 */
int oracle_attn_sparse(const oracle_sparse_args* a, int dtype, const void* q, const void* k, const void* v,
                       const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid, const int32_t* map,
                       double* o, uint32_t o_rows, double* lse, int nthreads);

/* The sparse rule for a list of (head, tile row) pairs: o_rows [n][128], lse_rows [n]. */
int oracle_attn_sparse_rows(const oracle_sparse_args* a, int dtype, const void* q, const void* k, const void* v,
                            const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                            const uint32_t* head_row, size_t n, double* o_rows, double* lse_rows, int nthreads);

/*
 * cube_select: q [heads][q_pad][dim], k [heads][k_pad][dim]; cnt u32 [n_cubes]; sel u16 [heads][n_cubes][kk],
 * nsel u16 [heads][n_cubes] with kk = min(topk, n_cubes). qp / kp / sc may be NULL (else [heads][n][dim],
 * [heads][n][dim], [heads][n][n] doubles). Returns 0, or -1 on the arguments the reference refuses.
 */
int oracle_cube_select(uint32_t heads, uint32_t dim, int dtype, const void* q, uint32_t q_pad, const void* k,
                       uint32_t k_pad, uint32_t n_cubes, const uint32_t* cnt, uint32_t topk, uint32_t local,
                       uint32_t stride, uint16_t* sel, uint16_t* nsel, double* qp, double* kp, double* sc);

/*
 * Batched single-token decode: q [batch][heads][dim] (one row a sequence), k and v [batch][kv_heads][cap][dim],
 * ctx u32 [batch] (keys [0, ctx) of each sequence); o [batch][heads * dim], lse [batch][heads] (may be NULL).
 */
int oracle_attn_decode(uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t dim, uint32_t cap, float scale,
                       int dtype, const void* q, const void* k, const void* v, const uint32_t* ctx, double* o,
                       double* lse, int nthreads);

/* The decode rule for a list of (sequence, head) pairs: o_rows [n][dim], lse_rows [n]. */
int oracle_attn_decode_rows(uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t dim, uint32_t cap,
                            float scale, int dtype, const void* q, const void* k, const void* v,
                            const uint32_t* ctx, const uint32_t* seq_head, size_t n, double* o_rows,
                            double* lse_rows, int nthreads);

/* Merges n partial results of one row: o_i [n][dim] (each normalised), lse_i [n] -> o [dim], *lse. */
/* HeadsArgs, HeadsNormArgs and HeadsPartialArgs (src/kernels/ops.metal:11-19, 371-374, 577-585) in one struct:
 * rope 1 pairs value i with i + rot / 2, rope 2 pairs 2p with 2p + 1; cs holds rot / 2 (cos, sin) pairs a row;
 * eps 0: no norm; clear: zero rows [row0 + rows, n_pad) of every head. */
typedef struct oracle_heads_args {
    uint32_t rows, ld, col0, stride, dim, heads, n_pad, row0, rope, rot;
    float eps;
    uint32_t clear;
} oracle_heads_args;

/* y [heads][n_pad][dim] as f16 or bf16 bits (out_dtype); y row row0 + t from x row t, or from x row map[t] (and
 * its angles) when map is not NULL, a zero row where map[t] < 0. Rows it does not write are left as they are. */
int oracle_heads(const oracle_heads_args* a, int out_dtype, const float* x, const float* cs, const float* w,
                 const int32_t* map, uint16_t* y);

/* attn_pv: partial [ceil(n_kv / kps)][heads][dim] from p f32 [heads][n_kv] and kv f16 bits [n_kv][dim]. */
int oracle_attn_pv(uint32_t heads, uint32_t dim, uint32_t n_kv, uint32_t kps, const float* p, const uint16_t* kv,
                   double* partial);
/* attn_gather_scores: scores [tokens][heads][stride] from q f16 bits [tokens][heads][dim], kv [*][dim]. */
int oracle_gather_scores(uint32_t heads, uint32_t dim, uint32_t stride, uint32_t tokens, const uint16_t* q,
                         const uint16_t* kv, const uint32_t* list, const uint32_t* count, double* scores);
/* attn_gather_pv: partial [splits][tokens][heads][dim] from p f32 [tokens][heads][stride]. */
int oracle_gather_pv(uint32_t heads, uint32_t dim, uint32_t stride, uint32_t splits, uint32_t tokens,
                     const float* p, const uint16_t* kv, const uint32_t* list, const uint32_t* count,
                     double* partial);
/* idx_dots: dots [tokens][heads][stride] (columns p < pools written) from q f32 [tokens][heads][dim] and pooled
 * f32 [pools][dim]. */
int oracle_idx_dots(uint32_t heads, uint32_t dim, uint32_t pools, uint32_t stride, uint32_t tokens, const float* q,
                    const float* pooled, double* dots);

/* Runtime::proj with BF16 weights (src/gpu/runtime.cpp:164-205): y [t][ldy] (columns < n written) from w bf16 bits
 * [n][k] and x [t][ldx], f32 (rounded to bf16 first, plus the remainder's product when split) or bf16 bits. */
int oracle_proj_bf16(uint32_t t, uint32_t k, uint32_t n, uint32_t ldx, uint32_t ldy, int x_dtype, int split,
                     const uint16_t* w, const void* x, double* y);

/* kda_scan (src/kernels/ops.metal:459-519): state double [heads][head_dim][head_dim], transposed as the reference
 * stores it (state[h][j][i] = S[i][j]), read and updated in place; o double at t * inner + h * head_dim; snap_state
 * (may be NULL when snap is 0) the state after `snap` tokens. */
int oracle_kda_scan(uint32_t head_dim, uint32_t tokens, uint32_t qkv_stride, uint32_t inner, uint32_t heads,
                    uint32_t snap, const float* q, const float* k, const float* v, const float* g, const float* beta,
                    double* state, double* o, double* snap_state);

void oracle_lse_merge(uint32_t n, uint32_t dim, const double* o_i, const double* lse_i, double* o, double* lse);

#ifdef __cplusplus
}
#endif

#endif
