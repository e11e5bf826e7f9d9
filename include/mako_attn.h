/*
 * mako_attn: the attention path of mako-common on MI355X (gfx950), as a C ABI.
 *
 * Each entry point replaces one kernel dispatch (or one group of dispatches) that the reference's
 * TransformerRuntime encodes into a Metal command encoder; the reference interface it stands for is cited
 * beside it. Buffers are device pointers (hipMalloc'd, or any device-resident memory), sizes are element
 * counts, `stream` is a hipStream_t passed as void* (NULL: the default stream). Every call only enqueues
 * work; results are visible once the stream is synchronised, as they were after Runtime::finish
 * (src/gpu/runtime.cpp:453-475). Calls never throw; they return MAKO_OK or an error code, and
 * mako_last_error() gives the message for the calling thread.
 *
 * Layouts (as the reference's tiles, src/models/runtime.hpp:90-111):
 *   q    [heads][q_pad][dim]        query tiles, one head after another
 *   k, v [kv_heads][k_pad][dim]     key / value tiles; head h reads kv head h / (heads / kv_heads)
 *   o    [n_q][width]               head h at columns [h * dim, (h + 1) * dim); rows >= n_q untouched
 *   lse  [heads][n_q] float          natural-log sum of exponentials of the scaled scores (may be NULL)
 * Element types: q, k, v in f16 or bf16; o in f32 (the reference's output), or the input's type.
 */
#ifndef MAKO_ATTN_H
#define MAKO_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MAKO_ATTN_ABI_VERSION 1

typedef enum mako_dtype { MAKO_F32 = 0, MAKO_F16 = 1, MAKO_BF16 = 2 } mako_dtype;

enum mako_status {
    MAKO_OK = 0,
    MAKO_EINVAL = 1,       /* arguments the reference refuses, or a precondition not met */
    MAKO_EUNSUPPORTED = 2, /* a head width or element type with no kernel in this build */
    MAKO_EWORKSPACE = 3,   /* workspace missing or smaller than the matching *_workspace() size */
    MAKO_EHIP = 4          /* a HIP call failed (launch or stream error) */
};

/* AttnArgs, field for field (src/kernels/ops.metal:54-64; src/models/runtime.cpp:26-29). */
typedef struct mako_attn_args {
    uint32_t n_q;      /* queries */
    uint32_t q_pad;    /* rows of a query head in q (>= n_q) */
    uint32_t n_k;      /* keys */
    uint32_t k_pad;    /* rows of a key / value head in k and v (>= n_k) */
    uint32_t heads, kv_heads;
    uint32_t q_pos0;   /* the position of query 0 among the keys */
    uint32_t block;    /* positions from here on see each other both ways; below, causal (0: bidirectional,
                          UINT32_MAX: causal) */
    uint32_t width;    /* o row length in elements (>= heads * dim) */
    float scale;       /* softmax scale, 1 / sqrt(dim) in the reference */
} mako_attn_args;

/* SparseAttnArgs (src/kernels/ops.metal:1029-1034; src/models/runtime.cpp:279-283) and two fields the
 * reference does not have: causal (a key j is seen by tile row r only when j <= r) and sel_heads (the rows of
 * sel / nsel: heads, one list per query head as cube_select writes them, or kv_heads, one list shared by the
 * query heads of a group). */
typedef struct mako_sparse_args {
    uint32_t n_q, q_pad, n_k, k_pad, heads, kv_heads, width;
    float scale;
    uint32_t n_cubes; /* the first n_cubes 64-row query tiles are cubes */
    uint32_t max_sel; /* entries a row of sel holds (min(topk, n_cubes)) */
    uint32_t dense0, dense1;
    uint32_t causal;
    uint32_t sel_heads;
} mako_sparse_args;

/* Batched single-token decode against a contiguous KV cache (no counterpart struct in the reference). */
typedef struct mako_decode_args {
    uint32_t batch;   /* sequences */
    uint32_t heads, kv_heads;
    uint32_t dim;     /* 128 */
    uint32_t cap;     /* rows of a kv head of one sequence in the cache (the cache's k_pad) */
    uint32_t max_ctx; /* an upper bound on every ctx_len[b] (<= cap); sizes the split-K partials */
    uint32_t split;   /* keys per split (a multiple of 64; 0: chosen by the library) */
    float scale;
} mako_decode_args;

/* ABI version of the loaded library (MAKO_ATTN_ABI_VERSION it was built with). */
int mako_attn_abi_version(void);

/* The message of the calling thread's last failed call ("" after a success). */
const char* mako_last_error(void);

/*
 * Dense flash attention: causal (block = UINT32_MAX), bidirectional (block = 0) or prefix-causal, GQA, one
 * launch. Replaces TransformerRuntime::attention (src/models/runtime.hpp:90-95; src/models/runtime.cpp:262-273)
 * and the kernels it dispatches, flash_attn_coop_{64,128}_32 and flash_attn_sg_256_16x32_4
 * (src/kernels/ops.metal:106-214, 230-369). dim 64, 128 or 256; heads a multiple of kv_heads. Keys past n_k
 * are masked (their rows need not be zero); fully masked rows give 0 and lse = -inf. Precision: P (the softmax
 * numerators) is rounded to the input type for P V, as the reference rounds it to half (src/kernels/ops.metal:329):
 * f16 inputs f16 P (relative error <= 2^-11 a probability), bf16 inputs bf16 P (<= 2^-8; rows that see fewer than 64
 * keys get probabilities to ~16 bits). V is used in its own type, bf16 V over its whole range, except at dim 256
 * past the heads-of-256 kernel's 32-bit offsets (calls of several GB), whose kernel converts bf16 V to f16 rounding
 * toward zero (|v| above 65504 saturates, below 6.1e-5 loses bits). The sums and the LSE add the unrounded f32
 * exponentials. Heads of 64 and 128 take one of two routes: a few query rows (n_q x heads / kv_heads <= 64, as the
 * reference's decode, attention with n_q = 1) split-K over the keys, with its partials in a workspace; more rows,
 * the prefill kernel, one launch with no workspace. Heads of 256 take one launch with no workspace, or past its
 * offsets first write V as f16 V^T tiles into a workspace. mako_attn_fwd keeps that workspace itself, per (device, stream),
 * allocated stream-ordered the first time a call needs it (or more of it) and held until mako_attn_release(stream);
 * under graph capture a call that would grow it fails with MAKO_EWORKSPACE.
 */
int mako_attn_fwd(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q,
                  const void* k, const void* v, void* o, float* lse, void* stream);

/*
 * mako_attn_fwd with the caller's workspace, for callers that own their scratch (the reference's Runtime owns it as
 * named scratch buffers: src/gpu/runtime.cpp:117-125; TransformerRuntime::attention passes scratch("attn_fwd")).
 * It allocates nothing; MAKO_EWORKSPACE when workspace_bytes is below mako_attn_fwd_workspace(a, dim) (0 for the
 * prefill routes: workspace may then be NULL). The workspace's contents do not matter before or after a call;
 * calls that overlap in time need separate workspaces.
 */
size_t mako_attn_fwd_workspace(const mako_attn_args* a, uint32_t dim);
int mako_attn_fwd_ws(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q,
                     const void* k, const void* v, void* o, float* lse, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * The workspaces the entry points without a workspace argument keep for a stream (on the current device): waits for
 * the stream, then frees them. No counterpart in the reference (its Runtime frees its scratch at destruction).
 * mako_attn_held_bytes: the bytes held on the current device, over all streams.
 */
int mako_attn_release(void* stream);
size_t mako_attn_held_bytes(void);

/*
 * Cube selection for block-sparse attention: per head and query cube, the topk key cubes by the dot product
 * of the cubes' mean q and k. Replaces TransformerRuntime::cube_select (src/models/runtime.hpp:96-107;
 * src/models/runtime.cpp:286-303) and cube_pool / cube_scores / cube_topk (src/kernels/ops.metal:926-1027).
 * q [heads][q_pad][128], k [heads][k_pad][128] (f16 or bf16), cnt u32 [n_cubes]; writes sel u16
 * [heads][n_cubes][min(topk, n_cubes)] and nsel u16 [heads][n_cubes]. workspace: at least
 * mako_cube_select_workspace(heads, n_cubes) bytes of device memory. Refuses (MAKO_EINVAL) what the reference
 * refuses: n_cubes > 4096, topk == 0, local not 0, 1 or 3. The selection is exact: means and scores in double,
 * in the order of the reference test's double check (tests/sparse_attn_test.cpp:98-129), ties to the smaller index.
 */
size_t mako_cube_select_workspace(uint32_t heads, uint32_t n_cubes);
int mako_cube_select(uint32_t heads, uint32_t q_pad, uint32_t k_pad, uint32_t n_cubes, uint32_t topk,
                     uint32_t local, uint32_t stride, mako_dtype in, const void* q, const void* k,
                     const uint32_t* cnt, uint16_t* sel, uint16_t* nsel, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Block-sparse attention over a pass list, D = 128. Replaces TransformerRuntime::attention_sparse
 * (src/models/runtime.hpp:108-111; src/models/runtime.cpp:305-317) and flash_attn_sparse_128
 * (src/kernels/ops.metal:1036-1185). Query tile t < n_cubes attends the 64-row key cubes sel lists for it and the
 * dense rows [dense0, dense1); a later tile attends [0, n_k); keys with valid[j] == 0 are masked; query row r's
 * output goes to o row map[r] (dropped when map[r] < 0). Requires q_pad % 64 == 0, k_pad % 128 == 0,
 * dense0 % 32 == 0 (the reference's checks) and n_cubes * 64 <= k_pad. lse [heads][q_pad] by tile row (may be
 * NULL). Lists shared by a kv head's query heads (sel_heads == kv_heads) in groups of 4, with dense0 % 64 == 0
 * and valid 16-byte aligned, take a route that first writes a pass table into a workspace (kept as mako_attn_fwd
 * keeps its own); P rounds as in mako_attn_fwd (bf16 P for bf16 inputs; rows whose first pass is not a full one get
 * tile-0 probabilities to ~16 bits). Other calls need no workspace and convert bf16 V and P to f16 (V rounding
 * toward zero: |v| above 65504 saturates).
 */
int mako_attn_sparse(const mako_sparse_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                     const void* v, void* o, const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                     const int32_t* map, float* lse, void* stream);

/* mako_attn_sparse with the caller's workspace, as mako_attn_fwd_ws (TransformerRuntime::attention_sparse passes
 * scratch("attn_sparse")); mako_attn_sparse_workspace(a) bytes (the pass table when the call can take that route). */
size_t mako_attn_sparse_workspace(const mako_sparse_args* a);
int mako_attn_sparse_ws(const mako_sparse_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                        const void* v, void* o, const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                        const int32_t* map, float* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Batched single-token decode, split-K over each sequence's context with fp32 partials merged by their LSE.
 * New beside TransformerRuntime::attention: the reference decodes one sequence at a time through attention()
 * with n_q = 1, q_pos0 = ctx - 1 (src/kernels/ops.metal:289), and its split-K primitive attn_pv
 * (src/kernels/gemm.metal:683-730) leaves the softmax and the merge to its caller; this does all three.
 * q [batch][heads][dim]; k, v [batch][kv_heads][cap][dim]; ctx_len u32 [batch] in device memory (sequence b
 * attends keys [0, min(ctx_len[b], max_ctx))); o [batch][heads * dim]; lse [batch][heads] (may be
 * NULL). workspace: at least mako_attn_decode_workspace(a) bytes of device memory.
 */
size_t mako_attn_decode_workspace(const mako_decode_args* a);
int mako_attn_decode(const mako_decode_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                     const void* v, const uint32_t* ctx_len, void* o, float* lse, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * mako_attn_decode with no workspace argument and no allocation of any kind: the split-K partials live in a
 * static device array of MAKO_DECODE_SCRATCH_BYTES inside the library (one copy on each GPU it runs on, held
 * until the process ends). No counterpart in the reference: it is for callers that cannot allocate device memory
 * while they run (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). Same arguments,
 * split and results as mako_attn_decode; MAKO_EWORKSPACE when the partials that split needs
 * (mako_attn_decode_workspace(a) bytes) exceed the static array. Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (two streams, two threads) race and must be serialised by the caller.
 */
#define MAKO_DECODE_SCRATCH_BYTES ((size_t)16 << 20)
int mako_attn_decode_noalloc(const mako_decode_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                             const void* v, const uint32_t* ctx_len, void* o, float* lse, void* stream);

/*
 * Head tiles from fp32 rows: head h of token t, x[t][col0 + h * stride .. + dim), written as y row
 * [h][row0 + t][dim] in f16 (the reference's half tiles) or bf16, optionally RMS-normed (times w) and then rotated by
 * the angle table cs. One call stands for each of the reference's tile producers (src/kernels/ops.metal:11-52,
 * 371-408, 576-620):
 *   TransformerRuntime::heads (src/models/runtime.cpp:215-226; heads_half + heads_clear): stride = dim = 128,
 *     eps = 0, rope 0 / 1 / 2 over rot = dim, clear = 1;
 *   TransformerRuntime::heads_norm (runtime.cpp:228-241; heads_norm_half): as heads with eps > 0 and w, any row0,
 *     clear = 0 (the rows past T are left as they are);
 *   TransformerRuntime::heads_partial (runtime.cpp:243-260; heads_partial): any stride, dim a multiple of 32 up to
 *     256, rope 1 over the first rot values, eps 0 (no norm) or > 0 with w, row0 = 0, clear = 0, and map: y row t
 *     takes x row map[t] (and its angles), a zero row where map[t] < 0.
 * Rotation: a pair (u, v) becomes (u c - v s, v c + u s) with (c, s) = cs[t][p] (float pairs, rot / 2 a row):
 * rope 1 pairs value i with i + rot / 2 (p = i), rope 2 pairs 2p with 2p + 1. The norm is
 * x * w / sqrt(mean(x^2) + eps) over the head's dim values, before the rotation. cs, w and map may be NULL when
 * unused. Refuses (MAKO_EINVAL) what the reference refuses (heads_partial: dim > 256, dim % 32, odd rot) and
 * shapes it cannot address.
 */
typedef struct mako_heads_args {
    uint32_t rows;   /* tokens T */
    uint32_t ld;     /* x row stride in elements */
    uint32_t col0;   /* the first head's column in x */
    uint32_t stride; /* columns from one head to the next in x */
    uint32_t dim;    /* values a head: a multiple of 32, at most 256 */
    uint32_t heads;  /* heads produced */
    uint32_t n_pad;  /* rows of a head in y (>= row0 + rows) */
    uint32_t row0;   /* y row of token 0 */
    uint32_t rope;   /* 0 none; 1 value i with i + rot / 2; 2 value 2i with 2i + 1 */
    uint32_t rot;    /* leading values rotated (even, at most dim) */
    float eps;       /* 0: no norm */
    uint32_t clear;  /* 1: zero y rows [row0 + rows, n_pad) of every head */
} mako_heads_args;

int mako_heads(const mako_heads_args* a, mako_dtype out, const float* x, const float* cs, const float* w,
               const int32_t* map, void* y, void* stream);

/*
 * Attention straight from fp32 projection rows. No counterpart in the reference, whose prefill steps produce the
 * head tiles and then attend (TransformerRuntime::heads / heads_norm / heads_partial, then attention:
 * src/models/qwen_text.cpp:308-311 and 414-418, src/models/h3_vae.cpp:219); it is for callers that keep those
 * tiles only for the attention call. cs holds the angles of key positions 0 .. n_k - 1 (one row a key, as the key
 * producer reads it); query row t sits at position q_pos0 + t and is rotated by row q_pos0 + t, so a rotated query
 * head needs q_pos0 + n_q <= n_k (MAKO_EINVAL otherwise; with n_k = 0 the queries are unused and no angle is read).
 * The result is that of
 *   mako_heads(hq, in, xq, cs + q_pos0 * hq->rot, wq, NULL, qt); mako_heads(hk, in, xk, cs, wk, NULL, kt);
 *   mako_heads(hv, in, xv, cs, NULL, NULL, vt); mako_attn_fwd(a, hq->dim, in, out, qt, kt, vt, o, lse)
 * bit for bit, with the tiles [heads][rows][dim] in the stream's workspace: each of hq / hk / hv is read as
 * mako_heads reads it except n_pad, row0 and clear (the tiles hold exactly `rows` rows); a is read as
 * mako_attn_fwd reads it except q_pad and k_pad. hq->rows must be a->n_q, hk->rows and hv->rows a->n_k, hq->heads
 * a->heads, hk->heads and hv->heads a->kv_heads, and the three dims equal (64, 128 or 256).
 * Heads of 64, 128 or 256 with 16-byte aligned rows (mako_heads' vector path), values neither normed nor rotated,
 * and more rows than the split-K route takes run as two launches: one that writes the query, key and value tiles
 * (heads of 256 past the prefill kernel's offsets: the f16 V^T images their kernel stages from instead of the value
 * tiles), then the prefill kernel mako_attn_fwd takes for the same call.
 * Other calls run the four launches above. The tiles live in a workspace (kept as mako_attn_fwd keeps its own).
 */
int mako_attn_fwd_rows(const mako_attn_args* a, const mako_heads_args* hq, const mako_heads_args* hk,
                       const mako_heads_args* hv, mako_dtype in, mako_dtype out, const float* xq, const float* xk,
                       const float* xv, const float* cs, const float* wq, const float* wk, void* o, float* lse,
                       void* stream);

/* mako_attn_fwd_rows with the caller's workspace, as mako_attn_fwd_ws (TransformerRuntime::attention_rows passes
 * scratch("attn_rows")): mako_attn_fwd_rows_workspace(a, dim) bytes, the head tiles and the attention's own. */
size_t mako_attn_fwd_rows_workspace(const mako_attn_args* a, uint32_t dim);
int mako_attn_fwd_rows_ws(const mako_attn_args* a, const mako_heads_args* hq, const mako_heads_args* hk,
                          const mako_heads_args* hv, mako_dtype in, mako_dtype out, const float* xq, const float* xk,
                          const float* xv, const float* cs, const float* wq, const float* wk, void* o, float* lse,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Split-K and gathered latent-cache primitives of the sparse latent decode (src/kernels/gemm.metal:683-870; no call
 * site in the reference's own engines: they serve a caller that computes the softmax between them). f16 latent rows
 * kv [*][dim], f32 accumulate, f32 outputs.
 *
 * mako_attn_pv (attn_pv, gemm.metal:683-730, PvArgs field for field): partial [splits][heads][dim], splits =
 *   ceil(n_kv / keys_per_split), partial[z][h][d] = sum over keys t of split z of half(p[h][t]) * kv[t][d], with
 *   p f32 [heads][n_kv]. Any number of heads (grid y of ceil(heads / 64), as the reference); dim and keys_per_split
 *   multiples of 64; at most 65535 splits.
 * mako_attn_gather_scores (attn_gather_scores, gemm.metal:743-786, GatherArgs field for field): scores f32
 *   [tokens][heads][stride], scores[t][h][s] = q[t][h] . kv[list[t][s]] for s < count[t], 0 up to stride; q f16
 *   [tokens][heads][dim], list u32 [tokens][stride], count u32 [tokens]. heads <= 64, dim a multiple of 256.
 * mako_attn_gather_pv (attn_gather_pv, gemm.metal:788-844): partial f32 [splits][tokens][heads][dim],
 *   partial[z][t][h][d] = sum over entries s of split z (per = ceil(stride / (splits * 64)) * 64 entries a split,
 *   s < count[t]) of half(p[t][h][s]) * kv[list[t][s]][d]; p f32 [tokens][heads][stride]. heads <= 64, dim a
 *   multiple of 128.
 * mako_idx_dots (idx_dots, gemm.metal:846-870, IdxDotArgs field for field): dots f32 [tokens][heads][stride],
 *   dots[t][h][p] = q[t][h] . pooled[p] in f32 for p < pools; q f32 [tokens][heads][dim], pooled f32 [pools][dim].
 *   heads <= 32.
 */
typedef struct mako_pv_args {
    uint32_t heads, dim, n_kv;
    uint32_t keys_per_split;
} mako_pv_args;

typedef struct mako_gather_args {
    uint32_t heads, dim, stride, splits, tokens;
} mako_gather_args;

typedef struct mako_idx_dot_args {
    uint32_t heads, dim, pools, stride;
} mako_idx_dot_args;

int mako_attn_pv(const mako_pv_args* a, const float* p, const void* kv, float* partial, void* stream);
int mako_attn_gather_scores(const mako_gather_args* a, const void* q, const void* kv, const uint32_t* list,
                            const uint32_t* count, float* scores, void* stream);
int mako_attn_gather_pv(const mako_gather_args* a, const float* p, const void* kv, const uint32_t* list,
                        const uint32_t* count, float* partial, void* stream);
int mako_idx_dots(const mako_idx_dot_args* a, uint32_t tokens, const float* q, const float* pooled, float* dots,
                  void* stream);

/*
 * The output projection after attention: Runtime::proj with BF16 weights (src/gpu/runtime.cpp:164-205; its call
 * after attention at src/models/qwen_text.cpp:312 and src/models/h3.cpp:366), the dense BF16 GEMM gemm_dense
 * (src/kernels/gemm.metal:251-296) behind it.
 *
 *   y[r][c] = sum_j w[c][j] * bf16(x[r][j])   (f32 accumulate), r < t, c < n, j < k
 *
 * mako_gemm_args is GemmArgs (gemm.metal:18-22, src/mtl/gemm.cpp:13-15) field for field: row_bytes is the weight
 * row's bytes (2 k for BF16), ldy / ldx the row strides of y / x in elements (0: n / k). w bf16 [n][k]; y f32
 * [t][ldy]. x_dtype MAKO_BF16: x is bf16 [t][ldx], e.g. the attention output written in bf16 by mako_attn_fwd (no
 * conversion pass); MAKO_F32: x is f32 [t][ldx] and its rounding to bf16 (to_bf16, gemm.metal:676-681) happens in
 * the GEMM's loads. split (f32 x only): Runtime's bf16_split_ (src/gpu/runtime.cpp:184-203; set by the Qwen encoders,
 * src/models/qwen_text.cpp:271): the rounding's remainder bf16(x - bf16(x)) goes through the GEMM too and adds into
 * y. k a multiple of 64 (the reference's "BF16 {k}x{n}: k must be a multiple of 64"); w and x 16-byte aligned, ldx a
 * multiple of 8 elements; t x ldx and n x k at most 2^32 elements, and with bf16 x, 256 rows of x (of w) plus 2 k + 128
 * bytes within 2^32 bytes (ldx and k below about 8.4M elements): MAKO_EINVAL otherwise.
 */
typedef struct mako_gemm_args {
    uint32_t t, k, n, row_bytes;
    uint32_t ldy, ldx;
} mako_gemm_args;

int mako_proj_bf16(const mako_gemm_args* a, int x_dtype, int split, const void* w, const void* x, float* y,
                   void* stream);

/*
 * The gated delta rule with a decay per channel: kda_scan (src/kernels/ops.metal:459-519), run by the linear-
 * attention layers that sit beside attention in Qwen3.5's encoder (src/models/qwen_text.cpp:332-391). Per head h,
 * with S the head's state (stored transposed, state[h][j][i] = S[i][j], head_dim x head_dim f32) and, for each token
 * t in order,
 *   S[i][:] *= exp(g[t][i]);  delta[j] = (v[t][j] - sum_i S[i][j] k[t][i]) * beta[t][h]
 *   S[i][j] += k[t][i] * delta[j];  o[t][j] = sum_i S[i][j] q[t][i] / sqrt(head_dim)
 * q, k, v at t * qkv_stride + h * head_dim, g and o at t * inner + h * head_dim, beta at t * heads + h (all f32).
 * state is read at the start and holds the state after the last token at the end; when snap is nonzero the state
 * after `snap` tokens is also written to snap_state (the reference's rollback snapshot). mako_scan_args is ScanArgs
 * (ops.metal:459-466) field for field; head_dim must be 128, as in the reference.
 */
typedef struct mako_scan_args {
    uint32_t head_dim, tokens, qkv_stride, inner, heads, snap;
} mako_scan_args;

int mako_kda_scan(const mako_scan_args* a, const float* q, const float* k, const float* v, const float* g,
                  const float* beta, float* state, float* o, float* snap_state, void* stream);

#ifdef __cplusplus
}
#endif

#endif
