// Split-K and gathered latent-cache helpers of the decode path: the reference's attn_pv, attn_gather_scores,
// attn_gather_pv and idx_dots (src/kernels/gemm.metal:683-870), on v_mfma_f32_32x32x16_f16 (32x32x2_f32 for the
// float indexer dot products).
//
// Semantics (reference file:line):
//   attn_pv            partial[split][h][d] = sum over the split's keys t of half(p[h][t]) * kv[t][d]; keys past
//                      n_kv count as zero; splits of keys_per_split keys (gemm.metal:683-730).
//   attn_gather_scores scores[t][h][s] = q[t][h] . kv[list[t][s]] for s < count[t], 0 for count[t] <= s < stride
//                      (gemm.metal:743-786).
//   attn_gather_pv     partial[split][t][h][d] = sum over the split's entries s < count[t] of
//                      half(p[t][h][s]) * kv[list[t][s]][d]; a split covers per = ceil(stride / (splits * 64)) * 64
//                      entries (gemm.metal:788-844).
//   idx_dots           dots[t][h][p] = q[t][h] . pooled[p] in float for p < pools, rows `stride` apart
//                      (gemm.metal:846-870).
// All accumulate in f32; heads <= 64 for the gathered forms, <= 32 for idx_dots, any number for attn_pv.
//
// The design is this one's own. Bound: HBM (the latent rows, or the probabilities, read once a launch). A
// workgroup of 4 waves computes a 64 x 64 output tile as 2 x 2 MFMA blocks of 32 x 32. The contraction over the
// latent dimension (scores, dots) reads each gathered row's 16-byte runs straight from global memory as the MFMA's
// B operand (8 consecutive values a lane); the contraction over keys (pv) stages a 64-key chunk in LDS, the
// probabilities as f16 rows and the latent rows transposed, so each MFMA operand is one 16-byte LDS read.
#include "device.hpp"

namespace mako {
namespace {

constexpr int kT = 64;  // output tile edge and key chunk

typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---- P V over keys (attn_pv, attn_gather_pv) --------------------------------------------------------------------

struct PvParams {
    const float* p;         // probabilities, row h at p + h * p_ld (+ token offset)
    const _Float16* kv;     // latent rows [*][dim]
    const uint32_t* list;   // gathered: entry s of token t is row list[t * stride + s]
    const uint32_t* count;  // gathered: entries of token t
    float* partial;
    uint32_t heads, dim, p_ld;
    uint32_t n_kv, per;     // plain: keys and keys a split; gathered: stride and entries a split
    uint32_t splits, tokens;
    uint32_t gathered;
};

// Grid (dim / 64, ceil(heads / 64), splits * tokens); 4 waves: wave w computes heads h0 + 32 (w / 2) .., dims
// d0 + 32 (w % 2) ...
__global__ __launch_bounds__(256) void pv_tiles(const PvParams a)
{
    // P chunk [64 heads][64 keys] f16 (row pitch 72), kv chunk transposed [64 dims][64 keys] f16 (pitch 72).
    constexpr int PP = kT + 8;
    __shared__ __attribute__((aligned(16))) _Float16 ps[kT * PP];
    __shared__ __attribute__((aligned(16))) _Float16 ks[kT * PP];
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t d0 = blockIdx.x * kT, h0 = blockIdx.y * kT;
    const uint32_t split = blockIdx.z % a.splits, t = blockIdx.z / a.splits;
    uint32_t k_begin, k_end;
    const float* p = a.p;
    const uint32_t* list = a.list;
    if (a.gathered) {
        const uint32_t cnt = a.count[t];
        k_begin = split * a.per;
        k_end = min(min(cnt, a.p_ld), k_begin + a.per);  // entries past the list row count as zero
        p += (size_t)t * a.heads * a.p_ld;
        list += (size_t)t * a.p_ld;
    } else {
        k_begin = split * a.per;
        k_end = min(a.n_kv, k_begin + a.per);
    }
    f32x16 acc = {};
    const uint32_t hb = 32 * (w >> 1), db = 32 * (w & 1);
    // Loads of a chunk: thread tid fills 16 probabilities of head h0 + tid / 4 and 16 latent values (2 x 16 bytes)
    // of key tid / 4.
    const uint32_t r = tid >> 2, c = (tid & 3) * 16;
    const bool r_ok = h0 + r < a.heads;
    p += (size_t)(r_ok ? h0 + r : 0u) * a.p_ld;
    for (uint32_t k0 = k_begin; k0 < k_end; k0 += kT) {
        {
            _Float16* po = ps + r * PP + c;
            #pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const uint32_t kk = k0 + c + i;
                const float x0 = (r_ok && kk < k_end) ? p[kk] : 0.0f;
                const float x1 = (r_ok && kk + 1 < k_end) ? p[kk + 1] : 0.0f;
                *reinterpret_cast<uint32_t*>(po + i) = Elem<_Float16>::pack2(x0, x1);
            }
            const uint32_t kr = k0 + r;
            u32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
            if (kr < k_end) {
                const uint32_t row = a.gathered ? list[kr] : kr;
                const u32x4* src = reinterpret_cast<const u32x4*>(a.kv + (size_t)row * a.dim + d0 + c);
                v0 = src[0];
                v1 = src[1];
            }
            // transposed: value e of this thread's 16 (dim d0 + c + e) to ks[(c + e) * PP + r]
            #pragma unroll
            for (int e = 0; e < 16; ++e) {
                const u32x4& v = e < 8 ? v0 : v1;
                ks[(c + e) * PP + r] = __builtin_bit_cast(_Float16, (uint16_t)half_of(v, e & 7));
            }
        }
        __syncthreads();
        #pragma unroll
        for (int kk = 0; kk < kT / 16; ++kk) {
            const f16x8 av = *reinterpret_cast<const f16x8*>(ps + (hb + c32) * PP + 16 * kk + 8 * g);
            const f16x8 bv = *reinterpret_cast<const f16x8*>(ks + (db + c32) * PP + 16 * kk + 8 * g);
            acc = Elem<_Float16>::mfma32(av, bv, acc);
        }
        __syncthreads();
    }
    // acc register r of lane (c32, g): head h0 + hb + 8 (r / 4) + 4 g + r % 4, dim d0 + db + c32
    float* out = a.partial + ((size_t)split * a.tokens + t) * a.heads * a.dim;
    #pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
        const uint32_t h = h0 + hb + 8 * (rr >> 2) + 4 * g + (rr & 3);
        if (h < a.heads)
            out[(size_t)h * a.dim + d0 + db + c32] = acc[rr];
    }
}

// ---- q . kv rows over the latent dimension (attn_gather_scores) -------------------------------------------------

struct ScoreParams {
    const _Float16* q;  // [tokens][heads][dim]
    const _Float16* kv;
    const uint32_t* list;
    const uint32_t* count;
    float* scores;      // [tokens][heads][stride]
    uint32_t heads, dim, stride;
};

// Grid (ceil(stride / 64), 1, tokens); wave w: heads 32 (w / 2) .., entries n0 + 32 (w % 2) ...
__global__ __launch_bounds__(256) void gather_scores(const ScoreParams a)
{
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t t = blockIdx.z, cnt = a.count[t];
    const uint32_t hb = 32 * (w >> 1), s = blockIdx.x * kT + 32 * (w & 1) + c32;  // this lane's entry (B column)
    const uint32_t h = hb + c32;                                                    // this lane's head (A row)
    const bool row_ok = s < cnt && s < a.stride;
    const uint32_t row = row_ok ? a.list[(size_t)t * a.stride + s] : 0u;
    const auto krs = buffer_rsrc(a.kv + (size_t)row * a.dim, row_ok ? a.dim * 2u : 0u);
    const auto qrs = buffer_rsrc(a.q + ((size_t)t * a.heads + h) * a.dim, h < a.heads ? a.dim * 2u : 0u);
    f32x16 acc = {};
    for (uint32_t k0 = 0; k0 < a.dim; k0 += 16) {
        const f16x8 av = __builtin_bit_cast(f16x8, buffer_load16(qrs, (k0 + 8 * g) * 2));
        const f16x8 bv = __builtin_bit_cast(f16x8, buffer_load16(krs, (k0 + 8 * g) * 2));
        acc = Elem<_Float16>::mfma32(av, bv, acc);
    }
    // acc register r of lane (c32, g): head hb + 8 (r / 4) + 4 g + r % 4, entry s (column c32)
    if (s < a.stride) {
        float* out = a.scores + (size_t)t * a.heads * a.stride + s;
        #pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const uint32_t hh = hb + 8 * (rr >> 2) + 4 * g + (rr & 3);
            if (hh < a.heads)
                out[(size_t)hh * a.stride] = acc[rr];
        }
    }
}

// ---- float q . pooled rows (idx_dots) ---------------------------------------------------------------------------

struct DotParams {
    const float* q;       // [tokens][heads][dim]
    const float* pooled;  // [pools][dim]
    float* dots;          // [tokens][heads][stride]
    uint32_t heads, dim, pools, stride;
};

// Grid (ceil(pools / 64), 1, tokens); waves 0 and 1 take pools p0 .. p0 + 31 and p0 + 32 .. (heads <= 32).
__global__ __launch_bounds__(128) void idx_dots_k(const DotParams a)
{
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t t = blockIdx.z, pl = blockIdx.x * kT + 32 * w + c32;
    const bool p_ok = pl < a.pools, h_ok = c32 < a.heads;
    const float* qr = a.q + ((size_t)t * a.heads + (h_ok ? c32 : 0u)) * a.dim;
    const float* kr = a.pooled + (size_t)(p_ok ? pl : 0u) * a.dim;
    f32x16 acc = {};
    for (uint32_t k0 = 0; k0 < a.dim; k0 += 2) {
        const uint32_t k = k0 + g;
        const float av = h_ok && k < a.dim ? qr[k] : 0.0f;
        const float bv = p_ok && k < a.dim ? kr[k] : 0.0f;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
    }
    if (p_ok) {
        float* out = a.dots + (size_t)t * a.heads * a.stride + pl;
        #pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const uint32_t hh = 8 * (rr >> 2) + 4 * g + (rr & 3);
            if (hh < a.heads)
                out[(size_t)hh * a.stride] = acc[rr];
        }
    }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mako

using namespace mako;

extern "C" int mako_attn_pv(const mako_pv_args* a, const float* p, const void* kv, float* partial, void* stream)
{
    if (!a || !p || !kv || !partial)
        return fail(MAKO_EINVAL, "attn_pv: a null argument");
    if (!a->heads || !a->dim || a->dim % 64 || !a->keys_per_split || a->keys_per_split % 64)
        return fail(MAKO_EINVAL, "attn_pv: %u heads of %u, %u keys a split (dim and keys a split multiples of 64)",
                    a->heads, a->dim, a->keys_per_split);
    if (a->heads > 64u * 65535u)
        return fail(MAKO_EINVAL, "attn_pv: %u heads exceed the grid", a->heads);
    if (!al16(kv))
        return fail(MAKO_EINVAL, "attn_pv: kv must be 16-byte aligned");
    const uint32_t splits = (a->n_kv + a->keys_per_split - 1) / a->keys_per_split;
    if (splits == 0)
        return ok();
    if (splits > 65535u)
        return fail(MAKO_EINVAL, "attn_pv: %u splits exceed the grid (at most 65535)", splits);
    PvParams pp{p, static_cast<const _Float16*>(kv), nullptr, nullptr, partial, a->heads, a->dim, a->n_kv,
                a->n_kv, a->keys_per_split, splits, 1, 0};
    hipLaunchKernelGGL(pv_tiles, dim3(a->dim / kT, (a->heads + kT - 1) / kT, splits), dim3(256), 0,
                       static_cast<hipStream_t>(stream), pp);
    return check_launch("attn_pv");
}

extern "C" int mako_attn_gather_scores(const mako_gather_args* a, const void* q, const void* kv,
                                       const uint32_t* list, const uint32_t* count, float* scores, void* stream)
{
    if (!a || !q || !kv || !list || !count || !scores)
        return fail(MAKO_EINVAL, "attn_gather_scores: a null argument");
    if (!a->heads || a->heads > 64 || !a->dim || a->dim % 256 || !a->stride)
        return fail(MAKO_EINVAL, "attn_gather_scores: %u heads of %u, lists of %u (heads <= 64, dim a multiple of "
                    "256)", a->heads, a->dim, a->stride);
    if (!al16(q) || !al16(kv))
        return fail(MAKO_EINVAL, "attn_gather_scores: q and kv must be 16-byte aligned");
    if (a->tokens == 0)
        return ok();
    if (a->tokens > 65535u || a->stride > 0x7fffffffu - kT)
        return fail(MAKO_EINVAL, "attn_gather_scores: %u tokens exceed the grid (at most 65535)", a->tokens);
    ScoreParams sp{static_cast<const _Float16*>(q), static_cast<const _Float16*>(kv), list, count, scores, a->heads,
                   a->dim, a->stride};
    hipLaunchKernelGGL(gather_scores, dim3((a->stride + kT - 1) / kT, 1, a->tokens), dim3(256), 0,
                       static_cast<hipStream_t>(stream), sp);
    return check_launch("attn_gather_scores");
}

extern "C" int mako_attn_gather_pv(const mako_gather_args* a, const float* p, const void* kv, const uint32_t* list,
                                   const uint32_t* count, float* partial, void* stream)
{
    if (!a || !p || !kv || !list || !count || !partial)
        return fail(MAKO_EINVAL, "attn_gather_pv: a null argument");
    if (!a->heads || a->heads > 64 || !a->dim || a->dim % 128 || !a->stride || !a->splits)
        return fail(MAKO_EINVAL, "attn_gather_pv: %u heads of %u, lists of %u in %u splits (heads <= 64, dim a "
                    "multiple of 128)", a->heads, a->dim, a->stride, a->splits);
    if (!al16(kv))
        return fail(MAKO_EINVAL, "attn_gather_pv: kv must be 16-byte aligned");
    if (a->tokens == 0)
        return ok();
    const uint32_t per = (a->stride + a->splits * kT - 1) / (a->splits * kT) * kT;
    PvParams pp{p, static_cast<const _Float16*>(kv), list, count, partial, a->heads, a->dim, a->stride, a->stride,
                per, a->splits, a->tokens, 1};
    if ((uint64_t)a->splits * a->tokens > 65535u)
        return fail(MAKO_EINVAL, "attn_gather_pv: %u tokens x %u splits exceed the grid (at most 65535)", a->tokens,
                    a->splits);
    hipLaunchKernelGGL(pv_tiles, dim3(a->dim / kT, 1, a->splits * a->tokens), dim3(256), 0,
                       static_cast<hipStream_t>(stream), pp);
    return check_launch("attn_gather_pv");
}

extern "C" int mako_idx_dots(const mako_idx_dot_args* a, uint32_t tokens, const float* q, const float* pooled,
                             float* dots, void* stream)
{
    if (!a || !q || !pooled || !dots)
        return fail(MAKO_EINVAL, "idx_dots: a null argument");
    if (!a->heads || a->heads > 32 || !a->dim || a->stride < a->pools)
        return fail(MAKO_EINVAL, "idx_dots: %u heads of %u, %u pools in rows of %u (heads <= 32, rows >= pools)",
                    a->heads, a->dim, a->pools, a->stride);
    if (tokens == 0 || a->pools == 0)
        return ok();
    if (tokens > 65535u || a->pools > 0x7fffffffu - kT)
        return fail(MAKO_EINVAL, "idx_dots: %u tokens exceed the grid (at most 65535)", tokens);
    DotParams dp{q, pooled, dots, a->heads, a->dim, a->pools, a->stride};
    hipLaunchKernelGGL(idx_dots_k, dim3((a->pools + kT - 1) / kT, 1, tokens), dim3(128), 0,
                       static_cast<hipStream_t>(stream), dp);
    return check_launch("idx_dots");
}
