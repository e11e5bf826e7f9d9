// Batched single-token decode for gfx950: split-K over each sequence's context, fp32 partials merged by LSE.
//
// Semantics: sequence b's one query row sits at position ctx[b] - 1 and sees keys [0, ctx[b]) (the reference's
// mask rule, src/kernels/ops.metal:289, with n_q = 1 and q_pos0 = ctx - 1); head h reads kv head
// h / (heads / kv_heads) (:242); the running maximum moves only when a score passes it by 8 (base 2, :303-316);
// an empty context gives 0 and lse = -inf (:355); P and V meet in f16 for the P V product (V converted from
// bf16 as it is staged). The reference splits the P V product over keys
// (attn_pv, src/kernels/gemm.metal:688-730) and leaves the softmax and the merge to its caller; here one kernel
// does the split softmax and products, and a second merges the splits.
//
// Design (bandwidth-bound: every K / V byte is read once from HBM):
// * Work unit: one wave, one (sequence, kv head, chunk of `split` keys). The wave stages 32-key K / V tiles in
//   its own LDS slice (coalesced 16-byte loads, four whole 256-byte rows an instruction; the next tile's loads
//   are in flight while the current one is used), so the four waves of a workgroup never wait on each other.
// * The group's query heads are the columns of S^T = K Q^T on v_mfma_f32_32x32x16 (4 of 32 columns used at
//   GQA 4): the matrix unit has ~20x the rate this needs, and it keeps the VALU free of per-key dot products and
//   cross-lane reductions. K rows are stored with bits 2 and 3 of the row swapped so the exponentiated scores are
//   already the B operand of O^T = V^T P^T; V is transposed into LDS through registers.
// * Workgroups are numbered sequence by sequence over the chunks that exist (the grid's upper bound comes from
//   max_ctx; the surplus workgroups come last and exit), with the kv head as the fastest index.
// * Partials: the unnormalised O^T columns, the running maximum and the row sum, per (sequence, chunk, head);
//   the merge kernel rescales them to the common maximum and divides once.
#include "device.hpp"

namespace mako {
namespace {

constexpr int kWaves = 4;
constexpr int kTK = 32;  // keys a tile
constexpr int kD = 128;
constexpr float kRescale = 8.0f;
constexpr uint32_t kDefaultSplit = 512;

struct DecParams {
    const void* q;
    const void* k;
    const void* v;
    const uint32_t* ctx;
    float* part_o;   // [batch][max_chunks][heads][kD]
    float* part_ml;  // [batch][max_chunks][heads][2]: maximum (base 2), sum
    uint32_t batch, heads, kv_heads, group, cap, split, max_chunks, max_ctx;
    float scale_log2;
};

// A sequence's context, clamped to max_ctx so no index can leave the cache or the partials.
__device__ __forceinline__ uint32_t ctx_of(const uint32_t* ctx, uint32_t b, uint32_t max_ctx)
{
    return min(ctx[b], max_ctx);
}

__device__ __forceinline__ uint32_t slot_of(uint32_t row)
{
    return (row & ~12u) | ((row & 4u) << 1) | ((row & 8u) >> 1);
}

// XOR swizzle of the four 16-byte key chunks in row d of a transposed 32-key V tile.
__device__ __forceinline__ uint32_t vt_swz(uint32_t d) { return ((d >> 1) ^ (d >> 3)) & 3u; }

template <class T>
__global__ __launch_bounds__(kWaves * 64, 2) void decode_split(const DecParams p)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int KS = kD + 8;
    __shared__ __attribute__((aligned(16))) T ks_all[kWaves][kTK * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt_all[kWaves][kD * kTK];

    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t kvh = blockIdx.x;
    // Which sequence and chunk group: workgroups are numbered over the chunk groups that exist.
    const uint32_t per_wg = kWaves * p.split;
    uint32_t x = blockIdx.y, b = p.batch;
    for (uint32_t i = 0; i < p.batch; ++i) {
        const uint32_t n = (ctx_of(p.ctx, i, p.max_ctx) + per_wg - 1) / per_wg;
        if (x < n) {
            b = i;
            break;
        }
        x -= n;
    }
    if (b == p.batch)
        return;
    const uint32_t ctx = ctx_of(p.ctx, b, p.max_ctx);
    const uint32_t chunk = x * kWaves + w;
    const uint32_t k_begin = chunk * p.split;
    if (k_begin >= ctx)
        return;
    const uint32_t k_end = min(k_begin + p.split, ctx);

    T* ks = ks_all[w];
    _Float16* vt = vt_all[w];
    // Q: the B operand; column c32 is query head kvh * group + c32 (zero past the group).
    V8 qreg[kD / 16];
    {
        const uint32_t hq = kvh * p.group + c32;
        const T* src = static_cast<const T*>(p.q) + ((size_t)b * p.heads + hq) * kD + 8 * g;
        for (int kk = 0; kk < kD / 16; ++kk)
            qreg[kk] = c32 < p.group ? *reinterpret_cast<const V8*>(src + 16 * kk) : V8{};
    }
    const size_t head_off = ((size_t)b * p.kv_heads + kvh) * p.cap * kD;
    const T* kbase = static_cast<const T*>(p.k) + head_off;
    const T* vbase = static_cast<const T*>(p.v) + head_off;
    // Loads: K chunk i of this lane is row 4 i + lane / 16, head dims 8 (lane % 16) ..; V rows 8 kg + i (kg =
    // lane / 16), the same head dims.
    const uint32_t cc = lane % 16, kg = lane / 16;
    u32x4 kreg[8], vreg[8];
    auto load_tile = [&](uint32_t j0) {
        for (int i = 0; i < 8; ++i) {
            const uint32_t key = j0 + 4 * i + kg;
            kreg[i] = key < k_end ? *reinterpret_cast<const u32x4*>(kbase + (size_t)key * kD + cc * 8) : u32x4{};
        }
        for (int i = 0; i < 8; ++i) {
            const uint32_t key = j0 + 8 * kg + i;
            vreg[i] = key < k_end ? *reinterpret_cast<const u32x4*>(vbase + (size_t)key * kD + cc * 8) : u32x4{};
        }
    };
    auto store_tile = [&]() {
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4*>(&ks[slot_of(4 * i + kg) * KS + cc * 8]) = kreg[i];
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = cc * 8 + e;
            *reinterpret_cast<u32x4*>(&vt[d * kTK + ((kg ^ vt_swz(d)) * 8)]) =
                u32x4{f16_pair<T>(vreg[0], vreg[1], e), f16_pair<T>(vreg[2], vreg[3], e),
                      f16_pair<T>(vreg[4], vreg[5], e), f16_pair<T>(vreg[6], vreg[7], e)};
        }
    };

    f32x16 oacc[kD / 32];
    for (int db = 0; db < kD / 32; ++db)
        oacc[db] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    const float c = p.scale_log2;
    load_tile(k_begin);
    for (uint32_t j0 = k_begin; j0 < k_end; j0 += kTK) {
        store_tile();
        if (j0 + kTK < k_end)
            load_tile(j0 + kTK);
        asm volatile("" ::: "memory");  // LDS writes before the reads of other lanes (a wave's LDS ops run in order)
        f32x16 s = f32x16{};
        {
            const T* kr = &ks[c32 * KS + 8 * g];
            for (int kk = 0; kk < kD / 16; ++kk)
                s = E::mfma32(*reinterpret_cast<const V8*>(kr + 16 * kk), qreg[kk], s);
        }
        // Register r holds key j0 + 16 (r / 8) + 8 g + r % 8.
        float mx = -INFINITY;
        if (j0 + kTK > k_end) {
            for (int r = 0; r < 16; ++r) {
                const uint32_t j = j0 + 16 * (r >> 3) + 8 * g + (r & 7);
                if (j >= k_end)
                    s[r] = -INFINITY;
            }
        }
        for (int r = 0; r < 16; ++r)
            mx = fmaxf(mx, s[r]);
        mx = fmaxf(mx, swap_halves(mx)) * c;
        float f = 1.0f;
        if (mx > m + kRescale) {
            f = exp2f(m - mx);
            m = mx;
        }
        l *= f;
        if (__any(f != 1.0f))
            for (int db = 0; db < kD / 32; ++db)
                for (int r = 0; r < 16; ++r)
                    oacc[db][r] *= f;
        const float mu = m == -INFINITY ? 0.0f : m;
        H8 pb[2];
        for (int a = 0; a < 2; ++a) {
            u32x4 pk;
            for (int jj = 0; jj < 4; ++jj) {
                const float e0 = exp2f(fmaf(s[8 * a + 2 * jj], c, -mu));
                const float e1 = exp2f(fmaf(s[8 * a + 2 * jj + 1], c, -mu));
                l += e0 + e1;
                pk[jj] = H::pack2(e0, e1);
            }
            pb[a] = __builtin_bit_cast(H8, pk);
        }
        for (int a = 0; a < 2; ++a)
            for (int db = 0; db < kD / 32; ++db) {
                const uint32_t d = 32 * db + c32;
                const _Float16* vr = &vt[d * kTK + (((2 * a + g) ^ vt_swz(d)) * 8)];
                oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb[a], oacc[db]);
            }
        asm volatile("" ::: "memory");
    }
    // The partial: unnormalised O^T column c32 (head dims 32 db + 8 (r / 4) + 4 g + r % 4), maximum and sum.
    const float lt = l + swap_halves(l);
    if (c32 < p.group) {
        const uint32_t hq = kvh * p.group + c32;
        const size_t row = ((size_t)b * p.max_chunks + chunk) * p.heads + hq;
        float* po = p.part_o + row * kD;
        for (int db = 0; db < kD / 32; ++db)
            for (int r4 = 0; r4 < 4; ++r4)
                *reinterpret_cast<f32x4*>(po + 32 * db + 8 * r4 + 4 * g) =
                    f32x4{oacc[db][4 * r4], oacc[db][4 * r4 + 1], oacc[db][4 * r4 + 2], oacc[db][4 * r4 + 3]};
        if (g == 0)
            *reinterpret_cast<float2*>(p.part_ml + row * 2) = float2{m, lt};
    }
}

// One workgroup of 128 threads per (head, sequence): the splits rescaled to their common maximum, summed,
// divided by the total sum; lse = (max + log2 sum) ln 2.
template <class TO>
__global__ __launch_bounds__(128) void decode_merge(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                    const uint32_t* __restrict__ ctx, TO* __restrict__ o,
                                                    float* __restrict__ lse, uint32_t heads, uint32_t max_chunks,
                                                    uint32_t split, uint32_t max_ctx)
{
    const uint32_t h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const uint32_t n = (ctx_of(ctx, b, max_ctx) + split - 1) / split;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        mx = fmaxf(mx, part_ml[(((size_t)b * max_chunks + i) * heads + h) * 2]);
    float sum = 0.0f, acc = 0.0f;
    if (mx != -INFINITY)
        for (uint32_t i = 0; i < n; ++i) {
            const size_t row = ((size_t)b * max_chunks + i) * heads + h;
            const float2 ml = *reinterpret_cast<const float2*>(part_ml + row * 2);
            const float wgt = exp2f(ml.x - mx);  // 0 for a chunk that saw nothing
            sum += ml.y * wgt;
            acc += part_o[row * kD + d] * wgt;
        }
    const float r = sum > 0.0f ? acc / sum : 0.0f;
    o[((size_t)b * heads + h) * kD + d] = (TO)r;
    if (lse && d == 0)
        lse[(size_t)b * heads + h] = sum > 0.0f ? (mx + __log2f(sum)) * kLn2 : -INFINITY;
}

uint32_t split_of(const mako_decode_args* a) { return a->split ? a->split : kDefaultSplit; }

uint32_t max_chunks_of(const mako_decode_args* a)
{
    const uint32_t s = split_of(a);
    const uint32_t per_wg = kWaves * s;
    return (a->max_ctx + per_wg - 1) / per_wg * kWaves;  // whole workgroups of chunks
}

size_t part_o_bytes(const mako_decode_args* a)
{
    return ((size_t)a->batch * max_chunks_of(a) * a->heads * kD * sizeof(float) + 255) / 256 * 256;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mako

using namespace mako;

extern "C" size_t mako_attn_decode_workspace(const mako_decode_args* a)
{
    if (!a)
        return 0;
    return part_o_bytes(a) + (size_t)a->batch * max_chunks_of(a) * a->heads * 2 * sizeof(float);
}

extern "C" int mako_attn_decode(const mako_decode_args* a, mako_dtype in, mako_dtype out, const void* q,
                                const void* k, const void* v, const uint32_t* ctx_len, void* o, float* lse,
                                void* workspace, size_t workspace_bytes, void* stream)
{
    if (!a || !q || !k || !v || !ctx_len || !o)
        return fail(MAKO_EINVAL, "attention_decode: a null argument");
    if (a->dim != kD)
        return fail(MAKO_EUNSUPPORTED, "attention_decode: heads of %u (128)", a->dim);
    if (in != MAKO_F16 && in != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "attention_decode: input type %d (f16 or bf16)", (int)in);
    if (out != MAKO_F32 && out != in)
        return fail(MAKO_EUNSUPPORTED, "attention_decode: output type %d (f32 or the input's)", (int)out);
    if (!a->heads || !a->kv_heads || a->heads % a->kv_heads || a->heads / a->kv_heads > 32)
        return fail(MAKO_EINVAL, "attention_decode: %u heads over %u kv heads (groups of at most 32)", a->heads,
                    a->kv_heads);
    if (a->max_ctx > a->cap)
        return fail(MAKO_EINVAL, "attention_decode: max_ctx %u over the cache's %u rows", a->max_ctx, a->cap);
    const uint32_t split = split_of(a);
    if (split % 64 || split > (1u << 20))
        return fail(MAKO_EINVAL, "attention_decode: %u keys a split (a multiple of 64)", split);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(MAKO_EINVAL, "attention_decode: q, k, v and o must be 16-byte aligned");
    if (!workspace || workspace_bytes < mako_attn_decode_workspace(a) || !aligned16(workspace))
        return fail(MAKO_EWORKSPACE, "attention_decode: workspace of %zu bytes, %zu needed (16-byte aligned)",
                    workspace_bytes, mako_attn_decode_workspace(a));
    if (a->batch == 0)
        return ok();
    const uint32_t max_chunks = max_chunks_of(a);
    float* part_o = static_cast<float*>(workspace);
    float* part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_o_bytes(a));
    const uint32_t groups = a->batch * (max_chunks / kWaves);
    if (groups > 65535u * 64u)
        return fail(MAKO_EINVAL, "attention_decode: %u chunk groups exceed the grid", groups);
    const DecParams p{q, k, v, ctx_len, part_o, part_ml, a->batch, a->heads, a->kv_heads,
                      a->heads / a->kv_heads, a->cap, split, max_chunks, a->max_ctx, a->scale * kLog2e};
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(a->kv_heads, groups), mgrid(a->heads, a->batch);
    if (in == MAKO_BF16)
        hipLaunchKernelGGL(decode_split<__bf16>, grid, dim3(kWaves * 64), 0, s, p);
    else
        hipLaunchKernelGGL(decode_split<_Float16>, grid, dim3(kWaves * 64), 0, s, p);
    if (out == MAKO_F32)
        hipLaunchKernelGGL(decode_merge<float>, mgrid, dim3(kD), 0, s, part_o, part_ml, ctx_len,
                           static_cast<float*>(o), lse, a->heads, max_chunks, split, a->max_ctx);
    else if (out == MAKO_BF16)
        hipLaunchKernelGGL(decode_merge<__bf16>, mgrid, dim3(kD), 0, s, part_o, part_ml, ctx_len,
                           static_cast<__bf16*>(o), lse, a->heads, max_chunks, split, a->max_ctx);
    else
        hipLaunchKernelGGL(decode_merge<_Float16>, mgrid, dim3(kD), 0, s, part_o, part_ml, ctx_len,
                           static_cast<_Float16*>(o), lse, a->heads, max_chunks, split, a->max_ctx);
    return check_launch("attention_decode");
}
