// The gated delta rule with a decay per channel: the reference's kda_scan (src/kernels/ops.metal:459-519), the
// recurrence of the linear-attention layers beside attention in Qwen3.5's encoder (src/models/qwen_text.cpp:374-382).
// For each head, with S its 128 x 128 state (stored transposed: state[h][j][i] = S[i][j]) and each token in order:
//   S[i][:] *= exp(g[i]);  delta[j] = (v[j] - sum_i S[i][j] k[i]) * beta
//   S[i][j] += k[i] * delta[j];  o[j] = sum_i S[i][j] q[i] / sqrt(128)
//
// The design is this one's own. Row j of a head's transposed state evolves on its own: it needs the token's shared
// q, k, g and its own v[j]. A row is 16 lanes (one DPP row) of 8 values each, lane l holding channels 4l .. 4l + 3
// and 64 + 4l .. 64 + 4l + 3, so the two sums over channels are 8 fused multiply-adds a lane and four DPP adds
// (quad swaps, half-row and row mirrors), with no LDS and no barrier. A workgroup of 4 waves takes 16 rows of one
// head (grid: heads x 8), so 1024 waves cover 32 heads. Tokens go through LDS in batches of 16, two buffers: the
// workgroup stages a batch's q, k and exp(g) rows once (coalesced 16-byte loads fetched into registers while the
// previous batch runs; the exponential computed once a channel, not once a row), its v and beta; each lane runs the
// batch's tokens out of LDS (the lane's 8 channels are two 16-byte reads a vector, 16 lanes reading 256 contiguous
// bytes), reading a token's operands one token ahead of the state's chain, and the batch's outputs leave as one
// coalesced store after the next barrier. One barrier a batch.
// Bound: the VALU (no packed FP32 here): 7 flops a channel a row a token.
#include "device.hpp"

namespace mako {
namespace {

constexpr int kD = 128, kRows = 16, kBatch = 16;

struct ScanParams {
    const float *q, *k, *v, *g, *beta;
    float* state;
    float* o;
    float* snap_state;
    uint32_t tokens, qkv_stride, inner, heads, snap;
};

// Sum over the 16 lanes of a DPP row, in every lane: xor 1 and xor 2 within quads, then the half-row and row mirrors.
// bound_ctrl set: every source lane of these patterns is inside the row, and the compiler then folds the move into
// the add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

__device__ __forceinline__ float row_sum16(float x)
{
    x += dpp<0xb1>(x);   // quad_perm [1, 0, 3, 2]
    x += dpp<0x4e>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp<0x141>(x);  // row_half_mirror
    x += dpp<0x140>(x);  // row_mirror
    return x;
}

__global__ __launch_bounds__(256) void kda_scan_rows(const ScanParams a)
{
    // two batch buffers: the next batch's rows are fetched into registers while this batch runs out of LDS
    __shared__ __attribute__((aligned(16))) float qs[2][kBatch][kD];
    __shared__ __attribute__((aligned(16))) float ks[2][kBatch][kD];
    __shared__ __attribute__((aligned(16))) float es[2][kBatch][kD];
    __shared__ float vs[2][kBatch][kRows], bs[2][kBatch], os[2][kBatch][kRows];
    const uint32_t tid = threadIdx.x, h = blockIdx.x, j0 = blockIdx.y * kRows, row = tid >> 4, l = tid & 15;
    const uint32_t c0 = 4 * l, c1 = 64 + 4 * l;  // this lane's channels: c0 .. c0 + 3 and c1 .. c1 + 3
    float* mg = a.state + ((size_t)h * kD + j0 + row) * kD;
    float m[8];
    {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(mg + c0), x1 = *reinterpret_cast<const f32x4*>(mg + c1);
        for (int n = 0; n < 4; ++n) {
            m[n] = x0[n];
            m[4 + n] = x1[n];
        }
    }
    const float scale = 0.08838834764831845f;  // 1 / sqrt(128)
    const size_t hq = (size_t)h * kD;
    // Staging of a batch: thread tid moves runs tid and tid + 256 (token run / 32, channels 4 (run % 32) ..) of q, k
    // and g, v of (token tid / 16, row tid % 16) and beta of token tid; loads past the last token are not issued.
    struct Stage {
        f32x4 q[2], k[2], g[2];
        float v, b;
    };
    auto fetch = [&](Stage& st, uint32_t t0) __attribute__((always_inline)) {
        const uint32_t np = min((uint32_t)kBatch, a.tokens - t0);
        #pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t e = tid + 256 * i, tt = e >> 5, c = 4 * (e & 31);
            if (tt < np) {
                const size_t qo = (size_t)(t0 + tt) * a.qkv_stride + hq + c, go = (size_t)(t0 + tt) * a.inner + hq + c;
                st.q[i] = *reinterpret_cast<const f32x4*>(a.q + qo);
                st.k[i] = *reinterpret_cast<const f32x4*>(a.k + qo);
                st.g[i] = *reinterpret_cast<const f32x4*>(a.g + go);
            }
        }
        if (tid < np * kRows)
            st.v = a.v[(size_t)(t0 + (tid >> 4)) * a.qkv_stride + hq + j0 + (tid & 15)];
        if (tid < np)
            st.b = a.beta[(size_t)(t0 + tid) * a.heads + h];
    };
    auto put = [&](const Stage& st, int b, uint32_t t0) __attribute__((always_inline)) {
        const uint32_t np = min((uint32_t)kBatch, a.tokens - t0);
        #pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t e = tid + 256 * i, tt = e >> 5, c = 4 * (e & 31);
            if (tt < np) {
                *reinterpret_cast<f32x4*>(&qs[b][tt][c]) = st.q[i];
                *reinterpret_cast<f32x4*>(&ks[b][tt][c]) = st.k[i];
                *reinterpret_cast<f32x4*>(&es[b][tt][c]) =
                    f32x4{__expf(st.g[i][0]), __expf(st.g[i][1]), __expf(st.g[i][2]), __expf(st.g[i][3])};
            }
        }
        if (tid < np * kRows)
            vs[b][tid >> 4][tid & 15] = st.v;
        if (tid < np)
            bs[b][tid] = st.b;
    };
    // One token out of buffer b; the operands of the token are read before the state's chain needs them.
    struct Ops {
        f32x4 e0, e1, k0, k1, q0, q1;
        float v, b;
    };
    auto ops = [&](Ops& x, int b, uint32_t tt) __attribute__((always_inline)) {
        x.e0 = *reinterpret_cast<const f32x4*>(&es[b][tt][c0]);
        x.e1 = *reinterpret_cast<const f32x4*>(&es[b][tt][c1]);
        x.k0 = *reinterpret_cast<const f32x4*>(&ks[b][tt][c0]);
        x.k1 = *reinterpret_cast<const f32x4*>(&ks[b][tt][c1]);
        x.q0 = *reinterpret_cast<const f32x4*>(&qs[b][tt][c0]);
        x.q1 = *reinterpret_cast<const f32x4*>(&qs[b][tt][c1]);
        x.v = vs[b][tt][row];
        x.b = bs[b][tt];
    };
    auto step = [&](const Ops& x, int b, uint32_t t, uint32_t tt) __attribute__((always_inline)) {
        const float ev[8] = {x.e0[0], x.e0[1], x.e0[2], x.e0[3], x.e1[0], x.e1[1], x.e1[2], x.e1[3]};
        const float kv[8] = {x.k0[0], x.k0[1], x.k0[2], x.k0[3], x.k1[0], x.k1[1], x.k1[2], x.k1[3]};
        const float qv[8] = {x.q0[0], x.q0[1], x.q0[2], x.q0[3], x.q1[0], x.q1[1], x.q1[2], x.q1[3]};
        float s0 = 0.0f, s1 = 0.0f;
        #pragma unroll
        for (int n = 0; n < 4; ++n) {
            m[n] *= ev[n];
            m[4 + n] *= ev[4 + n];
            s0 = fmaf(m[n], kv[n], s0);
            s1 = fmaf(m[4 + n], kv[4 + n], s1);
        }
        const float d = (x.v - row_sum16(s0 + s1)) * x.b;
        float u0 = 0.0f, u1 = 0.0f;
        #pragma unroll
        for (int n = 0; n < 4; ++n) {
            m[n] = fmaf(kv[n], d, m[n]);
            m[4 + n] = fmaf(kv[4 + n], d, m[4 + n]);
            u0 = fmaf(m[n], qv[n], u0);
            u1 = fmaf(m[4 + n], qv[4 + n], u1);
        }
        const float out = row_sum16(u0 + u1);
        if (l == 0)
            os[b][tt][row] = out * scale;
        if (t + 1 == a.snap) {  // the state after `snap` tokens (uniform across the workgroup)
            float* sg = a.snap_state + ((size_t)h * kD + j0 + row) * kD;
            *reinterpret_cast<f32x4*>(sg + c0) = f32x4{m[0], m[1], m[2], m[3]};
            *reinterpret_cast<f32x4*>(sg + c1) = f32x4{m[4], m[5], m[6], m[7]};
        }
    };
    auto store_out = [&](int b, uint32_t t0) __attribute__((always_inline)) {
        const uint32_t np = min((uint32_t)kBatch, a.tokens - t0);
        if (tid < np * kRows)
            a.o[(size_t)(t0 + (tid >> 4)) * a.inner + hq + j0 + (tid & 15)] = os[b][tid >> 4][tid & 15];
    };
    if (a.tokens > 0) {
        Stage st;
        fetch(st, 0);
        put(st, 0, 0);
        __syncthreads();
        int b = 0;
        for (uint32_t t0 = 0; t0 < a.tokens; t0 += kBatch, b ^= 1) {
            const bool more = t0 + kBatch < a.tokens;
            if (more)
                fetch(st, t0 + kBatch);  // in flight while this batch runs
            if (t0 > 0)
                store_out(b ^ 1, t0 - kBatch);  // the previous batch's outputs (written before the last barrier)
            const uint32_t np = min((uint32_t)kBatch, a.tokens - t0);
            Ops x0, x1;
            ops(x0, b, 0);
            uint32_t tt = 0;
            for (; tt + 1 < np; tt += 2) {  // two tokens a trip: each token's operands read a token ahead
                ops(x1, b, tt + 1);
                step(x0, b, t0 + tt, tt);
                if (tt + 2 < np)
                    ops(x0, b, tt + 2);
                step(x1, b, t0 + tt + 1, tt + 1);
            }
            if (tt < np)
                step(x0, b, t0 + tt, tt);
            if (more)
                put(st, b ^ 1, t0 + kBatch);  // buffer b ^ 1 was last read before the previous barrier
            __syncthreads();
        }
        store_out(b ^ 1, (a.tokens - 1) / kBatch * kBatch);
    }
    *reinterpret_cast<f32x4*>(mg + c0) = f32x4{m[0], m[1], m[2], m[3]};
    *reinterpret_cast<f32x4*>(mg + c1) = f32x4{m[4], m[5], m[6], m[7]};
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mako

using namespace mako;

extern "C" int mako_kda_scan(const mako_scan_args* a, const float* q, const float* k, const float* v, const float* g,
                             const float* beta, float* state, float* o, float* snap_state, void* stream)
{
    if (!a || !q || !k || !v || !g || !beta || !state || !o || (a->snap && !snap_state))
        return fail(MAKO_EINVAL, "kda_scan: a null argument");
    if (a->head_dim != kD)
        return fail(MAKO_EUNSUPPORTED, "kda_scan: head_dim %u (must be 128)", a->head_dim);
    if (!a->heads || a->qkv_stride < a->heads * kD || a->inner < a->heads * kD)
        return fail(MAKO_EINVAL, "kda_scan: %u heads of 128 in rows of %u (q, k, v) and %u (g, o)", a->heads,
                    a->qkv_stride, a->inner);
    if (a->qkv_stride % 4 || a->inner % 4 || !al16(q) || !al16(k) || !al16(g) || !al16(state) ||
        (a->snap && !al16(snap_state)))
        return fail(MAKO_EINVAL, "kda_scan: q, k, g and the states must be 16-byte aligned, row strides multiples of 4");
    if (a->snap > a->tokens)
        return fail(MAKO_EINVAL, "kda_scan: a snapshot after %u of %u tokens", a->snap, a->tokens);
    if (a->heads > 65535u)
        return fail(MAKO_EINVAL, "kda_scan: %u heads exceed the grid", a->heads);
    ScanParams p{q, k, v, g, beta, state, o, snap_state, a->tokens, a->qkv_stride, a->inner, a->heads, a->snap};
    hipLaunchKernelGGL(kda_scan_rows, dim3(a->heads, kD / kRows), dim3(256), 0, static_cast<hipStream_t>(stream), p);
    return check_launch("kda_scan");
}
