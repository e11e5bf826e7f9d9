// The gated delta rule with a decay per channel: the reference's kda_scan (src/kernels/ops.metal:459-519), the
// recurrence of the linear-attention layers beside attention in Qwen3.5's encoder (src/models/qwen_text.cpp:374-382).
// For each head, with S its 128 x 128 state (stored transposed: state[h][j][i] = S[i][j]) and each token in order:
//   S[i][:] *= exp(g[i]);  delta[j] = (v[j] - sum_i S[i][j] k[i]) * beta
//   S[i][j] += k[i] * delta[j];  o[j] = sum_i S[i][j] q[i] / sqrt(128)
//
// The design is this one's own. Row j of a head's transposed state evolves on its own: it needs the token's shared
// q, k, g and its own v[j]. A row is 16 lanes (one DPP row) of 8 values (lane l: channels 4l .. 4l + 3 and
// 64 + 4l .. 64 + 4l + 3), so the two sums over channels are 8 fused multiply-adds a lane and four v_add_f32_dpp:
// all VALU, no LDS round trip and no barrier inside a token. A workgroup of 4 waves takes 16 rows of one head
// (grid: heads x 8), so 32 heads make 1024 waves, one a SIMD. (The kernel also takes 32-lane rows of 4 values, the
// two DPP rows of a pair added by v_permlane16_swap: twice the waves, a third more instructions a token, slower.)
// Tokens go through LDS in batches of 16, two buffers: the workgroup stages a batch's q, k and exp(g) rows once
// (coalesced 16-byte loads fetched into registers while the previous batch runs; the exponential computed once a
// channel, not once a row), its v and beta; each lane runs the batch's tokens out of LDS (a lane reads its runs of
// a vector as 16-byte reads, a row's lanes reading contiguous 256-byte runs), reading a token's operands one token
// ahead of the state's chain, and the batch's outputs leave as one coalesced store after the next barrier. One
// barrier a batch. The token loop is one basic block: a token's output reduction is issued after the next token's
// state update (it is off the state's chain), the rollback snapshot has a loop of its own for the one batch that
// holds it, and nothing in the loop is conditional.
// Bound: the token recurrence (a dependent chain of decay, dot product, lane reduction and update per token) and
// the VALU (no packed FP32 here): 7 flops a channel a row a token.
#include "device.hpp"

#include <type_traits>

namespace mako {
namespace {

constexpr int kD = 128, kBatch = 16;

struct ScanParams {
    const float *q, *k, *v, *g, *beta;
    float* state;
    float* o;
    float* snap_state;
    uint32_t tokens, qkv_stride, inner, heads, snap;
};

// bound_ctrl set: every source lane of these patterns is inside the row, and the compiler then folds the move into
// the add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Sum over the LANES lanes of a state row, in every lane: xor 1 and xor 2 within quads, the half-row and row mirrors
// (16 lanes), then, for 32-lane rows, the two 16-lane rows of each pair added by v_permlane16_swap_b32 (with both
// operands x it returns the pair's even row and its odd row in every lane of the pair), a VALU exchange with no
// LDS round trip.
template <int LANES>
__device__ __forceinline__ float row_sum(float x)
{
    x += dpp<0xb1>(x);   // quad_perm [1, 0, 3, 2]
    x += dpp<0x4e>(x);   // quad_perm [2, 3, 0, 1]
    x += dpp<0x141>(x);  // row_half_mirror
    x += dpp<0x140>(x);  // row_mirror
    if (LANES == 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
        x = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    }
    return x;
}

// LANES lanes a state row, V = 128 / LANES values a lane in G = V / 4 runs of 4 channels: run r of lane l holds
// channels 4 LANES r + 4 l .. + 3, so a run of the lanes of a row is 16 LANES contiguous bytes of a vector.
template <int LANES>
__global__ __launch_bounds__(256) void kda_scan_rows(const ScanParams a)
{
    constexpr int V = kD / LANES, G = V / 4, ROWS = 256 / LANES;
    // two batch buffers: the next batch's rows are fetched into registers while this batch runs out of LDS
    __shared__ __attribute__((aligned(16))) float qs[2][kBatch][kD];
    __shared__ __attribute__((aligned(16))) float ks[2][kBatch][kD];
    __shared__ __attribute__((aligned(16))) float es[2][kBatch][kD];
    __shared__ float vs[2][kBatch][ROWS], bs[2][kBatch], os[2][kBatch][ROWS];
    const uint32_t tid = threadIdx.x, h = blockIdx.x, j0 = blockIdx.y * ROWS, row = tid / LANES, l = tid % LANES;
    uint32_t ch[G];
    #pragma unroll
    for (int r = 0; r < G; ++r)
        ch[r] = 4 * LANES * r + 4 * l;
    float* mg = a.state + ((size_t)h * kD + j0 + row) * kD;
    float m[V];
    #pragma unroll
    for (int r = 0; r < G; ++r) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(mg + ch[r]);
        for (int n = 0; n < 4; ++n)
            m[4 * r + n] = x[n];
    }
    const float scale = 0.08838834764831845f;  // 1 / sqrt(128)
    const size_t hq = (size_t)h * kD;
    // Staging of a batch: thread tid moves runs tid and tid + 256 (token run / 32, channels 4 (run % 32) ..) of q, k
    // and g, v of (token tid / ROWS, row tid % ROWS) and beta of token tid. Past the last token the loads read the
    // last token again (put skips them): loads issued on every path let the compiler wait for exactly the older
    // memory operations in the token loop, where a load under a branch made it wait for these too.
    struct Stage {
        f32x4 q[2], k[2], g[2];
        float v, b;
    };
    auto fetch = [&](Stage& st, uint32_t t0) __attribute__((always_inline)) {
        const uint32_t last = a.tokens - 1;
        #pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t e = tid + 256 * i, t = min(t0 + (e >> 5), last), c = 4 * (e & 31);
            const size_t qo = (size_t)t * a.qkv_stride + hq + c, go = (size_t)t * a.inner + hq + c;
            st.q[i] = *reinterpret_cast<const f32x4*>(a.q + qo);
            st.k[i] = *reinterpret_cast<const f32x4*>(a.k + qo);
            st.g[i] = *reinterpret_cast<const f32x4*>(a.g + go);
        }
        st.v = a.v[(size_t)min(t0 + tid / ROWS, last) * a.qkv_stride + hq + j0 + tid % ROWS];
        st.b = a.beta[(size_t)min(t0 + tid, last) * a.heads + h];
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
        if (tid < np * ROWS)
            vs[b][tid / ROWS][tid % ROWS] = st.v;
        if (tid < np)
            bs[b][tid] = st.b;
    };
    // One token out of buffer b; the operands of the token are read before the state's chain needs them.
    struct Ops {
        f32x4 e[G], k[G], q[G];
        float v, b;
    };
    auto ops = [&](Ops& x, int b, uint32_t tt) __attribute__((always_inline)) {
        #pragma unroll
        for (int r = 0; r < G; ++r) {
            x.e[r] = *reinterpret_cast<const f32x4*>(&es[b][tt][ch[r]]);
            x.k[r] = *reinterpret_cast<const f32x4*>(&ks[b][tt][ch[r]]);
            x.q[r] = *reinterpret_cast<const f32x4*>(&qs[b][tt][ch[r]]);
        }
        x.v = vs[b][tt][row];
        x.b = bs[b][tt];
    };
    // The state's update by one token; returns this lane's part of the token's output (its channels' terms). SNAP:
    // the batch holds token `snap` - 1, so the state after it is copied out.
    auto state = [&](auto SNAP_, const Ops& x, uint32_t t) __attribute__((always_inline)) {
        constexpr bool SNAP = decltype(SNAP_)::value;
        float ev[V], kv[V], qv[V];
        #pragma unroll
        for (int r = 0; r < G; ++r)
            #pragma unroll
            for (int n = 0; n < 4; ++n) {
                ev[4 * r + n] = x.e[r][n];
                kv[4 * r + n] = x.k[r][n];
                qv[4 * r + n] = x.q[r][n];
            }
        float s0 = 0.0f, s1 = 0.0f;
        #pragma unroll
        for (int n = 0; n < V; n += 2) {
            m[n] *= ev[n];
            m[n + 1] *= ev[n + 1];
            s0 = fmaf(m[n], kv[n], s0);
            s1 = fmaf(m[n + 1], kv[n + 1], s1);
        }
        const float d = (x.v - row_sum<LANES>(s0 + s1)) * x.b;
        float u0 = 0.0f, u1 = 0.0f;
        #pragma unroll
        for (int n = 0; n < V; n += 2) {
            m[n] = fmaf(kv[n], d, m[n]);
            m[n + 1] = fmaf(kv[n + 1], d, m[n + 1]);
            u0 = fmaf(m[n], qv[n], u0);
            u1 = fmaf(m[n + 1], qv[n + 1], u1);
        }
        if (SNAP && t + 1 == a.snap) {  // the state after `snap` tokens (uniform across the workgroup)
            float* sg = a.snap_state + ((size_t)h * kD + j0 + row) * kD;
            #pragma unroll
            for (int r = 0; r < G; ++r)
                *reinterpret_cast<f32x4*>(sg + ch[r]) = f32x4{m[4 * r], m[4 * r + 1], m[4 * r + 2], m[4 * r + 3]};
        }
        return u0 + u1;
    };
    // The token's output: the row's sum of the lanes' parts, into the batch's output buffer.
    auto emit = [&](float u, int b, uint32_t tt) __attribute__((always_inline)) {
        const float out = row_sum<LANES>(u);
        os[b][tt][row] = out * scale;  // every lane of the row holds the same sum
    };
    auto store_out = [&](int b, uint32_t t0) __attribute__((always_inline)) {
        const uint32_t np = min((uint32_t)kBatch, a.tokens - t0);
        if (tid < np * ROWS)
            a.o[(size_t)(t0 + tid / ROWS) * a.inner + hq + j0 + tid % ROWS] = os[b][tid / ROWS][tid % ROWS];
    };
    if (a.tokens > 0) {
        Stage st;
        fetch(st, 0);
        put(st, 0, 0);
        __syncthreads();
        int b = 0;
        for (uint32_t t0 = 0; t0 < a.tokens; t0 += kBatch, b ^= 1) {
            const bool more = t0 + kBatch < a.tokens;
            // The previous batch's outputs (written before the last barrier), stored before the next batch's loads
            // are issued: the token loop reuses the store's registers, and the wait for the store (memory
            // operations complete in order) then leaves the loads in flight.
            if (t0 > 0)
                store_out(b ^ 1, t0 - kBatch);
            if (more)
                fetch(st, t0 + kBatch);  // in flight while this batch runs
            const uint32_t np = min((uint32_t)kBatch, a.tokens - t0);
            auto tokens = [&](auto SNAP) __attribute__((always_inline)) {
                Ops x0, x1;
                ops(x0, b, 0);
                uint32_t tt = 0;
                for (; tt + 1 < np; tt += 2) {  // two tokens a trip: each token's operands read a token ahead
                    ops(x1, b, tt + 1);
                    const float u0 = state(SNAP, x0, t0 + tt);
                    ops(x0, b, min(tt + 2, (uint32_t)kBatch - 1));  // (past the batch: read, not used)
                    const float u1 = state(SNAP, x1, t0 + tt + 1);
                    emit(u0, b, tt);  // off the state's chain: its reduction fills the next token's wait states
                    emit(u1, b, tt + 1);
                }
                if (tt < np)
                    emit(state(SNAP, x0, t0 + tt), b, tt);
            };
            if (a.snap > t0 && a.snap <= t0 + np)
                tokens(std::true_type{});
            else
                tokens(std::false_type{});
            if (more)
                put(st, b ^ 1, t0 + kBatch);  // buffer b ^ 1 was last read before the previous barrier
            __syncthreads();
        }
        store_out(b ^ 1, (a.tokens - 1) / kBatch * kBatch);
    }
    #pragma unroll
    for (int r = 0; r < G; ++r)
        *reinterpret_cast<f32x4*>(mg + ch[r]) = f32x4{m[4 * r], m[4 * r + 1], m[4 * r + 2], m[4 * r + 3]};
}

constexpr int kScanLanes = 16;  // lanes a state row: 8 values a lane, one wave a SIMD at 32 heads

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
    hipLaunchKernelGGL(kda_scan_rows<kScanLanes>, dim3(a->heads, kD / (256 / kScanLanes)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p);
    return check_launch("kda_scan");
}
