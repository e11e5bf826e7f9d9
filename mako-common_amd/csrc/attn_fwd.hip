// Dense flash attention for gfx950: causal, bidirectional and prefix-causal (by `block`), GQA, head width 64,
// 128 or 256, f16 or bf16 in, f32 / f16 / bf16 out, optional LSE.
//
// The semantics are those of the reference's flash_attn_coop (src/kernels/ops.metal:216-369): key j is visible
// to query row r (position pos = q_pos0 + r) when j < n_k && (j <= pos || (pos >= block && j >= block))
// (ops.metal:289); head h reads kv head h / (heads / kv_heads) (:242); the running maximum moves only when a
// score passes it by 8 in the base-2 domain (:303-316), so most key blocks leave the output unscaled; P is
// rounded to f16 for the P V product (:329); a fully masked row gives 0 (:355); rows >= n_q are not stored
// (:359-362). One difference: the reference's row sum adds the unrounded exponentials (:330), the ping-pong kernel's
// adds the f16 values P V multiplies (v_dot2, half the instructions; the two differ by under 2^-12 relative). With bf16 inputs, V is converted to f16 as it is
// staged, so P keeps f16's 11 significant bits (bf16's 8 would put ~2^-9 |v| of error on rows of few keys).
//
// The design is this one's own, for CDNA4. Shared by both kernels below:
// * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16: Q (the B operand) stays in
//   registers for the whole kernel, K rows (the A operand) come from LDS. In the 32x32 result each lane holds
//   one query row (its column) and 16 keys, so the row's softmax is lane-local but for one exchange with lane
//   l ^ 32, and the output rescale is one scalar per lane.
// * K rows are stored in LDS with bits 2 and 3 of the row swapped within each 32 (slot_of); that makes the
//   registers of S^T, once exponentiated and packed, exactly the B operand of O^T = V^T P^T for 16 consecutive
//   keys, so P never goes through LDS.
// * V is stored transposed in LDS as f16 (one row per head dimension, 64 keys, XOR-swizzled 16-byte chunks),
//   written with an in-register transpose, so the V^T operand is one 16-byte LDS read.
// * Each wave owns 32 query rows of one head; a workgroup's waves cover hq query heads of one GQA group
//   (hq = 4, 2 or 1), so every key / value tile staged in LDS serves all of them.
// * Workgroups are launched heaviest rows first (causal work grows with the row), and the grid's fastest index
//   is the head group, so with 8 kv heads each XCD's L2 holds one kv head's K / V.
// flash_fwd (heads of 64 and 128) runs 8 waves in two groups that alternate matrix and vector phases; the
// running maximum's exchange between the two halves of a wave happens only when some lane's maximum passes its
// threshold. flash_fwd_wide (heads of 256) runs 4 waves with double-buffered tiles.
#include <cstdlib>

#include "device.hpp"

namespace mako {
namespace {

constexpr int kThreads = 256;
constexpr int kKB = 64;  // keys a tile
constexpr float kRescale = 8.0f;

struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    uint32_t n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, width;
    float scale_log2;  // scale * log2(e)
    uint32_t group;    // heads / kv_heads
    uint32_t hq;       // query heads a workgroup (4, 2 or 1; divides group)
    uint32_t rows_wg;  // query rows a workgroup (32 x waves / hq)
    uint32_t n_qblk;   // workgroups along the rows
};

// LDS slot of K row `row` of a tile: bits 2 and 3 swapped within each 32 rows.
__device__ __forceinline__ uint32_t slot_of(uint32_t row)
{
    return (row & ~12u) | ((row & 4u) << 1) | ((row & 8u) >> 1);
}

// XOR swizzle of the 16-byte key chunks in row d of the transposed V tile.
__device__ __forceinline__ uint32_t vt_swz(uint32_t d) { return (d ^ (d >> 3)) & 7u; }

template <class T, class TO, int D>
__global__ __launch_bounds__(kThreads, 1) void flash_fwd_wide(const FwdParams p)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int KS = D + 8;                 // K row stride in LDS (elements): 16 bytes of padding
    constexpr int VS = kKB;                   // V^T row stride (elements)
    constexpr int CPR = D / 8;                // 16-byte chunks a row
    constexpr int NV = kKB * CPR / kThreads;  // chunks a thread loads per tile, K and V each (= D / 32)
    constexpr int NDB = D / 32;               // 32-wide head-dimension blocks of the output
    constexpr int NKK = D / 16;               // 16-wide head-dimension steps of Q K^T
    static_assert(NV * kThreads == kKB * CPR && (NV == 2 || NV == 4 || NV == 8), "tile split");
    __shared__ __attribute__((aligned(16))) T ks[2][kKB * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][D * VS];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform over the wave
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t hg = blockIdx.x;
    const uint32_t qb = p.n_qblk - 1 - blockIdx.y;  // the latest rows (the most keys) first
    const uint32_t h = hg * p.hq + w % p.hq;
    const uint32_t kvh = hg * p.hq / p.group;
    const uint32_t wg_q0 = qb * p.rows_wg;
    const uint32_t q0 = wg_q0 + (w / p.hq) * 32;  // this wave's first row

    // Keys the workgroup visits (the causal bound), and this wave's own bound.
    const uint32_t wg_last = p.q_pos0 + min(wg_q0 + p.rows_wg, p.n_q) - 1;
    const uint32_t n_keys = wg_last >= p.block ? p.n_k : min(p.n_k, wg_last + 1);
    const bool live = q0 < p.n_q;
    const uint32_t w_last = p.q_pos0 + min(q0 + 32, p.n_q) - 1;
    const uint32_t w_keys = !live ? 0u : (w_last >= p.block ? p.n_k : min(p.n_k, w_last + 1));
    const uint32_t p0 = p.q_pos0 + q0;  // the wave's first position
    const uint32_t pos = p0 + c32;      // this lane's row's position

    // Q: the B operand, lane (c32, g) holds row q0 + c32, head dims 16 kk + 8 g .. + 7.
    V8 qreg[NKK];
    {
        // a buffer over this head's n_q rows: rows past n_q load as zeros
        const auto qrs = buffer_rsrc(static_cast<const T*>(p.q) + (size_t)h * p.q_pad * D, p.n_q * D * sizeof(T));
        const uint32_t off = ((q0 + c32) * D + 8 * g) * sizeof(T);
        #pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            qreg[kk] = __builtin_bit_cast(V8, buffer_load16(qrs, off + 16 * kk * sizeof(T)));
        #pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            settle(qreg[kk]);
    }

    // K / V of this kv head as buffer resources over its n_k valid rows: rows past n_k load as zeros.
    const auto krs = buffer_rsrc(static_cast<const T*>(p.k) + (size_t)kvh * p.k_pad * D, p.n_k * D * sizeof(T));
    const auto vrs = buffer_rsrc(static_cast<const T*>(p.v) + (size_t)kvh * p.k_pad * D, p.n_k * D * sizeof(T));
    // V loads: thread -> head-dim chunk cc and NV consecutive keys from NV * kg (kg XOR-ed by the half row so
    // that the transposed LDS writes of a 16-lane group spread over the banks).
    const uint32_t v_cc = tid % CPR;
    const uint32_t v_kg = (tid / CPR) ^ ((tid / (CPR / 2)) & 1u);
    u32x4 kreg[NV], vreg[NV];

    auto load_tile = [&](uint32_t j0) {
        #pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = tid + kThreads * i, row = c / CPR, col = c % CPR;
            kreg[i] = buffer_load16(krs, ((j0 + row) * D + col * 8) * sizeof(T));
        }
        #pragma unroll
        for (int i = 0; i < NV; ++i)
            vreg[i] = buffer_load16(vrs, ((j0 + NV * v_kg + i) * D + v_cc * 8) * sizeof(T));
    };
    auto store_tile = [&](int buf) {
        #pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = tid + kThreads * i, row = c / CPR, col = c % CPR;
            *reinterpret_cast<u32x4*>(&ks[buf][slot_of(row) * KS + col * 8]) = kreg[i];
        }
        const uint32_t key0 = NV * v_kg, kc = key0 / 8, off = key0 % 8;
        #pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = v_cc * 8 + e;
            _Float16* dst = &vt[buf][d * VS + ((kc ^ vt_swz(d)) * 8) + off];
            if constexpr (NV == 2) {
                *reinterpret_cast<uint32_t*>(dst) = f16_pair<T>(vreg[0], vreg[1], e);
            } else if constexpr (NV == 4) {
                *reinterpret_cast<u32x2*>(dst) =
                    u32x2{f16_pair<T>(vreg[0], vreg[1], e), f16_pair<T>(vreg[2], vreg[3], e)};
            } else {
                *reinterpret_cast<u32x4*>(dst) =
                    u32x4{f16_pair<T>(vreg[0], vreg[1], e), f16_pair<T>(vreg[2], vreg[3], e),
                          f16_pair<T>(vreg[4], vreg[5], e), f16_pair<T>(vreg[6], vreg[7], e)};
            }
        }
    };

    f32x16 oacc[NDB];
    #pragma unroll
    for (int db = 0; db < NDB; ++db)
        oacc[db] = f32x16{};
    float m = -INFINITY, l = 0.0f;  // running maximum (base-2 domain) and sum of this lane's keys
    const float c = p.scale_log2;

    const uint32_t nb = (n_keys + kKB - 1) / kKB;
    if (nb > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    for (uint32_t jb = 0; jb < nb; ++jb) {
        const int buf = jb & 1;
        const uint32_t j0 = jb * kKB;
        if (jb + 1 < nb)
            load_tile(j0 + kKB);
        if (j0 < w_keys) {
            // S^T for keys j0 .. j0 + 63: two 32x32 tiles; register r of tile t holds key
            // j0 + 32 t + 16 (r / 8) + 8 g + r % 8 for this lane's row.
            f32x16 s[2] = {f32x16{}, f32x16{}};
            {
                // the two 32-key tiles' products interleaved: two independent accumulation chains
                const T* kr0 = &ks[buf][c32 * KS + 8 * g];
                const T* kr1 = kr0 + 32 * KS;
                #pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    s[0] = E::mfma32(*reinterpret_cast<const V8*>(kr0 + 16 * kk), qreg[kk], s[0]);
                    s[1] = E::mfma32(*reinterpret_cast<const V8*>(kr1 + 16 * kk), qreg[kk], s[1]);
                }
            }
            const bool plain = j0 + kKB <= p.n_k && (j0 + kKB - 1 <= p0 || (p0 >= p.block && j0 >= p.block));
            if (!plain) {
                // the mask rule, branch-free per element
                const bool lane_open = pos >= p.block;
                #pragma unroll
                for (int t = 0; t < 2; ++t)
                    #pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t j = j0 + 32 * t + 16 * (r >> 3) + 8 * g + (r & 7);
                        const bool seen = (j < p.n_k) & ((j <= pos) | (lane_open & (j >= p.block)));
                        s[t][r] = seen ? s[t][r] : -INFINITY;
                    }
            }
            float mx = -INFINITY;
            #pragma unroll
            for (int t = 0; t < 2; ++t)
                #pragma unroll
                for (int r = 0; r < 16; ++r)
                    mx = fmaxf(mx, s[t][r]);
            mx = fmaxf(mx, swap_halves(mx)) * c;  // the row's maximum, base 2 (c > 0)
            float f = 1.0f;
            if (mx > m + kRescale) {
                f = exp2_fast(m - mx);  // 0 while nothing was seen
                m = mx;
            }
            l *= f;
            if (__any(f != 1.0f))
                #pragma unroll
                for (int db = 0; db < NDB; ++db)
                    #pragma unroll
                    for (int r = 0; r < 16; ++r)
                        oacc[db][r] *= f;
            const float mu = m == -INFINITY ? 0.0f : m;
            // P in f16, packed as the B operand of O^T += V^T P^T: chunk 2 t + a holds keys
            // j0 + 32 t + 16 a + 8 g + 0..7 of this lane's row.
            H8 pb[4];
            #pragma unroll
            for (int t = 0; t < 2; ++t)
                #pragma unroll
                for (int a = 0; a < 2; ++a) {
                    u32x4 pk;
                    #pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const float e0 = exp2_fast(fmaf(s[t][8 * a + 2 * jj], c, -mu));
                        const float e1 = exp2_fast(fmaf(s[t][8 * a + 2 * jj + 1], c, -mu));
                        l += e0 + e1;
                        pk[jj] = H::pack2(e0, e1);
                    }
                    pb[2 * t + a] = __builtin_bit_cast(H8, pk);
                }
            #pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                #pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const uint32_t d = 32 * db + c32;
                    const _Float16* vr = &vt[buf][d * VS + (((2 * cc + g) ^ vt_swz(d)) * 8)];
                    oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb[cc], oacc[db]);
                }
        }
        if (jb + 1 < nb)
            store_tile(buf ^ 1);
        __syncthreads();
    }

    // The row's sum over both halves of the wave; normalise and store. Register r of output block db holds head
    // dim 32 db + 8 (r / 4) + 4 g + r % 4.
    const float lt = l + swap_halves(l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const uint32_t row = q0 + c32;
    if (live && row < p.n_q) {
        TO* orow = static_cast<TO*>(p.o) + (size_t)row * p.width + (size_t)h * D;
        #pragma unroll
        for (int db = 0; db < NDB; ++db)
            #pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                store4<TO>(orow + 32 * db + 8 * r4 + 4 * g, oacc[db][4 * r4] * inv, oacc[db][4 * r4 + 1] * inv,
                           oacc[db][4 * r4 + 2] * inv, oacc[db][4 * r4 + 3] * inv);
        if (p.lse && g == 0)
            p.lse[(size_t)h * p.n_q + row] = lt > 0.0f ? (m + __log2f(lt)) * kLn2 : -INFINITY;
    }
}

constexpr int kWaves8 = 8;  // waves a workgroup of the ping-pong kernel

// Heads of 64 and 128. A workgroup is 8 waves, each owning 32 query rows; waves 0-3 and 4-7 form two groups with
// one wave of each on every SIMD. A wave alternates a matrix phase (Q K^T of the next 64-key tile and P V of the
// current one: MFMAs fed from LDS) and a vector phase (the softmax of the next tile's scores, and staging half of
// a later K / V tile into LDS). The groups run one phase apart, separated by workgroup barriers, so on every SIMD
// one wave issues matrix work while the other does vector work. Tiles rotate through three LDS buffers.
template <class T, class TO, int D>
__global__ __launch_bounds__(kWaves8 * 64) void flash_fwd(const FwdParams p)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int NBUF = 3;            // LDS tile buffers
    constexpr int KS = D + 8;          // K row stride in LDS (elements)
    constexpr int VS = kKB;            // V^T row stride (elements)
    constexpr int CPR = D / 8;         // 16-byte chunks a row
    constexpr int GRPI = 256 / CPR;    // K rows one group-wide staging instruction covers
    constexpr int NKG = 32 / GRPI;     // K chunks a thread stages per half tile (2 or 1)
    constexpr int NVP = 16 * CPR;      // (key pair, chunk) units of V in a half tile (threads staging V)
    constexpr int NDB = D / 32;
    constexpr int NKK = D / 16;
    static_assert(D == 64 || D == 128, "ping-pong path: heads of 64 or 128");
    static_assert(NKG * GRPI == 32 && NVP <= 256, "half-tile split");
    __shared__ __attribute__((aligned(16))) T ks[NBUF][kKB * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt[NBUF][D * VS];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform over the wave
    const uint32_t grp = w >> 2;                                  // 0: waves 0-3, 1: waves 4-7
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t hg = blockIdx.x;
    const uint32_t qb = p.n_qblk - 1 - blockIdx.y;  // the latest rows (the most keys) first
    const uint32_t h = hg * p.hq + w % p.hq;
    const uint32_t kvh = hg * p.hq / p.group;
    const uint32_t wg_q0 = qb * p.rows_wg;
    const uint32_t q0 = wg_q0 + (w / p.hq) * 32;  // this wave's first row

    // Keys the workgroup visits (the causal bound), and this wave's own bound.
    const uint32_t wg_last = p.q_pos0 + min(wg_q0 + p.rows_wg, p.n_q) - 1;
    const uint32_t n_keys = wg_last >= p.block ? p.n_k : min(p.n_k, wg_last + 1);
    const bool live = q0 < p.n_q;
    const uint32_t w_last = p.q_pos0 + min(q0 + 32, p.n_q) - 1;
    const uint32_t w_keys = !live ? 0u : (w_last >= p.block ? p.n_k : min(p.n_k, w_last + 1));
    const uint32_t p0 = p.q_pos0 + q0;  // the wave's first position
    const uint32_t pos = p0 + c32;      // this lane's row's position

    // Q: the B operand, lane (c32, g) holds row q0 + c32, head dims 16 kk + 8 g .. + 7 (rows past n_q load as 0).
    V8 qreg[NKK];
    {
        const auto qrs = buffer_rsrc(static_cast<const T*>(p.q) + (size_t)h * p.q_pad * D, p.n_q * D * sizeof(T));
        const uint32_t off = ((q0 + c32) * D + 8 * g) * sizeof(T);
        #pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            qreg[kk] = __builtin_bit_cast(V8, buffer_load16(qrs, off + 16 * kk * sizeof(T)));
        // (settled after the first tiles' loads are in flight too: one round trip for both)
    }

    // Staging: group grp stages keys 32 grp .. 32 grp + 31 of a tile, global -> registers (a buffer resource
    // that starts at the tile, so rows past n_k load as zeros) -> LDS: K row-major in slot order, V transposed to
    // f16. A V thread holds two consecutive keys of one 8-wide head-dimension chunk; the pair's place within its
    // 16-byte chunk is XOR-ed with twice bit 3 of the chunk index so that the 32 lanes of a write cover 32
    // distinct banks.
    const T* kbase = static_cast<const T*>(p.k) + (size_t)kvh * p.k_pad * D;
    const T* vbase = static_cast<const T*>(p.v) + (size_t)kvh * p.k_pad * D;
    const uint32_t gt = tid & 255, hk = 32 * grp;
    const uint32_t k_row = gt / CPR, k_col = gt % CPR;
    const bool v_on = gt < (uint32_t)NVP;
    const uint32_t v_cc = gt % CPR;
    const uint32_t v_kp = ((gt / CPR) & ~3u) | (((gt / CPR) ^ (2 * (v_cc >> 3))) & 3u);  // key pair 0 .. 15
    struct Half {
        u32x4 k[NKG], v[2];
    };
    // (Keys at or past n_keys are masked for every row of the workgroup, so they load as zeros; a tile past the
    // last fetches nothing.)
    auto load_half = [&](uint32_t tile, Half& st) __attribute__((always_inline)) {
        const uint32_t j0 = min(tile * kKB + hk, n_keys);
        const uint32_t left = (n_keys - j0) * D * (uint32_t)sizeof(T);
        const auto krs = buffer_rsrc(kbase + (size_t)j0 * D, left);
        #pragma unroll
        for (int i = 0; i < NKG; ++i)
            st.k[i] = buffer_load16(krs, ((k_row + GRPI * i) * D + k_col * 8) * sizeof(T));
        if (v_on) {
            const auto vrs = buffer_rsrc(vbase + (size_t)j0 * D, left);
            #pragma unroll
            for (int i = 0; i < 2; ++i)
                st.v[i] = buffer_load16(vrs, ((2 * v_kp + i) * D + v_cc * 8) * sizeof(T));
        }
    };
    // This lane's V^T positions in a buffer (the key pair's 8 dims), kept in registers: recomputing them beside
    // each store cost two VALU instructions a store.
    uint32_t vt_off[8];
    {
        const uint32_t key = hk + 2 * v_kp, kc = key / 8, off = key % 8;
        #pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = v_cc * 8 + e;
            vt_off[e] = d * VS + ((kc ^ vt_swz(d)) * 8) + off;
        }
        #pragma unroll
        for (int e = 0; e < 8; e += 4) {
            u32x4 u = {vt_off[e], vt_off[e + 1], vt_off[e + 2], vt_off[e + 3]};
            settle(u);
            for (int i = 0; i < 4; ++i)
                vt_off[e + i] = u[i];
        }
    }
    auto store_half = [&](uint32_t buf, const Half& st) __attribute__((always_inline)) {
        #pragma unroll
        for (int i = 0; i < NKG; ++i)
            *reinterpret_cast<u32x4*>(&ks[buf][(hk + slot_of(k_row + GRPI * i)) * KS + k_col * 8]) = st.k[i];
        if (v_on) {
            #pragma unroll
            for (int e = 0; e < 8; ++e)
                *reinterpret_cast<uint32_t*>(&vt[buf][vt_off[e]]) = f16_pair<T>(st.v[0], st.v[1], e);
        }
    };

    const float c = p.scale_log2;
    // Tile tt's keys all visible to all of this wave's rows.
    auto plain = [&](uint32_t tt) __attribute__((always_inline)) {
        const uint32_t j0 = tt * kKB;
        return j0 + kKB <= p.n_k && (j0 + kKB - 1 <= p0 || (p0 >= p.block && j0 >= p.block));
    };
    // Scores of a tile: s[t] register r holds key 64 tt + 32 t + 16 (r / 8) + 8 g + r % 8 of this lane's row.
    auto qk = [&](f32x16 (&s)[2], uint32_t buf) __attribute__((always_inline)) {
        const T* kr = &ks[buf][c32 * KS + 8 * g];
        s[0] = f32x16{};
        s[1] = f32x16{};
        #pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            s[0] = E::mfma32(*reinterpret_cast<const V8*>(kr + 16 * kk), qreg[kk], s[0]);
            s[1] = E::mfma32(*reinterpret_cast<const V8*>(kr + 32 * KS + 16 * kk), qreg[kk], s[1]);
        }
    };

    f32x16 oacc[NDB];
    #pragma unroll
    for (int db = 0; db < NDB; ++db)
        oacc[db] = f32x16{};
    // Running maximum m (base 2) and sum l of the row; the running maximum moves when a tile's maximum passes
    // m + kRescale, i.e. when a raw score passes thr = (m + kRescale) / c (c > 0).
    float m = -INFINITY, l = 0.0f, thr = -INFINITY;
    f32x16 s[2];  // scores of the next tile
    // P of the current tile, f16 pairs: pw[4 cc .. 4 cc + 3] hold keys 16 cc + 8 g + 0 .. 7 of this lane's row (kept
    // as dwords, not f16 vectors, so that the row sum reads them as whole registers)
    uint32_t pw[16];
    auto pb = [&](int cc) __attribute__((always_inline)) {
        return __builtin_bit_cast(H8, u32x4{pw[4 * cc], pw[4 * cc + 1], pw[4 * cc + 2], pw[4 * cc + 3]});
    };

    // The vector work on a tile's scores: mask, the rescale decision (the row's maximum is formed only when some
    // lane passes its threshold), exponentials, and the row sum of the f16 values the P V product multiplies.
    // Maxima and sums run as four independent chains.
    auto softmax = [&](uint32_t tt) __attribute__((always_inline)) {
        if (!plain(tt)) {
            const bool open = pos >= p.block;
            #pragma unroll
            for (int t = 0; t < 2; ++t)
                #pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t j = tt * kKB + 32 * t + 16 * (r >> 3) + 8 * g + (r & 7);
                    const bool seen = (j < p.n_k) & ((j <= pos) | (open & (j >= p.block)));
                    s[t][r] = seen ? s[t][r] : -INFINITY;
                }
        }
        float mx4[4];
        #pragma unroll
        for (int q = 0; q < 4; ++q)
            mx4[q] = fmaxf(s[q >> 1][8 * (q & 1)], s[q >> 1][8 * (q & 1) + 1]);
        #pragma unroll
        for (int q = 0; q < 4; ++q)
            #pragma unroll
            for (int r = 2; r < 8; ++r)
                mx4[q] = fmaxf(mx4[q], s[q >> 1][8 * (q & 1) + r]);
        const float lmx = fmaxf(fmaxf(mx4[0], mx4[1]), fmaxf(mx4[2], mx4[3]));
        if (__any(lmx > thr)) {
            const float mx = fmaxf(lmx, swap_halves(lmx)) * c;
            const bool up = mx > m + kRescale;
            const float f = up ? exp2_fast(m - mx) : 1.0f;  // 0 while nothing was seen
            m = up ? mx : m;
            thr = up ? (m + kRescale) / c : thr;
            l *= f;
            #pragma unroll
            for (int db = 0; db < NDB; ++db)
                #pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[db][r] *= f;
        }
        const float mu = m == -INFINITY ? 0.0f : m;
        #pragma unroll
        for (int q = 0; q < 16; ++q)
            pw[q] = H::pack2(exp2_fast(fmaf(s[q >> 3][2 * (q & 7)], c, -mu)),
                             exp2_fast(fmaf(s[q >> 3][2 * (q & 7) + 1], c, -mu)));
        float l4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        #pragma unroll
        for (int q = 0; q < 16; ++q)
            l4[q & 3] = sum_f16x2(pw[q], l4[q & 3]);
        l += (l4[0] + l4[1]) + (l4[2] + l4[3]);
    };
    // O^T += V^T P^T for the current tile (V^T in buffer buf).
    auto pv = [&](uint32_t buf) __attribute__((always_inline)) {
        #pragma unroll
        for (int cc = 0; cc < 4; ++cc)
            #pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const uint32_t d = 32 * db + c32;
                const _Float16* vr = &vt[buf][d * VS + (((2 * cc + g) ^ vt_swz(d)) * 8)];
                oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb(cc), oacc[db]);
            }
    };

    // The steady state's matrix phase in one stream: Q K^T of the next tile (2 NKK K fragments) then P V of the
    // current one (4 NDB V^T fragments), each operand read kRing reads ahead of its MFMA (a ring of registers the
    // scheduling groups keep in that order; the compiler alone kept two or three reads in flight).
    auto matrix = [&](uint32_t bk, uint32_t bv) __attribute__((always_inline)) {
        constexpr int NQ = 2 * NKK, N = NQ + 4 * NDB, kRing = 4;
        const T* kr = &ks[bk][c32 * KS + 8 * g];
        auto rd = [&](int i) __attribute__((always_inline)) {
            if (i < NQ)
                return *reinterpret_cast<const u32x4*>(kr + (i & 1) * 32 * KS + 16 * (i >> 1));
            const int cc = (i - NQ) / NDB, db = (i - NQ) % NDB;
            const uint32_t d = 32 * db + c32;
            return *reinterpret_cast<const u32x4*>(&vt[bv][d * VS + (((2 * cc + g) ^ vt_swz(d)) * 8)]);
        };
        u32x4 ring[kRing];
        #pragma unroll
        for (int i = 0; i < kRing; ++i)
            ring[i] = rd(i);
        s[0] = f32x16{};
        s[1] = f32x16{};
        __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);  // the first kRing LDS reads
        #pragma unroll
        for (int i = 0; i < N; ++i) {
            const u32x4 op = ring[i % kRing];
            if (i + kRing < N)
                ring[i % kRing] = rd(i + kRing);
            if (i < NQ) {  // same order as qk: key half i % 2, head-dim step i / 2
                s[i & 1] = E::mfma32(__builtin_bit_cast(V8, op), qreg[i >> 1], s[i & 1]);
            } else {  // same order as pv
                const int cc = (i - NQ) / NDB, db = (i - NQ) % NDB;
                oacc[db] = H::mfma32(__builtin_bit_cast(H8, op), pb(cc), oacc[db]);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // this MFMA
            if (i + kRing < N)
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // then the read kRing ahead
        }
    };

    const uint32_t nt = (n_keys + kKB - 1) / kKB;
    const uint32_t nt_w = (w_keys + kKB - 1) / kKB;
    // Tiles 0 .. 2 by both groups (their loads in flight together); group 1's half of tile 3 into registers.
    Half st;
    {
        Half st1, st2;
        load_half(0, st);
        load_half(1, st1);
        load_half(2, st2);
        store_half(0, st);
        store_half(1, st1);
        store_half(2, st2);
    }
    if (grp == 1)
        load_half(3, st);
    #pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
        settle(qreg[kk]);
    __syncthreads();
    if (nt_w > 0) {
        qk(s, 0);
        softmax(0);
    }
    if (grp == 1)
        __syncthreads();  // group 1 runs one phase behind group 0

    // Vector phase j's staging: group 0 stores its half of tile j + 2 (j >= 1; tile 2 came with the prologue) and
    // loads tile j + 3, group 1 stores its half of tile j + 3 and loads tile j + 4. Loads past the last tile fetch
    // nothing; one code path for both groups.
    uint32_t b0 = 0, b1 = 1, b2 = 2;  // buffers of tiles j, j + 1, j + 2
    auto stage = [&](uint32_t j) __attribute__((always_inline)) {
        const bool put = grp ? j + 3 < nt : j >= 1 && j + 2 < nt;
        if (put)
            store_half(grp ? b0 : b2, st);
        load_half(j + 3 + grp, st);
    };
    auto rotate = [&]() __attribute__((always_inline)) {
        const uint32_t t = b0;
        b0 = b1;
        b1 = b2;
        b2 = t;
    };
    // Three loops with one barrier pattern (two a tile), so that the matrix work of the steady state has no branch
    // around it: tiles this wave computes that have a next one, this wave's last tile, then tiles only the
    // workgroup's other waves compute.
    uint32_t j = 0;
    for (; j + 1 < nt_w; ++j) {
        // matrix phase: scores of tile j + 1, P V of tile j
        __builtin_amdgcn_s_setprio(1);
        __builtin_amdgcn_sched_barrier(0);
        matrix(b1, b0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        // vector phase: softmax of tile j + 1 and the staging
        softmax(j + 1);
        stage(j);
        __syncthreads();
        rotate();
    }
    if (j < nt_w) {
        __builtin_amdgcn_s_setprio(1);
        pv(b0);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        stage(j);
        __syncthreads();
        rotate();
        ++j;
    }
    for (; j < nt; ++j) {
        __syncthreads();
        stage(j);
        __syncthreads();
        rotate();
    }
    if (grp == 0)
        __syncthreads();  // the barrier count of group 1's offset

    // The row's sum over both halves of the wave; normalise and store. Register r of output block db holds head
    // dim 32 db + 8 (r / 4) + 4 g + r % 4.
    const float lt = l + swap_halves(l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const uint32_t row = q0 + c32;
    if (live && row < p.n_q) {
        TO* orow = static_cast<TO*>(p.o) + (size_t)row * p.width + (size_t)h * D;
        #pragma unroll
        for (int db = 0; db < NDB; ++db)
            #pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                store4<TO>(orow + 32 * db + 8 * r4 + 4 * g, oacc[db][4 * r4] * inv, oacc[db][4 * r4 + 1] * inv,
                           oacc[db][4 * r4 + 2] * inv, oacc[db][4 * r4 + 3] * inv);
        if (p.lse && g == 0)
            p.lse[(size_t)h * p.n_q + row] = lt > 0.0f ? (m + __log2f(lt)) * kLn2 : -INFINITY;
    }
}

// Query rows a workgroup covers for heads of `dim` with hq heads a workgroup.
uint32_t rows_per_wg(uint32_t dim, uint32_t hq) { return (dim == 256 ? 4u : (uint32_t)kWaves8) * 32u / hq; }

}  // namespace

// The split-K route for a few query rows (attn_decode.hip): 1 launched, 0 when the case does not take it, -1 when
// its workspace could not be had (the error recorded); splitk_workspace: the bytes it needs.
bool splitk_takes(const mako_attn_args* a, uint32_t dim);
size_t splitk_workspace(const mako_attn_args* a);
int launch_attn_splitk(const mako_attn_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                       const void* v, void* o, float* lse, hipStream_t s, const Workspace& work);

// flash_fwd_r64 (attn_fwd64.hip): heads of 128 and 64 with 64 rows a wave; 1 launched, 0 when a size does not fit
// its offsets. flash_fwd_d256: heads of 256; the same, or -1 when its workspace could not be had (the error
// recorded); d256_workspace: the bytes it needs.
template <class T, class TO, int D>
int launch_fwd64(const mako_attn_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                 float* lse, hipStream_t s);
size_t d256_workspace(const mako_attn_args* a);
// flash_fwd_r32 (attn_fwd_r32.hip): heads of 256 with 32 rows a wave, staged from K and V's rows (no workspace);
// 1 launched, 0 when a size does not fit its offsets (flash_fwd_d256 then takes the call).
bool r32_fits(const mako_attn_args* a, uint32_t out_bytes);
template <class T, class TO>
int launch_fwd_r32(const mako_attn_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                   float* lse, hipStream_t s);
template <class T, class TO>
int launch_fwd_d256(const mako_attn_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                    float* lse, hipStream_t s, const void* vt_ready, const Workspace* work);

namespace {

// MAKO_ATTN_FALLBACK=1 in the environment sends every dense call that reaches the prefill kernels to flash_fwd /
// flash_fwd_wide, the kernels otherwise taken only past the r64 / d256 kernels' 32-bit offsets (calls of several GB),
// so that tests reach them at ordinary sizes. Read at each call.
bool force_fallback()
{
    const char* e = std::getenv("MAKO_ATTN_FALLBACK");
    return e && e[0] == '1';
}

// false when flash_fwd_d256's workspace could not be had (nothing was launched, the error recorded).
template <class T, class TO>
bool launch_d(const mako_attn_args* a, uint32_t dim, const FwdParams& p, dim3 grid, hipStream_t s,
              const Workspace& work)
{
    if (!force_fallback()) {
        const int r = dim == 128 ? launch_fwd64<T, TO, 128>(a, p.scale_log2, p.q, p.k, p.v, p.o, p.lse, s)
                      : dim == 64 ? launch_fwd64<T, TO, 64>(a, p.scale_log2, p.q, p.k, p.v, p.o, p.lse, s)
                      : launch_fwd_r32<T, TO>(a, p.scale_log2, p.q, p.k, p.v, p.o, p.lse, s)
                          ? 1
                          : launch_fwd_d256<T, TO>(a, p.scale_log2, p.q, p.k, p.v, p.o, p.lse, s, nullptr, &work);
        if (r)
            return r > 0;
    }
    switch (dim) {
    case 64:
        hipLaunchKernelGGL((flash_fwd<T, TO, 64>), grid, dim3(kWaves8 * 64), 0, s, p);
        break;
    case 128:
        hipLaunchKernelGGL((flash_fwd<T, TO, 128>), grid, dim3(kWaves8 * 64), 0, s, p);
        break;
    default:
        hipLaunchKernelGGL((flash_fwd_wide<T, TO, 256>), grid, dim3(kThreads), 0, s, p);
        break;
    }
    return true;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mako

using namespace mako;

namespace mako {

int attn_check(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q, const void* k,
               const void* v, const void* o)
{
    if (!a || !q || !k || !v || !o)
        return fail(MAKO_EINVAL, "attention: a null argument");
    if (dim != 64 && dim != 128 && dim != 256)
        return fail(MAKO_EUNSUPPORTED, "attention: heads of %u", dim);
    if (in != MAKO_F16 && in != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "attention: input type %d (f16 or bf16)", (int)in);
    if (out != MAKO_F32 && out != in)
        return fail(MAKO_EUNSUPPORTED, "attention: output type %d (f32 or the input's)", (int)out);
    if (!a->heads || !a->kv_heads || a->heads % a->kv_heads)
        return fail(MAKO_EINVAL, "attention: %u heads over %u kv heads", a->heads, a->kv_heads);
    if (a->n_q > a->q_pad || a->n_k > a->k_pad)
        return fail(MAKO_EINVAL, "attention: %u queries in %u rows, %u keys in %u rows", a->n_q, a->q_pad, a->n_k,
                    a->k_pad);
    if ((uint64_t)a->heads * dim > a->width || a->width % 4)
        return fail(MAKO_EINVAL, "attention: o rows of %u for %u heads of %u (a multiple of 4, at least their width)",
                    a->width, a->heads, dim);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(MAKO_EINVAL, "attention: q, k, v and o must be 16-byte aligned");
    if ((uint64_t)a->k_pad * dim * 2 > 0x7fffffffu || (uint64_t)a->q_pad * dim * 2 > 0x7fffffffu)
        return fail(MAKO_EINVAL, "attention: %u query / %u key rows of %u exceed 2 GiB a head", a->q_pad, a->k_pad,
                    dim);
    if (!(a->scale > 0.0f) || a->scale == INFINITY)
        return fail(MAKO_EINVAL, "attention: scale %g (positive and finite)", (double)a->scale);
    const uint32_t group = a->heads / a->kv_heads;
    const uint32_t hq = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    if ((a->n_q + rows_per_wg(dim, hq) - 1) / rows_per_wg(dim, hq) > 65535)
        return fail(MAKO_EINVAL, "attention: %u queries exceed the grid", a->n_q);
    return MAKO_OK;
}

// The workspace a dense call needs: the split-K partials (heads of 128, a few rows) or, for heads of 256 past
// flash_fwd_r32's offsets (sized for an f32 output, the larger), flash_fwd_d256's V^T images; the prefill kernels
// for heads of 64 and 128, and flash_fwd_r32, need none.
size_t attn_fwd_workspace(const mako_attn_args* a, uint32_t dim)
{
    if (dim == 128 && splitk_takes(a, dim))
        return splitk_workspace(a);
    return dim == 256 && !r32_fits(a, 4) ? d256_workspace(a) : 0;
}

int attn_fwd_core(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q, const void* k,
                  const void* v, void* o, float* lse, const Workspace& work, void* stream)
{
    if (const int e = attn_check(a, dim, in, out, q, k, v, o))
        return e;
    if (a->n_q == 0)
        return ok();
    const uint32_t group = a->heads / a->kv_heads;
    const uint32_t hq = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    FwdParams p{q, k, v, o, lse, a->n_q, a->q_pad, a->n_k, a->k_pad, a->heads, a->kv_heads, a->q_pos0, a->block,
                a->width, a->scale * kLog2e, group, hq, rows_per_wg(dim, hq), 0};
    p.n_qblk = (a->n_q + p.rows_wg - 1) / p.rows_wg;
    const dim3 grid(a->heads / hq, p.n_qblk);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dim == 128) {
        // a few query rows (the reference's decode is attention with n_q = 1): split-K over the keys
        const int r = launch_attn_splitk(a, in, out, q, k, v, o, lse, s, work);
        if (r < 0)
            return last_code() != MAKO_OK ? last_code() : MAKO_EHIP;
        if (r > 0)
            return check_launch("attention");
    }
    bool launched;
    if (in == MAKO_BF16)
        launched = out == MAKO_F32 ? launch_d<__bf16, float>(a, dim, p, grid, s, work)
                                   : launch_d<__bf16, __bf16>(a, dim, p, grid, s, work);
    else
        launched = out == MAKO_F32 ? launch_d<_Float16, float>(a, dim, p, grid, s, work)
                                   : launch_d<_Float16, _Float16>(a, dim, p, grid, s, work);
    if (!launched)
        return last_code() != MAKO_OK ? last_code() : MAKO_EHIP;
    return check_launch("attention");
}

}  // namespace mako

extern "C" size_t mako_attn_fwd_workspace(const mako_attn_args* a, uint32_t dim)
{
    return a ? mako::attn_fwd_workspace(a, dim) : 0;
}

extern "C" int mako_attn_fwd(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q,
                             const void* k, const void* v, void* o, float* lse, void* stream)
{
    return mako::attn_fwd_core(a, dim, in, out, q, k, v, o, lse,
                               mako::library_workspace(dim == 128 ? mako::kWsSplitK : mako::kWsVtImages, "attention"),
                               stream);
}

extern "C" int mako_attn_fwd_ws(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out,
                                const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                                size_t workspace_bytes, void* stream)
{
    return mako::attn_fwd_core(a, dim, in, out, q, k, v, o, lse,
                               mako::caller_workspace(workspace, workspace_bytes, "attention"), stream);
}
