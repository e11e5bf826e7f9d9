// The persistent ping-pong flash loop shared by dense prefill (attn_fwd.hip, heads of 64 and 128) and block-sparse
// attention over shared lists (attn_sparse.hip).
//
// One workgroup a CU walks a list of work items (an item: one block of query rows of a few heads, and the key
// tiles it visits); the tile pipeline runs through item boundaries, so a workgroup pays for one prologue and
// one epilogue however many items it runs.
//
// * A workgroup is 8 waves, two a SIMD, each owning 32 query rows of one head (the schedule maps waves to heads
//   and rows). Waves 0-3 and 4-7 form two groups, one wave of each on every SIMD.
// * A wave alternates a matrix phase (S^T = K Q^T of the next tile, O^T += V^T P^T of the current one, on
//   v_mfma_f32_32x32x16 fed from LDS) and a vector phase (the next tile's mask, the rescale decision, the
//   exponentials and row sums, and staging half of a later K / V tile). The groups run one phase apart with
//   workgroup barriers between phases, so on every SIMD one wave issues MFMAs while the other issues VALU.
// * Q (the B operand) stays in registers; an item's Q is loaded in the vector phase before its first product.
//   At an item's last tile, the vector phase stores the finished output and clears the accumulators.
// * Scores are transposed: a lane holds one query row (its column) and 16 keys. K rows sit in LDS with bits 2 and
//   3 of the row swapped (pp_slot_of), which makes the exponentiated, packed scores exactly the B operand of
//   O^T = V^T P^T. V is stored transposed as f16 with XOR-swizzled 16-byte chunks (pp_vt_swz).
// * The running maximum moves only when a tile's maximum passes it by kPPRescale (base 2); the two halves of a wave
//   exchange their maxima only when some lane passes its threshold.
// * K / V tiles of 64 keys rotate through three LDS buffers. Tile j + 2's half of group 0 and tile j + 3's half of
//   group 1 are stored in vector phase j (buffers nothing reads then) and the next halves loaded.
#pragma once

#include "device.hpp"

namespace mako {

constexpr int kPPWaves = 8;      // waves a ping-pong workgroup
constexpr int kPPKeys = 64;      // keys a tile
constexpr float kPPRescale = 8.0f;

// LDS slot of K row `row` of a tile: bits 2 and 3 swapped within each 32 rows.
__device__ __forceinline__ uint32_t pp_slot_of(uint32_t row)
{
    return (row & ~12u) | ((row & 4u) << 1) | ((row & 8u) >> 1);
}

// XOR swizzle of the 16-byte key chunks in row d of the transposed 64-key V tile.
__device__ __forceinline__ uint32_t pp_vt_swz(uint32_t d) { return (d ^ (d >> 3)) & 7u; }

// The assignment of work items to persistent workgroups. Items are (group, rank) pairs: n_groups head groups of
// n_ranks items each, rank 0 the heaviest. Snake order deals items sorted by decreasing work to workgroups 0, 1, ..,
// G - 1, then G - 1, .., 0, and so on, so the heaviest and the lightest share a workgroup. When the workgroups
// divide evenly among the groups, workgroup w serves only group w % n_groups (dealt the same way among that
// group's workgroups): workgroups are spread over the XCDs round robin, so with 8 groups each XCD's L2 then holds
// a single group's K / V.
struct PPDeal {
    uint32_t n_groups, n_ranks, n_wg, wg;
    __device__ bool grouped() const { return n_wg % n_groups == 0; }
    __device__ static uint32_t snake_count(uint32_t n, uint32_t g, uint32_t w)
    {
        const uint32_t full = n / g, rem = n % g;
        const uint32_t pos = (full & 1u) ? g - 1 - w : w;
        return full + (pos < rem ? 1u : 0u);
    }
    __device__ static uint32_t snake_at(uint32_t i, uint32_t g, uint32_t w)
    {
        return i * g + ((i & 1u) ? g - 1 - w : w);
    }
    __device__ uint32_t count() const
    {
        return grouped() ? snake_count(n_ranks, n_wg / n_groups, wg / n_groups)
                         : snake_count(n_groups * n_ranks, n_wg, wg);
    }
    // This workgroup's i-th item: its group and rank.
    __device__ void at(uint32_t i, uint32_t& group, uint32_t& rank) const
    {
        if (grouped()) {
            group = wg % n_groups;
            rank = snake_at(i, n_wg / n_groups, wg / n_groups);
        } else {
            const uint32_t k = snake_at(i, n_wg, wg);
            group = k % n_groups;
            rank = k / n_groups;
        }
    }
};

// An item as the loop sees it: a schedule fills the fields it needs; nt >= 1 (an item with no keys runs one
// fully masked tile, so its output is still written).
struct PPItem {
    uint32_t a, b;  // schedule-defined coordinates (head group, query block)
    uint32_t nt;    // tiles
    uint32_t x;     // schedule-defined (e.g. the pass list length)
    uint32_t kv;    // the kv head
};

// A wave's view of an item.
struct PPWave {
    uint32_t h, kvh;  // query head, kv head
    uint32_t q0;      // first of the wave's 32 rows
    uint32_t nt_w;    // tiles this wave computes (a causal bound), <= the item's nt
};

// The loop. S is the schedule (see DenseSched in attn_fwd.hip and SparseSched in attn_sparse.hip):
//   S::kValid                      tiles carry per-key validity flags (a byte load a lane, balloted)
//   scale_log2()                   the softmax scale times log2(e) (positive)
//   n_items()                      items of this workgroup
//   item(i, it)                    this workgroup's i-th item
//   wave(it, w)                    wave w's view of item it
//   keys(it, t, j0, hi)            tile t's keys start at j0; keys at or past hi are masked
//   extent()                       K / V rows of a kv head that may be loaded (loads past them return zeros)
//   kv_row0(it) / q_row0(wv)       first row of the item's kv head in K / V, of the wave's head in Q; q_rows() of
//                                  them are loadable (rows past return zeros)
//   valid_flag(j, hi)              (kValid) key j's validity
//   plain(it, wv, t, vmask)        every key of tile t visible to every row of the wave
//   seen(j, hi, kbit, pos, open, vmask)         key j (bit kbit of its tile) visible to the lane's row
//   pos_of(wv, lane_row) / open_of(pos)         the lane's row position and whether it sees everything past block
//   finish<TO, D>(it, wv, oacc, l, m, c32, g)   store the item's output rows
template <class T, class TO, int D, class S>
__device__ __forceinline__ void pingpong(const S& sc, const void* q, const void* k, const void* v)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int NBUF = 3;
    constexpr int KS = D + 8;          // K row stride in LDS (elements): 16 bytes of padding
    constexpr int VS = kPPKeys;        // V^T row stride (elements)
    constexpr int CPR = D / 8;         // 16-byte chunks a row
    constexpr int GRPI = 256 / CPR;    // K rows one group-wide staging instruction covers
    constexpr int NKG = 32 / GRPI;     // K chunks a thread stages per half tile (2 or 1)
    constexpr int NVP = 16 * CPR;      // (key pair, chunk) units of V in a half tile (threads staging V)
    constexpr int NDB = D / 32;
    constexpr int NKK = D / 16;
    static_assert(D == 64 || D == 128, "ping-pong loop: heads of 64 or 128");
    static_assert(NKG * GRPI == 32 && NVP <= 256, "half-tile split");
    __shared__ __attribute__((aligned(16))) T ks[NBUF][kPPKeys * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt[NBUF][D * VS];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform over the wave
    const uint32_t grp = w >> 2;                                  // 0: waves 0-3, 1: waves 4-7
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t n_items = sc.n_items();
    if (n_items == 0)
        return;  // (uniform over the workgroup)

    // Tile cursors: an item index in this workgroup's list, a tile within it, and the item. Past the last item a
    // cursor's item has nt = 1 and index n_items (its tile is staged from nowhere and never computed).
    struct Cur {
        uint32_t i, t;
        PPItem it;
    };
    auto fetch = [&](Cur& cu) {
        if (cu.i < n_items)
            sc.item(cu.i, cu.it);
        else
            cu.it = PPItem{0, 0, 1, 0, 0};
    };
    auto advance = [&](Cur& cu) {
        if (++cu.t >= cu.it.nt) {
            ++cu.i;
            cu.t = 0;
            fetch(cu);
        }
    };
    uint32_t total = 0;  // tiles over all items
    for (uint32_t i = 0; i < n_items; ++i) {
        PPItem it;
        sc.item(i, it);
        total += it.nt;
    }
    Cur cA{0, 0, {}};  // tile j: P V, and the item finished after it
    fetch(cA);
    Cur cB = cA, c2 = cA, c3 = cA, c4 = cA;  // tiles j + 1 .. j + 4
    advance(cB);
    advance(c2), advance(c2);
    advance(c3), advance(c3), advance(c3);
    advance(c4), advance(c4), advance(c4), advance(c4);

    // Q of an item: the B operand, lane (c32, g) holds row q0 + c32, head dims 16 kk + 8 g .. + 7.
    V8 qreg[NKK];
    auto load_q = [&](const PPItem& it) {
        const PPWave wv = sc.wave(it, w);
        const auto qrs = buffer_rsrc(static_cast<const T*>(q) + sc.q_row0(wv) * D, sc.q_rows() * D * sizeof(T));
        const uint32_t off = ((wv.q0 + c32) * D + 8 * g) * sizeof(T);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            qreg[kk] = __builtin_bit_cast(V8, buffer_load16(qrs, off + 16 * kk * sizeof(T)));
    };

    // Staging: group grp stages keys 32 grp .. 32 grp + 31 of a tile, global -> registers -> LDS: K row-major in
    // slot order, V transposed to f16. A V thread holds two consecutive keys of one 8-wide head-dimension chunk; the
    // pair's place within its 16-byte chunk is XOR-ed with twice bit 3 of the chunk index so that the 32 lanes of a
    // write cover 32 distinct banks.
    const uint32_t gt = tid & 255, hk = 32 * grp;
    const uint32_t k_row = gt / CPR, k_col = gt % CPR;
    const bool v_on = gt < (uint32_t)NVP;
    const uint32_t v_cc = gt % CPR;
    const uint32_t v_kp = ((gt / CPR) & ~3u) | (((gt / CPR) ^ (2 * (v_cc >> 3))) & 3u);  // key pair 0 .. 15
    struct Half {
        u32x4 k[NKG], v[2];
    };
    auto load_half = [&](const Cur& cu, Half& st) {
        uint32_t j0 = 0, hi = 0, left = 0;
        const T* kb = nullptr;
        const T* vb = nullptr;
        if (cu.i < n_items) {
            sc.keys(cu.it, cu.t, j0, hi);
            j0 += hk;
            const uint32_t ext = sc.extent();
            left = j0 < ext ? (ext - j0) * D * (uint32_t)sizeof(T) : 0u;
            const size_t r0 = sc.kv_row0(cu.it) + min(j0, ext);
            kb = static_cast<const T*>(k) + r0 * D;
            vb = static_cast<const T*>(v) + r0 * D;
        }
        const auto krs = buffer_rsrc(kb, left);
#pragma unroll
        for (int i = 0; i < NKG; ++i)
            st.k[i] = buffer_load16(krs, ((k_row + GRPI * i) * D + k_col * 8) * sizeof(T));
        if (v_on) {
            const auto vrs = buffer_rsrc(vb, left);
#pragma unroll
            for (int i = 0; i < 2; ++i)
                st.v[i] = buffer_load16(vrs, ((2 * v_kp + i) * D + v_cc * 8) * sizeof(T));
        }
    };
    auto store_half = [&](uint32_t buf, const Half& st) {
#pragma unroll
        for (int i = 0; i < NKG; ++i)
            *reinterpret_cast<u32x4*>(&ks[buf][(hk + pp_slot_of(k_row + GRPI * i)) * KS + k_col * 8]) = st.k[i];
        if (v_on) {
            const uint32_t key = hk + 2 * v_kp, kc = key / 8, off = key % 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t d = v_cc * 8 + e;
                *reinterpret_cast<uint32_t*>(&vt[buf][d * VS + ((kc ^ pp_vt_swz(d)) * 8) + off]) =
                    f16_pair<T>(st.v[0], st.v[1], e);
            }
        }
    };

    // Scores of a tile: s[t] register r holds key j0 + 32 t + 16 (r / 8) + 8 g + r % 8 of this lane's row.
    auto qk = [&](f32x16 (&s)[2], uint32_t buf) {
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
    // m + kPPRescale, i.e. when a raw score passes thr = (m + kPPRescale) / c (c > 0).
    const float c = sc.scale_log2();
    float m = -INFINITY, l = 0.0f, thr = -INFINITY;
    f32x16 s[2];  // scores of the next tile
    H8 pb[4];     // P of the current tile in f16: pb[cc] holds keys 16 cc + 8 g + 0 .. 7 of this lane's row

    // The vector work on a tile's scores: mask, the rescale decision, exponentials and the row sum.
    auto softmax = [&](const Cur& cu, const PPWave& wv, uint64_t vmask) {
        if (!sc.plain(cu.it, wv, cu.t, vmask)) {
            uint32_t j0, hi;
            sc.keys(cu.it, cu.t, j0, hi);
            const uint32_t pos = sc.pos_of(wv, wv.q0 + c32);
            const bool open = sc.open_of(pos);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t kbit = 32 * t + 16 * (r >> 3) + 8 * g + (r & 7);
                    s[t][r] = sc.seen(j0 + kbit, hi, kbit, pos, open, vmask) ? s[t][r] : -INFINITY;
                }
        }
        float lmx = s[0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                lmx = fmaxf(lmx, s[t][r]);
        if (__any(lmx > thr)) {
            // some row's maximum moves: the row's maximum over both halves of the wave, then the rescale
            const float mx = fmaxf(lmx, swap_halves(lmx)) * c;
            const bool up = mx > m + kPPRescale;
            const float f = up ? exp2_fast(m - mx) : 1.0f;  // 0 while nothing was seen
            m = up ? mx : m;
            thr = up ? (m + kPPRescale) / c : thr;
            l *= f;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[db][r] *= f;
        }
        const float mu = m == -INFINITY ? 0.0f : m;
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
    };
    // O^T += V^T P^T for the current tile (V^T in buffer buf).
    auto pv = [&](uint32_t buf) {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const uint32_t d = 32 * db + c32;
                const _Float16* vr = &vt[buf][d * VS + (((2 * cc + g) ^ pp_vt_swz(d)) * 8)];
                oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb[cc], oacc[db]);
            }
    };
    // A tile's validity flag for this lane's key (kValid schedules; loaded a phase before its ballot).
    auto vflag_of = [&](const Cur& cu) -> uint32_t {
        if constexpr (S::kValid) {
            if (cu.i >= n_items)
                return 0u;
            uint32_t j0, hi;
            sc.keys(cu.it, cu.t, j0, hi);
            return sc.valid_flag(j0 + lane, hi);
        } else {
            return 1u;
        }
    };
    // The wave's view of the items of tiles j and j + 1 (refreshed when their cursors enter a new item).
    PPWave wvA = sc.wave(cA.it, w), wvB = sc.wave(cB.it, w);
    auto computes = [&](const Cur& cu, const PPWave& wv) { return cu.i < n_items && cu.t < wv.nt_w; };

    // Prologue: the first item's Q and tiles 0 .. 2 by both groups, loads in flight together; group 1's half of
    // tile 3; the first tile's scores and softmax; the next item's Q when tile 1 starts one.
    load_q(cA.it);
    {
        Half h0, h1, h2;
        Cur t1 = cB, t2 = c2;
        load_half(cA, h0);
        load_half(t1, h1);
        load_half(t2, h2);
        store_half(0, h0);
        store_half(1, h1);
        store_half(2, h2);
    }
    Half st;
    if (grp == 1)
        load_half(c3, st);
    uint32_t vflag = vflag_of(cA);
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
        settle(qreg[kk]);
    __syncthreads();
    if (computes(cA, wvA)) {
        qk(s, 0);
        softmax(cA, wvA, __ballot(vflag != 0));
    }
    if (cB.t == 0 && cB.i < n_items) {
        // (a one-tile first item: its successor's Q, settled here so that the loop's waits for Q only ever cover
        // a load issued in the previous vector phase, ahead of that phase's staging loads)
        load_q(cB.it);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            settle(qreg[kk]);
    }
    if (grp == 1)
        __syncthreads();  // group 1 runs one phase behind group 0

    uint32_t b0 = 0, b1 = 1, b2 = 2;  // buffers of tiles j, j + 1, j + 2
    for (uint32_t j = 0; j < total; ++j) {
        // matrix phase: scores of tile j + 1, P V of tile j; tile j + 1's validity flags in flight
        vflag = vflag_of(cB);
        const bool do_qk = computes(cB, wvB), do_pv = computes(cA, wvA);
        __builtin_amdgcn_s_setprio(1);
        if (do_qk)
            qk(s, b1);
        if (do_pv)
            pv(b0);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        // vector phase: the finished item's output, softmax of tile j + 1, the Q of an item starting at tile
        // j + 2, and staging
        if (cA.t + 1 == cA.it.nt) {
            sc.template finish<TO, D>(cA.it, wvA, oacc, l, m, c32, g);
#pragma unroll
            for (int db = 0; db < NDB; ++db)
                oacc[db] = f32x16{};
            m = -INFINITY;
            l = 0.0f;
            thr = -INFINITY;
        }
        if (do_qk)
            softmax(cB, wvB, __ballot(vflag != 0));
        if (c2.t == 0 && c2.i < n_items)
            load_q(c2.it);
        // group 0: tile j + 2 into b2 (tile 2 came with the prologue), then tile j + 3's loads; group 1: tile j + 3
        // into b0, then tile j + 4's
        if (grp == 1 || j >= 1)
            store_half(grp == 0 ? b2 : b0, st);
        load_half(grp == 0 ? c3 : c4, st);
        __syncthreads();
        const uint32_t t = b0;
        b0 = b1;
        b1 = b2;
        b2 = t;
        advance(cA);
        advance(cB);
        advance(c2);
        advance(c3);
        advance(c4);
        if (cA.t == 0)
            wvA = sc.wave(cA.it, w);
        if (cB.t == 0)
            wvB = sc.wave(cB.it, w);
    }
    if (grp == 0)
        __syncthreads();  // the barrier count of group 1's offset
}

}  // namespace mako
