// Block-sparse attention with one selection list per query head (sel_heads == heads: the lists cube_select writes,
// as MiniMax-H3's engine calls it, src/models/h3.cpp:357-363) for f16 heads of 128: flash_sparse_lists. The
// semantics are the reference's attention_sparse (src/kernels/ops.metal:1036-1185) as attn_sparse.hip states them:
// query tile t (64 rows) < n_cubes visits the key cubes its list names, then the dense rows [dense0, dense1); a later
// tile visits [0, n_k); keys with valid[j] == 0 are masked; causal: key j is seen by tile row r only when j <= r;
// query row r's output goes to o row map[r], dropped when map[r] < 0 or r >= n_q; lse [heads][q_pad] by tile row.
//
// Why a kernel of its own: with a list per query head, no two query tiles of a head and no two heads visit the same
// key tiles, so a staged K / V tile serves only the 64 rows of its own (head, query tile). The r64 route's sharing
// (one staged tile for the 4 waves of a workgroup) does not exist here, and a 64-rows-a-wave stream would need a ring
// of 64-key tiles per wave: more LDS than a CU holds for one wave a SIMD. So a workgroup is one (head, query tile):
// 2 waves of 32 rows over 32-key tiles, 17 KiB a tile buffer and two buffers, so that 4 workgroups (8 waves, 2 a
// SIMD) share a CU and one wave's softmax runs beside another's MFMAs.
//
// Staging is raw, by LDS DMA (16 bytes a lane, no conversion): the K image in slot order (slot s holds key
// slot_of(s), so the exponentiated scores fall in the lanes and registers of the P V B operand) with rows padded to
// 272 bytes (the 16 rows a b128 read spans start in distinct banks); the V image as the r64 stream lays it out
// (32-byte units permuted by row) and read by ds_read_b64_tr_b16 as the V^T A operand; and the tile's 32 validity
// bytes. S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16_f16, with P rounded to f16 (to nearest) as the
// reference rounds it (ops.metal:329) and the sums of the unrounded exponentials (:330); the running maximum moves
// only when a tile's passes it by more than 8 (base 2, :303-316). Tile t + 1 is in flight while tile t is computed.
// Items (head, query tile) go head-major, with every head on one XCD at a time when the heads are a multiple of 8
// (the head's K / V then stay in that XCD's L2), and the query tiles from the last (dense tiles, which see every key)
// to the first.
#include "fwd64_common.hpp"

namespace mako {
namespace {

constexpr uint32_t kLD = 128;                     // head dims
constexpr uint32_t kLKeys = 32;                   // keys a tile
constexpr uint32_t kLKRow = 2 * kLD + 16;         // 272: LDS bytes of a K image row
constexpr uint32_t kLKImg = 9 * 1024;             // the K image (8704 bytes) and what its ninth 1 KiB piece spills
constexpr uint32_t kLVImg = kLKeys * 2 * kLD;     // 8 KiB: the V image
constexpr uint32_t kLBuf = kLKImg + kLVImg + 64;  // and the tile's 32 validity bytes
constexpr uint32_t kLMaxSel = 256;                 // list entries a query tile (two cube tiles each)
constexpr float kLRescale = 8.0f;

struct ListsParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const uint16_t* sel;
    const uint16_t* nsel;
    const uint8_t* valid;
    const int32_t* map;
    uint32_t n_q, q_pad, n_k, k_pad, heads, group, width;
    float scale_log2;
    uint32_t n_cubes, max_sel, dense0, dense1, causal, n_qt, xcd_major;
};

// An LDS DMA of 16 bytes a lane: rsrc + voff + soff to LDS m0 + 16 lane.
__device__ __forceinline__ void dma16_at(uint32_t m0, uint32_t voff, uint32_t soff, u32x4 rsrc)
{
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m0), "v"(voff),
                 "s"(rsrc), "s"(soff)
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// Where 32-byte unit u (head dims 16 u .. 16 u + 15) of V row k sits in its LDS row: u ^ (k % 4) ^ 4 (u % 2), a
// bijection of the row's 8 units for each k. A transpose read's 32-lane pass addresses units 2 db and 2 db + 1 of
// four rows k % 4 = 0 .. 3: the XOR with k % 4 spreads the rows over four units and the 4 (u % 2) term puts the odd
// unit's group in the other half of the row, so the pass covers the 64 banks once (without it, twice the 32 of one
// half: a 2-way conflict).
__device__ __forceinline__ uint32_t lv_unit(uint32_t u, uint32_t k) { return u ^ (k & 3u) ^ (4u * (u & 1u)); }
// The V byte, relative to a 1 KiB V image piece, that lane's LDS slot holds (byte 16 lane of the piece: row r,
// physical unit pu, half): the unit lv_unit places at pu, its own inverse up to the parity term.
__device__ __forceinline__ uint32_t lv_src(uint32_t lane)
{
    const uint32_t b = 16 * lane, r = b / 256, pos = b % 256, pu = pos / 32;
    const uint32_t x = pu ^ (r & 3u);
    const uint32_t u = x ^ (4u * (x & 1u));
    return r * 256 + 32 * u + 16 * ((pos / 16) & 1u);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// x over lanes l and l ^ 32 (the two halves of a wave hold the two key halves of a row): the larger and the sum,
// both halves getting the same bits. v_permlane32_swap exchanges the upper 32 lanes of its first operand with the
// lower 32 of its second, so with x in both, one holds x of lanes 0-31 in every lane and the other x of lanes 32-63:
// no LDS round trip. The instruction goes through inline asm because this compiler's builtin returns the first
// operand for both results; the s_nop gives the preceding VALU write its wait states.
__device__ __forceinline__ void lane_halves(float x, float& lo, float& hi)
{
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    lo = __builtin_bit_cast(float, a);
    hi = __builtin_bit_cast(float, b);
}
// max(a, b, c) by one v_max3_f32: fmaxf on values the compiler cannot prove canonical (MFMA results) is a
// canonicalising v_max per operand and then the v_max, three instructions for two values.
__device__ __forceinline__ float max3(float a, float b, float c)
{
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// x where the lane's bit of the wave mask `keep` is set, -inf elsewhere: one v_cndmask on a scalar lane mask.
__device__ __forceinline__ float keep_or_ninf(float x, uint64_t keep)
{
    float r;
    asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(-INFINITY), "v"(x), "s"(keep));
    return r;
}

__device__ __forceinline__ float pair_max(float x)
{
    float lo, hi;
    lane_halves(x, lo, hi);
    return max3(lo, hi, -INFINITY);
}
__device__ __forceinline__ float pair_sum(float x)
{
    float lo, hi;
    lane_halves(x, lo, hi);
    return lo + hi;
}

// Four f16 of V^T by a transpose read at LDS byte `at` of this wave's group pattern.
__device__ __forceinline__ s16x4 tr_read(const unsigned char* at)
{
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at));
}

template <class TO, bool CAUSAL>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2, 2))) void flash_sparse_lists(
    const ListsParams p)
{
    using E = Elem<_Float16>;
    using V8 = f16x8;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * kLBuf];
    __shared__ uint32_t lst[2 * kLMaxSel];  // the first keys of the cube tiles visited, in list order
    __shared__ uint32_t lcnt[2];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 5, c32 = lane & 31;
    // The item: head-major, XCD b % 8 taking heads b % 8, b % 8 + 8, ... when xcd_major.
    uint32_t h, qt;
    {
        const uint32_t b = blockIdx.x;
        const uint32_t s = p.xcd_major ? b / 8 : b;
        h = p.xcd_major ? b % 8 + 8 * (s / p.n_qt) : s / p.n_qt;
        qt = p.n_qt - 1 - s % p.n_qt;
        if (h >= p.heads)
            return;
    }
    const uint32_t kvh = h / p.group;
    const uint32_t q0 = qt * 64 + 32 * w, row = q0 + c32;  // this wave's first row, this lane's row
    const bool live = q0 < p.n_q;

    // The tiles: a cube tile's selected cubes (two tiles each), then its dense rows; a later tile's keys [0, n_k).
    const bool cube = qt < p.n_cubes;
    const uint16_t* my_sel = p.sel + ((size_t)h * p.n_cubes + (cube ? qt : 0u)) * p.max_sel;
    const uint32_t ns = cube ? min(uniform_u16(p.nsel, (size_t)h * p.n_cubes + qt), p.max_sel) : 0u;
    const uint32_t dlo = cube ? p.dense0 : 0u, dhi = cube ? p.dense1 : p.n_k;
    const uint32_t nd = dhi > dlo ? (dhi - dlo + kLKeys - 1) / kLKeys : 0u;

    // Sources: the kv head's k_pad rows of K and V, the k_pad validity bytes (offsets past them load zeros).
    u32x4 krs = rsrc_of(static_cast<const _Float16*>(p.k) + (size_t)kvh * p.k_pad * kLD, p.k_pad * 2 * kLD);
    u32x4 vrs = rsrc_of(static_cast<const _Float16*>(p.v) + (size_t)kvh * p.k_pad * kLD, p.k_pad * 2 * kLD);
    u32x4 brs = rsrc_of(p.valid, p.k_pad);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        krs[i] = __builtin_amdgcn_readfirstlane(krs[i]);
        vrs[i] = __builtin_amdgcn_readfirstlane(vrs[i]);
        brs[i] = __builtin_amdgcn_readfirstlane(brs[i]);
    }
    // K image piece i (1 KiB): lane l's 16 bytes are byte 1024 i + 16 l of the image, row R = that / 272 (key
    // slot_of(R) of the tile), chunk (that % 272) / 16; chunk 16 (the row's padding) and rows past 31 (the spill of
    // piece 8) load any bytes of the tile. Wave w DMAs pieces 4 w .. 4 w + 3 and piece 8 (both waves: the same bytes
    // to the same place). V image piece i: keys 4 i .. 4 i + 3, lane l's slot holds the unit lv_unit places there.
    auto kd_of = [&](uint32_t i) {
        const uint32_t b = 1024 * i + 16 * lane, r = b / kLKRow, ch = b % kLKRow / 16;
        return r < kLKeys && ch < 16 ? slot_of(r) * (2 * kLD) + 16 * ch : 0u;
    };
    uint32_t kd[5], vd[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        kd[m] = kd_of(4 * w + m);
        vd[m] = 1024 * (4 * w + m) + lv_src(lane);
    }
    kd[4] = kd_of(8);
    const uint32_t lbase = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(lds));
    // A tile's K image and validity bytes, and its V image, into buffer buf.
    auto dma_k = [&](uint32_t j0, uint32_t buf) __attribute__((always_inline)) {
        const uint32_t kb = lbase + buf * kLBuf;
        const uint32_t so = __builtin_amdgcn_readfirstlane(j0 * 2 * kLD);
#pragma unroll
        for (int m = 0; m < 4; ++m)
            dma16_at(kb + 1024 * (4 * w + m), kd[m], so, krs);
        dma16_at(kb + 1024 * 8, kd[4], so, krs);
        if (w == 0 && lane < 2)
            dma16_at(kb + kLKImg + kLVImg, 16 * lane, j0, brs);
    };
    auto dma_v = [&](uint32_t j0, uint32_t buf) __attribute__((always_inline)) {
        const uint32_t vb = lbase + buf * kLBuf + kLKImg;
        const uint32_t so = __builtin_amdgcn_readfirstlane(j0 * 2 * kLD);
#pragma unroll
        for (int m = 0; m < 4; ++m)
            dma16_at(vb + 1024 * (4 * w + m), vd[m], so, vrs);
    };

    // Q: the B operand, lane (c32, g) holds row q0 + c32, head dims 16 kk + 8 g .. + 7 (rows past n_q load as 0).
    V8 qreg[8];
    {
        const auto qrs = buffer_rsrc(static_cast<const _Float16*>(p.q) + (size_t)h * p.q_pad * kLD, p.n_q * 2 * kLD);
        const uint32_t off = (row * kLD + 8 * g) * 2;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            qreg[kk] = __builtin_bit_cast(V8, buffer_load16(qrs, off + 32 * kk));
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            settle(qreg[kk]);
    }
    // V^T reads: in each 16-lane group G, lane 4 j + y addresses head dims 16 (G % 2) + 4 y .. + 3 of key 8 (G / 2)
    // + j (+ 4 for the second read, + 16 for keys 16 .. 31) of 32-dim block db, and receives those dims' values for
    // four keys: unit u = 2 db + G % 2 of key row j, at lv_unit(u, j) = 4 ((db / 2) ^ (G % 2)) + ((2 (db % 2) + G % 2)
    // ^ j). Four bases, one for each db % 4; db / 4 is an immediate (none at 128 dims).
    const uint32_t gj = (lane >> 2) & 3u, gy = lane & 3u, gg = (lane >> 4) & 1u;
    uint32_t vbase[4];
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4)
        vbase[d4] = (8 * g + gj) * (2 * kLD) + 32 * lv_unit(2 * d4 + gg, gj) + 8 * gy;

    // The tile sequence: the cube tiles of the list that hold a valid key (not the padding halves of partly
    // filled cubes) and, causal, start at or before the workgroup's last row, then the dense tiles. The cube tiles
    // are found once, before the loop: thread i takes candidate i of each 128 (list entry i / 2, half i % 2), reads
    // its 32 validity bytes, and the kept ones are packed in order into lst (ballot, then each lane's rank). The
    // loop then reads one LDS word a tile instead of two dependent scalar loads a candidate.
    const uint32_t wg_last = qt * 64 + 63;
    uint32_t ncl = 0;
    for (uint32_t r0 = 0; r0 < 2 * ns; r0 += 128) {
        const uint32_t r = r0 + tid;
        bool keep = false;
        uint32_t j0 = 0;
        if (r < 2 * ns) {
            j0 = (uint32_t)my_sel[r >> 1] * 64 + kLKeys * (r & 1);
            const u32x4 a = *reinterpret_cast<const u32x4*>(p.valid + j0);
            const u32x4 b = *reinterpret_cast<const u32x4*>(p.valid + j0 + 16);
            keep = ((a[0] | a[1]) | (a[2] | a[3]) | (b[0] | b[1]) | (b[2] | b[3])) != 0 && (!CAUSAL || j0 <= wg_last);
        }
        const uint64_t bal = __ballot(keep);
        if (lane == 0)
            lcnt[w] = (uint32_t)__builtin_popcountll(bal);
        __syncthreads();
        const uint32_t base = ncl + (w == 1 ? lcnt[0] : 0u);
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (keep)
            lst[base + rank] = j0;
        ncl += lcnt[0] + lcnt[1];
        __syncthreads();  // lcnt is rewritten by the next round; lst is complete after the last
    }
    ncl = __builtin_amdgcn_readfirstlane(ncl);
    const uint32_t ntl = ncl + nd;
    auto next_tile = [&](uint32_t& r, uint32_t& j0, uint32_t& hi) __attribute__((always_inline)) {
        if (r >= ntl)
            return false;
        if (r < ncl) {
            j0 = __builtin_amdgcn_readfirstlane(lst[r]);
            hi = (j0 | 63u) + 1;  // the cube's end
        } else {
            j0 = dlo + kLKeys * (r - ncl);
            hi = dhi;
            if (CAUSAL && j0 > wg_last)  // the dense tiles ascend: none after this one either
                return false;
        }
        ++r;
        return true;
    };

    // S^T of the tile whose K image is in buffer buf: register r holds key j0 + 16 (r / 8) + 8 g + r % 8.
    auto k_scores = [&](uint32_t buf) __attribute__((always_inline)) {
        f32x16 sc = f32x16{};
        const unsigned char* kr = lds + buf * kLBuf + c32 * kLKRow + 16 * g;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            sc = E::mfma32(*reinterpret_cast<const V8*>(kr + 32 * kk), qreg[kk], sc);
        return sc;
    };
    // bit i: key j0 + i of the tile in buffer buf valid and before the pass's end
    auto tile_mask = [&](uint32_t j0, uint32_t hi, uint32_t buf) __attribute__((always_inline)) {
        const uint32_t vflag = lds[buf * kLBuf + kLKImg + kLVImg + c32];
        return (uint32_t)__ballot(vflag != 0 && j0 + c32 < hi);
    };
    // -inf for the scores of keys not seen: invalid, past the pass's end or (causal) past the lane's row. Without
    // the causal limit, register r's key is a wave-uniform bit of vmask for each lane half (8 g + r % 8 + 16 (r / 8)),
    // so its lane mask is two bit tests on the scalar unit and the masking one v_cndmask a register.
    auto mask_scores = [&](f32x16& sc, uint32_t vmask, uint32_t j0) __attribute__((always_inline)) {
        if (!CAUSAL && vmask != 0xffffffffu) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int b = 16 * (r >> 3) + (r & 7);
                const uint64_t keep = (((vmask >> b) & 1u) ? 0x00000000ffffffffull : 0ull) |
                                      (((vmask >> (b + 8)) & 1u) ? 0xffffffff00000000ull : 0ull);
                sc[r] = keep_or_ninf(sc[r], keep);
            }
        } else if (CAUSAL && (vmask != 0xffffffffu || j0 + kLKeys - 1 > q0)) {
            const uint32_t lm = ((vmask >> (8 * g)) & 0xffu) | (((vmask >> (16 + 8 * g)) & 0xffu) << 8);
            const int lim = CAUSAL ? (int)row - (int)j0 : 1 << 30;  // keys j0 + kidx <= row
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kidx = 16 * (r >> 3) + 8 * (int)g + (r & 7);
                const bool seen = ((lm >> r) & 1u) && (!CAUSAL || kidx <= lim);
                sc[r] = seen ? sc[r] : -INFINITY;
            }
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
        oacc[db] = f32x16{};
    float m = -INFINITY, l = 0.0f;  // running maximum (base-2 domain) and sum of this lane's keys
    const float c = p.scale_log2;

    // Two stages: iteration t computes tile t + 1's scores (its K image, DMA'd an iteration ahead of V) beside
    // tile t's exponentials and P V. Buffer t % 2 holds K(t) and V(t); at iteration t, K(t + 2) and its validity
    // bytes go to the slot K(t) left and V(t + 1) to the slot V(t - 1) left.
    uint32_t r = 0, ja = 0, ha = 0, jb = 0, hb = 0;
    const bool ta = next_tile(r, ja, ha);
    bool tb = ta && next_tile(r, jb, hb);
    if (ta) {
        dma_k(ja, 0);
        dma_v(ja, 0);
    }
    if (tb)
        dma_k(jb, 1);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // A wave none of whose 32 rows has an output (the padding rows of a partly filled cube: in H3's layout the
    // second wave of every cube of the last, one-frame cube layer) computes nothing: it stages its share of each
    // tile and keeps the barriers of the other wave's loop, then leaves.
    if (__ballot(live && row < p.n_q && p.map[row] >= 0) == 0) {
        uint32_t bl = 0;
        for (bool have_l = ta; have_l;) {
            uint32_t jc = 0, hc = 0;
            const bool tc = tb && next_tile(r, jc, hc);
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
            if (tc)
                dma_k(jc, bl);
            if (tb)
                dma_v(jb, bl ^ 1);
            have_l = tb;
            tb = tc;
            jb = jc;
            bl ^= 1;
        }
        return;
    }
    f32x16 s_cur = k_scores(0);
    mask_scores(s_cur, tile_mask(ja, ha, 0), ja);
    uint32_t b = 0;
    bool have = ta;
    while (have) {
        uint32_t jc = 0, hc = 0;
        const bool tc = tb && next_tile(r, jc, hc);
        // this wave's DMAs of K(t + 1) and V(t) have landed; past the barrier, the other wave's too, and neither
        // reads the slots of K(t) and V(t - 1) any more
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (tc)
            dma_k(jc, b);
        if (tb)
            dma_v(jb, b ^ 1);
        // tile t's row maxima and the rescale decision
        const float mx0 = max3(s_cur[0], s_cur[1], s_cur[2]), mx1 = max3(s_cur[3], s_cur[4], s_cur[5]);
        const float mx2 = max3(s_cur[6], s_cur[7], s_cur[8]), mx3 = max3(s_cur[9], s_cur[10], s_cur[11]);
        const float mx4 = max3(s_cur[12], s_cur[13], s_cur[14]);
        const float mx = pair_max(max3(max3(mx0, mx1, mx2), max3(mx3, mx4, s_cur[15]), -INFINITY)) * c;
        float f = 1.0f;
        if (mx > m + kLRescale) {
            f = exp2_fast(m - mx);
            m = mx;
        }
        l *= f;
        if (__any(f != 1.0f))
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr)
                    oacc[db][rr] *= f;
        // tile t + 1's scores (stale bytes when there is none: never used) beside tile t's exponentials
        const uint32_t vmask_n = tile_mask(jb, hb, b ^ 1);
        f32x16 s_nxt = k_scores(b ^ 1);
        const float mu = m == -INFINITY ? 0.0f : m;
        V8 pb[2];
        float l4[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four chains of the row sum
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            f16x8 pv;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = exp2_fast(fmaf(s_cur[8 * cc + e], c, -mu));
                l4[e & 3] += x;
                pv[e] = (_Float16)x;
            }
            pb[cc] = pv;
        }
        l += (l4[0] + l4[1]) + (l4[2] + l4[3]);
        // O^T += V^T P^T for tile t: keys 16 cc .. 16 cc + 15, head dims 32 db .. 32 db + 31.
        const unsigned char* vbuf = lds + b * kLBuf + kLKImg;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const unsigned char* va = vbuf + vbase[db] + 16 * cc * (2 * kLD);
                const s16x4 lo = tr_read(va), hi4 = tr_read(va + 4 * (2 * kLD));
                const V8 a = __builtin_bit_cast(V8, __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                oacc[db] = E::mfma32(a, pb[cc], oacc[db]);
            }
        mask_scores(s_nxt, vmask_n, jb);
        s_cur = s_nxt;
        have = tb;
        tb = tc;
        jb = jc;
        hb = hc;
        b ^= 1;
    }

    // Normalise and store through the row map; the LSE by tile row.
    const float lt = pair_sum(l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (live && row < p.n_q) {
        const int32_t dst = p.map[row];
        if (dst >= 0) {
            TO* orow = static_cast<TO*>(p.o) + (size_t)dst * p.width + (size_t)h * kLD;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    store4<TO>(orow + 32 * db + 8 * r4 + 4 * g, oacc[db][4 * r4] * inv, oacc[db][4 * r4 + 1] * inv,
                               oacc[db][4 * r4 + 2] * inv, oacc[db][4 * r4 + 3] * inv);
            if (p.lse && g == 0)
                p.lse[(size_t)h * p.q_pad + row] = lt > 0.0f ? (m + __log2f(lt)) * kLn2 : -INFINITY;
        }
    }
}

}  // namespace

// Whether a call takes flash_sparse_lists: f16 inputs, a list per query head, dense0 and k_pad multiples of 32 (so
// every tile's validity bytes lie inside valid's k_pad), valid 16-byte aligned, and the offsets in range.
bool sparse_lists_fits(const mako_sparse_args* a, mako_dtype in, const void* valid)
{
    return in == MAKO_F16 && a->kv_heads && a->heads % a->kv_heads == 0 && a->sel_heads == a->heads &&
           a->max_sel <= kLMaxSel && a->dense0 % 32 == 0 && a->k_pad % 32 == 0 &&
           (reinterpret_cast<uintptr_t>(valid) & 15u) == 0 &&
           (uint64_t)a->q_pad * 256 < (1ull << 31) && (uint64_t)a->k_pad * 256 < (1ull << 32) &&
           (uint64_t)a->heads * ((a->n_q + 63) / 64) < (1ull << 31);
}

template <class TO>
void launch_sparse_lists(const mako_sparse_args* a, float scale_log2, const void* q, const void* k, const void* v,
                         void* o, const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                         const int32_t* map, float* lse, hipStream_t s)
{
    const uint32_t n_qt = (a->n_q + 63) / 64;
    const ListsParams p{q,        k,          v,           o,         lse,       sel,       nsel,
                        valid,    map,        a->n_q,      a->q_pad,  a->n_k,    a->k_pad,  a->heads,
                        a->heads / a->kv_heads, a->width,  scale_log2, a->n_cubes, a->max_sel, a->dense0,
                        a->dense1, a->causal ? 1u : 0u, n_qt, a->heads % 8 == 0 ? 1u : 0u};
    if (a->causal)
        hipLaunchKernelGGL((flash_sparse_lists<TO, true>), dim3(a->heads * n_qt), dim3(128), 0, s, p);
    else
        hipLaunchKernelGGL((flash_sparse_lists<TO, false>), dim3(a->heads * n_qt), dim3(128), 0, s, p);
}

template void launch_sparse_lists<float>(const mako_sparse_args*, float, const void*, const void*, const void*,
                                         void*, const uint16_t*, const uint16_t*, const uint8_t*, const int32_t*,
                                         float*, hipStream_t);
template void launch_sparse_lists<_Float16>(const mako_sparse_args*, float, const void*, const void*, const void*,
                                            void*, const uint16_t*, const uint16_t*, const uint8_t*,
                                            const int32_t*, float*, hipStream_t);

}  // namespace mako
