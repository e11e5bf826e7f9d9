// Split-K attention for gfx950 over each sequence's context, fp32 partials merged by LSE: batched single-token decode
// (one query row a sequence), and the reference's attention() with a few query rows (mako_attn_fwd routes n_q rows
// x the GQA group <= 64 columns here; the prefill kernels would leave the GPU nearly empty).
//
// Semantics: decode: sequence b's one query row sits at position ctx[b] - 1 and sees keys [0, ctx[b]) (the
// reference's mask rule, src/kernels/ops.metal:289, with n_q = 1 and q_pos0 = ctx - 1); attention: one sequence, row r
// at position q_pos0 + r sees key j < n_k when j <= q_pos0 + r or both are >= block (:289); head h reads kv head
// h / (heads / kv_heads) (:242); the running maximum moves only when a score passes it by 8 (base 2, :303-316);
// an empty context gives 0 and lse = -inf (:355); P and V meet in f16 for the P V product (V converted from
// bf16 as it is staged). The reference splits the P V product over keys (attn_pv, src/kernels/gemm.metal:688-730)
// and leaves the softmax and the merge to its caller; here one kernel does the split softmax and products, and
// a second merges the splits.
//
// Design (bandwidth-bound: every K / V byte is read once from HBM):
// * Work split: the K / V rows of all (sequence, kv head) segments, laid end to end, are cut into equal ranges,
//   one per resident wave (2 workgroups of 4 waves per CU), so every wave streams the same number of rows and
//   no workgroup tail is left. A wave's range covers one segment or a few; each (wave, segment) overlap is one
//   piece and writes one partial, stored at index wave + segment (pieces are intervals between consecutive
//   wave and segment boundaries, so that index is unique).
// * Each wave stages 32-key K / V tiles in its own LDS slice (buffer loads that return zeros past the piece's
//   end, four whole 256-byte rows an instruction; the next tile's loads are in flight while the current one is
//   used), so the four waves of a workgroup never wait on each other.
// * The columns of S^T = K Q^T on v_mfma_f32_32x32x16 are (query row, head of the group) pairs, col = r group + hg
//   (decode at GQA 4 uses 4 of the 32): the matrix unit has ~20x the rate this needs, and it keeps the VALU free of
//   per-key dot products and cross-lane reductions. More than 32 columns (up to 64) make each kv head two segments,
//   one a column group, which read the same K / V at the same time (the second read mostly hits the cache), so a
//   wave never needs a second block of accumulators. A column masks the keys its row does not see (only tiles past
//   the first row's limit need it). K rows are stored with bits 2 and 3 of the row swapped so the exponentiated scores are
//   already the B operand of O^T = V^T P^T; V is transposed into LDS through registers.
// * Partials: the unnormalised O^T columns, the running maximum and the row sum; the merge rescales a
//   segment's pieces to their common maximum and divides once. With many columns a wave takes more keys (at least
//   8 a column), so the partials stay a small share of the K / V bytes.
#include <algorithm>
#include <mutex>

#include "device.hpp"

namespace mako {
namespace {

constexpr int kWaves = 4;
constexpr int kWgPerCu = 2;
constexpr int kTK = 32;  // keys a tile
constexpr int kD = 128;
constexpr float kRescale = 8.0f;

struct DecParams {
    const void* q;
    const void* k;
    const void* v;
    const uint32_t* ctx;  // keys of each sequence's segment; null: every sequence has max_ctx
    float* part_o;   // [pieces][nc][kD]
    float* part_ml;  // [pieces][nc][2]: maximum (base 2), sum
    uint32_t batch, heads, kv_heads, group, cap, max_ctx, n_waves;
    float scale_log2;
    uint32_t nq;          // query rows a sequence; nc = nq * group columns (<= 64)
    uint32_t ncg, ncs;    // column groups a kv head (segments a kv head), columns a segment (<= 32)
    uint32_t q_pos0;      // position of row 0 (UINT32_MAX: ctx - nq, the decode case)
    uint32_t block, n_k;  // the visibility rule's block and key count
    uint32_t qs_b, qs_h, qs_r;  // q element strides: sequence, head, row
    uint32_t os_b, os_r;        // o element strides: sequence, row (head h at h * kD)
    uint32_t ls_b, ls_h, ls_r;  // lse strides
};

// A sequence's context, clamped to max_ctx so no index can leave the cache.
__device__ __forceinline__ uint32_t ctx_of(const uint32_t* ctx, uint32_t b, uint32_t max_ctx)
{
    return ctx ? min(ctx[b], max_ctx) : max_ctx;
}

// The sum of the contexts of sequences [0, n) (every lane gets it), read 64 at a time: lane-parallel loads and a
// wave reduction, not n dependent steps.
__device__ __forceinline__ uint32_t ctx_sum(const DecParams& p, uint32_t n, uint32_t lane)
{
    if (!p.ctx)
        return n * p.max_ctx;
    uint32_t s = 0;
    for (uint32_t i0 = 0; i0 < n; i0 += 64) {
        uint32_t v = i0 + lane < n ? min(p.ctx[i0 + lane], p.max_ctx) : 0u;
        #pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            v += __shfl_xor(v, o);
        s += v;
    }
    return s;
}

// The sequence b whose rows (laid end to end, nseg rows a key) hold row r, and the first row of its segments;
// b = batch when r is past them all. Lane-parallel as ctx_sum: an inclusive prefix over 64 sequences at a time, the
// first lane whose end passes r.
__device__ __forceinline__ void seq_of(const DecParams& p, uint32_t r, uint32_t lane, uint32_t nseg, uint32_t& b,
                                       uint32_t& seg0)
{
    if (!p.ctx) {
        const uint32_t per = p.max_ctx * nseg;
        b = per ? min(r / per, p.batch) : p.batch;
        seg0 = b * per;
        return;
    }
    uint32_t base = 0;
    for (uint32_t i0 = 0; i0 < p.batch; i0 += 64) {
        const uint32_t i = i0 + lane;
        const uint32_t len = i < p.batch ? min(p.ctx[i], p.max_ctx) * nseg : 0u;
        uint32_t inc = len;
        #pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(inc, o);
            inc += lane >= (uint32_t)o ? t : 0u;
        }
        const uint64_t hit = __ballot(i < p.batch && r < base + inc);
        if (hit) {
            const uint32_t first = (uint32_t)__builtin_ctzll(hit);
            b = i0 + first;
            seg0 = base + __shfl(inc - len, first);
            return;
        }
        base += __shfl(inc, 63);
    }
    b = p.batch;
    seg0 = base;
}

// A value the whole wave holds (the index arithmetic of seq_of goes through lane shuffles, so the compiler cannot
// prove it uniform; buffer resources built from it would need a waterfall loop around every load).
__device__ __forceinline__ uint32_t uniform(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane(x); }

// The keys row r of a sequence with context ctx sees: [0, lim).
__device__ __forceinline__ uint32_t lim_of(const DecParams& p, uint32_t ctx, uint32_t r)
{
    const uint32_t pos = (p.q_pos0 == 0xffffffffu ? ctx - p.nq : p.q_pos0) + r;
    return pos >= p.block ? ctx : min(ctx, pos + 1);
}

// The rows of all segments laid end to end, cut into n equal ranges: range w starts at floor(w T / n), computed
// as w q + (w r) / n with q, r = T divmod n (w r < n^2 fits 32 bits), so no 64-bit division is needed.
// T < 2^32 always (2^32 K / V rows of 128 f16 values would be 2 TB).
struct Ranges {
    uint32_t T, n, q, r;
    __device__ Ranges(uint32_t total, uint32_t n_waves) : T(total), n(n_waves), q(total / n_waves), r(total % n_waves) {}
    __device__ __forceinline__ uint32_t start(uint32_t w) const { return w * q + (w * r) / n; }
    __device__ __forceinline__ bool empty(uint32_t w) const { return start(w) == start(w + 1); }
    // The wave whose range holds row x.
    __device__ __forceinline__ uint32_t wave_of(uint32_t x) const
    {
        uint32_t w = (uint32_t)(((uint64_t)x * n) / T);
        while (w + 1 < n && start(w + 1) <= x)
            ++w;
        while (w > 0 && start(w) > x)
            --w;
        return w;
    }
};

__device__ __forceinline__ uint32_t slot_of(uint32_t row)
{
    return (row & ~12u) | ((row & 4u) << 1) | ((row & 8u) >> 1);
}

// XOR swizzle of the four 16-byte key chunks in row d of a transposed 32-key V tile.
__device__ __forceinline__ uint32_t vt_swz(uint32_t d) { return ((d >> 1) ^ (d >> 3)) & 3u; }

// One wave's keys of a piece: the 32-key tiles at j_first, j_first + step, ... below k_end of one segment (K / V
// through krs / vrs, rows at or past k_end loading as zeros), against its 32 columns' Q (the B operand, qreg). The
// wave stages each tile in its own LDS slice (ks: K rows with bits 2 and 3 swapped, so the exponentiated scores are
// already the B operand of O^T = V^T P^T; vt: V^T in f16, through registers), with the next tile's loads in flight
// while the current one is used. Keys at or past min(k_end, lim) are masked (tiles below lim_all need no mask).
// Leaves the unnormalised O^T (register r of block db: head dim 32 db + 8 (r / 4) + 4 g + r % 4 of column c32), the
// running maximum m (base 2, scaled; the same in both halves; -inf when no key was seen) and this lane's share l of
// the row sum.
template <class T>
__device__ __forceinline__ void wave_keys(const DecParams& p, T* ks, _Float16* vt, typename Elem<T>::vec8* qreg,
                                          __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs, uint32_t j_first,
                                          uint32_t step, uint32_t k_end, uint32_t lim, uint32_t lim_all,
                                          f32x16 (&oacc)[kD / 32], float& m, float& l)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int KS = kD + 8;
    const uint32_t lane = threadIdx.x & 63, g = lane >> 5, c32 = lane & 31;
    // Loads: K chunk i of this lane is row 4 i + lane / 16, head dims 8 (lane % 16) ..; V rows 8 kg + i, the same
    // head dims.
    // Streaming (non-temporal) loads, or plain ones when two column groups read each tile (the second read then
    // hits the L2 line the first brought in).
    const uint32_t cc = lane % 16, kg = lane / 16;
    const bool shared = p.ncg > 1;
    u32x4 kreg[8], vreg[8];
    auto load16 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off) {
        return shared ? buffer_load16(r, off) : buffer_load16_nt(r, off);
    };
    auto load_tile = [&](uint32_t j0) {
        #pragma unroll
        for (int i = 0; i < 8; ++i)
            kreg[i] = load16(krs, ((j0 + 4 * i + kg) * kD + cc * 8) * sizeof(T));
        #pragma unroll
        for (int i = 0; i < 8; ++i)
            vreg[i] = load16(vrs, ((j0 + 8 * kg + i) * kD + cc * 8) * sizeof(T));
    };
    auto store_tile = [&]() {
        #pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4*>(&ks[slot_of(4 * i + kg) * KS + cc * 8]) = kreg[i];
        #pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = cc * 8 + e;
            *reinterpret_cast<u32x4*>(&vt[d * kTK + ((kg ^ vt_swz(d)) * 8)]) =
                u32x4{f16_pair<T>(vreg[0], vreg[1], e), f16_pair<T>(vreg[2], vreg[3], e),
                      f16_pair<T>(vreg[4], vreg[5], e), f16_pair<T>(vreg[6], vreg[7], e)};
        }
    };

    #pragma unroll
    for (int db = 0; db < kD / 32; ++db)
        oacc[db] = f32x16{};
    m = -INFINITY;
    l = 0.0f;
    if (j_first >= k_end)
        return;
    const float c = p.scale_log2;
    load_tile(j_first);
    // Q (loaded by load_q, before the first tile) arrives: waiting here for it does not wait for the tile
    #pragma unroll
    for (int kk = 0; kk < kD / 16; ++kk)
        settle(qreg[kk]);
    for (uint32_t j0 = j_first; j0 < k_end; j0 += step) {
        store_tile();
        if (j0 + step < k_end)
            load_tile(j0 + step);
        asm volatile("" ::: "memory");  // LDS writes before other lanes' reads (a wave's LDS ops run in order)
        f32x16 s = f32x16{};
        {
            const T* kr = &ks[c32 * KS + 8 * g];
            #pragma unroll
            for (int kk = 0; kk < kD / 16; ++kk)
                s = E::mfma32(*reinterpret_cast<const V8*>(kr + 16 * kk), qreg[kk], s);
        }
        // Register r holds key j0 + 16 (r / 8) + 8 g + r % 8; keys past the piece or the column's row are masked.
        if (j0 + kTK > min(k_end, lim_all)) {
            const uint32_t end = min(k_end, lim);
            #pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t j = j0 + 16 * (r >> 3) + 8 * g + (r & 7);
                s[r] = j < end ? s[r] : -INFINITY;
            }
        }
        float mx = -INFINITY;
        #pragma unroll
        for (int r = 0; r < 16; ++r)
            mx = fmaxf(mx, s[r]);
        mx = fmaxf(mx, swap_halves(mx)) * c;
        float f = 1.0f;
        if (mx > m + kRescale) {
            f = exp2_fast(m - mx);
            m = mx;
        }
        l *= f;
        if (__any(f != 1.0f))
            #pragma unroll
            for (int db = 0; db < kD / 32; ++db)
                #pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[db][r] *= f;
        const float mu = m == -INFINITY ? 0.0f : m;
        H8 pb[2];
        #pragma unroll
        for (int a = 0; a < 2; ++a) {
            u32x4 pk;
            #pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const float e0 = exp2_fast(fmaf(s[8 * a + 2 * jj], c, -mu));
                const float e1 = exp2_fast(fmaf(s[8 * a + 2 * jj + 1], c, -mu));
                l += e0 + e1;
                pk[jj] = H::pack2(e0, e1);
            }
            pb[a] = __builtin_bit_cast(H8, pk);
        }
        #pragma unroll
        for (int a = 0; a < 2; ++a)
            #pragma unroll
            for (int db = 0; db < kD / 32; ++db) {
                const uint32_t d = 32 * db + c32;
                const _Float16* vr = &vt[d * kTK + (((2 * a + g) ^ vt_swz(d)) * 8)];
                oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb[a], oacc[db]);
            }
        asm volatile("" ::: "memory");
    }
}

// Q of a wave's 32 columns as the MFMA's B operand: lane (c32, g) holds head dims 16 kk + 8 g .. + 7 of column
// c32 (zero when has_col is false). The loads stay in flight: wave_keys waits for them after issuing its first
// tile's loads, so the two round trips overlap.
template <class T>
__device__ __forceinline__ void load_q(const DecParams& p, uint32_t b, uint32_t kvh, uint32_t col, bool has_col,
                                       typename Elem<T>::vec8 (&qreg)[kD / 16])
{
    using V8 = typename Elem<T>::vec8;
    const uint32_t g = (threadIdx.x & 63) >> 5;
    const uint32_t r = col / p.group, hq = kvh * p.group + col % p.group;
    const T* src = static_cast<const T*>(p.q) + (size_t)b * p.qs_b + (size_t)hq * p.qs_h + (size_t)r * p.qs_r + 8 * g;
    #pragma unroll
    for (int kk = 0; kk < kD / 16; ++kk)
        qreg[kk] = has_col ? *reinterpret_cast<const V8*>(src + 16 * kk) : V8{};
}

template <class T>
__global__ __launch_bounds__(kWaves * 64, 2) void decode_split(const DecParams p)
{
    using V8 = typename Elem<T>::vec8;
    constexpr int KS = kD + 8;
    __shared__ __attribute__((aligned(16))) T ks_all[kWaves][kTK * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt_all[kWaves][kD * kTK];

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t wave = blockIdx.x * kWaves + wl;
    const uint32_t nc = p.nq * p.group, nseg = p.kv_heads * p.ncg;

    // The rows laid end to end: segment (b, sh) = b * nseg + sh (kv head sh / ncg, column group sh % ncg) holds
    // ctx[b] rows.
    const uint32_t total = uniform(ctx_sum(p, p.batch, lane) * nseg);
    if (total == 0)
        return;
    const Ranges rg(total, p.n_waves);
    const uint32_t r0 = rg.start(wave), r1 = rg.start(wave + 1);
    if (r0 >= r1)
        return;
    // The segment holding r0 (seg0: the first row of sequence b's segments).
    uint32_t b, seg0;
    seq_of(p, r0, lane, nseg, b, seg0);
    b = uniform(b);
    seg0 = uniform(seg0);
    uint32_t ctx = uniform(ctx_of(p.ctx, b, p.max_ctx));
    uint32_t sh = (r0 - seg0) / ctx;
    uint32_t row = r0;

    while (row < r1) {
        // One piece: segment (b, sh), keys [k_begin, k_end).
        const uint32_t s_start = seg0 + sh * ctx;
        const uint32_t k_begin = row - s_start;
        const uint32_t k_end = min(ctx, r1 - s_start);
        const uint32_t seg = b * nseg + sh;
        const uint32_t kvh = sh / p.ncg;
        // Column of the lane: col = 32 (sh % ncg) + c32, row col / group, head kvh * group + col % group; its keys
        // [0, lim) (none past the segment's columns). Tiles below lim_all need no mask: every column sees them.
        const uint32_t col = 32 * (sh % p.ncg) + c32;
        const bool has_col = c32 < p.ncs && col < nc;
        const uint32_t lim = has_col ? lim_of(p, ctx, col / p.group) : 0u;
        const uint32_t lim_all = lim_of(p, ctx, 0);
        V8 qreg[kD / 16];
        load_q<T>(p, b, kvh, col, has_col, qreg);
        const size_t head_off = ((size_t)b * p.kv_heads + kvh) * p.cap * kD;
        const auto krs = buffer_rsrc(static_cast<const T*>(p.k) + head_off, k_end * kD * sizeof(T));
        const auto vrs = buffer_rsrc(static_cast<const T*>(p.v) + head_off, k_end * kD * sizeof(T));
        f32x16 oacc[kD / 32];
        float m, l;
        wave_keys<T>(p, ks_all[wl], vt_all[wl], qreg, krs, vrs, k_begin, kTK, k_end, lim, lim_all, oacc, m, l);
        // The piece's partial at index wave + segment: unnormalised O^T column c32 of the segment (head dims
        // 32 db + 8 (r / 4) + 4 g + r % 4), maximum and sum.
        const float lt = l + swap_halves(l);
        if (has_col) {
            const size_t prow = ((size_t)wave + seg) * p.ncs + c32;
            float* po = p.part_o + prow * kD;
            #pragma unroll
            for (int db = 0; db < kD / 32; ++db)
                #pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *reinterpret_cast<f32x4*>(po + 32 * db + 8 * r4 + 4 * g) =
                        f32x4{oacc[db][4 * r4], oacc[db][4 * r4 + 1], oacc[db][4 * r4 + 2], oacc[db][4 * r4 + 3]};
            if (g == 0)
                *reinterpret_cast<float2*>(p.part_ml + prow * 2) = float2{m, lt};
        }
        // The next segment (sequences with an empty context hold no rows and are skipped).
        row = s_start + k_end;
        if (++sh == nseg) {
            sh = 0;
            seg0 += ctx * nseg;
            do {
                ++b;
            } while (b < p.batch && ctx_of(p.ctx, b, p.max_ctx) == 0);
            if (b >= p.batch)
                break;
            ctx = uniform(ctx_of(p.ctx, b, p.max_ctx));
        }
    }
}

// A whole workgroup on each piece (mako_attn_fwd's few-row route):
// * One workgroup of kCoopWaves waves a CU; the rows of all (sequence, kv head) segments, laid end to end, are cut
//   into equal ranges, one a workgroup. Column groups do not make segments here: wave w takes column group
//   w % ncg and every (kCoopWaves / ncg)-th 32-key tile of the piece (the waves of the two column groups read the
//   same tiles at about the same time, so the second read is served by the L2).
// * The waves of a column group combine their partials through LDS (rescaled to their common maximum), and the
//   workgroup writes one partial a piece and column, at index workgroup + segment as in decode_split: a
//   workgroup's 8 waves leave one partial where decode_split's would leave 8, so the merge (decode_merge, with one
//   column group of nc columns) reads 8 times fewer.
constexpr int kCoopWaves = 8;
constexpr int kSliceBytes = kTK * (kD + 8) * 2 + kD * kTK * 2;  // a wave's K tile and V^T tile

template <class T>
__global__ __launch_bounds__(kCoopWaves * 64, 1) void decode_coop(const DecParams p)
{
    using V8 = typename Elem<T>::vec8;
    constexpr uint32_t kThreads = kCoopWaves * 64;
    __shared__ __attribute__((aligned(16))) unsigned char slices[kCoopWaves][kSliceBytes];
    __shared__ float2 s_ml[kCoopWaves][32];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wl = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t nc = p.nq * p.group, nseg = p.kv_heads;
    const uint32_t cg = wl % p.ncg, kw = wl / p.ncg, n_kw = kCoopWaves / p.ncg;
    T* ks = reinterpret_cast<T*>(slices[wl]);
    _Float16* vt = reinterpret_cast<_Float16*>(slices[wl] + kTK * (kD + 8) * sizeof(T));

    // The rows laid end to end: segment (b, kvh) = b * kv_heads + kvh holds ctx[b] rows.
    const uint32_t total = uniform(ctx_sum(p, p.batch, lane) * nseg);
    if (total == 0)
        return;
    const Ranges rg(total, gridDim.x);
    const uint32_t r0 = rg.start(blockIdx.x), r1 = rg.start(blockIdx.x + 1);
    if (r0 >= r1)
        return;
    uint32_t b, seg0;
    seq_of(p, r0, lane, nseg, b, seg0);
    b = uniform(b);
    seg0 = uniform(seg0);
    uint32_t ctx = uniform(ctx_of(p.ctx, b, p.max_ctx));
    uint32_t kvh = (r0 - seg0) / ctx;
    uint32_t row = r0;

    while (row < r1) {
        // One piece: segment (b, kvh), keys [k_begin, k_end).
        const uint32_t s_start = seg0 + kvh * ctx;
        const uint32_t k_begin = row - s_start;
        const uint32_t k_end = min(ctx, r1 - s_start);
        const uint32_t seg = b * nseg + kvh;
        const uint32_t col = 32 * cg + c32;
        const bool has_col = c32 < p.ncs && col < nc;
        const uint32_t lim = has_col ? lim_of(p, ctx, col / p.group) : 0u;
        const uint32_t lim_all = lim_of(p, ctx, 0);
        V8 qreg[kD / 16];
        load_q<T>(p, b, kvh, col, has_col, qreg);
        const size_t head_off = ((size_t)b * p.kv_heads + kvh) * p.cap * kD;
        const auto krs = buffer_rsrc(static_cast<const T*>(p.k) + head_off, k_end * kD * sizeof(T));
        const auto vrs = buffer_rsrc(static_cast<const T*>(p.v) + head_off, k_end * kD * sizeof(T));
        f32x16 oacc[kD / 32];
        float m, l;
        wave_keys<T>(p, ks, vt, qreg, krs, vrs, k_begin + kTK * kw, kTK * n_kw, k_end, lim, lim_all, oacc, m, l);

        // This wave's share into its own slice: quad q (registers 4 (q % 4) .. + 3 of block q / 4: head dims
        // 32 (q / 4) + 8 (q % 4) + 4 g .. + 3) of lane l at f32x4 q * 64 + l; maximum and row sum a column.
        {
            f32x4* red = reinterpret_cast<f32x4*>(slices[wl]);
            #pragma unroll
            for (int q = 0; q < 16; ++q)
                red[q * 64 + lane] = f32x4{oacc[q / 4][4 * (q % 4)], oacc[q / 4][4 * (q % 4) + 1],
                                           oacc[q / 4][4 * (q % 4) + 2], oacc[q / 4][4 * (q % 4) + 3]};
            const float lt = l + swap_halves(l);
            if (g == 0)
                s_ml[wl][c32] = float2{m, lt};
        }
        __syncthreads();
        // The piece's partial a column: items (column group, column, half, quad) over the workgroup.
        {
            const uint32_t per_cg = p.ncs * 32, items = per_cg * p.ncg;
            for (uint32_t it = tid; it < items; it += kThreads) {
                const uint32_t icg = it / per_cg, rest = it % per_cg;
                const uint32_t c = rest / 32, h = (rest / 16) % 2, q = rest % 16, ccol = 32 * icg + c;
                if (ccol >= nc)
                    continue;
                float mx = -INFINITY;
                for (uint32_t j = 0; j < n_kw; ++j)
                    mx = fmaxf(mx, s_ml[icg + p.ncg * j][c].x);
                float sum = 0.0f;
                f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                for (uint32_t j = 0; j < n_kw; ++j) {
                    const uint32_t w = icg + p.ncg * j;
                    const float2 ml = s_ml[w][c];
                    const float f = ml.x == -INFINITY ? 0.0f : exp2_fast(ml.x - mx);
                    sum += ml.y * f;
                    acc += reinterpret_cast<const f32x4*>(slices[w])[q * 64 + 32 * h + c] * f;
                }
                const size_t prow = ((size_t)blockIdx.x + seg) * nc + ccol;
                *reinterpret_cast<f32x4*>(p.part_o + prow * kD + 32 * (q / 4) + 8 * (q % 4) + 4 * h) = acc;
                if (h == 0 && q == 0)
                    *reinterpret_cast<float2*>(p.part_ml + prow * 2) = float2{mx, sum};
            }
        }
        __syncthreads();  // the slices are free again
        // The next segment (sequences with an empty context hold no rows and are skipped).
        row = s_start + k_end;
        if (++kvh == nseg) {
            kvh = 0;
            seg0 += ctx * nseg;
            do {
                ++b;
            } while (b < p.batch && ctx_of(p.ctx, b, p.max_ctx) == 0);
            if (b >= p.batch)
                break;
            ctx = uniform(ctx_of(p.ctx, b, p.max_ctx));
        }
    }
}

// One workgroup of 256 threads per (head, sequence, row), as kMergeGroups groups of 32 lanes (a lane holds 4 head
// dims): group gi takes every kMergeGroups-th of the segment's pieces, one pass with a running maximum (all of its
// pieces' loads in flight at once for up to 8 each: one round trip for up to 64 pieces), then the groups' (maximum,
// sum, output) meet in LDS and group 0 divides once; lse = (max + log2 sum) ln 2. Small workgroups so that every
// (head, sequence, row) of a call is resident at once.
constexpr int kMergeGroups = 8;
constexpr int kMergeThreads = kMergeGroups * 32;

template <class TO>
__global__ __launch_bounds__(kMergeThreads) void decode_merge(const DecParams p, TO* __restrict__ o,
                                                              float* __restrict__ lse)
{
    __shared__ float s_ml[kMergeGroups][2];
    __shared__ f32x4 s_acc[kMergeGroups][kD / 4];
    const uint32_t h = blockIdx.x, b = blockIdx.y, rq = blockIdx.z, gi = threadIdx.x / 32, d4 = threadIdx.x % 32;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t kvh = h / p.group, col = rq * p.group + h % p.group, nseg = p.kv_heads * p.ncg;
    const uint32_t sh = kvh * p.ncg + col / p.ncs, cs = col % p.ncs;  // the column's segment and place in it
    const uint32_t total = ctx_sum(p, p.batch, lane) * nseg;
    const uint32_t seq0 = ctx_sum(p, b, lane);
    const uint32_t ctx = ctx_of(p.ctx, b, p.max_ctx);
    float mx = -INFINITY, sum = 0.0f;
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (ctx > 0) {
        const Ranges rg(total, p.n_waves);
        const uint32_t s_start = seq0 * nseg + sh * ctx;
        const uint32_t w_lo = rg.wave_of(s_start), w_hi = rg.wave_of(s_start + ctx - 1);
        const uint32_t seg = b * nseg + sh;
        constexpr int U = 8;
        for (uint32_t w0 = w_lo + gi; w0 <= w_hi; w0 += U * kMergeGroups) {
            float2 ml[U];
            f32x4 ov[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t w = w0 + u * kMergeGroups;
                // waves with an empty range wrote nothing (only possible with fewer rows than waves, q = 0)
                const bool live = w <= w_hi && (rg.q > 0 || !rg.empty(w));
                const size_t prow = ((size_t)(live ? w : w_lo) + seg) * p.ncs + cs;
                ml[u] = live ? *reinterpret_cast<const float2*>(p.part_ml + prow * 2) : float2{-INFINITY, 0.0f};
                ov[u] = live ? *reinterpret_cast<const f32x4*>(p.part_o + prow * kD + 4 * d4) : f32x4{};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float nm = fmaxf(mx, ml[u].x);
                if (nm == -INFINITY)
                    continue;  // nothing seen yet
                const float a = exp2_fast(mx - nm), wgt = exp2_fast(ml[u].x - nm);
                sum = sum * a + ml[u].y * wgt;
                acc = acc * a + ov[u] * wgt;
                mx = nm;
            }
        }
    }
    if (d4 == 0) {
        s_ml[gi][0] = mx;
        s_ml[gi][1] = sum;
    }
    s_acc[gi][d4] = acc;
    __syncthreads();
    if (gi != 0)
        return;
    for (uint32_t j = 1; j < kMergeGroups; ++j) {
        const float jm = s_ml[j][0];
        const float nm = fmaxf(mx, jm);
        if (nm == -INFINITY)
            continue;
        const float a = exp2_fast(mx - nm), wgt = exp2_fast(jm - nm);
        sum = sum * a + s_ml[j][1] * wgt;
        acc = acc * a + s_acc[j][d4] * wgt;
        mx = nm;
    }
    TO* orow = o + (size_t)b * p.os_b + (size_t)rq * p.os_r + (size_t)h * kD + 4 * d4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        orow[i] = (TO)(sum > 0.0f ? acc[i] / sum : 0.0f);
    if (lse && d4 == 0)
        lse[(size_t)b * p.ls_b + (size_t)h * p.ls_h + (size_t)rq * p.ls_r] =
            sum > 0.0f ? (mx + __log2f(sum)) * kLn2 : -INFINITY;
}

// Resident waves: kWgPerCu workgroups of kWaves waves on every CU of the current device (0: no device).
uint32_t resident_waves() { return device_cus() * kWgPerCu * kWaves; }

// Waves a call launches: the resident ones, or fewer when split asks for at most `split` keys a wave.
uint32_t waves_for(const mako_decode_args* a, uint32_t resident)
{
    if (!a->split)
        return resident;
    const uint64_t want = ((uint64_t)a->batch * a->kv_heads * a->max_ctx + a->split - 1) / a->split;
    const uint64_t n = std::min<uint64_t>(std::max<uint64_t>(want, 1), resident);
    return (uint32_t)((n + kWaves - 1) / kWaves * kWaves);
}

// Partials: one a piece (at most n_waves + segments pieces) and column (nc = rows x group).
size_t part_o_bytes(size_t pieces, uint32_t nc) { return (pieces * nc * kD * sizeof(float) + 255) / 256 * 256; }
size_t partials_bytes(size_t pieces, uint32_t nc) { return part_o_bytes(pieces, nc) + pieces * nc * 2 * sizeof(float); }

size_t pieces_of(uint32_t n_waves, const mako_decode_args* a) { return (size_t)n_waves + (size_t)a->batch * a->kv_heads; }
// (the decode's group is at most 32 columns: one segment a kv head)

size_t workspace_for(uint32_t n_waves, const mako_decode_args* a)
{
    return partials_bytes(pieces_of(n_waves, a), a->heads / a->kv_heads);
}

// The split kernel and the merge on stream s.
template <class T>
void launch_split_merge(const DecParams& p, mako_dtype out, void* o, float* lse, hipStream_t s)
{
    const dim3 grid(p.n_waves / kWaves), mgrid(p.heads, p.batch, p.nq);
    hipLaunchKernelGGL((decode_split<T>), grid, dim3(kWaves * 64), 0, s, p);
    const dim3 mblock(kMergeThreads);
    if (out == MAKO_F32)
        hipLaunchKernelGGL(decode_merge<float>, mgrid, mblock, 0, s, p, static_cast<float*>(o), lse);
    else if (out == MAKO_BF16)
        hipLaunchKernelGGL(decode_merge<__bf16>, mgrid, mblock, 0, s, p, static_cast<__bf16*>(o), lse);
    else
        hipLaunchKernelGGL(decode_merge<_Float16>, mgrid, mblock, 0, s, p, static_cast<_Float16*>(o), lse);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The split-K partials of mako_attn_decode_noalloc: a file-scope device array, one copy on every GPU the library
// runs on, held until the process ends. Its host-side name is not a device address: kernels and copies take the
// address hipGetSymbolAddress returns for the current device (scratch_ptr).
constexpr size_t kScratchBytes = MAKO_DECODE_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices];  // per device: the address of its copy of `scratch` (null until looked up)

// The current device's copy of `scratch`, looked up once per device with that device current; null (with the
// error recorded) when the lookup fails.
void* scratch_ptr()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fail(MAKO_EHIP, "attention_decode_noalloc: no current device (or more than %d)", kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            fail(MAKO_EHIP, "attention_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                 hipGetErrorString(e));
            return nullptr;
        }
        scratch_dev[dev] = ptr;
    }
    return scratch_dev[dev];
}

}  // namespace
}  // namespace mako

using namespace mako;

extern "C" size_t mako_attn_decode_workspace(const mako_decode_args* a)
{
    if (!a || !a->kv_heads || !a->heads || a->heads % a->kv_heads)
        return 0;
    const uint32_t resident = resident_waves();
    return resident ? workspace_for(waves_for(a, resident), a) : 0;
}

namespace {

// The checks both decode entry points make (what: the name in the messages).
int check_args(const mako_decode_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k, const void* v,
               const uint32_t* ctx_len, const void* o, const char* what)
{
    if (!a || !q || !k || !v || !ctx_len || !o)
        return fail(MAKO_EINVAL, "%s: a null argument", what);
    if (a->dim != kD)
        return fail(MAKO_EUNSUPPORTED, "%s: heads of %u (128)", what, a->dim);
    if (in != MAKO_F16 && in != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "%s: input type %d (f16 or bf16)", what, (int)in);
    if (out != MAKO_F32 && out != in)
        return fail(MAKO_EUNSUPPORTED, "%s: output type %d (f32 or the input's)", what, (int)out);
    if (!a->heads || !a->kv_heads || a->heads % a->kv_heads || a->heads / a->kv_heads > 32)
        return fail(MAKO_EINVAL, "%s: %u heads over %u kv heads (groups of at most 32)", what, a->heads, a->kv_heads);
    if (a->max_ctx > a->cap)
        return fail(MAKO_EINVAL, "%s: max_ctx %u over the cache's %u rows", what, a->max_ctx, a->cap);
    if ((uint64_t)a->cap * kD * 2 > 0x7fffffffu)
        return fail(MAKO_EINVAL, "%s: %u cache rows exceed 2 GiB a head", what, a->cap);
    if ((uint64_t)a->batch * a->kv_heads * a->max_ctx >= (1ull << 32))
        return fail(MAKO_EINVAL, "%s: %u x %u x %u rows exceed 2^32", what, a->batch, a->kv_heads, a->max_ctx);
    if (a->split % 64)
        return fail(MAKO_EINVAL, "%s: %u keys a split (a multiple of 64, or 0)", what, a->split);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(MAKO_EINVAL, "%s: q, k, v and o must be 16-byte aligned", what);
    if (!(a->scale > 0.0f) || a->scale == INFINITY)
        return fail(MAKO_EINVAL, "%s: scale %g (positive and finite)", what, (double)a->scale);
    return MAKO_OK;
}

// The split kernel and the merge on `stream`, with the partials in `ws` (at least workspace_for(n_waves, a) bytes).
int launch_decode(const mako_decode_args* a, uint32_t n_waves, mako_dtype in, mako_dtype out, const void* q,
                  const void* k, const void* v, const uint32_t* ctx_len, void* o, float* lse, void* ws, void* stream,
                  const char* what)
{
    const uint32_t group = a->heads / a->kv_heads;
    float* part_o = static_cast<float*>(ws);
    float* part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + part_o_bytes(pieces_of(n_waves, a), group));
    // one query row a sequence at position ctx - 1: q [batch][heads][kD], o likewise, lse [batch][heads]
    const DecParams p{q, k, v, ctx_len, part_o, part_ml, a->batch, a->heads, a->kv_heads, group, a->cap,
                      a->max_ctx, n_waves, a->scale * kLog2e, 1u, 1u, group, 0xffffffffu, 0xffffffffu, 0u,
                      a->heads * kD, kD, 0u, a->heads * kD, 0u, a->heads, 1u, 0u};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (in == MAKO_BF16)
        launch_split_merge<__bf16>(p, out, o, lse, s);
    else
        launch_split_merge<_Float16>(p, out, o, lse, s);
    return check_launch(what);
}

}  // namespace

namespace mako {

// mako_attn_fwd's route for a few query rows (heads of 128): when the columns (n_q rows x the GQA group) are at most
// 64, decode_coop over each kv head's keys (those the last row sees), one workgroup a CU taking at least
// kCoopMinRows keys, partials in the call's workspace (splitk_workspace bytes), then decode_merge into o [n_q][width]
// and lse [heads][n_q]. With no key to see, only the merge runs (it writes zeros and lse = -inf). Returns 1 when
// launched, 0 when the case does not take this route (splitk_takes false), -1 when the workspace could not be had
// (the error recorded).
bool splitk_takes(const mako_attn_args* a, uint32_t dim)
{
    return dim == 128 && a->n_q > 0 && (uint64_t)a->n_q * (a->heads / a->kv_heads) <= 64 &&
           (uint64_t)a->q_pos0 + a->n_q < 0xffffffffull;
}

namespace {
constexpr uint32_t kCoopMinRows = kCoopWaves * 128;

// The split-K route's shape: keys the last row sees, and workgroups (one a CU at most, each >= kCoopMinRows keys).
void splitk_shape(const mako_attn_args* a, uint32_t cus, uint32_t& n_keys, uint32_t& n_wg)
{
    const uint32_t last = a->q_pos0 + a->n_q - 1;  // the last row's position: it sees the most keys
    n_keys = last >= a->block ? a->n_k : std::min(a->n_k, last + 1);
    const uint64_t rows = (uint64_t)a->kv_heads * n_keys;
    n_wg = (uint32_t)std::min<uint64_t>(std::max<uint64_t>((rows + kCoopMinRows - 1) / kCoopMinRows, 1), cus);
}
}  // namespace

size_t splitk_workspace(const mako_attn_args* a)
{
    const uint32_t cus = device_cus();
    if (!splitk_takes(a, 128) || !cus)
        return 0;
    uint32_t n_keys, n_wg;
    splitk_shape(a, cus, n_keys, n_wg);
    return n_keys ? partials_bytes((size_t)n_wg + a->kv_heads, a->n_q * (a->heads / a->kv_heads)) : 0;
}

int launch_attn_splitk(const mako_attn_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                       const void* v, void* o, float* lse, hipStream_t s, const Workspace& work)
{
    const uint32_t group = a->heads / a->kv_heads, nc = a->n_q * group;
    if (!splitk_takes(a, 128))
        return 0;
    const uint32_t ncg = (nc + 31) / 32, ncs = std::min(nc, 32u);
    const uint32_t cus = device_cus();
    if (!cus)
        return fail(MAKO_EHIP, "attention: no device"), -1;
    uint32_t n_keys, n_wg;
    splitk_shape(a, cus, n_keys, n_wg);
    // one sequence of n_keys keys a kv head: q [heads][q_pad][kD], o [n_q][width], lse [heads][n_q]
    DecParams p{q, k, v, nullptr, nullptr, nullptr, 1u, a->heads, a->kv_heads, group, a->k_pad, n_keys,
                n_wg, a->scale * kLog2e, a->n_q, ncg, ncs, a->q_pos0, a->block, a->n_k,
                0u, a->q_pad * kD, kD, 0u, a->width, 0u, a->n_q, 1u};
    const auto merge = [&](const DecParams& pm) {
        const dim3 mgrid(pm.heads, pm.batch, pm.nq), mblock(kMergeThreads);
        if (out == MAKO_F32)
            hipLaunchKernelGGL(decode_merge<float>, mgrid, mblock, 0, s, pm, static_cast<float*>(o), lse);
        else if (out == MAKO_BF16)
            hipLaunchKernelGGL(decode_merge<__bf16>, mgrid, mblock, 0, s, pm, static_cast<__bf16*>(o), lse);
        else
            hipLaunchKernelGGL(decode_merge<_Float16>, mgrid, mblock, 0, s, pm, static_cast<_Float16*>(o), lse);
    };
    if (n_keys == 0) {
        merge(p);  // no partials are read: the context is empty
        return 1;
    }
    const size_t pieces = (size_t)n_wg + a->kv_heads;
    void* ws = work.get(partials_bytes(pieces, nc), s);
    if (!ws)
        return -1;
    p.part_o = static_cast<float*>(ws);
    p.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + part_o_bytes(pieces, nc));
    const dim3 grid(n_wg), block(kCoopWaves * 64);
    if (in == MAKO_BF16)
        hipLaunchKernelGGL(decode_coop<__bf16>, grid, block, 0, s, p);
    else
        hipLaunchKernelGGL(decode_coop<_Float16>, grid, block, 0, s, p);
    DecParams pm = p;  // the pieces hold all nc columns: one column group for the merge's lookup
    pm.ncg = 1;
    pm.ncs = nc;
    merge(pm);
    return 1;
}

}  // namespace mako

extern "C" int mako_attn_decode(const mako_decode_args* a, mako_dtype in, mako_dtype out, const void* q,
                                const void* k, const void* v, const uint32_t* ctx_len, void* o, float* lse,
                                void* workspace, size_t workspace_bytes, void* stream)
{
    const char* what = "attention_decode";
    if (const int rc = check_args(a, in, out, q, k, v, ctx_len, o, what))
        return rc;
    const uint32_t resident = resident_waves();
    if (!resident)
        return fail(MAKO_EHIP, "%s: no device to size the split for", what);
    const uint32_t n_waves = waves_for(a, resident);
    const size_t need = workspace_for(n_waves, a);
    if (!workspace || workspace_bytes < need || !aligned16(workspace))
        return fail(MAKO_EWORKSPACE, "%s: workspace of %zu bytes, %zu needed (16-byte aligned)", what,
                    workspace_bytes, need);
    if (a->batch == 0)
        return ok();
    return launch_decode(a, n_waves, in, out, q, k, v, ctx_len, o, lse, workspace, stream, what);
}

extern "C" int mako_attn_decode_noalloc(const mako_decode_args* a, mako_dtype in, mako_dtype out, const void* q,
                                        const void* k, const void* v, const uint32_t* ctx_len, void* o, float* lse,
                                        void* stream)
{
    const char* what = "attention_decode_noalloc";
    if (const int rc = check_args(a, in, out, q, k, v, ctx_len, o, what))
        return rc;
    const uint32_t resident = resident_waves();
    if (!resident)
        return fail(MAKO_EHIP, "%s: no device to size the split for", what);
    const uint32_t n_waves = waves_for(a, resident);
    const size_t need = workspace_for(n_waves, a);
    if (need > kScratchBytes)
        return fail(MAKO_EWORKSPACE,
                    "%s: the split-K partials need %zu bytes, over the library's static scratch of %zu bytes "
                    "(fewer sequences, kv heads or query heads a group, or a larger split, or mako_attn_decode "
                    "with a workspace)", what, need, kScratchBytes);
    void* ws = scratch_ptr();
    if (!ws)
        return MAKO_EHIP;
    if (a->batch == 0)
        return ok();
    return launch_decode(a, n_waves, in, out, q, k, v, ctx_len, o, lse, ws, stream, what);
}
