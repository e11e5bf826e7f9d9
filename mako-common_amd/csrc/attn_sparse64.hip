// Block-sparse attention for heads of 128 on gfx950 with 64 query rows a wave: flash_sparse_r64, the stream of
// flash_fwd_r64 (attn_fwd64.hip, gen_attn_fwd64.py) driven by a pass table.
//
// Semantics (the reference's attention_sparse, src/kernels/ops.metal:1036-1185, as attn_sparse.hip states them): query
// tile t (64 rows) < n_cubes visits the key cubes its list names, then the dense rows [dense0, dense1); a later tile
// visits [0, n_k); keys with valid[j] == 0 are masked; causal: key j is seen by tile row r only when j <= r; query
// row r's output goes to o row map[r], dropped when map[r] < 0 or r >= n_q; lse [heads][q_pad] by tile row.
//
// The route (mako_attn_sparse takes it when its conditions hold, else flash_sparse8 / flash_sparse): lists shared by
// a kv head's query heads (sel_heads == kv_heads) in groups of 4, so a workgroup is one 64-row query tile of 4 query
// heads (one wave a head) over one list, and every K / V tile staged in LDS serves all four; dense0 a multiple of
// 64 and valid 16-byte aligned, so every pass is one 64-key tile. K and V are staged from their rows (rows past n_k
// too, since only valid masks keys; as the reference, masked keys need finite values).
//
// Before it, sparse_prep (one launch) writes the pass table: for each (kv head, query tile) list, entry ps =
// {first key of pass ps, 0, W0, W1}, -1 (none) past the list. W_g holds the validity of the 32 keys the lanes of half
// g of a wave hold (bit 16 t + r: key 32 t + 16 (r / 8) + 8 g + r % 8 of the tile): valid and before the pass's end.
// A causal pass wholly after the tile's rows is none (its keys are all masked anyway; none stages zeros), and the
// first pass that no bound cuts comes first (it sets the rows' running maximum from all of its keys). The stream
// reads each tile's entry with scalar loads an iteration ahead: the first key sets the tile's K and V sources, and
// a tile whose words are not all ones is masked by them as well as by the causal row limit.
#include "fwd64_common.hpp"

namespace mako {
namespace {

constexpr uint32_t kNone = 0xffffffffu;

struct SparsePlan {
    const uint16_t* sel;
    const uint16_t* nsel;
    const uint8_t* valid;
    u32x4* table;          // [kv_heads][n_qt][n_ent]
    uint32_t kv_heads, n_qt, n_ent, n_cubes, max_sel, dense0, dense1, n_k, causal;
};

// The passes of list (kvh, qt): ns selected cubes, then nd 64-key steps of the dense rows [lo, hi).
struct Passes {
    uint32_t ns, nd, lo, hi;
};

__device__ __forceinline__ Passes passes_of(const uint16_t* nsel, uint32_t kvh, uint32_t qt, uint32_t n_cubes,
                                            uint32_t max_sel, uint32_t dense0, uint32_t dense1, uint32_t n_k)
{
    const bool cube = qt < n_cubes;
    Passes r;
    r.ns = cube ? min((uint32_t)nsel[(size_t)kvh * n_cubes + qt], max_sel) : 0u;
    r.lo = cube ? dense0 : 0u;
    r.hi = cube ? dense1 : n_k;
    r.nd = r.hi > r.lo ? (r.hi - r.lo + 63) / 64 : 0u;
    return r;
}

// The pass-table entries, one a thread.
__global__ __launch_bounds__(256) void sparse_prep(const SparsePlan p)
{
    const uint32_t idx = blockIdx.x * 256 + threadIdx.x;
    const uint32_t list = idx / p.n_ent, ps = idx % p.n_ent;
    if (list >= p.kv_heads * p.n_qt)
        return;
    const uint32_t kvh = list / p.n_qt, qt = list % p.n_qt;
    const Passes pa = passes_of(p.nsel, kvh, qt, p.n_cubes, p.max_sel, p.dense0, p.dense1, p.n_k);
    const uint32_t nt = pa.ns + pa.nd;
    auto range = [&](uint32_t i, uint32_t& j0, uint32_t& hi) {
        if (i < pa.ns) {
            j0 = (uint32_t)p.sel[((size_t)kvh * p.n_cubes + qt) * p.max_sel + i] * 64;
            hi = j0 + 64;
        } else {
            j0 = pa.lo + (i - pa.ns) * 64;
            hi = min(j0 + 64, pa.hi);
        }
    };
    // The stream's first pass sets every row's running maximum; a pass the causal bound or the pass's end cuts
    // would set it from a few scores for some rows, and later passes would then overshoot it by more than 8 (the
    // exact path, every few tiles). So pass 0 trades places with the first pass that neither cuts: the same passes,
    // in another order.
    uint32_t first = 0;
    for (; first < nt; ++first) {
        uint32_t j0, hi;
        range(first, j0, hi);
        if (hi == j0 + 64 && !(p.causal && j0 + 64 > 64 * qt + 1))
            break;
    }
    const uint32_t src = first == nt ? ps : ps == 0 ? first : ps == first ? 0u : ps;
    u32x4 entry = u32x4{kNone, 0u, 0u, 0u};
    if (ps < nt) {
        uint32_t j0, hi;
        range(src, j0, hi);
        if (!(p.causal && j0 > 64 * qt + 63)) {
            uint64_t m = 0;  // bit i: key j0 + i may be seen
            const u32x4* vp = reinterpret_cast<const u32x4*>(p.valid + j0);
            #pragma unroll
            for (int c = 0; c < 4; ++c) {
                const u32x4 x = vp[c];
                #pragma unroll
                for (int d = 0; d < 4; ++d)
                    #pragma unroll
                    for (int b = 0; b < 4; ++b)
                        m |= (uint64_t)(((x[d] >> (8 * b)) & 0xffu) != 0u) << (16 * c + 4 * d + b);
            }
            const uint32_t n_in = hi - j0;  // 1 .. 64
            if (n_in < 64)
                m &= (1ull << n_in) - 1;
            uint32_t w0 = 0, w1 = 0;
            #pragma unroll
            for (int b = 0; b < 32; ++b) {
                const int key = 32 * (b >> 4) + 16 * ((b & 15) >> 3) + (b & 7);
                w0 |= (uint32_t)((m >> key) & 1u) << b;
                w1 |= (uint32_t)((m >> (key + 8)) & 1u) << b;
            }
            entry = u32x4{j0, 0u, w0, w1};
        }
    }
    p.table[(size_t)list * p.n_ent + ps] = entry;
}

struct Sparse64Params {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const uint16_t* nsel;
    const int32_t* map;
    const u32x4* table;      // the pass table: [kv_heads][n_qt][n_ent]
    uint32_t n_q, q_pad, n_k, k_pad, heads, kv_heads, width;
    float scale_log2;
    uint32_t n_cubes, max_sel, dense0, dense1, causal;
    uint32_t group, n_hg, n_qt, n_ent, n_items;
};

template <class T, class TO>
__global__ __launch_bounds__(256, 1) void flash_sparse_r64(const Sparse64Params p)
{
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kLdsBytes];
    const uint32_t tid = threadIdx.x, lane = tid & 63, g = lane >> 5, c32 = lane & 31;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);

    // A persistent grid as flash_fwd_r64's: item i (query tile n_qt - 1 - i / n_hg, head group i % n_hg: the dense
    // later tiles first) belongs to XCD i % 8; the g8 workgroups of an XCD walk its items in rounds of g8, the order
    // reversed every other round.
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const bool by_xcd = G % 8 == 0;
    const uint32_t g8 = G / 8, bx = b % 8, bk = b / 8;
    for (uint32_t round = 0;; ++round) {
    const uint32_t item = by_xcd ? bx + 8 * (round * g8 + (round % 2 == 0 ? bk : g8 - 1 - bk)) : b + round * G;
    if (item >= p.n_items)
        break;
    const uint32_t hg = item % p.n_hg, qt = p.n_qt - 1 - item / p.n_hg;
    const uint32_t h = hg * 4 + w;
    const uint32_t kvh = hg * 4 / p.group;
    const uint32_t q0 = qt * 64;
    const Passes pa = passes_of(p.nsel, kvh, qt, p.n_cubes, p.max_sel, p.dense0, p.dense1, p.n_k);
    const uint32_t nt = pa.ns + pa.nd;

    // The row limit (causal: keys up to the row; otherwise none, every pass's keys coming from the table's words).
    constexpr uint32_t kNoLimit = 0x7fffffffu;
    const uint32_t lmin = p.causal ? q0 + 1 : kNoLimit;
    const uint32_t lim0 = p.causal ? q0 + c32 + 1 - 8 * g : kNoLimit;
    const uint32_t lim1 = p.causal ? q0 + 32 + c32 + 1 - 8 * g : kNoLimit;

    // LDS and staging: as flash_fwd_r64.
    const uint32_t lbase = (uint32_t)reinterpret_cast<uintptr_t>(lds);
    const uint32_t vbase = lbase + kNBuf * kKTile;
    uint32_t kr = lbase + c32 * kKRow + 16 * g;
    const uint32_t kr0 = kr;
    const uint32_t th = (lane >> 4) & 1u, ti = lane & 15u;
    const uint32_t vrow = vbase + (8 * g + ti / 4) * 256 + 8 * (ti % 4);
    uint32_t vr0 = vrow + 32 * v_unit(th, ti / 4);
    uint32_t vr1 = vrow + 32 * v_unit(2 + th, ti / 4);
    auto kd_of = [&](uint32_t i) {
        const uint32_t by = 1024 * i + 16 * lane, row = by / kKRow, ch = by % kKRow / 16;
        return slot_of(row) * 256 + 16 * (ch < 16 ? ch : 0);
    };
    const uint32_t kd0 = kd_of(w), kd1 = kd_of(w + 4), kd2 = kd_of(w + 8), kd3 = kd_of(w + 12), kd4 = kd_of(16);
    const uint32_t vd = 4096 * w + vd_of<128>(lane);
    const uint32_t skw = __builtin_amdgcn_readfirstlane(lbase), skww = __builtin_amdgcn_readfirstlane(lbase + 1024 * w);
    const uint32_t svww = __builtin_amdgcn_readfirstlane(vbase + 4096 * w);
    const uint32_t qo = ((q0 + c32) * 128 + 8 * g) * 2;
    // Epilogue: O rows through the wave's LDS region as flash_fwd_r64's, then to o row map[q0 + row] at 64-bit
    // addresses (row x width x bytes + ocol); mp: the bpermute address of the lane that holds row (lane / lpr)'s map
    // entry; mlive: the lane's row is below n_q (others are dropped).
    constexpr uint32_t so = sizeof(TO), orow = 128 * so, lpr = orow / 16;
    const uint32_t obase = lbase + w * 64 * orow;
    const uint32_t ew = so == 4 ? obase + c32 * orow + 16 * ((c32 & 7u) ^ g)
                                : obase + c32 * orow + 8 * g + 16 * (c32 & 7u);
    const uint32_t er = obase + (lane / lpr) * orow + 16 * ((lane % lpr) ^ (lane / lpr));
    const uint32_t mp = 4 * (lane / lpr);
    const uint64_t ocol = reinterpret_cast<uint64_t>(p.o) + h * orow + 16 * (lane % lpr);
    const uint32_t ows = __builtin_amdgcn_readfirstlane(p.width * so);
    const uint32_t mlive = q0 + lane < p.n_q ? 1u : 0u;
    const uint32_t mo = (q0 + lane) * 4;
    const uint32_t lo0 = q0 + c32 < p.n_q ? (h * p.q_pad + q0 + c32) * 4 : 0xffffffffu;
    const uint32_t lo1 = q0 + 32 + c32 < p.n_q ? (h * p.q_pad + q0 + 32 + c32) * 4 : 0xffffffffu;
    const uint32_t swp = (lane ^ 32) * 4;
    const uint32_t g32 = 32 * g;

    const u32x4 qrs = rsrc_of(static_cast<const T*>(p.q) + (size_t)h * p.q_pad * 128, p.n_q * 256);
    const u32x4 lrs = rsrc_of(p.lse, p.lse ? p.heads * p.q_pad * 4 : 0);
    const u32x4 mrs = rsrc_of(p.map, p.n_q * 4);
    const uint64_t ent = reinterpret_cast<uint64_t>(p.table + ((size_t)kvh * p.n_qt + qt) * p.n_ent);
    const uint64_t kbase = reinterpret_cast<uint64_t>(static_cast<const T*>(p.k) + (size_t)kvh * p.k_pad * 128);
    const uint64_t vtbase = reinterpret_cast<uint64_t>(static_cast<const T*>(p.v) + (size_t)kvh * p.k_pad * 128);
    const uint32_t has_lse = __builtin_amdgcn_readfirstlane(p.lse ? 1u : 0u);
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, p.scale_log2)));
    const uint32_t s_nt = __builtin_amdgcn_readfirstlane(nt);
    const uint32_t s_lmin = __builtin_amdgcn_readfirstlane(lmin);
    const uint32_t kb0 = __builtin_amdgcn_readfirstlane((uint32_t)kbase);
    const uint32_t kb1 = __builtin_amdgcn_readfirstlane((uint32_t)(kbase >> 32) & 0xffffu);
    const uint32_t vb0 = __builtin_amdgcn_readfirstlane((uint32_t)vtbase);
    const uint32_t vb1 = __builtin_amdgcn_readfirstlane((uint32_t)(vtbase >> 32) & 0xffffu);
    const uint32_t zero = __builtin_amdgcn_readfirstlane(0u);
    // readfirstlane yields an int: each half goes through uint32_t, or the low half would sign-extend into the high
    const uint64_t s_ent = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(ent >> 32)) << 32) |
                           (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)ent);

#define MAKO_SPARSE64_OPERANDS                                                                                  \
    : [kr] "+v"(kr), [vr0] "+v"(vr0), [vr1] "+v"(vr1)                                                           \
    : [kd0] "v"(kd0), [kd1] "v"(kd1), [kd2] "v"(kd2), [kd3] "v"(kd3), [kd4] "v"(kd4), [vd] "v"(vd),              \
      [lim0] "v"(lim0), [lim1] "v"(lim1), [kr0] "v"(kr0), [qo] "v"(qo), [lo0] "v"(lo0), [lo1] "v"(lo1),          \
      [swp] "v"(swp), [ew] "v"(ew), [er] "v"(er), [mp] "v"(mp), [ocol] "v"(ocol), [mlive] "v"(mlive),            \
      [mo] "v"(mo), [g32] "v"(g32), [qrs] "s"(qrs), [lrs] "s"(lrs), [mrs] "s"(mrs), [ent] "s"(s_ent),           \
      [c] "s"(c), [nt] "s"(s_nt), [ntw] "s"(s_nt), [lmin] "s"(s_lmin), [has_lse] "s"(has_lse), [ows] "s"(ows),   \
      [kb0] "s"(kb0), [kb1] "s"(kb1), [kn] "s"(zero), [vb0] "s"(vb0), [vb1] "s"(vb1), [vn] "s"(zero),            \
      [skw] "s"(skw), [skww] "s"(skww), [svww] "s"(svww)                                                          \
    : MAKO_SPARSE64_CLOBBERS, "vcc", "scc", "memory"

    if constexpr (__is_same(T, __bf16)) {
        if constexpr (__is_same(TO, float))
            asm volatile(MAKO_SPARSE64_ASM_BF16_F32 MAKO_SPARSE64_OPERANDS);
        else
            asm volatile(MAKO_SPARSE64_ASM_BF16_BF16 MAKO_SPARSE64_OPERANDS);
    } else {
        if constexpr (__is_same(TO, float))
            asm volatile(MAKO_SPARSE64_ASM_F16_F32 MAKO_SPARSE64_OPERANDS);
        else
            asm volatile(MAKO_SPARSE64_ASM_F16_F16 MAKO_SPARSE64_OPERANDS);
    }
    // every wave's stream has ended (its LDS reads landed) before the next item's staging overwrites LDS
    asm volatile("s_barrier" ::: "memory");
    }
#undef MAKO_SPARSE64_OPERANDS
}

}  // namespace

// Whether flash_sparse_r64 takes the call (see the file comment for the conditions; valid null: taken as aligned).
bool sparse64_fits(const mako_sparse_args* a, const void* valid)
{
    const uint32_t group = a->kv_heads ? a->heads / a->kv_heads : 0u;
    return a->kv_heads && a->sel_heads == a->kv_heads && group % 4 == 0 && a->dense0 % 64 == 0 &&
           (reinterpret_cast<uintptr_t>(valid) & 15u) == 0 && (uint64_t)a->q_pad * 256 < (1ull << 31) &&
           (uint64_t)a->heads * a->q_pad * 4 < (1ull << 32) && (uint64_t)a->k_pad * 256 < (1ull << 32);
}

// Entries of a pass-table list: the passes a query tile can have, and four past them (the stream reads ahead).
uint32_t pass_entries(const mako_sparse_args* a)
{
    const uint32_t n_qt = (a->n_q + 63) / 64;
    const uint32_t nd_c = a->dense1 > a->dense0 ? (a->dense1 - a->dense0 + 63) / 64 : 0u;
    const uint32_t nd_l = n_qt > a->n_cubes ? (a->n_k + 63) / 64 : 0u;
    return std::max(a->max_sel + nd_c, nd_l) + 4;
}

// The pass table's bytes: 16 an entry, an entry list a (kv head, query tile).
size_t sparse64_workspace(const mako_sparse_args* a)
{
    return (size_t)a->kv_heads * ((a->n_q + 63) / 64) * pass_entries(a) * 16;
}

// sparse_prep then flash_sparse_r64 on stream s, the pass table in the call's workspace (work). Returns 1 when
// launched, -1 when the workspace could not be had (the error recorded).
template <class T, class TO>
int launch_sparse64(const mako_sparse_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                    const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid, const int32_t* map, float* lse,
                    hipStream_t s, const Workspace& work)
{
    const uint32_t n_qt = (a->n_q + 63) / 64;
    const uint32_t n_ent = pass_entries(a);
    const size_t entries = (size_t)a->kv_heads * n_qt * n_ent;
    u32x4* table = static_cast<u32x4*>(work.get(entries * 16, s));
    if (!table)
        return -1;
    const SparsePlan plan{sel, nsel, valid, table, a->kv_heads, n_qt, n_ent, a->n_cubes, a->max_sel, a->dense0,
                          a->dense1, a->n_k, a->causal ? 1u : 0u};
    const uint32_t plan_blocks = (uint32_t)((entries + 255) / 256);
    hipLaunchKernelGGL(sparse_prep, dim3(plan_blocks), dim3(256), 0, s, plan);
    const uint32_t n_hg = a->heads / 4;
    const Sparse64Params p{q, k, v, o, lse, nsel, map, table, a->n_q, a->q_pad, a->n_k, a->k_pad, a->heads,
                           a->kv_heads, a->width, scale_log2, a->n_cubes, a->max_sel, a->dense0, a->dense1,
                           a->causal ? 1u : 0u, a->heads / a->kv_heads, n_hg, n_qt, n_ent, n_hg * n_qt};
    const uint32_t grid = std::min<uint32_t>(p.n_items, std::max<uint32_t>(1, device_cus()));
    hipLaunchKernelGGL((flash_sparse_r64<T, TO>), dim3(grid), dim3(256), 0, s, p);
    return 1;
}

#define MAKO_SPARSE64_INSTANCE(T, TO)                                                                            \
    template int launch_sparse64<T, TO>(const mako_sparse_args*, float, const void*, const void*, const void*, void*, \
                                        const uint16_t*, const uint16_t*, const uint8_t*, const int32_t*, float*,    \
                                        hipStream_t, const Workspace&);
MAKO_SPARSE64_INSTANCE(__bf16, float)
MAKO_SPARSE64_INSTANCE(__bf16, __bf16)
MAKO_SPARSE64_INSTANCE(_Float16, float)
MAKO_SPARSE64_INSTANCE(_Float16, _Float16)
#undef MAKO_SPARSE64_INSTANCE

}  // namespace mako
