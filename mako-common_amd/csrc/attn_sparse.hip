// Block-sparse attention for gfx950 (Video Sparse Attention's training-free form) and its cube selection.
//
// Semantics (the reference's, src/kernels/ops.metal:914-1185; host checks src/models/runtime.cpp:286-317):
// * cube_pool: the mean of a cube's 64 rows of q or k over its cnt[c] valid rows (0 when cnt is 0; the padding
//   rows are zero by the tiles' construction) (ops.metal:926-939).
// * cube_scores: sc[h][qc][kc] = qp[h][qc] . kp[h][kc] (:941-955).
//   The selection is index work, so it is exact: pooling and scores run in double, in the order of the double CPU
//   check the reference's own test sorts by (tests/sparse_attn_test.cpp:98-129; the rows summed in order, the mean
//   by one correctly rounded division, the dot products as a sequential sum of separately rounded products, no
//   fused multiply-add), so the scores, and with them every comparison the top-k makes, are the check's bit for bit.
// * cube_topk: the `local` cubes {qc, qc - stride, qc + stride} (those in range) first, their scores taken out of
//   the running, then repeated argmax, the larger score first and the smaller index on ties; nsel = min(topk, n)
//   (:957-1027). Here one wave per (query cube, head) with the scores in registers and a shuffle argmax a pick.
// * attention_sparse: query tile t (64 rows) < n_cubes visits the key cubes sel lists for it (64 keys each), then
//   the dense rows [dense0, dense1); a later tile visits [0, n_k); keys with valid[j] == 0 are masked (:1079-1113);
//   query row r's output goes to o row map[r], dropped when map[r] < 0 or r >= n_q (:1173-1184). Two fields the
//   reference does not have: causal (key j is seen by tile row r only when j <= r) and sel_heads (one list per
//   kv head, shared by the group's query heads, instead of one per query head).
//
// Design: the flash tile loop of attn_fwd.hip (S^T = K Q^T on v_mfma_f32_32x32x16, K rows in bit-swapped LDS
// slots, V transposed to f16 in LDS, P in registers, lazy rescale) driven by a pass list. A workgroup is one
// 64-row query tile of hs query heads (hs = 2 when a kv head's list is shared by at least two query heads, else
// 1), two waves a head, so every gathered K / V tile serves 2 hs waves. Each wave builds the tile's validity mask
// with one byte load a lane and a ballot; a tile whose 64 keys are all valid (and not cut by the causal bound)
// skips per-element masking.
#include "device.hpp"

namespace mako {

// attn_sparse64.hip: the r64 route for lists shared in groups of 4 (valid null: taken as aligned), the bytes of its
// pass table, and its launch (-1: the workspace could not be had, the error recorded).
bool sparse64_fits(const mako_sparse_args* a, const void* valid);
size_t sparse64_workspace(const mako_sparse_args* a);
// attn_sparse_lists.hip: the route for a list per query head with f16 inputs, and its launch.
bool sparse_lists_fits(const mako_sparse_args* a, mako_dtype in, const void* valid);
template <class TO>
void launch_sparse_lists(const mako_sparse_args* a, float scale_log2, const void* q, const void* k, const void* v,
                         void* o, const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                         const int32_t* map, float* lse, hipStream_t s);
template <class T, class TO>
int launch_sparse64(const mako_sparse_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                    const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid, const int32_t* map, float* lse,
                    hipStream_t s, const Workspace& work);

namespace {

constexpr int kD = 128;
constexpr int kKB = 64;  // keys a tile (one cube)
constexpr int kCube = 64;
constexpr float kRescale = 8.0f;

__device__ __forceinline__ uint32_t slot_of(uint32_t row)
{
    return (row & ~12u) | ((row & 4u) << 1) | ((row & 8u) >> 1);
}
__device__ __forceinline__ uint32_t vt_swz(uint32_t d) { return (d ^ (d >> 3)) & 7u; }

struct SparseParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const uint16_t* sel;
    const uint16_t* nsel;
    const uint8_t* valid;
    const int32_t* map;
    uint32_t n_q, q_pad, n_k, k_pad, heads, kv_heads, width;
    float scale_log2;
    uint32_t n_cubes, max_sel, dense0, dense1, causal, sel_heads;
    uint32_t group, hs, n_qt;
    uint32_t n_hg, xcd_major;  // head groups (heads / hs); items dealt by XCD (n_hg % 8 == 0)
};

// Workgroup b's item (head group, query tile), head-group-major so that the chip streams the K / V of about one head
// group at a time (per-head lists gather cubes from anywhere in a head's keys: with every head live at once the
// gathered tiles come from HBM). With xcd_major, workgroup b runs on XCD b % 8 and XCD x takes head groups x, x + 8,
// ... one after another, so each XCD's L2 serves one head group's keys. Query tiles run from the last (dense tiles,
// which see every key) to the first. False past the last item.
__device__ __forceinline__ bool sparse_item(const SparseParams& p, uint32_t b, uint32_t& hg, uint32_t& qt)
{
    uint32_t s = b;
    hg = 0;
    if (p.xcd_major) {
        s = b / 8;
        hg = b % 8 + 8 * (s / p.n_qt);
    } else {
        hg = s / p.n_qt;
    }
    qt = p.n_qt - 1 - s % p.n_qt;
    return hg < p.n_hg;
}

template <class T, class TO, int NW>
__global__ __launch_bounds__(NW * 64, 2) void flash_sparse(const SparseParams p)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int NT = NW * 64;
    constexpr int KS = kD + 8;
    constexpr int CPR = kD / 8;          // 16-byte chunks a row
    constexpr int NV = kKB * CPR / NT;   // chunks a thread loads per tile, K and V each
    constexpr int NKK = kD / 16, NDB = kD / 32;
    __shared__ __attribute__((aligned(16))) T ks[2][kKB * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][kD * kKB];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = lane >> 5, c32 = lane & 31;
    uint32_t hg, qt;
    if (!sparse_item(p, blockIdx.x, hg, qt))
        return;
    const uint32_t h = hg * p.hs + (w >> 1);
    const uint32_t kvh = h / p.group;
    const uint32_t q0 = qt * kCube + (w & 1) * 32;  // this wave's first row
    const uint32_t row = q0 + c32;

    // The pass list: a cube tile's selected cubes, then its dense rows; a later tile's all keys.
    const bool cube = qt < p.n_cubes;
    const uint32_t sh = p.sel_heads == p.heads ? h : kvh;  // uniform within the workgroup when hs > 1
    uint32_t ns = 0;
    const uint16_t* my_sel = p.sel + ((size_t)sh * p.n_cubes + qt) * p.max_sel;
    if (cube)
        ns = min(uniform_u16(p.nsel, (size_t)sh * p.n_cubes + qt), p.max_sel);
    const uint32_t dense_lo = cube ? p.dense0 : 0u, dense_hi = cube ? p.dense1 : p.n_k;
    const uint32_t n_dense = dense_hi > dense_lo ? (dense_hi - dense_lo + kKB - 1) / kKB : 0u;
    const uint32_t n_pass = ns + n_dense;
    auto pass_range = [&](uint32_t ps, uint32_t& j0, uint32_t& hi) {
        if (ps < ns) {
            j0 = uniform_u16(my_sel, ps) * kCube;
            hi = j0 + kCube;
        } else {
            j0 = dense_lo + (ps - ns) * kKB;
            hi = min(j0 + kKB, dense_hi);
        }
    };

    V8 qreg[NKK];
    {
        const auto qrs = buffer_rsrc(static_cast<const T*>(p.q) + (size_t)h * p.q_pad * kD, p.n_q * kD * sizeof(T));
        const uint32_t off = (row * kD + 8 * g) * sizeof(T);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            qreg[kk] = __builtin_bit_cast(V8, buffer_load16(qrs, off + 16 * kk * sizeof(T)));
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            settle(qreg[kk]);
    }
    // K / V over the kv head's k_pad rows (cube passes may read keys past n_k; valid masks them); the valid
    // flags over k_pad bytes. Loads past the end return zeros.
    const auto krs = buffer_rsrc(static_cast<const T*>(p.k) + (size_t)kvh * p.k_pad * kD, p.k_pad * kD * sizeof(T));
    const auto vrs = buffer_rsrc(static_cast<const T*>(p.v) + (size_t)kvh * p.k_pad * kD, p.k_pad * kD * sizeof(T));
    const auto valid_rs = buffer_rsrc(p.valid, p.k_pad);
    const uint32_t v_cc = tid % CPR;
    const uint32_t v_kg = (tid / CPR) ^ ((tid / (CPR / 2)) & 1u);
    u32x4 kreg[NV], vreg[NV];
    auto load_tile = [&](uint32_t j0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = tid + NT * i, r = c / CPR, col = c % CPR;
            kreg[i] = buffer_load16(krs, ((j0 + r) * kD + col * 8) * sizeof(T));
        }
#pragma unroll
        for (int i = 0; i < NV; ++i)
            vreg[i] = buffer_load16(vrs, ((j0 + NV * v_kg + i) * kD + v_cc * 8) * sizeof(T));
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = tid + NT * i, r = c / CPR, col = c % CPR;
            *reinterpret_cast<u32x4*>(&ks[buf][slot_of(r) * KS + col * 8]) = kreg[i];
        }
        const uint32_t key0 = NV * v_kg, kc = key0 / 8, off = key0 % 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = v_cc * 8 + e;
            _Float16* dst = &vt[buf][d * kKB + ((kc ^ vt_swz(d)) * 8) + off];
            if constexpr (NV == 4)
                *reinterpret_cast<u32x2*>(dst) =
                    u32x2{f16_pair<T>(vreg[0], vreg[1], e), f16_pair<T>(vreg[2], vreg[3], e)};
            else
                *reinterpret_cast<u32x4*>(dst) =
                    u32x4{f16_pair<T>(vreg[0], vreg[1], e), f16_pair<T>(vreg[2], vreg[3], e),
                          f16_pair<T>(vreg[4], vreg[5], e), f16_pair<T>(vreg[6], vreg[7], e)};
        }
    };

    f32x16 oacc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
        oacc[db] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    const float c = p.scale_log2;
    const bool live = q0 < p.n_q;

    uint32_t j0 = 0, hi = 0;
    if (n_pass > 0) {
        pass_range(0, j0, hi);
        load_tile(j0);
        store_tile(0);
    }
    __syncthreads();
    for (uint32_t ps = 0; ps < n_pass; ++ps) {
        const int buf = ps & 1;
        const uint32_t cj0 = j0, chi = hi;
        if (ps + 1 < n_pass) {
            pass_range(ps + 1, j0, hi);
            load_tile(j0);
        }
        // This tile's validity: bit i for key cj0 + i in range and valid.
        const uint32_t vflag = __builtin_amdgcn_raw_buffer_load_b8(valid_rs, (int)(cj0 + lane), 0, 0);
        const uint64_t vmask = __ballot(cj0 + lane < chi && vflag != 0);
        // nothing to do when no key of the tile is valid, or (causal) every key lies past every row of the wave
        if (live && vmask != 0 && !(p.causal && cj0 > q0 + 31)) {
            f32x16 s[2] = {f32x16{}, f32x16{}};
            {
                const T* kr0 = &ks[buf][c32 * KS + 8 * g];
                const T* kr1 = kr0 + 32 * KS;
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    s[0] = E::mfma32(*reinterpret_cast<const V8*>(kr0 + 16 * kk), qreg[kk], s[0]);
                    s[1] = E::mfma32(*reinterpret_cast<const V8*>(kr1 + 16 * kk), qreg[kk], s[1]);
                }
            }
            // Register r of tile t holds key cj0 + 32 t + 16 (r / 8) + 8 g + r % 8.
            const bool causal_cut = p.causal && cj0 + kKB - 1 > q0;
            if (vmask != ~0ull || causal_cut) {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int a = 0; a < 2; ++a) {
                        const uint32_t kbase = 32 * t + 16 * a + 8 * g;
                        const uint32_t bits = (uint32_t)(vmask >> kbase) & 0xffu;
#pragma unroll
                        for (int jj = 0; jj < 8; ++jj) {
                            const bool seen = ((bits >> jj) & 1u) && (!p.causal || cj0 + kbase + jj <= row);
                            s[t][8 * a + jj] = seen ? s[t][8 * a + jj] : -INFINITY;
                        }
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    mx = fmaxf(mx, s[t][r]);
            mx = fmaxf(mx, swap_halves(mx)) * c;
            float f = 1.0f;
            if (mx > m + kRescale) {
                f = exp2_fast(m - mx);
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
                    const _Float16* vr = &vt[buf][d * kKB + (((2 * cc + g) ^ vt_swz(d)) * 8)];
                    oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb[cc], oacc[db]);
                }
        }
        if (ps + 1 < n_pass)
            store_tile(buf ^ 1);
        __syncthreads();
    }

    // Normalise and store through the row map; the LSE by tile row.
    const float lt = l + swap_halves(l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (live && row < p.n_q) {
        const int32_t dst = p.map[row];
        if (dst >= 0) {
            TO* orow = static_cast<TO*>(p.o) + (size_t)dst * p.width + (size_t)h * kD;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    store4<TO>(orow + 32 * db + 8 * r4 + 4 * g, oacc[db][4 * r4] * inv, oacc[db][4 * r4 + 1] * inv,
                               oacc[db][4 * r4 + 2] * inv, oacc[db][4 * r4 + 3] * inv);
            if (p.lse && g == 0)
                p.lse[(size_t)h * p.q_pad + row] = lt > 0.0f ? (m + __log2f(lt)) * kLn2 : -INFINITY;
        }
    }
}

// ---- cube selection ------------------------------------------------------------------------------------------

// out[h][c][d] = (sum of the 64 rows of cube c) / cnt[c], 0 when cnt[c] is 0. Grid (n_cubes, heads, 2): z = 0 pools
// q (rows q_pad apart per head), z = 1 pools k (k_pad). 128 threads, one per head dimension.
template <class T>
__global__ __launch_bounds__(kD) void cube_pool(const T* __restrict__ q, const T* __restrict__ k,
                                                 const uint32_t* __restrict__ cnt, double* __restrict__ qp,
                                                 double* __restrict__ kp, uint32_t n_cubes, uint32_t q_pad,
                                                 uint32_t k_pad)
{
    const uint32_t cb = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    const bool is_k = blockIdx.z == 1;
    const T* x = (is_k ? k + (size_t)h * k_pad * kD : q + (size_t)h * q_pad * kD) + (size_t)cb * kCube * kD + d;
    double s = 0.0;
#pragma unroll 16
    for (uint32_t r = 0; r < kCube; ++r)
        s += (double)to_float(x[(size_t)r * kD]);
    const uint32_t n = cnt[cb];
    (is_k ? kp : qp)[((size_t)h * n_cubes + cb) * kD + d] = n ? s / (double)n : 0.0;
}

// sc[h][qc][kc] = qp[h][qc] . kp[h][kc]. A workgroup computes a 64 x 64 tile of scores, 4 x 4 a thread (16
// independent sums), with the pooled rows staged through LDS 32 dimensions at a time; each sum still adds its
// products in dimension order. Grid (ceil(n / 64), ceil(n / 64), heads), 256 threads.
constexpr uint32_t kScoreTile = 64, kScoreChunk = 32;

__global__ __launch_bounds__(256) void cube_scores(const double* __restrict__ qp, const double* __restrict__ kp,
                                                   double* __restrict__ sc, uint32_t n)
{
    // row stride 33 doubles: the 16 rows a read spans fall in distinct banks
    __shared__ double qs[kScoreTile][kScoreChunk + 1], ks[kScoreTile][kScoreChunk + 1];
    const uint32_t kc0 = blockIdx.x * kScoreTile, qc0 = blockIdx.y * kScoreTile, h = blockIdx.z, t = threadIdx.x;
    const uint32_t qr = t / 16, kr = t % 16;  // rows qr + 16 i and columns kr + 16 j of the tile
    const double* qh = qp + (size_t)h * n * kD;
    const double* kh = kp + (size_t)h * n * kD;
    double acc[4][4] = {};
    for (uint32_t d0 = 0; d0 < kD; d0 += kScoreChunk) {
        for (uint32_t e = t; e < kScoreTile * kScoreChunk; e += 256) {
            const uint32_t r = e / kScoreChunk, d = e % kScoreChunk;
            qs[r][d] = qc0 + r < n ? qh[(size_t)(qc0 + r) * kD + d0 + d] : 0.0;
            ks[r][d] = kc0 + r < n ? kh[(size_t)(kc0 + r) * kD + d0 + d] : 0.0;
        }
        __syncthreads();
        for (uint32_t d = 0; d < kScoreChunk; ++d) {
            double a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = qs[qr + 16 * i][d];
                b[i] = ks[kr + 16 * i][d];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    acc[i][jj] = __dadd_rn(acc[i][jj], __dmul_rn(a[i], b[jj]));  // no contraction
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
            if (qc0 + qr + 16 * i < n && kc0 + kr + 16 * jj < n)
                sc[((size_t)h * n + qc0 + qr + 16 * i) * n + kc0 + kr + 16 * jj] = acc[i][jj];
}

// sel[h][qc][0 .. kk) (kk = min(topk, n)): the local cubes first, then repeated argmax (the larger score, the
// smaller index on ties); nsel[h][qc] = kk. One wave per (qc, h), n <= 64 P: lane l keeps scores l, l + 64, ...
// (P doubles) in registers and the best of them (value, index: a strict > scan in index order keeps the smaller
// index of equal values; no score yet: -inf at index 0). A pick is the wave's best pair by six pairing steps (the
// larger value, the smaller index on ties): four DPP moves inside 16-lane rows, then the row and half swaps; the
// lane that holds it drops that score (-inf) and rescans its own. So a pick is a few dozen vector instructions and
// one lane's rescan of P registers, with no LDS round trip or workgroup barrier.
// As the reference's rule: a local cube's score is dropped once picked; when every remaining score is -inf the
// pick is index 0.
// Folds (ov, oi) into (v, i): the larger value, the smaller index on ties (the selection's order).
__device__ __forceinline__ void take_better(double& v, uint32_t& i, double ov, uint32_t oi)
{
    const bool take = ov > v || (ov == v && oi < i);
    v = take ? ov : v;
    i = take ? oi : i;
}

// One step of the wave's argmax on the DPP path: each lane takes the better of its pair and its partner's, the
// partner given by CTRL (quad_perm [1, 0, 3, 2]: lane ^ 1; [2, 3, 0, 1]: lane ^ 2; row half-mirror: 7 - lane within
// 8; row mirror: 15 - lane within 16), all moves inside a 16-lane row.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(double& v, uint32_t& i)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
    const uint32_t oi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)i, CTRL, 0xf, 0xf, false);
    take_better(v, i, __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo), oi);
}

// The steps across rows: v_permlane16_swap exchanges the odd rows of its first operand with the even rows of its
// second, v_permlane32_swap the upper half of the first with the lower half of the second; given the pair twice,
// the two results hold the values of the two rows (halves) being joined, in the same order in every lane of both,
// so both end with the same pair. Inline asm: this compiler's builtins return the first operand for both results;
// the s_nops give the preceding VALU writes, and the swaps' own results, their wait states.
template <bool HALVES>
__device__ __forceinline__ void argmax_swap(double& v, uint32_t& i)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    uint32_t l0 = (uint32_t)b, l1 = l0, h0 = (uint32_t)(b >> 32), h1 = h0, i0 = i, i1 = i;
    if (HALVES)
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_permlane32_swap_b32 %2, %3\n\t"
                     "v_permlane32_swap_b32 %4, %5\n\ts_nop 1"
                     : "+v"(l0), "+v"(l1), "+v"(h0), "+v"(h1), "+v"(i0), "+v"(i1));
    else
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_permlane16_swap_b32 %2, %3\n\t"
                     "v_permlane16_swap_b32 %4, %5\n\ts_nop 1"
                     : "+v"(l0), "+v"(l1), "+v"(h0), "+v"(h1), "+v"(i0), "+v"(i1));
    v = __builtin_bit_cast(double, ((uint64_t)h0 << 32) | l0);
    i = i0;
    take_better(v, i, __builtin_bit_cast(double, ((uint64_t)h1 << 32) | l1), i1);
}

template <uint32_t P>
__device__ __forceinline__ void best_of(const double (&v)[P], uint32_t lane, uint32_t n, double& bv, uint32_t& bi)
{
    bv = -INFINITY;
    bi = 0;
#pragma unroll
    for (uint32_t j = 0; j < P; ++j)
        if (lane + 64 * j < n && v[j] > bv) {
            bv = v[j];
            bi = lane + 64 * j;
        }
}

template <uint32_t P>
__global__ __launch_bounds__(64) void cube_topk(const double* __restrict__ sc, uint16_t* __restrict__ sel,
                                                uint16_t* __restrict__ nsel, uint32_t n, uint32_t kk, uint32_t local,
                                                uint32_t stride)
{
    const uint32_t qc = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const double* rowp = sc + ((size_t)h * n + qc) * n;
    double v[P];
#pragma unroll
    for (uint32_t j = 0; j < P; ++j)
        v[j] = lane + 64 * j < n ? rowp[lane + 64 * j] : -INFINITY;
    uint16_t* out = sel + ((size_t)h * n + qc) * kk;
    const auto drop = [&](uint32_t idx) {  // the lane holding idx sets it to -inf
#pragma unroll
        for (uint32_t j = 0; j < P; ++j)
            if (lane + 64 * j == idx)
                v[j] = -INFINITY;
    };
    uint32_t it = 0;
    if (local) {
        const uint32_t picks[3] = {qc, qc >= stride ? qc - stride : n, qc + stride < n ? qc + stride : n};
        for (uint32_t j = 0; j < local && it < kk; ++j)
            if (picks[j] < n) {
                if (lane == 0)
                    out[it] = (uint16_t)picks[j];
                ++it;
                drop(picks[j]);
            }
    }
    double bv;
    uint32_t bi;
    best_of<P>(v, lane, n, bv, bi);
    for (; it < kk; ++it) {
        double wv = bv;
        uint32_t wi = bi;
        argmax_dpp<0xb1>(wv, wi);    // quad_perm [1, 0, 3, 2]
        argmax_dpp<0x4e>(wv, wi);    // quad_perm [2, 3, 0, 1]
        argmax_dpp<0x141>(wv, wi);   // row half-mirror
        argmax_dpp<0x140>(wv, wi);   // row mirror
        argmax_swap<false>(wv, wi);  // rows 0 / 1 and 2 / 3
        argmax_swap<true>(wv, wi);   // halves
        if (lane == 0)
            out[it] = (uint16_t)wi;
        if (lane == wi % 64) {  // the holder drops the pick and finds its next best
            drop(wi);
            best_of<P>(v, lane, n, bv, bi);
        }
    }
    if (lane == 0)
        nsel[(size_t)h * n + qc] = (uint16_t)kk;
}

// The top-k launch with the smallest register array that holds n scores (n <= 4096).
void launch_topk(const double* sc, uint16_t* sel, uint16_t* nsel, uint32_t n, uint32_t heads, uint32_t kk,
                 uint32_t local, uint32_t stride, hipStream_t s)
{
    const dim3 grid(n, heads);
#define MAKO_TOPK_CASE(PL)                                                                                         \
    if (n <= 64 * (PL)) {                                                                                          \
        hipLaunchKernelGGL(cube_topk<PL>, grid, dim3(64), 0, s, sc, sel, nsel, n, kk, local, stride);             \
        return;                                                                                                    \
    }
    MAKO_TOPK_CASE(1)
    MAKO_TOPK_CASE(2)
    MAKO_TOPK_CASE(4)
    MAKO_TOPK_CASE(8)
    MAKO_TOPK_CASE(16)
    MAKO_TOPK_CASE(32)
    MAKO_TOPK_CASE(64)
#undef MAKO_TOPK_CASE
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

size_t pooled_bytes(uint32_t heads, uint32_t n) { return ((size_t)heads * n * kD * sizeof(double) + 255) / 256 * 256; }

constexpr int kWaves8 = 8;

// Lists shared by a kv head's query heads, in groups of 4: the ping-pong structure of attn_fwd.hip's flash_fwd
// driven by the pass list. A workgroup is one 64-row query tile of 4 query heads: 8 waves, wave w holding head
// w % 4's rows 32 (w / 4) .. + 31, so every gathered K / V tile serves all eight. Waves 0-3 and 4-7 alternate a
// matrix phase (Q K^T of the next pass's tile, P V of the current one) and a vector phase (that tile's masks,
// softmax and the staging of later tiles), one phase apart; tiles rotate through three LDS buffers. A tile's
// validity (valid flags and the pass's end) is one byte load a lane and a ballot, issued a phase ahead.
template <class T, class TO>
__global__ __launch_bounds__(kWaves8 * 64) void flash_sparse8(const SparseParams p)
{
    using E = Elem<T>;
    using V8 = typename E::vec8;
    using H = Elem<_Float16>;
    using H8 = f16x8;
    constexpr int NBUF = 3;
    constexpr int KS = kD + 8;
    constexpr int VS = kKB;
    constexpr int CPR = kD / 8;
    constexpr int GRPI = 256 / CPR;  // K rows one group-wide staging instruction covers
    constexpr int NKG = 32 / GRPI;   // K chunks a thread stages per half tile
    constexpr int NKK = kD / 16, NDB = kD / 32;
    __shared__ __attribute__((aligned(16))) T ks[NBUF][kKB * KS];
    __shared__ __attribute__((aligned(16))) _Float16 vt[NBUF][kD * VS];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t grp = w >> 2;
    const uint32_t g = lane >> 5, c32 = lane & 31;
    const uint32_t qt = p.n_qt - 1 - blockIdx.y;  // dense tiles (all keys) and late cubes first
    const uint32_t h = blockIdx.x * 4 + (w & 3);
    const uint32_t kvh = h / p.group;  // the same for the workgroup's 4 heads
    const uint32_t q0 = qt * kCube + 32 * (w >> 2);
    const uint32_t row = q0 + c32;
    const bool live = q0 < p.n_q;

    // The pass list: a cube tile's selected cubes, then its dense rows; a later tile's all keys. A pass past the
    // list is empty (its keys start at k_pad: loads fetch nothing and every key is masked).
    const bool cube = qt < p.n_cubes;
    const uint16_t* my_sel = p.sel + ((size_t)kvh * p.n_cubes + qt) * p.max_sel;
    const uint32_t ns = cube ? min(uniform_u16(p.nsel, (size_t)kvh * p.n_cubes + qt), p.max_sel) : 0u;
    const uint32_t dense_lo = cube ? p.dense0 : 0u, dense_hi = cube ? p.dense1 : p.n_k;
    const uint32_t n_dense = dense_hi > dense_lo ? (dense_hi - dense_lo + kKB - 1) / kKB : 0u;
    const uint32_t nt = ns + n_dense;
    auto pass_range = [&](uint32_t ps, uint32_t& j0, uint32_t& hi) {
        if (ps < ns) {
            j0 = uniform_u16(my_sel, ps) * kCube;
            hi = j0 + kCube;
        } else if (ps < nt) {
            j0 = dense_lo + (ps - ns) * kKB;
            hi = min(j0 + kKB, dense_hi);
        } else {
            j0 = p.k_pad;
            hi = j0;
        }
    };

    V8 qreg[NKK];
    {
        const auto qrs = buffer_rsrc(static_cast<const T*>(p.q) + (size_t)h * p.q_pad * kD, p.n_q * kD * sizeof(T));
        const uint32_t off = (row * kD + 8 * g) * sizeof(T);
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            qreg[kk] = __builtin_bit_cast(V8, buffer_load16(qrs, off + 16 * kk * sizeof(T)));
    }

    // Staging (as in flash_fwd): group grp stages keys 32 grp .. 32 grp + 31 of a pass's tile, K row-major in slot
    // order, V transposed to f16. The K / V resources span the kv head's k_pad rows (a cube may hold rows past n_k,
    // which valid masks); loads past k_pad return zeros.
    const T* kbase = static_cast<const T*>(p.k) + (size_t)kvh * p.k_pad * kD;
    const T* vbase = static_cast<const T*>(p.v) + (size_t)kvh * p.k_pad * kD;
    const uint32_t gt = tid & 255, hk = 32 * grp;
    const uint32_t k_row = gt / CPR, k_col = gt % CPR;
    const uint32_t v_cc = gt % CPR;
    const uint32_t v_kp = ((gt / CPR) & ~3u) | (((gt / CPR) ^ (2 * (v_cc >> 3))) & 3u);  // key pair 0 .. 15
    struct Half {
        u32x4 k[NKG], v[2];
    };
    auto load_half = [&](uint32_t ps, Half& st) __attribute__((always_inline)) {
        uint32_t j0, hi;
        pass_range(ps, j0, hi);
        j0 += hk;
        const uint32_t left = j0 < p.k_pad ? (p.k_pad - j0) * kD * (uint32_t)sizeof(T) : 0u;
        const auto krs = buffer_rsrc(kbase + (size_t)min(j0, p.k_pad) * kD, left);
        const auto vrs = buffer_rsrc(vbase + (size_t)min(j0, p.k_pad) * kD, left);
#pragma unroll
        for (int i = 0; i < NKG; ++i)
            st.k[i] = buffer_load16(krs, ((k_row + GRPI * i) * kD + k_col * 8) * sizeof(T));
#pragma unroll
        for (int i = 0; i < 2; ++i)
            st.v[i] = buffer_load16(vrs, ((2 * v_kp + i) * kD + v_cc * 8) * sizeof(T));
    };
    auto store_half = [&](uint32_t buf, const Half& st) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NKG; ++i)
            *reinterpret_cast<u32x4*>(&ks[buf][(hk + slot_of(k_row + GRPI * i)) * KS + k_col * 8]) = st.k[i];
        const uint32_t key = hk + 2 * v_kp, kc = key / 8, off = key % 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = v_cc * 8 + e;
            *reinterpret_cast<uint32_t*>(&vt[buf][d * VS + ((kc ^ vt_swz(d)) * 8) + off]) =
                f16_pair<T>(st.v[0], st.v[1], e);
        }
    };
    // A pass's validity flag for key j0 + lane (loaded a phase before its ballot).
    const auto valid_rs = buffer_rsrc(p.valid, p.k_pad);
    auto valid_flag = [&](uint32_t ps) {
        uint32_t j0, hi;
        pass_range(ps, j0, hi);
        const uint32_t f = __builtin_amdgcn_raw_buffer_load_b8(valid_rs, (int)(j0 + lane), 0, 0);
        return (j0 + lane < hi && f != 0) ? 1u : 0u;
    };

    const float c = p.scale_log2;
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
    float m = -INFINITY, l = 0.0f, thr = -INFINITY;
    f32x16 s[2];
    // P of the current pass as f16 pairs (dwords, so that the row sum reads whole registers)
    uint32_t pw[16];
    auto pb = [&](int cc) __attribute__((always_inline)) {
        return __builtin_bit_cast(H8, u32x4{pw[4 * cc], pw[4 * cc + 1], pw[4 * cc + 2], pw[4 * cc + 3]});
    };

    // The vector work on pass ps's scores (register r of s[t] holds key j0 + 32 t + 16 (r / 8) + 8 g + r % 8):
    // masks from the validity ballot and the causal bound, the rescale decision, exponentials and the row sum.
    auto softmax = [&](uint32_t ps, uint64_t vmask) __attribute__((always_inline)) {
        uint32_t j0, hi;
        pass_range(ps, j0, hi);
        const bool cut = p.causal && j0 + kKB - 1 > q0;
        if (vmask != ~0ull || cut) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int a = 0; a < 2; ++a) {
                    const uint32_t kb = 32 * t + 16 * a + 8 * g;
                    const uint32_t bits = (uint32_t)(vmask >> kb) & 0xffu;
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const bool seen = ((bits >> jj) & 1u) && (!p.causal || j0 + kb + jj <= row);
                        s[t][8 * a + jj] = seen ? s[t][8 * a + jj] : -INFINITY;
                    }
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
            const float f = up ? exp2_fast(m - mx) : 1.0f;
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
        float l4[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // the row sum of the f16 values P V multiplies
#pragma unroll
        for (int q = 0; q < 16; ++q)
            l4[q & 3] = sum_f16x2(pw[q], l4[q & 3]);
        l += (l4[0] + l4[1]) + (l4[2] + l4[3]);
    };
    auto pv = [&](uint32_t buf) {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const uint32_t d = 32 * db + c32;
                const _Float16* vr = &vt[buf][d * VS + (((2 * cc + g) ^ vt_swz(d)) * 8)];
                oacc[db] = H::mfma32(*reinterpret_cast<const H8*>(vr), pb(cc), oacc[db]);
            }
    };

    // The steady state's matrix phase in one stream, as in flash_fwd: Q K^T of the next pass then P V of the
    // current one, each operand read kRing reads ahead of its MFMA (the compiler alone kept two or three).
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
            if (i < NQ) {  // same order as qk
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

    // Prologue: passes 0 .. 2 by both groups (loads in flight together with Q's), group 1's half of pass 3.
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
    uint32_t vflag = valid_flag(0);
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
        settle(qreg[kk]);
    __syncthreads();
    if (nt > 0) {
        qk(s, 0);
        softmax(0, __ballot(vflag != 0));
    }
    if (grp == 1)
        __syncthreads();  // group 1 runs one phase behind group 0

    uint32_t b0 = 0, b1 = 1, b2 = 2;
    // The staging as in flash_fwd (loads past the list fetch nothing), and the buffer rotation.
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
    // Passes with a next one, then the last: no branch around the matrix work of the steady state.
    uint32_t j = 0;
    for (; j + 1 < nt; ++j) {
        // matrix phase: scores of pass j + 1, P V of pass j; pass j + 1's validity flags in flight
        vflag = valid_flag(j + 1);
        __builtin_amdgcn_s_setprio(1);
        __builtin_amdgcn_sched_barrier(0);
        matrix(b1, b0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        // vector phase: softmax of pass j + 1, and the staging
        softmax(j + 1, __ballot(vflag != 0));
        stage(j);
        __syncthreads();
        rotate();
    }
    if (j < nt) {
        __builtin_amdgcn_s_setprio(1);
        pv(b0);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        stage(j);
        __syncthreads();
    }
    if (grp == 0)
        __syncthreads();  // the barrier count of group 1's offset

    // Normalise and store through the row map; the LSE by tile row.
    const float lt = l + swap_halves(l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    if (live && row < p.n_q) {
        const int32_t dst = p.map[row];
        if (dst >= 0) {
            TO* orow = static_cast<TO*>(p.o) + (size_t)dst * p.width + (size_t)h * kD;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    store4<TO>(orow + 32 * db + 8 * r4 + 4 * g, oacc[db][4 * r4] * inv, oacc[db][4 * r4 + 1] * inv,
                               oacc[db][4 * r4 + 2] * inv, oacc[db][4 * r4 + 3] * inv);
            if (p.lse && g == 0)
                p.lse[(size_t)h * p.q_pad + row] = lt > 0.0f ? (m + __log2f(lt)) * kLn2 : -INFINITY;
        }
    }
}

template <class T, class TO>
void launch_sparse(const SparseParams& p, hipStream_t s)
{
    if (p.sel_heads == p.kv_heads && p.group % 4 == 0) {
        hipLaunchKernelGGL((flash_sparse8<T, TO>), dim3(p.heads / 4, p.n_qt), dim3(kWaves8 * 64), 0, s, p);
        return;
    }
    const dim3 grid(p.n_hg * p.n_qt);
    if (p.hs == 2)
        hipLaunchKernelGGL((flash_sparse<T, TO, 4>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((flash_sparse<T, TO, 2>), grid, dim3(128), 0, s, p);
}

}  // namespace
}  // namespace mako

using namespace mako;

extern "C" size_t mako_cube_select_workspace(uint32_t heads, uint32_t n_cubes)
{
    return 2 * pooled_bytes(heads, n_cubes) + (size_t)heads * n_cubes * n_cubes * sizeof(double);
}

extern "C" int mako_cube_select(uint32_t heads, uint32_t q_pad, uint32_t k_pad, uint32_t n_cubes, uint32_t topk,
                                uint32_t local, uint32_t stride, mako_dtype in, const void* q, const void* k,
                                const uint32_t* cnt, uint16_t* sel, uint16_t* nsel, void* workspace,
                                size_t workspace_bytes, void* stream)
{
    if (n_cubes > 4096 || !topk || (local != 0 && local != 1 && local != 3))
        return fail(MAKO_EINVAL, "cube_select: %u cubes, top %u, local %u", n_cubes, topk, local);
    if (!q || !k || !cnt || !sel || !nsel)
        return fail(MAKO_EINVAL, "cube_select: a null argument");
    if (in != MAKO_F16 && in != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "cube_select: input type %d (f16 or bf16)", (int)in);
    if ((uint64_t)n_cubes * kCube > q_pad || (uint64_t)n_cubes * kCube > k_pad)
        return fail(MAKO_EINVAL, "cube_select: %u cubes of 64 rows exceed the tiles' %u / %u rows", n_cubes, q_pad,
                    k_pad);
    if (!workspace || workspace_bytes < mako_cube_select_workspace(heads, n_cubes) || !aligned16(workspace))
        return fail(MAKO_EWORKSPACE, "cube_select: workspace of %zu bytes, %zu needed (16-byte aligned)",
                    workspace_bytes, mako_cube_select_workspace(heads, n_cubes));
    if (!heads || !n_cubes)
        return ok();
    double* qp = static_cast<double*>(workspace);
    double* kp = reinterpret_cast<double*>(static_cast<char*>(workspace) + pooled_bytes(heads, n_cubes));
    double* sc = reinterpret_cast<double*>(static_cast<char*>(workspace) + 2 * pooled_bytes(heads, n_cubes));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 pgrid(n_cubes, heads, 2),
        sgrid((n_cubes + kScoreTile - 1) / kScoreTile, (n_cubes + kScoreTile - 1) / kScoreTile, heads);
    if (in == MAKO_BF16)
        hipLaunchKernelGGL(cube_pool<__bf16>, pgrid, dim3(kD), 0, s, static_cast<const __bf16*>(q),
                           static_cast<const __bf16*>(k), cnt, qp, kp, n_cubes, q_pad, k_pad);
    else
        hipLaunchKernelGGL(cube_pool<_Float16>, pgrid, dim3(kD), 0, s, static_cast<const _Float16*>(q),
                           static_cast<const _Float16*>(k), cnt, qp, kp, n_cubes, q_pad, k_pad);
    hipLaunchKernelGGL(cube_scores, sgrid, dim3(256), 0, s, qp, kp, sc, n_cubes);
    launch_topk(sc, sel, nsel, n_cubes, heads, std::min(topk, n_cubes), local, stride, s);
    return check_launch("cube_select");
}

namespace {

int attn_sparse_core(const mako_sparse_args* a, mako_dtype in, mako_dtype out, const void* q, const void* k,
                     const void* v, void* o, const uint16_t* sel, const uint16_t* nsel, const uint8_t* valid,
                     const int32_t* map, float* lse, const Workspace& work, void* stream)
{
    if (!a || !q || !k || !v || !o || !valid || !map || ((!sel || !nsel) && a->n_cubes))
        return fail(MAKO_EINVAL, "attention_sparse: a null argument");
    if (a->q_pad % 64 || a->k_pad % 128 || a->dense0 % 32)
        return fail(MAKO_EINVAL,
                    "attention_sparse: q_pad a multiple of 64, k_pad of 128, the dense rows from a multiple of 32");
    if (in != MAKO_F16 && in != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "attention_sparse: input type %d (f16 or bf16)", (int)in);
    if (out != MAKO_F32 && out != in)
        return fail(MAKO_EUNSUPPORTED, "attention_sparse: output type %d (f32 or the input's)", (int)out);
    if (!a->heads || !a->kv_heads || a->heads % a->kv_heads)
        return fail(MAKO_EINVAL, "attention_sparse: %u heads over %u kv heads", a->heads, a->kv_heads);
    if (a->sel_heads != a->heads && a->sel_heads != a->kv_heads)
        return fail(MAKO_EINVAL, "attention_sparse: sel rows for %u heads (heads %u or kv heads %u)", a->sel_heads,
                    a->heads, a->kv_heads);
    if (a->n_q > a->q_pad || a->n_k > a->k_pad || a->dense0 > a->dense1 || a->dense1 > a->k_pad ||
        (uint64_t)a->n_cubes * kCube > a->k_pad || (a->n_cubes && !a->max_sel))
        return fail(MAKO_EINVAL, "attention_sparse: %u queries in %u rows, %u keys in %u, dense rows [%u, %u), %u "
                    "cubes of %u selections", a->n_q, a->q_pad, a->n_k, a->k_pad, a->dense0, a->dense1, a->n_cubes,
                    a->max_sel);
    if ((uint64_t)a->heads * kD > a->width || a->width % 4)
        return fail(MAKO_EINVAL, "attention_sparse: o rows of %u for %u heads of 128", a->width, a->heads);
    if ((uint64_t)a->k_pad * kD * 2 > 0x7fffffffu)
        return fail(MAKO_EINVAL, "attention_sparse: %u key rows exceed 2 GiB a head", a->k_pad);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(MAKO_EINVAL, "attention_sparse: q, k, v and o must be 16-byte aligned");
    if (!(a->scale > 0.0f) || a->scale == INFINITY)
        return fail(MAKO_EINVAL, "attention_sparse: scale %g (positive and finite)", (double)a->scale);
    if (a->n_q == 0)
        return ok();
    const uint32_t group = a->heads / a->kv_heads;
    const uint32_t hs = (a->sel_heads == a->kv_heads && group % 2 == 0) ? 2 : 1;
    const SparseParams p{q, k, v, o, lse, sel, nsel, valid, map, a->n_q, a->q_pad, a->n_k, a->k_pad, a->heads,
                         a->kv_heads, a->width, a->scale * kLog2e, a->n_cubes, a->max_sel, a->dense0, a->dense1,
                         a->causal ? 1u : 0u, a->sel_heads, group, hs, (a->n_q + kCube - 1) / kCube,
                         a->heads / hs, (a->heads / hs) % 8 == 0 ? 1u : 0u};
    if (p.n_qt > 65535)
        return fail(MAKO_EINVAL, "attention_sparse: %u query tiles exceed the grid", p.n_qt);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (sparse64_fits(a, valid)) {
        const float sl = a->scale * kLog2e;
        int r;
        if (in == MAKO_BF16)
            r = out == MAKO_F32
                    ? launch_sparse64<__bf16, float>(a, sl, q, k, v, o, sel, nsel, valid, map, lse, s, work)
                    : launch_sparse64<__bf16, __bf16>(a, sl, q, k, v, o, sel, nsel, valid, map, lse, s, work);
        else
            r = out == MAKO_F32
                    ? launch_sparse64<_Float16, float>(a, sl, q, k, v, o, sel, nsel, valid, map, lse, s, work)
                    : launch_sparse64<_Float16, _Float16>(a, sl, q, k, v, o, sel, nsel, valid, map, lse, s, work);
        if (r < 0)
            return last_code() != MAKO_OK ? last_code() : MAKO_EHIP;
        return check_launch("attention_sparse");
    }
    if (sparse_lists_fits(a, in, valid)) {
        if (out == MAKO_F32)
            launch_sparse_lists<float>(a, a->scale * kLog2e, q, k, v, o, sel, nsel, valid, map, lse, s);
        else
            launch_sparse_lists<_Float16>(a, a->scale * kLog2e, q, k, v, o, sel, nsel, valid, map, lse, s);
        return check_launch("attention_sparse");
    }
    if (in == MAKO_BF16) {
        if (out == MAKO_F32)
            launch_sparse<__bf16, float>(p, s);
        else
            launch_sparse<__bf16, __bf16>(p, s);
    } else {
        if (out == MAKO_F32)
            launch_sparse<_Float16, float>(p, s);
        else
            launch_sparse<_Float16, _Float16>(p, s);
    }
    return check_launch("attention_sparse");
}

}  // namespace

extern "C" size_t mako_attn_sparse_workspace(const mako_sparse_args* a)
{
    return a && a->n_q && sparse64_fits(a, nullptr) ? sparse64_workspace(a) : 0;
}

extern "C" int mako_attn_sparse(const mako_sparse_args* a, mako_dtype in, mako_dtype out, const void* q,
                                const void* k, const void* v, void* o, const uint16_t* sel, const uint16_t* nsel,
                                const uint8_t* valid, const int32_t* map, float* lse, void* stream)
{
    return attn_sparse_core(a, in, out, q, k, v, o, sel, nsel, valid, map, lse,
                            library_workspace(kWsPassTable, "attention_sparse"), stream);
}

extern "C" int mako_attn_sparse_ws(const mako_sparse_args* a, mako_dtype in, mako_dtype out, const void* q,
                                   const void* k, const void* v, void* o, const uint16_t* sel, const uint16_t* nsel,
                                   const uint8_t* valid, const int32_t* map, float* lse, void* workspace,
                                   size_t workspace_bytes, void* stream)
{
    return attn_sparse_core(a, in, out, q, k, v, o, sel, nsel, valid, map, lse,
                            caller_workspace(workspace, workspace_bytes, "attention_sparse"), stream);
}
