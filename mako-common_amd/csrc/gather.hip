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

// Workgroups run on XCD (linear id % 8): dispatch is round robin over the 8 XCDs, each with its own L2. The kernels
// below take a 1-D grid and give the `tiles` workgroups of one unit (the tiles that share an input: one token's
// probabilities or query rows) consecutive slots of one XCD, so the shared input comes from HBM once.
struct XcdSlot {
    uint32_t unit, tile;
};
__device__ __forceinline__ XcdSlot xcd_slot(uint32_t tiles)
{
    const uint32_t L = blockIdx.x, slot = L >> 3;
    return {(L & 7u) + 8u * (slot / tiles), slot % tiles};
}
inline uint32_t xcd_grid(uint32_t units, uint32_t tiles) { return 8u * tiles * ((units + 7u) / 8u); }

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
    uint32_t n_dt, n_ht, units;  // dim tiles, head tiles, units (head tile x split x token)
    uint32_t p_vec;              // probability rows 16-byte aligned: 4-float loads
};

// Unit = (head tile, split, token), tile = 64 dims; 4 waves: wave w computes heads h0 + 32 (w / 2) .., dims
// d0 + 32 (w % 2) ... A 64-key chunk goes through LDS, two buffers, one barrier a chunk:
//   probabilities as f16 rows ps[head][key] (thread tid: head tid / 4, keys 16 (tid % 4) ..);
//   latent rows transposed, ks[dim][key], written as key pairs (thread tid: keys 2 (tid / 8) and the next one, dims
//   8 (tid % 8) ..), the 16-byte group of 8 keys at position group ^ (dim / 8) % 8 so the pair writes of a wave hit
//   64 distinct banks.
// The loads of the next two chunks are in flight while a chunk's MFMAs run: every fetch issues the same loads
// (addresses clamped into the arrays, values past the ends zeroed when stored), so the steady loop's waits are fixed
// counts. Gathered rows take their list entries one chunk ahead.
template <bool GATHERED, bool PVEC>
__global__ __launch_bounds__(256) void pv_tiles(const PvParams a)
{
    constexpr int PP = kT + 8;  // LDS row pitch in halves
    __shared__ __attribute__((aligned(16))) _Float16 ps[2][kT * PP];
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][kT * PP];
    const XcdSlot xs = xcd_slot(a.n_dt);
    if (xs.unit >= a.units)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t d0 = xs.tile * kT, h0 = (xs.unit % a.n_ht) * kT, z = xs.unit / a.n_ht;
    const uint32_t split = z % a.splits, t = z / a.splits;
    const float* p = a.p;
    const uint32_t* list = a.list;
    const uint32_t k_begin = split * a.per;
    uint32_t k_end;
    if (GATHERED) {
        k_end = min(min(a.count[t], a.p_ld), k_begin + a.per);  // entries past the list row count as zero
        p += (size_t)t * a.heads * a.p_ld;
        list += (size_t)t * a.p_ld;
    } else {
        k_end = min(a.n_kv, k_begin + a.per);
    }
    const uint32_t nch = k_end > k_begin ? (k_end - k_begin + kT - 1) / kT : 0u;
    f32x16 acc = {};
    if (nch > 0) {
        const uint32_t r = tid >> 2, c = (tid & 3) * 16;     // probabilities: head h0 + r, keys c ..
        const uint32_t ep = tid >> 3, dg = tid & 7;          // latent: keys 2 ep, 2 ep + 1, dims 8 dg ..
        const bool r_ok = h0 + r < a.heads;
        const float* pr = p + (size_t)(r_ok ? h0 + r : h0) * a.p_ld;
        const _Float16* kvd = a.kv + d0 + 8 * dg;
        const uint32_t last = k_end - 1;
        struct Stage {
            float x[16];
            u32x4 v0, v1;
        };
        uint32_t i0 = 0, i1 = 0;  // gathered: the rows of the next chunk's keys 2 ep, 2 ep + 1
        if (GATHERED) {
            i0 = list[min(k_begin + 2 * ep, last)];
            i1 = list[min(k_begin + 2 * ep + 1, last)];
        }
        auto fetch = [&](Stage& st, uint32_t k0) __attribute__((always_inline)) {
            // the next chunk's list entries first: the next fetch then waits for them alone, not for this one's data
            uint32_t n0 = 0, n1 = 0;
            if (GATHERED) {
                n0 = list[min(k0 + kT + 2 * ep, last)];
                n1 = list[min(k0 + kT + 2 * ep + 1, last)];
            }
            const uint32_t kk = k0 + c;
            if (PVEC) {
                #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f32x4 y = *reinterpret_cast<const f32x4*>(pr + min(kk + 4 * i, a.p_ld - 4));
                    st.x[4 * i] = y[0];
                    st.x[4 * i + 1] = y[1];
                    st.x[4 * i + 2] = y[2];
                    st.x[4 * i + 3] = y[3];
                }
            } else {
                #pragma unroll
                for (int i = 0; i < 16; ++i)
                    st.x[i] = pr[min(kk + i, last)];
            }
            const uint32_t row0 = GATHERED ? i0 : min(k0 + 2 * ep, last);
            const uint32_t row1 = GATHERED ? i1 : min(k0 + 2 * ep + 1, last);
            st.v0 = *reinterpret_cast<const u32x4*>(kvd + (size_t)row0 * a.dim);
            st.v1 = *reinterpret_cast<const u32x4*>(kvd + (size_t)row1 * a.dim);
            i0 = n0;
            i1 = n1;
        };
        auto put = [&](const Stage& st, int b, uint32_t k0) __attribute__((always_inline)) {
            const uint32_t kk = k0 + c;
            u32x4 w0, w1;
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a0 = r_ok && kk + 2 * i < k_end ? st.x[2 * i] : 0.0f;
                const float a1 = r_ok && kk + 2 * i + 1 < k_end ? st.x[2 * i + 1] : 0.0f;
                const float b0 = r_ok && kk + 8 + 2 * i < k_end ? st.x[8 + 2 * i] : 0.0f;
                const float b1 = r_ok && kk + 9 + 2 * i < k_end ? st.x[9 + 2 * i] : 0.0f;
                w0[i] = Elem<_Float16>::pack2(a0, a1);
                w1[i] = Elem<_Float16>::pack2(b0, b1);
            }
            *reinterpret_cast<u32x4*>(ps[b] + r * PP + c) = w0;
            *reinterpret_cast<u32x4*>(ps[b] + r * PP + c + 8) = w1;
            const uint32_t m0 = k0 + 2 * ep < k_end ? 0xffffu : 0u, m1 = k0 + 2 * ep + 1 < k_end ? 0xffff0000u : 0u;
            const uint32_t col = (((ep >> 2) ^ dg) << 3) + 2 * (ep & 3);  // key 2 ep, swizzled
            uint32_t* kw = reinterpret_cast<uint32_t*>(ks[b] + 8 * dg * PP + col);
            #pragma unroll
            for (int i = 0; i < 8; ++i)
                kw[i * (PP / 2)] = (half_of(st.v0, i) & m0) | ((half_of(st.v1, i) << 16) & m1);
        };
        const uint32_t hb = 32 * (w >> 1), db = 32 * (w & 1), krow = db + c32, ksw = (krow >> 3) & 7;
        auto mma = [&](int b) __attribute__((always_inline)) {
            #pragma unroll
            for (int kk = 0; kk < kT / 16; ++kk) {
                const f16x8 av = *reinterpret_cast<const f16x8*>(ps[b] + (hb + c32) * PP + 16 * kk + 8 * g);
                const f16x8 bv = *reinterpret_cast<const f16x8*>(ks[b] + krow * PP + (((2 * kk + g) ^ ksw) << 3));
                acc = Elem<_Float16>::mfma32(av, bv, acc);
            }
        };
        // Even steps multiply out of buffer 0, odd steps out of buffer 1; a buffer is written only after the
        // barrier that ends the step reading it. sa / sb hold the chunks fetched but not yet stored.
        Stage sa, sb;
        fetch(sa, k_begin);
        if (nch > 1)
            fetch(sb, k_begin + kT);
        put(sa, 0, k_begin);
        __syncthreads();
        uint32_t j = 0;
        for (; j + 3 < nch; j += 2) {
            fetch(sa, k_begin + (j + 2) * kT);
            __builtin_amdgcn_sched_barrier(0);  // the loads go out before the stores of the older chunk wait
            mma(0);
            put(sb, 1, k_begin + (j + 1) * kT);
            __syncthreads();
            fetch(sb, k_begin + (j + 3) * kT);
            __builtin_amdgcn_sched_barrier(0);
            mma(1);
            put(sa, 0, k_begin + (j + 2) * kT);
            __syncthreads();
        }
        // chunks j .. nch - 1 are left (one to three): chunk j in buffer 0, chunk j + 1 (if any) in sb
        if (j + 2 < nch) {
            fetch(sa, k_begin + (j + 2) * kT);
            mma(0);
            put(sb, 1, k_begin + (j + 1) * kT);
            __syncthreads();
            mma(1);
            put(sa, 0, k_begin + (j + 2) * kT);
            __syncthreads();
            mma(0);
        } else if (j + 1 < nch) {
            mma(0);
            put(sb, 1, k_begin + (j + 1) * kT);
            __syncthreads();
            mma(1);
        } else {
            mma(0);
        }
    }
    // acc register r of lane (c32, g): head h0 + hb + 8 (r / 4) + 4 g + r % 4, dim d0 + db + c32
    const uint32_t hb = 32 * (w >> 1), db = 32 * (w & 1);
    float* out = a.partial + ((size_t)split * a.tokens + t) * a.heads * a.dim;
    #pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
        const uint32_t h = h0 + hb + 8 * (rr >> 2) + 4 * g + (rr & 3);
        if (h < a.heads)
            out[(size_t)h * a.dim + d0 + db + c32] = acc[rr];
    }
}

template <bool GATHERED>
void launch_pv(const PvParams& pp, hipStream_t stream)
{
    const dim3 grid(xcd_grid(pp.units, pp.n_dt));
    if (pp.p_vec)
        hipLaunchKernelGGL((pv_tiles<GATHERED, true>), grid, dim3(256), 0, stream, pp);
    else
        hipLaunchKernelGGL((pv_tiles<GATHERED, false>), grid, dim3(256), 0, stream, pp);
}

// ---- q . kv rows over the latent dimension (attn_gather_scores) -------------------------------------------------

struct ScoreParams {
    const _Float16* q;  // [tokens][heads][dim]
    const _Float16* kv;
    const uint32_t* list;
    const uint32_t* count;
    float* scores;      // [tokens][heads][stride]
    uint32_t heads, dim, stride;
    uint32_t n_et, tokens;  // entry tiles a token (EB * 128 entries each), tokens
};

// Unit = token, tile = EB * 128 list entries; 4 waves, wave w takes entries e0 + 32 (EB w + b) + c32 (b < EB)
// against all heads (two blocks of 32). q is staged in LDS QC dims at a time (QC = 512 or 256, pitch QC + 8 halves:
// 16 consecutive rows hit distinct bank groups); the gathered rows go straight from global memory into the MFMA's B operand, one 64-dim
// group ahead of the MFMAs. The contraction runs over the dims in an order both operands share: in group m, MFMA
// step i takes dims 64 m + 32 g + 8 i .. + 7 in lane half g, so a lane reads 64 contiguous bytes of its row a group
// (the two lane halves: one 128-byte line). Every group issues the same loads (entries past count[t] read a clamped
// valid row, heads past `heads` the last head; the last group reloads itself), so the loop's waits are fixed
// counts; entries past count[t] are stored as 0.
template <int EB, int QC>
__global__ __launch_bounds__(256) void gather_scores(const ScoreParams a)
{
    constexpr int QP = QC + 8, GN = QC / 64, QL = QC / 32;  // pitch, groups a chunk, staging loads a thread
    __shared__ __attribute__((aligned(16))) _Float16 qs[kT * QP];
    const XcdSlot xs = xcd_slot(a.n_et);
    if (xs.unit >= a.tokens)
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t t = xs.unit, cnt = min(a.count[t], a.stride);
    const uint32_t e0 = xs.tile * (EB * 128) + 32 * EB * w;
    f32x16 acc[2][EB];
    #pragma unroll
    for (int hb = 0; hb < 2; ++hb)
        #pragma unroll
        for (int b = 0; b < EB; ++b)
            acc[hb][b] = f32x16{};
    if (xs.tile * (EB * 128) < cnt) {  // workgroup-uniform: a workgroup wholly past count[t] only stores zeros
        const u32x4* row[EB];
        #pragma unroll
        for (int b = 0; b < EB; ++b) {
            const uint32_t s = min(e0 + 32 * b + c32, cnt - 1);
            row[b] = reinterpret_cast<const u32x4*>(a.kv + (size_t)a.list[(size_t)t * a.stride + s] * a.dim) + 4 * g;
        }
        const _Float16* qt = a.q + (size_t)t * a.heads * a.dim;
        u32x4 cur[EB][4], nxt[EB][4];
        auto load = [&](u32x4 (&v)[EB][4], uint32_t m) __attribute__((always_inline)) {
            #pragma unroll
            for (int b = 0; b < EB; ++b)
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[b][i] = row[b][8 * m + i];
        };
        const uint32_t groups = a.dim / 64;
        load(cur, 0);
        for (uint32_t m0 = 0; m0 < groups; m0 += GN) {
            __syncthreads();  // the previous chunk is no longer read
            // q[t][h][64 m0 .. + QC]: 64 rows x QC / 8 runs of 16 bytes, QL a thread, all loads first
            constexpr uint32_t RS = QC / 8;  // runs a row
            u32x4 st[QL];
            #pragma unroll
            for (int i = 0; i < QL; ++i) {
                const uint32_t u = tid + 256 * i, h = u / RS, cc = u % RS;
                st[i] = *reinterpret_cast<const u32x4*>(qt + (size_t)min(h, a.heads - 1) * a.dim + 64 * m0 + 8 * cc);
            }
            #pragma unroll
            for (int i = 0; i < QL; ++i) {
                const uint32_t u = tid + 256 * i, h = u / RS, cc = u % RS;
                *reinterpret_cast<u32x4*>(qs + h * QP + 8 * cc) = st[i];
            }
            __syncthreads();
            #pragma unroll 2
            for (uint32_t mm = 0; mm < GN; ++mm) {
                const uint32_t m = m0 + mm;
                load(nxt, min(m + 1, groups - 1));
                __builtin_amdgcn_sched_barrier(0);  // the loads go out before the MFMAs wait for the older group
                const uint32_t qc = 64 * mm + 32 * g;
                #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    #pragma unroll
                    for (int hb = 0; hb < 2; ++hb) {
                        const f16x8 av = *reinterpret_cast<const f16x8*>(qs + (32 * hb + c32) * QP + qc + 8 * i);
                        #pragma unroll
                        for (int b = 0; b < EB; ++b)
                            acc[hb][b] = Elem<_Float16>::mfma32(av, __builtin_bit_cast(f16x8, cur[b][i]), acc[hb][b]);
                    }
                }
                #pragma unroll
                for (int b = 0; b < EB; ++b)
                    #pragma unroll
                    for (int i = 0; i < 4; ++i)
                        cur[b][i] = nxt[b][i];
            }
        }
    }
    // acc[hb][b] register r of lane (c32, g): head 32 hb + 8 (r / 4) + 4 g + r % 4, entry e0 + 32 b + c32
    float* out = a.scores + (size_t)t * a.heads * a.stride;
    #pragma unroll
    for (int b = 0; b < EB; ++b) {
        const uint32_t s = e0 + 32 * b + c32;
        if (s < a.stride) {
            const bool live = s < cnt;
            #pragma unroll
            for (int hb = 0; hb < 2; ++hb)
                #pragma unroll
                for (int rr = 0; rr < 16; ++rr) {
                    const uint32_t hh = 32 * hb + 8 * (rr >> 2) + 4 * g + (rr & 3);
                    if (hh < a.heads)
                        out[(size_t)hh * a.stride + s] = live ? acc[hb][b][rr] : 0.0f;
                }
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

// Grid (ceil(pools / 64), 1, tokens); waves 0 and 1 take pools p0 .. p0 + 31 and p0 + 32 .. (heads <= 32); one
// float a lane a step, straight from global memory. For rows of any width.
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

// Rows a multiple of 4 floats, 16-byte aligned. Grid (ceil(pools / 128), 1, tokens); 4 waves, wave w takes pools
// p0 + 32 w .. + 31 against the token's heads. 32-float chunks of the q rows and of 128 pooled rows are staged in
// LDS by coalesced 16-byte loads (pitch 36 floats: 16 consecutive rows hit distinct bank groups), two buffers, the
// next chunk's loads in flight during the MFMAs. The contraction runs over a chunk's dims in an order both operands
// share: MFMA step i of group m takes dim 8 m + 4 g + i in lane half g, so each operand is one 16-byte LDS read for
// four steps.
constexpr int kDP = 36;

__global__ __launch_bounds__(256) void idx_dots_lds(const DotParams a)
{
    __shared__ __attribute__((aligned(16))) float qs[2][32 * kDP];
    __shared__ __attribute__((aligned(16))) float ks[2][128 * kDP];
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t t = blockIdx.z, p0 = blockIdx.x * 128;
    // staging: thread tid moves float4 (tid & 7) of q row tid / 8 and of pooled rows p0 + tid / 8 + 32 i; rows past
    // heads or pools read a valid row (their results are not stored), dims past dim read a valid float4 of the row
    // and are zeroed
    const uint32_t sr = tid >> 3, sc = (tid & 7) * 4;
    const float* qsrc = a.q + ((size_t)t * a.heads + min(sr, a.heads - 1)) * a.dim;
    const float* ksrc[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i)
        ksrc[i] = a.pooled + (size_t)min(p0 + sr + 32 * i, a.pools - 1) * a.dim;
    struct Stage {
        f32x4 q, k[4];
    };
    auto fetch = [&](Stage& st, uint32_t k0) __attribute__((always_inline)) {
        const uint32_t off = min(k0 + sc, a.dim - 4);  // in the row; values past dim are zeroed in put
        st.q = *reinterpret_cast<const f32x4*>(qsrc + off);
        #pragma unroll
        for (int i = 0; i < 4; ++i)
            st.k[i] = *reinterpret_cast<const f32x4*>(ksrc[i] + off);
    };
    auto put = [&](const Stage& st, int b, uint32_t k0) __attribute__((always_inline)) {
        const bool in = k0 + sc < a.dim;
        *reinterpret_cast<f32x4*>(qs[b] + sr * kDP + sc) = in ? st.q : f32x4{0, 0, 0, 0};
        #pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<f32x4*>(ks[b] + (sr + 32 * i) * kDP + sc) = in ? st.k[i] : f32x4{0, 0, 0, 0};
    };
    f32x16 acc = {};
    auto mma = [&](int b) __attribute__((always_inline)) {
        #pragma unroll
        for (int m = 0; m < 4; ++m) {
            const f32x4 av = *reinterpret_cast<const f32x4*>(qs[b] + c32 * kDP + 8 * m + 4 * g);
            const f32x4 bv = *reinterpret_cast<const f32x4*>(ks[b] + (32 * w + c32) * kDP + 8 * m + 4 * g);
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc, 0, 0, 0);
        }
    };
    // Chunks of 32 dims (values past dim zeroed), two buffers: even chunks
    // multiply out of buffer 0, odd ones out of buffer 1, and the loads of the next two chunks are in flight (sa /
    // sb hold the chunks fetched but not yet stored).
    const uint32_t nc = (a.dim + 31) / 32;
    Stage sa, sb;
    fetch(sa, 0);
    fetch(sb, 32);
    put(sa, 0, 0);
    __syncthreads();
    uint32_t c = 0;
    for (; c + 3 < nc; c += 2) {
        fetch(sa, 32 * (c + 2));
        __builtin_amdgcn_sched_barrier(0);
        mma(0);
        __builtin_amdgcn_sched_barrier(0);
        put(sb, 1, 32 * (c + 1));
        __syncthreads();
        fetch(sb, 32 * (c + 3));
        __builtin_amdgcn_sched_barrier(0);
        mma(1);
        __builtin_amdgcn_sched_barrier(0);
        put(sa, 0, 32 * (c + 2));
        __syncthreads();
    }
    // chunks c .. nc - 1 are left (one to three): chunk c in buffer 0, chunk c + 1 (if any) in sb
    if (c + 2 < nc) {
        fetch(sa, 32 * (c + 2));
        mma(0);
        put(sb, 1, 32 * (c + 1));
        __syncthreads();
        mma(1);
        put(sa, 0, 32 * (c + 2));
        __syncthreads();
        mma(0);
    } else if (c + 1 < nc) {
        mma(0);
        put(sb, 1, 32 * (c + 1));
        __syncthreads();
        mma(1);
    } else {
        mma(0);
    }
    // acc register r of lane (c32, g): head 8 (r / 4) + 4 g + r % 4, pool p0 + 32 w + c32
    const uint32_t pl = p0 + 32 * w + c32;
    if (pl < a.pools) {
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

constexpr uint64_t kMaxGrid = 1u << 24;  // workgroups of a 1-D launch of 256 work-items (32-bit grid size)

extern "C" int mako_attn_pv(const mako_pv_args* a, const float* p, const void* kv, float* partial, void* stream)
{
    if (!a || !p || !kv || !partial)
        return fail(MAKO_EINVAL, "attn_pv: a null argument");
    if (!a->heads || !a->dim || a->dim % 64 || !a->keys_per_split || a->keys_per_split % 64)
        return fail(MAKO_EINVAL, "attn_pv: %u heads of %u, %u keys a split (dim and keys a split multiples of 64)",
                    a->heads, a->dim, a->keys_per_split);
    if (!al16(kv))
        return fail(MAKO_EINVAL, "attn_pv: kv must be 16-byte aligned");
    const uint32_t splits = (a->n_kv + a->keys_per_split - 1) / a->keys_per_split;
    if (splits == 0)
        return ok();
    const uint32_t n_dt = a->dim / kT, n_ht = (a->heads + kT - 1) / kT;
    if ((uint64_t)n_ht * splits * n_dt + 8u * n_dt > kMaxGrid)
        return fail(MAKO_EINVAL, "attn_pv: %u splits of %u head tiles and %u dim tiles exceed the grid", splits,
                    n_ht, n_dt);
    PvParams pp{p, static_cast<const _Float16*>(kv), nullptr, nullptr, partial, a->heads, a->dim, a->n_kv,
                a->n_kv, a->keys_per_split, splits, 1, 0, n_dt, n_ht, n_ht * splits,
                a->n_kv % 4 == 0 && al16(p)};
    launch_pv<false>(pp, static_cast<hipStream_t>(stream));
    return check_launch("attn_pv");
}

constexpr int kScoreEB = 2;  // entry blocks of 32 a wave: 256 list entries a workgroup

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
    const uint32_t n_et = (a->stride + kScoreEB * 128 - 1) / (kScoreEB * 128);
    if ((uint64_t)n_et * a->tokens + 8u * n_et > kMaxGrid)
        return fail(MAKO_EINVAL, "attn_gather_scores: %u tokens of lists of %u exceed the grid", a->tokens,
                    a->stride);
    ScoreParams sp{static_cast<const _Float16*>(q), static_cast<const _Float16*>(kv), list, count, scores, a->heads,
                   a->dim, a->stride, n_et, a->tokens};
    const dim3 grid(xcd_grid(a->tokens, n_et));
    if (a->dim % 512 == 0)
        hipLaunchKernelGGL((gather_scores<kScoreEB, 512>), grid, dim3(256), 0, static_cast<hipStream_t>(stream), sp);
    else
        hipLaunchKernelGGL((gather_scores<kScoreEB, 256>), grid, dim3(256), 0, static_cast<hipStream_t>(stream), sp);
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
    const uint32_t n_dt = a->dim / kT;
    if ((uint64_t)a->splits * a->tokens * n_dt + 8u * n_dt > kMaxGrid)
        return fail(MAKO_EINVAL, "attn_gather_pv: %u tokens x %u splits exceed the grid", a->tokens, a->splits);
    const uint32_t per = (a->stride + a->splits * kT - 1) / (a->splits * kT) * kT;
    PvParams pp{p, static_cast<const _Float16*>(kv), list, count, partial, a->heads, a->dim, a->stride, a->stride,
                per, a->splits, a->tokens, 1, n_dt, 1, a->splits * a->tokens, a->stride % 4 == 0 && al16(p)};
    launch_pv<true>(pp, static_cast<hipStream_t>(stream));
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
    if (a->dim % 4 == 0 && al16(q) && al16(pooled))
        hipLaunchKernelGGL(idx_dots_lds, dim3((a->pools + 127) / 128, 1, tokens), dim3(256), 0,
                           static_cast<hipStream_t>(stream), dp);
    else
        hipLaunchKernelGGL(idx_dots_k, dim3((a->pools + kT - 1) / kT, 1, tokens), dim3(128), 0,
                           static_cast<hipStream_t>(stream), dp);
    return check_launch("idx_dots");
}
