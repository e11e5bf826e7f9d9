// The output projection after attention: Runtime::proj with BF16 weights (src/gpu/runtime.cpp:164-205), i.e. the
// to_bf16 rounding of the activations (src/kernels/gemm.metal:676-681), the dense BF16 GEMM gemm_dense
// (gemm.metal:251-296) and, with bf16_split_, the remainder's GEMM and add_rows (src/kernels/ops.metal:421-437):
//
//   y[r][c] = sum_j w[c][j] * bf16(x[r][j])  (+ sum_j w[c][j] * bf16(x[r][j] - bf16(x[r][j])) with split)
//
// The design is this one's own. Bound: MFMA (a 4096-token, 4096 x 4096 projection is 137 GFLOP against 67 MB of
// output and 64 MB of operands). A workgroup of 4 waves computes a BM x 256 tile of y (BM = 256; 128 with split),
// each wave a (BM / 2) x 128 block as 32 x 32 MFMA blocks (v_mfma_f32_32x32x16_bf16) accumulating in f32.
// 64-wide K chunks of x rows and w rows go through LDS, two buffers with one barrier a chunk; the next chunk waits in
// registers while the current one is multiplied, and is stored, and the one after fetched, behind the first MFMAs. Both operands are K-contiguous rows, so every 16-byte run of a row
// is one MFMA operand (8 consecutive k). LDS rows are 128 bytes; the 16-byte run c of row r sits at position
// c ^ ((r / 2) % 8), so the 16 lanes of a ds_read_b128 (16 consecutive rows, one run) and of a ds_write_b128 (two
// rows, eight runs) hit 64 distinct banks. f32 activations are rounded to bf16 (to nearest even) as they are
// staged: the reference's separate to_bf16 pass (and its bf16 copy of x in HBM) is gone.
#include "device.hpp"

namespace mako {
namespace {

constexpr int kBN = 256, kBK = 64;

struct ProjParams {
    const __bf16* w;  // [n][k]
    const void* x;    // [t][ldx], bf16 or f32
    float* y;         // [t][ldy]
    uint32_t t, k, n, ldy, ldx;
    uint32_t tiles_m, tiles_n, tiles, per_xcd;
};

// Tile q of the output walks bands of 4 tile rows column by column, and XCD x takes tiles x * per_xcd .. (workgroup
// L runs on XCD L % 8): with 16 x 16 tiles each XCD holds a 4 x 8 block, sharing 4 row panels of x and 8 of w in
// its L2.
__device__ __forceinline__ bool tile_of(const ProjParams& a, uint32_t& tm, uint32_t& tn)
{
    const uint32_t L = blockIdx.x, slot = L >> 3;
    const uint32_t q = (L & 7u) * a.per_xcd + slot;
    if (slot >= a.per_xcd || q >= a.tiles)
        return false;
    const uint32_t band = q / (4u * a.tiles_n), h = min(4u, a.tiles_m - 4u * band), in = q - band * 4u * a.tiles_n;
    tn = in / h;
    tm = 4u * band + in % h;
    return true;
}

__device__ __forceinline__ uint32_t lds_pos(uint32_t row, uint32_t run) { return row * kBK + ((run ^ ((row >> 1) & 7u)) << 3); }

template <int BM, bool XF32, bool SPLIT>
__global__ __launch_bounds__(256, 1) void proj_tiles(const ProjParams a)
{
    constexpr int MB = BM / 64;     // 32-row blocks of x a wave
    constexpr int RA = BM / 32;     // staging rounds of x rows (32 rows a round)
    constexpr int RB = kBN / 32;    // staging rounds of w rows
    __shared__ __attribute__((aligned(16))) __bf16 as[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) __bf16 al[SPLIT ? 2 : 1][SPLIT ? BM * kBK : 8];
    __shared__ __attribute__((aligned(16))) __bf16 bs[2][kBN * kBK];
    uint32_t tm, tn;
    if (!tile_of(a, tm, tn))
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t t0 = tm * BM, n0 = tn * kBN;
    // staging: thread tid moves run tid % 8 (8 values of k) of rows tid / 8 + 32 i; rows past t / n read the last
    // row (their results are not stored)
    const uint32_t sr = tid >> 3, run = tid & 7;
    uint32_t xo[RA], wo[RB];
    #pragma unroll
    for (int i = 0; i < RA; ++i)
        xo[i] = min(t0 + sr + 32u * i, a.t - 1) * a.ldx + 8 * run;
    #pragma unroll
    for (int i = 0; i < RB; ++i)
        wo[i] = min(n0 + sr + 32u * i, a.n - 1) * a.k + 8 * run;
    struct Stage {
        f32x4 xf[XF32 ? 2 * RA : 1];  // f32 activations, loaded as float vectors (see put)
        u32x4 x[XF32 ? 1 : RA];
        u32x4 w[RB];
    };
    auto fetch = [&](Stage& st, uint32_t k0) __attribute__((always_inline)) {
        #pragma unroll
        for (int i = 0; i < RA; ++i) {
            if (XF32) {
                const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + (size_t)xo[i] + k0);
                st.xf[2 * i] = p[0];
                st.xf[2 * i + 1] = p[1];
            } else {
                st.x[i] = *reinterpret_cast<const u32x4*>(static_cast<const __bf16*>(a.x) + (size_t)xo[i] + k0);
            }
        }
        #pragma unroll
        for (int i = 0; i < RB; ++i)
            st.w[i] = *reinterpret_cast<const u32x4*>(a.w + (size_t)wo[i] + k0);
    };
    auto put = [&](const Stage& st, int b) __attribute__((always_inline)) {
        #pragma unroll
        for (int i = 0; i < RA; ++i) {
            const uint32_t p = lds_pos(sr + 32u * i, run);
            if (XF32) {
                // Floats come straight from float vectors: hipcc (ROCm 7.2) miscompiles the bf16 packing of
                // floats bit-cast one by one out of a u32x4 (one source converted twice, the loads overlapped).
                const f32x4 v0 = st.xf[2 * i], v1 = st.xf[2 * i + 1];
                const float f[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                u32x4 hi, lo;
                #pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hi[e] = Elem<__bf16>::pack2(f[2 * e], f[2 * e + 1]);
                    if (SPLIT)  // bf16(x - float(bf16(x))), the remainder the reference's bf16_lo keeps
                        lo[e] = Elem<__bf16>::pack2(f[2 * e] - (float)(__bf16)f[2 * e],
                                                    f[2 * e + 1] - (float)(__bf16)f[2 * e + 1]);
                }
                *reinterpret_cast<u32x4*>(as[b] + p) = hi;
                if (SPLIT)
                    *reinterpret_cast<u32x4*>(al[b] + p) = lo;
            } else {
                *reinterpret_cast<u32x4*>(as[b] + p) = st.x[i];
            }
        }
        #pragma unroll
        for (int i = 0; i < RB; ++i)
            *reinterpret_cast<u32x4*>(bs[b] + lds_pos(sr + 32u * i, run)) = st.w[i];
    };
    f32x16 acc[MB][4];
    #pragma unroll
    for (int bi = 0; bi < MB; ++bi)
        #pragma unroll
        for (int bj = 0; bj < 4; ++bj)
            acc[bi][bj] = f32x16{};
    const uint32_t ra = (w >> 1) * (BM / 2), rb = (w & 1) * 128;  // this wave's first x row and w row in the tile
    struct Frag {
        bf16x8 x[MB], xl[SPLIT ? MB : 1], w[4];
    };
    auto read = [&](Frag& f, int b, int kk) __attribute__((always_inline)) {
        const uint32_t rn = 2 * kk + g;
        #pragma unroll
        for (int bi = 0; bi < MB; ++bi) {
            const uint32_t p = lds_pos(ra + 32 * bi + c32, rn);
            f.x[bi] = *reinterpret_cast<const bf16x8*>(as[b] + p);
            if (SPLIT)
                f.xl[bi] = *reinterpret_cast<const bf16x8*>(al[b] + p);
        }
        #pragma unroll
        for (int bj = 0; bj < 4; ++bj)
            f.w[bj] = *reinterpret_cast<const bf16x8*>(bs[b] + lds_pos(rb + 32 * bj + c32, rn));
    };
    auto mfmas = [&](const Frag& f) __attribute__((always_inline)) {
        #pragma unroll
        for (int bi = 0; bi < MB; ++bi)
            #pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                acc[bi][bj] = Elem<__bf16>::mfma32(f.x[bi], f.w[bj], acc[bi][bj]);
                if (SPLIT)
                    acc[bi][bj] = Elem<__bf16>::mfma32(f.xl[bi], f.w[bj], acc[bi][bj]);
            }
    };
    // One K chunk out of buffer b: the operands of step kk + 1 are read while step kk's MFMAs run, and between(kk)
    // (the staging of a later chunk) is issued behind step kk's MFMAs.
    // sched_barrier keeps each read group ahead of the MFMAs it overlaps (the scheduler otherwise sinks the reads to
    // their first use and the MFMAs wait for LDS).
    auto chunk = [&](int b, auto between) __attribute__((always_inline)) {
        Frag f0, f1;
        read(f0, b, 0);
        read(f1, b, 1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(f0);
        between(0);
        __builtin_amdgcn_sched_barrier(0);
        read(f0, b, 2);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(f1);
        between(1);
        __builtin_amdgcn_sched_barrier(0);
        read(f1, b, 3);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(f0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(f1);
    };
    const uint32_t nk = a.k / kBK;
    Stage st;
    fetch(st, 0);
    put(st, 0);
    if (nk > 1)
        fetch(st, kBK);
    __syncthreads();
    uint32_t j = 0;
    for (; j + 2 < nk; ++j) {  // chunk j + 1 goes to the other buffer (last read before the previous barrier)
        const int b = j & 1;
        chunk(b, [&](int kk) __attribute__((always_inline)) {
            if (kk == 0)
                put(st, b ^ 1);
            else
                fetch(st, (j + 2) * kBK);
        });
        __syncthreads();
    }
    if (j + 1 < nk) {
        const int b = j & 1;
        chunk(b, [&](int kk) __attribute__((always_inline)) {
            if (kk == 0)
                put(st, b ^ 1);
        });
        __syncthreads();
        ++j;
    }
    chunk(j & 1, [](int) {});
    // acc[bi][bj] register r of lane (c32, g): row t0 + ra + 32 bi + 8 (r / 4) + 4 g + r % 4, column n0 + rb + 32 bj + c32
    #pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
        const uint32_t c = n0 + rb + 32 * bj + c32;
        if (c >= a.n)
            continue;
        #pragma unroll
        for (int bi = 0; bi < MB; ++bi)
            #pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = t0 + ra + 32 * bi + 8 * (r >> 2) + 4 * g + (r & 3);
                if (row < a.t)
                    a.y[(size_t)row * a.ldy + c] = acc[bi][bj][r];
            }
    }
}

// A raw buffer descriptor over the rows of a tile's panel from `base` (rows of ld values, `rows` of them left in the
// operand): reads at or past the end return zeros.
__device__ __forceinline__ u32x4 panel_rsrc(const __bf16* base, uint32_t rows, uint32_t ld)
{
    const uint64_t a = reinterpret_cast<uint64_t>(base), bytes = (uint64_t)rows * ld * 2;
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, (uint32_t)min(bytes, (uint64_t)0xffffffffu), 0x00020000u};
}

// bf16 activations: both operands go global -> LDS by the LDS DMA (buffer_load_dwordx4 ... lds: lane l of a wave
// writes 16 bytes at the wave's LDS base + 16 l, from any offset of its choosing in the tile's panel), with no
// register staging. A stage holds 64 K values of the tile's 256 x rows and 256 w rows (128 bytes a row, so the DMA of
// a row reads whole 128-byte lines; 32-wide stages, which read half lines, ran 3 % slower), two stages (128 KB), one
// barrier a stage: the DMA of stage q + 1 goes out in the first 16 MFMA slots after barrier q, the fragment reads one
// every other slot, a K step ahead of their MFMAs. LDS rows are 128 bytes; the 16-byte run c of row r sits at
// position c ^ ((r / 2) % 8), so the 16 lanes of a ds_read_b128 (16 consecutive rows, one run) hit 64 distinct banks.
// A DMA instruction writes 8 rows (1 KB), lane l taking row l / 8 at position l % 8.
constexpr int kEK = 64;

__device__ __forceinline__ uint32_t epos(uint32_t row, uint32_t run) { return row * kEK + ((run ^ ((row >> 1) & 7u)) << 3); }

__global__ __launch_bounds__(256, 1) void proj_dma(const ProjParams a)
{
    __shared__ __attribute__((aligned(16))) __bf16 as[2][kBN * kEK];
    __shared__ __attribute__((aligned(16))) __bf16 bs[2][kBN * kEK];
    uint32_t tm, tn;
    if (!tile_of(a, tm, tn))
        return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c32 = lane & 31;
    const uint32_t t0 = tm * kBN, n0 = tn * kBN;
    const __bf16* x = static_cast<const __bf16*>(a.x);
    uint32_t xo[8], wo[8];
    #pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t row = 64 * w + 8 * i + (lane >> 3), run = (lane & 7) ^ ((row >> 1) & 7);
        xo[i] = (min(t0 + row, a.t - 1) - t0) * a.ldx * 2 + 16 * run;
        wo[i] = (min(n0 + row, a.n - 1) - n0) * a.k * 2 + 16 * run;
    }
    const u32x4 xrs = panel_rsrc(x + (size_t)t0 * a.ldx, a.t - t0, a.ldx);
    const u32x4 wrs = panel_rsrc(a.w + (size_t)n0 * a.k, a.n - n0, a.k);
    const uint32_t wl = __builtin_amdgcn_readfirstlane(64 * w * kEK * 2);  // this wave's first row, LDS bytes
    // The DMA is issued as inline asm: the compiler, seeing the builtin, waits for every DMA in flight before any LDS
    // read (it cannot tell the stages apart). Here the only waits are the stage barriers'. M0 (the DMA's LDS base) is
    // listed as clobbered; nothing else in this kernel uses it.
    auto dma = [&](uint32_t voff, uint32_t soff, u32x4 rs, uint32_t lds) __attribute__((always_inline)) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff),
                     "s"(rs), "s"(soff)
                     : "memory", "m0");
#pragma clang diagnostic pop
    };
    const uint32_t abase = (uint32_t)(uintptr_t)&as[0][0] + wl, bbase = (uint32_t)(uintptr_t)&bs[0][0] + wl;
    // DMA instruction i (0 .. 15) of K stage q (values 64 q .. 64 q + 63) into LDS stage q % 2: x piece i / 2 (8 rows)
    // for even i, w piece i / 2 for odd
    auto dma1 = [&](uint32_t q, int i) __attribute__((always_inline)) {
        const uint32_t so = 2 * kEK * q, st = (q & 1) * (kBN * kEK * 2) + 1024 * (i / 2);
        if (i % 2 == 0)
            dma(xo[i / 2], so, xrs, abase + st);
        else
            dma(wo[i / 2], so, wrs, bbase + st);
    };
    f32x16 acc[4][4];
    #pragma unroll
    for (int bi = 0; bi < 4; ++bi)
        #pragma unroll
        for (int bj = 0; bj < 4; ++bj)
            acc[bi][bj] = f32x16{};
    const uint32_t ra = (w >> 1) * 128, rb = (w & 1) * 128;
    struct Frag {
        bf16x8 x[4], w[4];
    };
    // pieces 0 .. 7 of a fragment: x0, w0, w1, w2, w3, x1, x2, x3, the order the MFMAs (bi outer, bj inner) use them
    auto read1 = [&](Frag& f, uint32_t st, int kk, int piece) __attribute__((always_inline)) {
        const uint32_t rn = 2 * kk + g;
        if (piece == 0 || piece >= 5) {
            const int bi = piece == 0 ? 0 : piece - 4;
            f.x[bi] = *reinterpret_cast<const bf16x8*>(as[st] + epos(ra + 32 * bi + c32, rn));
        } else {
            const int bj = piece - 1;
            f.w[bj] = *reinterpret_cast<const bf16x8*>(bs[st] + epos(rb + 32 * bj + c32, rn));
        }
    };
    // 16 MFMAs on `use`; the reads of `next` (LDS stage st, K step kk of its four) on the even slots; with DMA, the 16
    // instructions of K stage q, one a slot
    auto half = [&](const Frag& use, Frag& next, uint32_t st, int kk, auto DMA, uint32_t q) __attribute__((always_inline)) {
        #pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[i / 4][i % 4] = Elem<__bf16>::mfma32(use.x[i / 4], use.w[i % 4], acc[i / 4][i % 4]);
            __builtin_amdgcn_sched_barrier(0);
            if (i % 2 == 0 && kk >= 0)
                read1(next, st, kk, i / 2);
            if constexpr (decltype(DMA)::value)
                dma1(q, i);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using Y = std::true_type;
    using N = std::false_type;
    const uint32_t nq = a.k / kEK;  // >= 1
    Frag fa, fb;
    #pragma unroll
    for (int i = 0; i < 16; ++i)
        dma1(0, i);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    #pragma unroll
    for (int i = 0; i < 8; ++i)
        read1(fa, 0, 0, i);
    if (nq > 1) {
        #pragma unroll
        for (int i = 0; i < 16; ++i)
            dma1(1, i);
    }
    __builtin_amdgcn_sched_barrier(0);
    half(fa, fb, 0, 1, N{}, 0);
    half(fb, fa, 0, 2, N{}, 0);
    half(fa, fb, 0, 3, N{}, 0);
    // K stage q: its LDS stage has landed (this wave's DMA by the wait, every wave's by the barrier) and the reads of
    // stage q - 1 are done, so stage q + 1 goes to the other LDS stage while the last K step of q - 1 and the first
    // three of q run. The last K stage has nothing to fetch.
    uint32_t q = 1;
    for (; q + 1 < nq; ++q) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t st = q & 1;
        half(fb, fa, st, 0, Y{}, q + 1);
        half(fa, fb, st, 1, N{}, 0);
        half(fb, fa, st, 2, N{}, 0);
        half(fa, fb, st, 3, N{}, 0);
    }
    if (q < nq) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t st = q & 1;
        half(fb, fa, st, 0, N{}, 0);
        half(fa, fb, st, 1, N{}, 0);
        half(fb, fa, st, 2, N{}, 0);
        half(fa, fb, st, 3, N{}, 0);
    }
    half(fb, fa, 0, -1, N{}, 0);
    #pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
        const uint32_t c = n0 + rb + 32 * bj + c32;
        if (c >= a.n)
            continue;
        #pragma unroll
        for (int bi = 0; bi < 4; ++bi)
            #pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = t0 + ra + 32 * bi + 8 * (r >> 2) + 4 * g + (r & 3);
                if (row < a.t)
                    a.y[(size_t)row * a.ldy + c] = acc[bi][bj][r];
            }
    }
}

template <int BM, bool XF32, bool SPLIT>
void launch_proj(ProjParams p, hipStream_t stream)
{
    p.tiles_m = (p.t + BM - 1) / BM;
    p.tiles_n = (p.n + kBN - 1) / kBN;
    p.tiles = p.tiles_m * p.tiles_n;
    p.per_xcd = (p.tiles + 7) / 8;
    hipLaunchKernelGGL((proj_tiles<BM, XF32, SPLIT>), dim3(8 * p.per_xcd), dim3(256), 0, stream, p);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mako

using namespace mako;

extern "C" int mako_proj_bf16(const mako_gemm_args* a, int x_dtype, int split, const void* w, const void* x, float* y,
                              void* stream)
{
    if (!a || !w || !x || !y)
        return fail(MAKO_EINVAL, "proj: a null argument");
    if (x_dtype != MAKO_F32 && x_dtype != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "proj: activations of type %d (f32 or bf16)", x_dtype);
    if (a->k == 0 || a->k % 64)
        return fail(MAKO_EINVAL, "BF16 %ux%u: k must be a multiple of 64", a->k, a->n);
    if (a->row_bytes && a->row_bytes != 2 * a->k)
        return fail(MAKO_EINVAL, "proj: BF16 rows of %u values are %u bytes, not %u", a->k, 2 * a->k, a->row_bytes);
    if (split && x_dtype != MAKO_F32)
        return fail(MAKO_EINVAL, "proj: the bf16 split needs f32 activations");
    const uint32_t ldx = a->ldx ? a->ldx : a->k, ldy = a->ldy ? a->ldy : a->n;
    if (ldx < a->k || ldy < a->n)
        return fail(MAKO_EINVAL, "proj: rows of %u (x) and %u (y) are shorter than k = %u and n = %u", ldx, ldy, a->k,
                    a->n);
    if (!al16(w) || !al16(x) || ldx % 8)
        return fail(MAKO_EINVAL, "proj: w and x must be 16-byte aligned and ldx a multiple of 8");
    if ((uint64_t)a->t * ldx > 0xffffffffu || (uint64_t)a->n * a->k > 0xffffffffu)
        return fail(MAKO_EINVAL, "proj: %u x %u activations or %u x %u weights exceed 2^32 elements", a->t, ldx, a->n,
                    a->k);
    if (a->t == 0 || a->n == 0)
        return ok();
    ProjParams p{static_cast<const __bf16*>(w), x, y, a->t, a->k, a->n, ldy, ldx, 0, 0, 0, 0};
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (x_dtype == MAKO_BF16) {
        // a tile's DMA addresses its panels by 32-bit offsets (up to 256 rows, a row's k values, a margin)
        const auto span = [&](uint32_t rows, uint32_t ld) {
            return (uint64_t)std::min(rows, 256u) * ld * 2 + 2ull * a->k + 128;
        };
        if (span(a->t, ldx) > 0xffffffffu || span(a->n, a->k) > 0xffffffffu)
            return fail(MAKO_EINVAL, "proj: rows of %u (x) and %u (w) values are too long for 32-bit tile offsets", ldx,
                        a->k);
        p.tiles_m = (p.t + kBN - 1) / kBN;
        p.tiles_n = (p.n + kBN - 1) / kBN;
        p.tiles = p.tiles_m * p.tiles_n;
        p.per_xcd = (p.tiles + 7) / 8;
        hipLaunchKernelGGL(proj_dma, dim3(8 * p.per_xcd), dim3(256), 0, s, p);
    }
    else if (!split)
        launch_proj<256, true, false>(p, s);
    else
        launch_proj<128, true, true>(p, s);
    return check_launch("proj");
}
