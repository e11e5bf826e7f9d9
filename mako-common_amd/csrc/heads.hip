// Head tiles from fp32 rows (the step before attention): slice each head out of the token rows, RMS-norm it
// (times a weight), rotate it by the rotary angle table, and write it in f16 or bf16 as the [heads][n_pad][dim]
// tiles the attention kernels read; optionally through a row map, and with the padding rows zeroed.
//
// Semantics of the reference's producers (src/kernels/ops.metal): heads_half (:21-42) - a pair (u, v) becomes
// (u c - v s, v c + u s) with (c, s) = cs[t][i], pairing value i with i + dim / 2 (rope 1) or 2i with 2i + 1
// (rope 2); heads_clear (:44-52) - rows [T, n_pad) zeroed; heads_norm_half (:376-407) - x * rsqrt(mean(x^2) +
// eps) * w before the rotation; heads_partial (:587-620) - any head stride, dim a multiple of 32 up to 256, only the
// first rot values rotate (i with i + rot / 2, angles cs[t][i % (rot / 2)]), the norm optional, and y row t taken
// from x row map[t] (a zero row where map[t] < 0).
//
// The design is this one's own. Bound: HBM (4 bytes read and 2 written a value). Two kernels: heads_vec for the
// common shapes (heads of 64, 128 or 256 with 16-byte aligned rows; see there), and heads_tiles for the rest: one
// wave a (token, head) item, four items a workgroup, lane l holding values l, l + 64, ... (each load and store
// instruction of a wave covers one contiguous run of the row), the sum of squares a wave reduction, and the
// rotation partner of a value through the wave's own LDS row; items run head-major, so consecutive waves write
// consecutive tile rows.
#include "heads_common.hpp"

namespace mako {
namespace {

template <class TO>
__device__ __forceinline__ void store1(TO* p, float v);
template <>
__device__ __forceinline__ void store1<_Float16>(_Float16* p, float v)
{
    *p = (_Float16)v;  // round to nearest even
}
template <>
__device__ __forceinline__ void store1<__bf16>(__bf16* p, float v)
{
    *p = (__bf16)v;  // round to nearest even
}

template <class TO>
__global__ __launch_bounds__(kItems * 64) void heads_tiles(const HeadsParams p)
{
    __shared__ float vals[kItems][kMaxDim];
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint64_t it = (uint64_t)blockIdx.x * kItems + w;
    const uint32_t S = (p.dim + 63) / 64;  // values a lane

    // The item: a produced row (head h, token t, from x row src), or a padding row cleared, or nothing.
    uint32_t h = 0, yrow = 0, src = 0;
    bool prod = false, zero = true;
    if (it < p.n_prod) {
        h = (uint32_t)(it / p.rows);
        const uint32_t t = (uint32_t)(it % p.rows);
        yrow = p.row0 + t;
        prod = true;
        if (p.map) {
            const int32_t m = p.map[t];
            zero = m < 0;
            src = zero ? 0u : (uint32_t)m;
        } else {
            zero = false;
            src = t;
        }
    } else if (it < p.n_items) {
        const uint64_t c = it - p.n_prod;
        h = (uint32_t)(c / p.n_clear);
        yrow = p.row0 + p.rows + (uint32_t)(c % p.n_clear);
    }
    const bool live = prod && !zero;

    float v[kMaxDim / 64];
    const float* xr = p.x + (size_t)src * p.ld + p.col0 + (size_t)h * p.stride;
    #pragma unroll
    for (int s = 0; s < kMaxDim / 64; ++s) {
        const uint32_t i = lane + 64 * s;
        v[s] = (live && s < (int)S && i < p.dim) ? xr[i] : 0.0f;
    }
    if (p.eps > 0.0f) {
        float ss = 0.0f;
        #pragma unroll
        for (int s = 0; s < kMaxDim / 64; ++s)
            ss += v[s] * v[s];
        #pragma unroll
        for (int o = 32; o >= 1; o >>= 1)
            ss += __shfl_xor(ss, o);
        const float inv = rsqrtf(ss / (float)p.dim + p.eps);
        #pragma unroll
        for (int s = 0; s < kMaxDim / 64; ++s) {
            const uint32_t i = lane + 64 * s;
            if (live && s < (int)S && i < p.dim)
                v[s] *= inv * p.w[i];
        }
    }
    if (p.rope) {
        // (uniform over the launch, so every wave of the workgroup reaches the barrier)
        #pragma unroll
        for (int s = 0; s < kMaxDim / 64; ++s) {
            const uint32_t i = lane + 64 * s;
            if (s < (int)S && i < p.dim)
                vals[w][i] = v[s];
        }
        __syncthreads();
        const uint32_t half = p.rot / 2;
        const float2* cr = p.cs + (size_t)src * half;
        #pragma unroll
        for (int s = 0; s < kMaxDim / 64; ++s) {
            const uint32_t i = lane + 64 * s;
            if (!live || s >= (int)S || i >= p.rot)
                continue;
            const bool first = p.rope == 1 ? i < half : (i & 1u) == 0;
            const uint32_t j = p.rope == 1 ? (first ? i + half : i - half) : (i ^ 1u);
            const uint32_t pr = p.rope == 1 ? (first ? i : i - half) : (i >> 1);
            const float2 c = cr[pr];
            const float o = vals[w][j];
            v[s] = first ? v[s] * c.x - o * c.y : v[s] * c.x + o * c.y;
        }
    }
    if (it < p.n_items) {
        TO* yr = static_cast<TO*>(p.y) + ((size_t)h * p.n_pad + yrow) * p.dim;
        #pragma unroll
        for (int s = 0; s < kMaxDim / 64; ++s) {
            const uint32_t i = lane + 64 * s;
            if (s < (int)S && i < p.dim)
                store1<TO>(yr + i, live ? v[s] : 0.0f);
        }
    }
}

template <class TO, int LPH>
__global__ __launch_bounds__(kItems * 64) void heads_vec(const HeadsParams p)
{
    heads_vec_item<TO, LPH>(p, (uint64_t)blockIdx.x * kItems + (threadIdx.x >> 6));
}

}  // namespace
}  // namespace mako

using namespace mako;

namespace mako {

int heads_check(const mako_heads_args* a, mako_dtype out, const float* x, const float* cs, const float* w,
                const void* y)
{
    if (!a || !y || (a->rows && !x))
        return fail(MAKO_EINVAL, "heads: a null argument");
    if (out != MAKO_F16 && out != MAKO_BF16)
        return fail(MAKO_EUNSUPPORTED, "heads: output type %d (f16 or bf16)", (int)out);
    if (a->dim == 0 || a->dim > kMaxDim || a->dim % 32 || a->rot % 2)
        return fail(MAKO_EINVAL, "heads: heads of %u with %u rotated", a->dim, a->rot);
    if (a->rope > 2 || (a->rope && (a->rot == 0 || a->rot > a->dim || !cs)))
        return fail(MAKO_EINVAL, "heads: rope %u over %u of %u values%s", a->rope, a->rot, a->dim,
                    a->rope && !cs ? " without an angle table" : "");
    if (a->eps < 0.0f || a->eps != a->eps || (a->eps > 0.0f && !w))
        return fail(MAKO_EINVAL, "heads: eps %g%s", (double)a->eps, a->eps > 0.0f && !w ? " without a weight" : "");
    if ((uint64_t)a->row0 + a->rows > a->n_pad)
        return fail(MAKO_EINVAL, "heads: rows %u from %u exceed %u", a->rows, a->row0, a->n_pad);
    if (a->rows && (uint64_t)a->col0 + (uint64_t)(a->heads ? a->heads - 1 : 0) * a->stride + a->dim > a->ld)
        return fail(MAKO_EINVAL, "heads: %u heads of %u at %u apart from column %u exceed rows of %u", a->heads,
                    a->dim, a->stride, a->col0, a->ld);
    const uint32_t n_clear = a->clear ? a->n_pad - a->row0 - a->rows : 0u;
    const uint64_t n_items = (uint64_t)a->heads * a->rows + (uint64_t)a->heads * n_clear;
    if ((n_items + kItems - 1) / kItems > 0x7fffffffu)
        return fail(MAKO_EINVAL, "heads: %llu items exceed the grid", (unsigned long long)n_items);
    return MAKO_OK;
}

bool heads_vec_takes(const mako_heads_args* a, const float* x, const float* cs, const float* w, const void* y)
{
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    return (a->dim == 64 || a->dim == 128 || a->dim == 256) && a->ld % 4 == 0 && a->col0 % 4 == 0 &&
           a->stride % 4 == 0 && al16(x) && (!w || al16(w)) && (!cs || al16(cs)) && al16(y) &&
           (a->rope != 1 || a->rot % 8 == 0) && (a->rope != 2 || a->rot % 4 == 0);
}

HeadsParams heads_params(const mako_heads_args* a, const float* x, const float* cs, const float* w,
                         const int32_t* map, void* y, bool vec)
{
    const uint32_t n_clear = a->clear ? a->n_pad - a->row0 - a->rows : 0u;
    HeadsParams p{x, reinterpret_cast<const float2*>(cs), w, map, y, a->rows, a->ld, a->col0, a->stride, a->dim,
                  a->heads, a->n_pad, a->row0, a->rope, a->rope ? a->rot : 0u, a->eps, n_clear, 0, 0};
    if (vec) {
        const uint32_t hpw = 64 / (a->dim / 4), hg_n = (a->heads + hpw - 1) / hpw;
        p.n_prod = (uint64_t)((a->rows + kTok - 1) / kTok) * hg_n;
        p.n_items = p.n_prod + (uint64_t)((n_clear + kTok - 1) / kTok) * hg_n;
    } else {
        p.n_prod = (uint64_t)a->heads * a->rows;
        p.n_items = p.n_prod + (uint64_t)a->heads * n_clear;
    }
    return p;
}

}  // namespace mako

extern "C" int mako_heads(const mako_heads_args* a, mako_dtype out, const float* x, const float* cs, const float* w,
                          const int32_t* map, void* y, void* stream)
{
    if (const int e = heads_check(a, out, x, cs, w, y))
        return e;
    const bool vec = heads_vec_takes(a, x, cs, w, y);
    const HeadsParams p = heads_params(a, x, cs, w, map, y, vec);
    if (p.n_items == 0)
        return ok();
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((uint32_t)((p.n_items + kItems - 1) / kItems));
    if (vec) {
        if (out == MAKO_F16) {
            if (a->dim == 64)
                hipLaunchKernelGGL((heads_vec<_Float16, 16>), grid, dim3(kItems * 64), 0, s, p);
            else if (a->dim == 128)
                hipLaunchKernelGGL((heads_vec<_Float16, 32>), grid, dim3(kItems * 64), 0, s, p);
            else
                hipLaunchKernelGGL((heads_vec<_Float16, 64>), grid, dim3(kItems * 64), 0, s, p);
        } else {
            if (a->dim == 64)
                hipLaunchKernelGGL((heads_vec<__bf16, 16>), grid, dim3(kItems * 64), 0, s, p);
            else if (a->dim == 128)
                hipLaunchKernelGGL((heads_vec<__bf16, 32>), grid, dim3(kItems * 64), 0, s, p);
            else
                hipLaunchKernelGGL((heads_vec<__bf16, 64>), grid, dim3(kItems * 64), 0, s, p);
        }
        return check_launch("heads");
    }
    if (out == MAKO_F16)
        hipLaunchKernelGGL((heads_tiles<_Float16>), grid, dim3(kItems * 64), 0, s, p);
    else
        hipLaunchKernelGGL((heads_tiles<__bf16>), grid, dim3(kItems * 64), 0, s, p);
    return check_launch("heads");
}
