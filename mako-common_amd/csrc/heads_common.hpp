// The head producers' pieces that attention from projection rows (attn_rows.hip) shares with mako_heads
// (heads.hip): the launch parameters, the host checks, and the per-item body of the vector path.
#pragma once

#include "device.hpp"

namespace mako {

constexpr int kItems = 4;    // (token, head) items a workgroup, one a wave
constexpr int kMaxDim = 256;
constexpr int kTok = 2;      // tokens a heads_vec item

struct HeadsParams {
    const float* x;
    const float2* cs;
    const float* w;
    const int32_t* map;
    void* y;
    uint32_t rows, ld, col0, stride, dim, heads, n_pad, row0, rope, rot;
    float eps;
    uint32_t n_clear;  // rows cleared a head
    uint64_t n_prod;   // heads * rows
    uint64_t n_items;  // n_prod + heads * n_clear
};


// Host side. heads_check: MAKO_OK when mako_heads accepts *a with these buffers (else the error, recorded).
// heads_vec_takes: whether the vector path covers the call. heads_params: the launch parameters, items counted for
// heads_tiles (one a (token, head)) or, with vec, for heads_vec (kTok tokens of 64 / (dim / 4) heads).
int heads_check(const mako_heads_args* a, mako_dtype out, const float* x, const float* cs, const float* w,
                const void* y);
bool heads_vec_takes(const mako_heads_args* a, const float* x, const float* cs, const float* w, const void* y);
HeadsParams heads_params(const mako_heads_args* a, const float* x, const float* cs, const float* w,
                         const int32_t* map, void* y, bool vec);

namespace {

// The vector path (dim 64, 128 or 256; x rows, columns and the angle table 16-byte aligned; rope 2, or rope 1
// with rot a multiple of 8): a lane holds 4 consecutive values of a head (one 16-byte load, one 8-byte store),
// LPH = dim / 4 lanes a head, 64 / LPH heads of a token a wave, and a wave takes kTok consecutive tokens of its
// heads with all their loads in flight together. The norm is a reduction over the head's lanes; under rope 1 the
// partner values of a lane sit rot / 8 lanes away in the same head and come by lane shuffle; under rope 2 they are
// lane-local.
// heads_vec_item: item `it` (a wave's; heads_vec runs kItems a workgroup, one a wave).
template <class TO, int LPH>
__device__ __forceinline__ void heads_vec_item(const HeadsParams& p, uint64_t it)
{
    constexpr int HPW = 64 / LPH;  // heads a wave
    const uint32_t lane = threadIdx.x & 63, r = lane % LPH, hw = lane / LPH;
    const uint32_t hg_n = (p.heads + HPW - 1) / HPW;
    if (it >= p.n_items)
        return;  // (no barriers below)
    // Items: token blocks of produced rows (n_prod of them), then token blocks of padding rows.
    const bool prod = it < p.n_prod;
    const uint64_t c = prod ? it : it - p.n_prod;
    const uint32_t h = (uint32_t)(c % hg_n) * HPW + hw;
    const uint32_t t0 = (uint32_t)(c / hg_n) * kTok;  // first token (or padding row) of the block
    const uint32_t n_t = prod ? p.rows : p.n_clear;
    if (h >= p.heads)
        return;
    const uint32_t i0 = 4 * r;  // this lane's first value
    f32x4 v[kTok];
    uint32_t src[kTok];
    bool live[kTok];
    #pragma unroll
    for (int k = 0; k < kTok; ++k) {
        const uint32_t t = t0 + k;
        const int32_t m = !prod || t >= n_t ? -1 : p.map ? p.map[t] : (int32_t)t;
        live[k] = m >= 0;
        src[k] = live[k] ? (uint32_t)m : 0u;
        v[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (live[k])
            v[k] = *reinterpret_cast<const f32x4*>(p.x + (size_t)src[k] * p.ld + p.col0 + (size_t)h * p.stride + i0);
    }
    f32x4 wv = {1.0f, 1.0f, 1.0f, 1.0f};
    if (p.eps > 0.0f)
        wv = *reinterpret_cast<const f32x4*>(p.w + i0);
    #pragma unroll
    for (int k = 0; k < kTok; ++k) {
        if (p.eps > 0.0f) {
            float ss = v[k][0] * v[k][0] + v[k][1] * v[k][1] + v[k][2] * v[k][2] + v[k][3] * v[k][3];
            #pragma unroll
            for (int o = LPH / 2; o >= 1; o >>= 1)
                ss += __shfl_xor(ss, o);
            const float inv = rsqrtf(ss / (float)p.dim + p.eps);
            #pragma unroll
            for (int e = 0; e < 4; ++e)
                v[k][e] *= inv * wv[e];
        }
        if (p.rope == 1) {
            const uint32_t half = p.rot / 2, dl = half / 4;  // partner lane distance
            const bool first = i0 < half, rot = i0 < p.rot;
            const int src_lane = (int)lane + (first ? (int)dl : -(int)dl);
            f32x4 o;
            #pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = __shfl(v[k][e], rot ? src_lane : (int)lane);
            if (live[k] && rot) {
                const uint32_t pr = first ? i0 : i0 - half;
                const f32x4* c2 = reinterpret_cast<const f32x4*>(p.cs + (size_t)src[k] * half + pr);
                const f32x4 ca = c2[0], cb = c2[1];  // (c, s) of pairs pr .. pr + 3
                const float cc[4] = {ca[0], ca[2], cb[0], cb[2]}, sn[4] = {ca[1], ca[3], cb[1], cb[3]};
                #pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[k][e] = first ? v[k][e] * cc[e] - o[e] * sn[e] : v[k][e] * cc[e] + o[e] * sn[e];
            }
        } else if (p.rope == 2 && live[k] && i0 < p.rot) {
            const f32x4 cq = *reinterpret_cast<const f32x4*>(p.cs + (size_t)src[k] * (p.rot / 2) + i0 / 2);
            const float u0 = v[k][0], w0 = v[k][1], u1 = v[k][2], w1 = v[k][3];
            v[k][0] = u0 * cq[0] - w0 * cq[1];
            v[k][1] = w0 * cq[0] + u0 * cq[1];
            v[k][2] = u1 * cq[2] - w1 * cq[3];
            v[k][3] = w1 * cq[2] + u1 * cq[3];
        }
        const uint32_t t = t0 + k;
        if (t < n_t) {
            const uint32_t yrow = p.row0 + (prod ? 0u : p.rows) + t;
            TO* yr = static_cast<TO*>(p.y) + ((size_t)h * p.n_pad + yrow) * p.dim + i0;
            store4<TO>(yr, v[k][0], v[k][1], v[k][2], v[k][3]);
        }
    }
}

}  // namespace
}  // namespace mako
