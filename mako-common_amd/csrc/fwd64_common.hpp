// Pieces the r64 attention kernels share (attn_fwd64.hip: dense, attn_sparse64.hip: block-sparse): the LDS tile
// geometry their generated stream assumes (gen_attn_fwd64.py), the K slot order and V unit order, and the f16 V^T
// tile images flash_fwd_d256 stages from. Internal linkage: each file gets its own copies.
#pragma once

#include "attn_fwd64_asm.inc"
#include "device.hpp"

namespace mako {
namespace {

constexpr uint32_t kNBuf = MAKO_FWD64_NBUF; // LDS tile buffers

// The LDS tile geometry of the stream for heads of D (128 or 64; gen_attn_fwd64.set_dim).
template <int D>
struct R64 {
    static constexpr uint32_t kKRow = 2 * D + 16;                    // LDS bytes of a K row: 2 D + 16 of padding
    static constexpr uint32_t kKTile = 64 * kKRow;                   // a K tile of 64 keys (17 or 9 KiB)
    static constexpr uint32_t kVRow = 2 * D;                         // LDS bytes of a V row (r64 stream)
    static constexpr uint32_t kVTile = D * 64 * 2;                   // a V tile: 64 rows (r64), or a V^T image
                                                                     // tile of D head dims x 64 keys in f16 (d256)
    static constexpr uint32_t kNKP = (kKTile / 1024 - 1) / 4;        // K image KiB pieces a wave DMAs: w + 4 m
    static constexpr uint32_t kLdsBytes = kNBuf * (kKTile + kVTile);
};
constexpr uint32_t kKRow = R64<128>::kKRow;
constexpr uint32_t kKTile = R64<128>::kKTile;
constexpr uint32_t kVTile = R64<128>::kVTile;
constexpr uint32_t kLdsBytes = R64<128>::kLdsBytes;

__device__ __forceinline__ uint32_t slot_of(uint32_t row)
{
    return (row & ~12u) | ((row & 4u) << 1) | ((row & 8u) >> 1);
}

// Where 32-byte unit u (head dims 16 u .. 16 u + 15) of V row k sits in that row's LDS image (the r64 stream): the
// unit's low two bits XOR the row's, so the four rows a transpose read's 16-lane group addresses (k % 4 = 0 .. 3, one
// unit each) cover the 128 bytes of banks once (gen_attn_fwd64.v_unit). Its own inverse for a given row.
__device__ __forceinline__ uint32_t v_unit(uint32_t u, uint32_t k) { return (u & ~3u) | ((u & 3u) ^ (k & 3u)); }

// The V byte, relative to a 1 KiB V image piece, that lane's LDS slot holds (byte 16 lane of the piece: row r,
// unit p, half): unit v_unit(p, r) of that row. Pieces start on a multiple of 4 rows, so r % 4 is the tile row's.
template <int D>
__device__ __forceinline__ uint32_t vd_of(uint32_t lane)
{
    constexpr uint32_t rowb = 2 * D;
    const uint32_t b = 16 * lane, r = b / rowb, pos = b % rowb;
    return r * rowb + 32 * v_unit(pos / 32, r) + 16 * ((pos / 16) & 1u);
}

// XOR swizzle of the 16-byte key chunks in row d of a V^T tile: a bijection on d mod 8 (eight consecutive rows read
// one chunk column from eight distinct bank groups) that depends on d mod 32 only (the four 32-row blocks of a
// fragment read differ by an immediate offset).
__device__ __forceinline__ uint32_t vt_swz(uint32_t d) { return (d & 7u) ^ ((d >> 3) & 3u); }

// The stores of a vt_image thread: x[i][m] holds head dims 8 e + 2 m, + 1 of key 8 c + i (f16 pairs); it writes
// the eight 16-byte chunks of head dims 8 e .. 8 e + 7 (keys 8 c .. 8 c + 7) of the tile at dst.
template <int D>
__device__ __forceinline__ void vt_store_block(uint32_t* dst, const uint32_t (&x)[8][4], uint32_t c, uint32_t e)
{
    #pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {  // head dim d = 8 e + j: keys 8 c + 2 q, + 1 in dword q
        const uint32_t d = 8 * e + j, m = j >> 1, sh = 16 * (j & 1);
        u32x4 out;
        #pragma unroll
        for (uint32_t q = 0; q < 4; ++q)
            out[q] = ((x[2 * q][m] >> sh) & 0xffffu) | (((x[2 * q + 1][m] >> sh) & 0xffffu) << 16);
        *reinterpret_cast<u32x4*>(dst + d * 32 + 4 * (c ^ vt_swz(d))) = out;
    }
}

// f16 bits of a pair of T values (bf16 rounds toward zero, as the attention kernels' staging does).
template <class T>
__device__ __forceinline__ uint32_t f16_pair_of(uint32_t t2)
{
    if constexpr (__is_same(T, __bf16)) {
        const float lo = __builtin_bit_cast(float, t2 << 16);
        const float hi = __builtin_bit_cast(float, t2 & 0xffff0000u);
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    } else {
        return t2;
    }
}

// The V^T tile images: tile t of kv head h is D x 128 bytes (16 or 8 KiB), row d (head dim) of 128 bytes holding keys
// 64 t .. 64 t + 63 in f16, the 16-byte chunk of keys 64 t + 8 c .. + 7 at slot c ^ vt_swz(d): the LDS layout the
// kernel reads, so its staging copies tiles unchanged. Keys >= n_k are zero. bf16 becomes f16 rounding toward zero
// (v_cvt_pkrtz), as the staging of the other attention kernels does. D threads make a tile: thread (c, e) loads keys
// 8 c .. 8 c + 7, head dims 8 e .. 8 e + 7 (eight 16-byte loads; D / 8 threads cover a key row), transposes the
// 8 x 8 block in registers and stores the eight 16-byte chunks of its head dims.
// vt_image_tiles: the 256 / D tiles (256 / D) bx .. of kv head kvh (a workgroup of 256 threads).
template <class T, int D = 128>
__device__ __forceinline__ void vt_image_tiles(const T* v, uint32_t* img, uint32_t n_k, uint32_t k_pad, uint32_t n_vt,
                                               uint32_t bx, uint32_t kvh)
{
    constexpr uint32_t CPR = D / 8;  // 16-byte chunks of a key row
    const uint32_t tile = bx * (256 / D) + threadIdx.x / D;
    if (tile >= n_vt)
        return;
    const uint32_t t = threadIdx.x % D, e = t % CPR, c = t / CPR;
    const u32x4* src = reinterpret_cast<const u32x4*>(v + ((size_t)kvh * k_pad + (size_t)tile * 64 + 8 * c) * D) + e;
    uint32_t x[8][4];  // x[i][m]: head dims 8 e + 2 m, + 1 of key 8 c + i (f16 pairs)
    #pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        u32x4 r = u32x4{0u, 0u, 0u, 0u};
        if (tile * 64 + 8 * c + i < n_k)
            r = __builtin_nontemporal_load(src + CPR * i);
        #pragma unroll
        for (uint32_t m = 0; m < 4; ++m)
            x[i][m] = f16_pair_of<T>(r[m]);
    }
    vt_store_block<D>(img + ((size_t)kvh * n_vt + tile) * (D * 32), x, c, e);
}

// vt_rows_tiles: the same images straight from fp32 rows (attention from projection rows): value d of key j of kv
// head kvh is x[j * ld + col0 + kvh * stride + d], rounded to T to nearest even (as mako_heads writes a value tile)
// and then to f16 as vt_image_tiles converts T, so the images equal vt_image's of the tiles mako_heads would write.
// Thread (c, e) loads two 16-byte pieces of each of its eight keys. x, ld, col0 and stride: 16-byte aligned.
template <class T, int D>
__device__ __forceinline__ void vt_rows_tiles(const float* xr, uint32_t ld, uint32_t col0, uint32_t stride,
                                              uint32_t* img, uint32_t n_k, uint32_t n_vt, uint32_t bx, uint32_t kvh)
{
    constexpr uint32_t CPR = D / 8;
    const uint32_t tile = bx * (256 / D) + threadIdx.x / D;
    if (tile >= n_vt)
        return;
    const uint32_t t = threadIdx.x % D, e = t % CPR, c = t / CPR;
    const float* src = xr + (size_t)(tile * 64 + 8 * c) * ld + col0 + (size_t)kvh * stride + 8 * e;
    uint32_t x[8][4];
    #pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        f32x4 a = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, b = a;
        if (tile * 64 + 8 * c + i < n_k) {
            a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + (size_t)i * ld));
            b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + (size_t)i * ld + 4));
        }
        x[i][0] = f16_pair_of<T>(Elem<T>::pack2(a[0], a[1]));
        x[i][1] = f16_pair_of<T>(Elem<T>::pack2(a[2], a[3]));
        x[i][2] = f16_pair_of<T>(Elem<T>::pack2(b[0], b[1]));
        x[i][3] = f16_pair_of<T>(Elem<T>::pack2(b[2], b[3]));
    }
    vt_store_block<D>(img + ((size_t)kvh * n_vt + tile) * (D * 32), x, c, e);
}

template <class T, int D = 128>
__global__ __launch_bounds__(256) void vt_image(const T* v, uint32_t* img, uint32_t n_k, uint32_t k_pad, uint32_t n_vt)
{
    vt_image_tiles<T, D>(v, img, n_k, k_pad, n_vt, blockIdx.x, blockIdx.y);
}

// A raw buffer descriptor (gfx9 layout) over `bytes` bytes at `base`: offsets at or past the end load zeros and drop
// stores.
__device__ __forceinline__ u32x4 rsrc_of(const void* base, uint32_t bytes)
{
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

}  // namespace
}  // namespace mako
