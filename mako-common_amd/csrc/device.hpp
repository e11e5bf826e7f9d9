// Device helpers shared by the attention kernels: vector types, the gfx950 MFMA wrappers per element type,
// conversions, and the error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mako_attn.h"

namespace mako {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Per input element type: the 8-wide operand of v_mfma_f32_32x32x16_{bf16,f16} and two floats packed into one
// dword (round to nearest even).
template <class T>
struct Elem;

template <>
struct Elem<__bf16> {
    using vec8 = bf16x8;
    static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c)
    {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi)
    {
        bf16x2 v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
};

template <>
struct Elem<_Float16> {
    using vec8 = f16x8;
    static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c)
    {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi)
    {
        f16x2 v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
};

// Output stores: four consecutive floats of one row as the output type.
template <class TO>
__device__ __forceinline__ void store4(TO* p, float a, float b, float c, float d);

template <>
__device__ __forceinline__ void store4<float>(float* p, float a, float b, float c, float d)
{
    *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}

template <>
__device__ __forceinline__ void store4<__bf16>(__bf16* p, float a, float b, float c, float d)
{
    *reinterpret_cast<u32x2*>(p) = u32x2{Elem<__bf16>::pack2(a, b), Elem<__bf16>::pack2(c, d)};
}

template <>
__device__ __forceinline__ void store4<_Float16>(_Float16* p, float a, float b, float c, float d)
{
    *reinterpret_cast<u32x2*>(p) = u32x2{Elem<_Float16>::pack2(a, b), Elem<_Float16>::pack2(c, d)};
}

template <class T>
__device__ __forceinline__ float to_float(T x)
{
    return (float)x;
}

// Element e (0..7) of a 16-byte chunk of 16-bit values, in the low 16 bits.
__device__ __forceinline__ uint32_t half_of(const u32x4& c, int e)
{
    const uint32_t w = c[e >> 1];
    return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

// Element e of chunk a and element e of chunk b (inputs of type T) as one dword of two f16 values. The P V
// product always runs in f16 (P in f16 has 11 significant bits, bf16 only 8); bf16 values convert exactly within
// f16's normal range, and round toward zero below it and saturate at +-65504 above it.
template <class T>
__device__ __forceinline__ uint32_t f16_pair(const u32x4& a, const u32x4& b, int e);

template <>
__device__ __forceinline__ uint32_t f16_pair<_Float16>(const u32x4& a, const u32x4& b, int e)
{
    return half_of(a, e) | (half_of(b, e) << 16);
}

template <>
__device__ __forceinline__ uint32_t f16_pair<__bf16>(const u32x4& a, const u32x4& b, int e)
{
    const uint32_t wa = a[e >> 1], wb = b[e >> 1];
    const float fa = __builtin_bit_cast(float, (e & 1) ? (wa & 0xffff0000u) : (wa << 16));
    const float fb = __builtin_bit_cast(float, (e & 1) ? (wb & 0xffff0000u) : (wb << 16));
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(fa, fb));
}

// A raw buffer resource over `bytes` bytes at `base`: loads at offsets past the end return zero (the gfx9
// range check), which masks rows past a tensor's valid extent without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off)
{
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}

// The same as a streaming (non-temporal) load, for data read once: it does not displace reused lines in the
// caches, and sustains more of HBM's read bandwidth than a plain load.
__device__ __forceinline__ u32x4 buffer_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off)
{
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 2));
}

// A 16-bit entry of a read-only device array at a wave-uniform index, read through the scalar cache (a dword
// load of the aligned dword holding it: that dword lies in the same page as the entry, so it is always mapped).
// Unlike a vector load, it does not wait behind the wave's outstanding vector-memory loads.
__device__ __forceinline__ uint32_t uniform_u16(const uint16_t* base, size_t i)
{
    typedef const __attribute__((address_space(4))) uint32_t const_u32;
    const uintptr_t a = reinterpret_cast<uintptr_t>(base + i);
    const uint32_t w = *reinterpret_cast<const_u32*>(a & ~(uintptr_t)3);
    return (a & 2) ? w >> 16 : w & 0xffffu;
}

// 2^x by v_exp_f32 alone (no denormal-range fix-up: results below 2^-126 flush to zero, which the softmax
// sums cannot tell apart).
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// acc + lo(x) + hi(x) for the two f16 halves of x, summed in f32 (v_dot2_f32_f16 against (1, 1)). Pass a whole
// register: when the operand was a dword extracted from a wider f16 vector, this compiler selected the vector's
// first dword instead (the half pair's offset lost).
__device__ __forceinline__ float sum_f16x2(uint32_t x, float acc)
{
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), f16x2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
}

// Marks a loaded value as arrived: the compiler waits for its load here, once, instead of treating it as still
// in flight inside a later loop (where the in-order vmcnt wait would also wait for that loop's prefetches).
template <class V>
__device__ __forceinline__ void settle(V& x)
{
    u32x4 u = __builtin_bit_cast(u32x4, x);
    asm volatile("" : "+v"(u));
    x = __builtin_bit_cast(V, u);
}

// The other half of a 64-lane wave (lane l <-> l ^ 32).
__device__ __forceinline__ float swap_halves(float x)
{
    return __shfl_xor(x, 32);
}

__device__ __forceinline__ uint32_t as_u32(float x) { return __builtin_bit_cast(uint32_t, x); }

}  // namespace mako

// ---- host side: error plumbing of the C ABI ----------------------------------------------------------------------

namespace mako {

// Records the message for mako_last_error() and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message; returns MAKO_OK.
int ok();
// The code of the calling thread's last fail() (MAKO_OK after ok()).
int last_code();
// MAKO_OK, or MAKO_EHIP with the launch error recorded (hipGetLastError after a launch).
int check_launch(const char* what);
// Compute units of the current device (cached per device and thread); 0 when there is none.
uint32_t device_cus();

// Workspaces the library keeps for callers that pass none: one buffer per (purpose, device, stream), grown (stream-
// ordered) when a call needs more. Calls on one stream are ordered by the stream and calls on different streams use
// different buffers, so no call waits on the host or inserts a GPU-side wait. A stream's buffers stay until
// mako_attn_release(stream) frees them (a stream destroyed without it leaves them to a later stream with its
// handle). Returns null, with nothing allocated and the error recorded, when the allocation fails (MAKO_EHIP) or
// when the stream is capturing a graph and the buffer would have to grow (MAKO_EWORKSPACE: an allocation in a
// capture would belong to the graph).
enum WorkspacePurpose { kWsVtImages = 0, kWsSplitK = 1, kWsRowTiles = 2, kWsPassTable = 3, kWsPurposes = 4 };
void* stream_workspace(WorkspacePurpose purpose, size_t bytes, hipStream_t s, const char* what);

// A call's workspace: the caller's buffer (given, from an entry point that takes one: never allocates) or the
// library's buffer for (purpose, device, stream). get(need) returns memory of at least need bytes, or null with the
// error recorded (MAKO_EWORKSPACE when the caller's buffer is smaller, else as stream_workspace). Slices of a given
// workspace are taken with at(offset).
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool given = false;
    WorkspacePurpose purpose = kWsVtImages;
    const char* what = "";
    void* get(size_t need, hipStream_t s) const;
    Workspace at(size_t offset) const;
};
inline Workspace caller_workspace(void* p, size_t bytes, const char* what)
{
    Workspace w;
    w.ptr = p;
    w.bytes = bytes;
    w.given = true;
    w.what = what;
    return w;
}
inline Workspace library_workspace(WorkspacePurpose purpose, const char* what)
{
    Workspace w;
    w.purpose = purpose;
    w.what = what;
    return w;
}

}  // namespace mako
