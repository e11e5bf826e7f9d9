// The C ABI's error plumbing: a per-thread message for mako_last_error().
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "device.hpp"
#include "mako_attn.h"

namespace mako {

namespace {
thread_local std::string last_error;
thread_local int last_status = MAKO_OK;
}

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error = buf;
    last_status = code;
    return code;
}

int ok()
{
    last_error.clear();
    last_status = MAKO_OK;
    return MAKO_OK;
}

int last_code() { return last_status; }

int check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(MAKO_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

uint32_t device_cus()
{
    static thread_local int dev_cached = -1;
    static thread_local uint32_t cus_cached = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return 0;
    if (dev != dev_cached) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return 0;
        cus_cached = (uint32_t)cus;
        dev_cached = dev;
    }
    return cus_cached;
}

namespace {
struct Held {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex ws_mu;
std::map<std::tuple<int, int, hipStream_t>, Held> ws_all;  // (purpose, device, stream)
}  // namespace

void* stream_workspace(WorkspacePurpose purpose, size_t bytes, hipStream_t s, const char* what)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return fail(MAKO_EHIP, "%s: no current device", what), nullptr;
    std::lock_guard<std::mutex> lock(ws_mu);
    Held& ws = ws_all[{(int)purpose, dev, s}];
    if (ws.bytes < bytes) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cap) != hipSuccess)
            (void)hipGetLastError();
        if (cap != hipStreamCaptureStatusNone)
            return fail(MAKO_EWORKSPACE,
                        "%s: the stream is capturing a graph and the library's workspace would grow to %zu bytes; "
                        "pass a workspace (the *_ws entry point) or make the call once before the capture",
                        what, bytes), nullptr;
        if (ws.ptr)
            (void)hipFreeAsync(ws.ptr, s);  // after the previous use on this stream
        ws.ptr = nullptr;
        ws.bytes = 0;
        if (hipMallocAsync(&ws.ptr, bytes, s) != hipSuccess) {
            (void)hipGetLastError();
            ws.ptr = nullptr;
            return fail(MAKO_EHIP, "%s: no device memory for a workspace of %zu bytes", what, bytes), nullptr;
        }
        ws.bytes = bytes;
    }
    return ws.ptr;
}

void* Workspace::get(size_t need, hipStream_t s) const
{
    if (!given)
        return stream_workspace(purpose, need, s, what);
    if (bytes < need || (need && !ptr))
        return fail(MAKO_EWORKSPACE, "%s: a workspace of %zu bytes, the call needs %zu", what, bytes, need), nullptr;
    return ptr;
}

Workspace Workspace::at(size_t offset) const
{
    Workspace w = *this;
    if (given) {
        w.ptr = offset <= bytes ? static_cast<char*>(ptr) + offset : nullptr;
        w.bytes = offset <= bytes ? bytes - offset : 0;
    }
    return w;
}

}  // namespace mako

extern "C" int mako_attn_abi_version(void) { return MAKO_ATTN_ABI_VERSION; }

extern "C" int mako_attn_release(void* stream)
{
    using namespace mako;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return fail(MAKO_EHIP, "release: no current device");
    if (hipStreamSynchronize(s) != hipSuccess)
        return fail(MAKO_EHIP, "release: %s", hipGetErrorString(hipGetLastError()));
    std::lock_guard<std::mutex> lock(ws_mu);
    for (auto it = ws_all.begin(); it != ws_all.end();) {
        if (std::get<1>(it->first) == dev && std::get<2>(it->first) == s) {
            if (it->second.ptr && hipFree(it->second.ptr) != hipSuccess)
                return fail(MAKO_EHIP, "release: %s", hipGetErrorString(hipGetLastError()));
            it = ws_all.erase(it);
        } else {
            ++it;
        }
    }
    return ok();
}

extern "C" size_t mako_attn_held_bytes(void)
{
    using namespace mako;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return 0;
    std::lock_guard<std::mutex> lock(ws_mu);
    size_t n = 0;
    for (const auto& kv : ws_all)
        if (std::get<1>(kv.first) == dev)
            n += kv.second.bytes;
    return n;
}

extern "C" const char* mako_last_error(void) { return mako::last_error.c_str(); }
