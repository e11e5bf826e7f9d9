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
}

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error = buf;
    return code;
}

int ok()
{
    last_error.clear();
    return MAKO_OK;
}

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
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex ws_mu;
std::map<std::tuple<int, int, hipStream_t>, Workspace> ws_all;
}  // namespace

void* stream_workspace(WorkspacePurpose purpose, size_t bytes, hipStream_t s)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return nullptr;
    std::lock_guard<std::mutex> lock(ws_mu);
    Workspace& ws = ws_all[{(int)purpose, dev, s}];
    if (ws.bytes < bytes) {
        if (ws.ptr)
            (void)hipFreeAsync(ws.ptr, s);  // after the previous use on this stream
        ws.ptr = nullptr;
        ws.bytes = 0;
        if (hipMallocAsync(&ws.ptr, bytes, s) != hipSuccess) {
            (void)hipGetLastError();
            ws.ptr = nullptr;
            return nullptr;
        }
        ws.bytes = bytes;
    }
    return ws.ptr;
}

}  // namespace mako

extern "C" int mako_attn_abi_version(void) { return MAKO_ATTN_ABI_VERSION; }

extern "C" const char* mako_last_error(void) { return mako::last_error.c_str(); }
