#include "gpu_runtime.hpp"

#include <algorithm>
#include <cstdio>
#include <stdexcept>

#include "mako_attn.h"

namespace mako::gpu {

namespace {

using Clock = std::chrono::steady_clock;

void hip_check(hipError_t e, const char* what)
{
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

std::optional<Telemetry> parse_telemetry(std::string_view s)
{
    if (s == "off")
        return Telemetry::off;
    if (s == "summary")
        return Telemetry::summary;
    if (s == "steps")
        return Telemetry::steps;
    if (s == "layers")
        return Telemetry::layers;
    if (s == "kernels")
        return Telemetry::kernels;
    return std::nullopt;
}

Runtime::Runtime(Telemetry telemetry, int device) : device_(device), tel_(telemetry)
{
    hip_check(hipSetDevice(device_), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&enc_.stream, hipStreamNonBlocking), "hipStreamCreate");
}

Runtime::~Runtime()
{
    if (enc_.stream)
        (void)hipStreamSynchronize(enc_.stream);
    for (auto& t : timed_) {
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.end);
    }
    for (hipEvent_t e : spare_events_)
        (void)hipEventDestroy(e);
    for (auto& [name, b] : scratch_)
        (void)hipFree(b.ptr);
    if (enc_.stream)
        (void)hipStreamDestroy(enc_.stream);
}

uint64_t Runtime::scratch_bytes() const
{
    uint64_t n = 0;
    for (const auto& [name, b] : scratch_)
        n += b.bytes;
    return n;
}

Buffer* Runtime::scratch(const std::string& name, uint64_t bytes)
{
    auto it = scratch_.find(name);
    if (it == scratch_.end() || it->second.bytes < bytes) {
        if (it != scratch_.end()) {
            hip_check(hipStreamSynchronize(enc_.stream), "scratch: waiting for the queue");
            hip_check(hipFree(it->second.ptr), "hipFree");
        }
        Buffer b;
        b.bytes = std::max<uint64_t>(bytes, 256);
        hip_check(hipMalloc(&b.ptr, b.bytes), ("scratch " + name).c_str());
        it = scratch_.insert_or_assign(name, b).first;
    }
    return &it->second;
}

void Runtime::drop_scratch(const std::string& name)
{
    auto it = scratch_.find(name);
    if (it == scratch_.end())
        return;
    hip_check(hipStreamSynchronize(enc_.stream), "drop_scratch: waiting for the queue");
    hip_check(hipFree(it->second.ptr), "hipFree");
    scratch_.erase(it);
}

Encoder* Runtime::encoder()
{
    if (!encoding_) {
        step_start_ = Clock::now();
        encoding_ = true;
    }
    return &enc_;
}

hipEvent_t Runtime::event()
{
    if (!spare_events_.empty()) {
        hipEvent_t e = spare_events_.back();
        spare_events_.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    hip_check(hipEventCreate(&e), "hipEventCreate");
    return e;
}

void Runtime::before(Encoder* enc)
{
    if (tel_ != Telemetry::kernels)
        return;
    Timed t;
    t.start = event();
    t.end = event();
    hip_check(hipEventRecord(t.start, enc->stream), "hipEventRecord");
    timed_.push_back(std::move(t));
}

void Runtime::after(Encoder*& enc, std::string_view kernel)
{
    if (tel_ != Telemetry::kernels || timed_.empty())
        return;
    timed_.back().kernel = kernel;
    hip_check(hipEventRecord(timed_.back().end, enc->stream), "hipEventRecord");
}

void Runtime::finish(Encoder* enc)
{
    const auto t0 = Clock::now();
    if (encoding_) {
        stats_.encode_ms += std::chrono::duration<double, std::milli>(t0 - step_start_).count();
        encoding_ = false;
    }
    const hipError_t e = hipStreamSynchronize(enc->stream);
    stats_.gpu_wait_ms += std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
    if (e != hipSuccess)
        throw std::runtime_error(std::string("launch queue failed: ") + hipGetErrorString(e));
    const hipError_t last = hipGetLastError();
    if (last != hipSuccess)
        throw std::runtime_error(std::string("launch queue failed: ") + hipGetErrorString(last));
    resolve_times();
}

void Runtime::resolve_times()
{
    for (auto& t : timed_) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, t.start, t.end) == hipSuccess) {
            auto it = std::find_if(kernels_.begin(), kernels_.end(),
                                   [&](const KernelTime& k) { return k.kernel == t.kernel; });
            if (it == kernels_.end())
                it = kernels_.insert(kernels_.end(), KernelTime{t.kernel, 0, 0});
            it->ms += ms;
            ++it->count;
            stats_.gpu_exec_ms += ms;
        }
        spare_events_.push_back(t.start);
        spare_events_.push_back(t.end);
    }
    timed_.clear();
}

std::vector<KernelTime> Runtime::kernel_times()
{
    std::vector<KernelTime> out;
    out.swap(kernels_);
    return out;
}

void Runtime::check(int status)
{
    if (status != MAKO_OK)
        throw std::runtime_error(mako_last_error());
}

void Runtime::proj(Encoder*& enc, const Weight& w, Buffer* x, uint64_t x_off, Buffer* y, uint64_t y_off, uint32_t T,
                   uint32_t ldy, bool x_bf16)
{
    if (w.k % 64) {  // the reference's message (src/gpu/runtime.cpp:179-180)
        char msg[96];
        std::snprintf(msg, sizeof msg, "BF16 %ux%u: k must be a multiple of 64", w.k, w.n);
        throw std::runtime_error(msg);
    }
    const mako_gemm_args a{T, w.k, w.n, 2 * w.k, ldy, 0};
    before(enc);
    check(mako_proj_bf16(&a, x_bf16 ? MAKO_BF16 : MAKO_F32, bf16_split_ && !x_bf16 ? 1 : 0,
                         static_cast<const char*>(w.buf->ptr) + w.off, static_cast<const char*>(x->ptr) + x_off,
                         reinterpret_cast<float*>(static_cast<char*>(y->ptr) + y_off), enc->stream));
    after(enc, bf16_split_ && !x_bf16 ? "proj BF16 split" : "proj BF16");
}

}  // namespace mako::gpu
