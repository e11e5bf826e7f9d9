#include "gpu_runtime.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <utility>
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

namespace {

// The telemetry level names, in the order of the levels.
constexpr std::pair<std::string_view, Telemetry> kTelemetryNames[] = {
    {"off", Telemetry::off}, {"summary", Telemetry::summary}, {"steps", Telemetry::steps},
    {"layers", Telemetry::layers}, {"kernels", Telemetry::kernels}};

}  // namespace

std::optional<Telemetry> parse_telemetry(std::string_view s)
{
    for (const auto& [name, level] : kTelemetryNames)
        if (name == s)
            return level;
    return std::nullopt;
}

RepeatSpec RepeatSpec::parse(std::string_view spec)
{
    const size_t colon = spec.rfind(':');
    if (colon == std::string_view::npos)
        throw std::runtime_error("MAKO_REPEAT wants <label substring>:<n>");
    RepeatSpec r;
    // The count: the integer that starts the text after the last ':' (leading blanks skipped); none, or below 0: 0.
    const std::string count(spec.substr(colon + 1));
    const long n = std::strtol(count.c_str(), nullptr, 10);
    r.times = static_cast<int>(std::clamp<long>(n, 0, std::numeric_limits<int>::max()));
    // The labels: the comma-separated parts before it; empty parts match nothing.
    std::string_view rest = spec.substr(0, colon);
    while (!rest.empty()) {
        const std::string_view part = rest.substr(0, rest.find(','));
        if (!part.empty())
            r.labels.emplace_back(part);
        rest.remove_prefix(std::min(rest.size(), part.size() + 1));
    }
    return r;
}

bool RepeatSpec::matches(std::string_view label) const
{
    return std::any_of(labels.begin(), labels.end(),
                       [&](const std::string& sub) { return label.find(sub) != std::string_view::npos; });
}

Runtime::Runtime(Telemetry telemetry, int device) : device_(device), tel_(telemetry)
{
    if (const char* r = std::getenv("MAKO_REPEAT"))
        repeat_ = RepeatSpec::parse(r);
    hip_check(hipSetDevice(device_), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&enc_.stream, hipStreamNonBlocking), "hipStreamCreate");
}

int Runtime::repeats(std::string_view label) const
{
    return repeat_.times != 1 && repeat_.matches(label) ? repeat_.times : 1;
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
    for (auto& m : marks_)
        (void)hipEventDestroy(m.ev);
    for (auto& p : pending_probes_)
        (void)hipHostFree(p.host);
    for (auto& [ptr, n] : spare_host_)
        (void)hipHostFree(ptr);
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
    end_marks(enc);
    on_committed(enc);
    const hipError_t e = hipStreamSynchronize(enc->stream);
    stats_.gpu_wait_ms += std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
    on_completed();
    if (e != hipSuccess)
        throw std::runtime_error(std::string("launch queue failed: ") + hipGetErrorString(e));
    const hipError_t last = hipGetLastError();
    if (last != hipSuccess)
        throw std::runtime_error(std::string("launch queue failed: ") + hipGetErrorString(last));
    resolve_times();
    resolve_sections();
    deliver_probes();
}

void Runtime::end_marks(Encoder* enc)
{
    if (marks_.empty() || marks_.back().section < 0)  // no open section or part
        return;
    Mark end;
    end.ev = event();
    end.section = -1;
    hip_check(hipEventRecord(end.ev, enc->stream), "hipEventRecord");
    marks_.push_back(std::move(end));
}

void Runtime::submit(Encoder*& enc)
{
    finish(enc);
    enc = encoder();
}

void Runtime::commit_ahead(Encoder*& enc)
{
    if (!commit_ahead_ok())
        return;
    const auto now = Clock::now();
    if (encoding_)
        stats_.encode_ms += std::chrono::duration<double, std::milli>(now - step_start_).count();
    step_start_ = now;  // the next stretch's encode time starts here
    encoding_ = true;
    end_marks(enc);
    ++stats_.commits_ahead;
}

void Runtime::section(Encoder*& enc, uint32_t layer, int section)
{
    if (tel_ != Telemetry::layers)
        return;
    Mark m;
    m.ev = event();
    m.layer = layer;
    m.section = section;
    hip_check(hipEventRecord(m.ev, enc->stream), "hipEventRecord");
    marks_.push_back(std::move(m));
}

void Runtime::part(Encoder*& enc, std::string_view name)
{
    if (!part_timing_ || marks_.empty() || marks_.back().section < 0)
        return;
    Mark m;
    m.ev = event();
    m.layer = marks_.back().layer;
    m.section = marks_.back().section;
    m.part = name;
    hip_check(hipEventRecord(m.ev, enc->stream), "hipEventRecord");
    marks_.push_back(std::move(m));
}

// Each interval between consecutive marks belongs to the section of its first mark, and to that mark's part if it
// names one.
void Runtime::resolve_sections()
{
    for (size_t i = 0; i + 1 < marks_.size(); ++i) {
        const Mark& m = marks_[i];
        float ms = 0.0f;
        if (m.section < 0 || hipEventElapsedTime(&ms, m.ev, marks_[i + 1].ev) != hipSuccess)
            continue;  // an end mark opens no interval
        auto sec = std::find_if(sections_.begin(), sections_.end(), [&](const SectionTime& t) {
            return t.layer == m.layer && t.section == m.section;
        });
        if (sec == sections_.end())
            sec = sections_.insert(sections_.end(), SectionTime{m.layer, m.section, 0});
        sec->ms += ms;
        if (!m.part.empty()) {
            auto it = std::find_if(parts_.begin(), parts_.end(), [&](const KernelTime& k) { return k.kernel == m.part; });
            if (it == parts_.end())
                it = parts_.insert(parts_.end(), KernelTime{m.part, 0, 0});
            it->ms += ms;
            ++it->count;
        }
    }
    for (auto& m : marks_)
        spare_events_.push_back(m.ev);
    marks_.clear();
}

std::vector<Runtime::SectionTime> Runtime::section_times()
{
    std::vector<SectionTime> out;
    out.swap(sections_);
    return out;
}

std::vector<KernelTime> Runtime::part_times()
{
    std::vector<KernelTime> out;
    out.swap(parts_);
    return out;
}

void Runtime::probe(Encoder*& enc, const std::string& name, int layer, Buffer* buf, size_t n, uint64_t off)
{
    if (!probe_)
        return;
    if (off + n * sizeof(float) > buf->bytes)
        throw std::runtime_error("probe " + name + ": " + std::to_string(n) + " values at byte " + std::to_string(off) +
                                 " run past the buffer's " + std::to_string(buf->bytes));
    PendingProbe p;
    p.name = name;
    p.layer = layer;
    p.n = n;
    // a spare pinned buffer large enough, or a new one
    auto it = std::find_if(spare_host_.begin(), spare_host_.end(), [&](const auto& h) { return h.second >= n; });
    if (it != spare_host_.end()) {
        p.host = it->first;
        p.cap = it->second;
        spare_host_.erase(it);
    } else {
        hip_check(hipHostMalloc(reinterpret_cast<void**>(&p.host), std::max<size_t>(n, 1) * sizeof(float),
                                hipHostMallocDefault), "probe: hipHostMalloc");
        p.cap = std::max<size_t>(n, 1);
    }
    pending_probes_.push_back(p);
    hip_check(hipMemcpyAsync(p.host, static_cast<const char*>(buf->ptr) + off, n * sizeof(float),
                             hipMemcpyDeviceToHost, enc->stream), "probe: hipMemcpyAsync");
}

void Runtime::deliver_probes()
{
    std::vector<PendingProbe> ps;
    ps.swap(pending_probes_);
    for (auto& p : ps) {
        if (probe_)
            probe_(p.name, p.layer, p.host, p.n);
        spare_host_.emplace_back(p.host, p.cap);
    }
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
    const char* label = bf16_split_ && !x_bf16 ? "proj BF16 split" : "proj BF16";
    before(enc);
    for (int r = repeats(label); r > 0; --r)
        check(mako_proj_bf16(&a, x_bf16 ? MAKO_BF16 : MAKO_F32, bf16_split_ && !x_bf16 ? 1 : 0,
                             static_cast<const char*>(w.buf->ptr) + w.off, static_cast<const char*>(x->ptr) + x_off,
                             reinterpret_cast<float*>(static_cast<char*>(y->ptr) + y_off), enc->stream));
    after(enc, label);
}

}  // namespace mako::gpu
