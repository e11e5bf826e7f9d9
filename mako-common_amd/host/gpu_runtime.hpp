// The launch side of the attention path on HIP: what src/gpu/runtime.hpp gives the reference's engines, for the
// parts the attention path uses (named scratch buffers, one in-order launch queue, finish() raising device errors,
// per-kernel and per-section telemetry, the probe hook for parity checks, MAKO_REPEAT, the step statistics). Kernels are reached through the C ABI of include/mako_attn.h, not
// by name: the typed entry points replace the pipeline lookup (src/gpu/runtime.cpp:127-135).
#pragma once

#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdint>
#include <functional>
#include <map>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace mako::gpu {

// How much a step measures (src/gpu/runtime.hpp:21-26): at the layers level each section (and, with part timing on,
// each named part) of a step is timed by HIP events on the queue; at the kernels level every launch is bracketed by
// a pair of HIP events and labelled.
enum class Telemetry { off, summary, steps, layers, kernels };
std::optional<Telemetry> parse_telemetry(std::string_view s);

// The value of MAKO_REPEAT, <label substrings, comma-separated>:<n> (src/gpu/runtime.cpp:52-59): the substrings and
// the launch count. parse() throws std::runtime_error for a value with no ':'.
struct RepeatSpec {
    std::vector<std::string> labels;
    int times = 1;
    static RepeatSpec parse(std::string_view spec);
    // Whether one of the substrings occurs in `label`.
    bool matches(std::string_view label) const;
};

struct KernelTime {
    std::string kernel;
    double ms = 0;
    uint32_t count = 0;
};

// Device memory (what an MTL::Buffer at offset 0 was): a hipMalloc'd pointer and its size.
struct Buffer {
    void* ptr = nullptr;
    uint64_t bytes = 0;
};

// The launch queue a step records into (what the compute command encoder was): one HIP stream at the default
// priority, launches in order, results visible after Runtime::finish.
struct Encoder {
    hipStream_t stream = nullptr;
};

class Runtime {
public:
    // Called after each named stage of a step with the fp32 values it produced, for parity checks
    // (src/gpu/runtime.hpp:45-47). Probes are delivered by finish(), in the order they were taken.
    using Probe = std::function<void(const std::string& name, int layer, const float* data, size_t n)>;
    void set_probe(Probe probe) { probe_ = std::move(probe); }

    struct Stats {
        double gpu_wait_ms = 0, gpu_exec_ms = 0;  // wait: finish() blocked; exec: timed launches, summed
        double encode_ms = 0, step_ms = 0;        // encode: step start to finish(), less the commit_ahead() gaps
        uint32_t commits_ahead = 0;               // commit_ahead() calls that ended a stretch
    };
    const Stats& stats() const { return stats_; }
    // Bytes of all scratch buffers allocated so far.
    uint64_t scratch_bytes() const;
    // At the kernels level: the launches' GPU times since the last call, summed per kernel.
    std::vector<KernelTime> kernel_times();
    // At the layers level: each timed section's GPU time (layer, section, ms) and the named parts' times summed per
    // name, since the last call (the reference's resolve_times, src/gpu/runtime.hpp:147-152).
    struct SectionTime {
        uint32_t layer = 0;
        int section = 0;
        double ms = 0;
    };
    std::vector<SectionTime> section_times();
    std::vector<KernelTime> part_times();
    // MAKO_REPEAT=<label substrings, comma-separated>:<n>: launches whose label holds one of the substrings run n
    // times (0: not at all), so the extra step time measures their cost in place (src/gpu/runtime.hpp:158-172).
    int repeats(std::string_view label) const;

    Runtime(const Runtime&) = delete;
    Runtime& operator=(const Runtime&) = delete;

protected:
    explicit Runtime(Telemetry telemetry, int device = 0);
    virtual ~Runtime();

    // A named device buffer of at least `bytes`, reallocated (after the queue drains) when too small
    // (src/gpu/runtime.cpp:117-125). Its contents survive until then.
    Buffer* scratch(const std::string& name, uint64_t bytes);
    void drop_scratch(const std::string& name);
    // The step's launch queue; `enc` stays valid for the Runtime's life.
    Encoder* encoder();
    // Before / after a launch: at the kernels level, events around it, labelled `kernel` (the reference closed
    // and reopened the encoder, src/gpu/runtime.cpp:362-370).
    void before(Encoder* enc);
    void after(Encoder*& enc, std::string_view kernel);
    // Waits for every launch of the queue and raises std::runtime_error if one failed (src/gpu/runtime.cpp:453-475);
    // then resolves the step's times and delivers its probes.
    void finish(Encoder* enc);
    // finish(), then the next launches start a new step on the same queue (src/gpu/runtime.cpp:493-500).
    void submit(Encoder*& enc);
    // Ends the step's current stretch without waiting (src/gpu/runtime.cpp:477-491; src/gpu/runtime.hpp:121-123):
    // the launches made so far are already on the in-order queue and running, so what remains of the reference's
    // commit is its bookkeeping. The stretch's encode time is added to the stats, a timed section or part ends here
    // (the launches up to the next section() are untimed, as the reference's encoder of section -1 was), and
    // finish() waits for and accounts every stretch. Does nothing while commit_ahead_ok() says no.
    void commit_ahead(Encoder*& enc);
    // finish()'s hooks (src/gpu/runtime.hpp:124-128): on_committed after the last launch is queued and before the
    // wait (host work the GPU may be waiting for), on_completed after the wait, before errors are raised.
    virtual void on_committed(Encoder*) {}
    virtual void on_completed() {}
    virtual bool commit_ahead_ok() const { return true; }
    // With a probe set: n f32 values of buf at off bytes copied on the queue (after what was launched before) into
    // host memory, handed to the probe by finish() as (name, layer) (src/gpu/runtime.cpp:502-517).
    void probe(Encoder*& enc, const std::string& name, int layer, Buffer* buf, size_t n, uint64_t off = 0);
    // Hands the taken probes to the probe (src/gpu/runtime.cpp:519-524); finish() calls it.
    void deliver_probes();
    // At the layers level: the launches from here to the next section() (or finish()) are timed as section
    // `section` of layer `layer` (the reference's timed encoder of a section).
    bool timing() const { return tel_ == Telemetry::layers; }
    void section(Encoder*& enc, uint32_t layer, int section);
    // At the layers level with part timing on: the launches from here to the next part() or section() (or finish())
    // are timed as `name` within the current section (src/gpu/runtime.hpp:137-146).
    void enable_part_timing(bool on) { part_timing_ = on && tel_ == Telemetry::layers; }
    void part(Encoder*& enc, std::string_view name);
    // Turns a nonzero C ABI status into std::runtime_error carrying the library's message.
    static void check(int status);

    // A BF16 weight matrix as proj() reads it (the reference's Tensor of type BF16 with dims {k, n}): n rows of k
    // bf16 values, `off` bytes into buf.
    struct Weight {
        Buffer* buf = nullptr;
        uint64_t off = 0;
        uint32_t k = 0, n = 0;
    };
    // y[t] = W x[t] for T tokens, the BF16 branch of the reference's proj (src/gpu/runtime.cpp:164-205): x rows of k
    // f32 values at x_off bytes (bf16 rows when x_bf16, e.g. attention output written in bf16), y f32 rows ldy
    // apart (0: n) at y_off bytes; with bf16_split_ the rounding's remainder goes through the product too. Throws
    // "BF16 {k}x{n}: k must be a multiple of 64" as the reference does.
    void proj(Encoder*& enc, const Weight& w, Buffer* x, uint64_t x_off, Buffer* y, uint64_t y_off, uint32_t T,
              uint32_t ldy = 0, bool x_bf16 = false);
    bool bf16_split_ = false;

    int device_ = 0;
    Telemetry tel_ = Telemetry::off;
    Encoder enc_;
    std::map<std::string, Buffer> scratch_;
    Stats stats_;

private:
    struct Timed {
        hipEvent_t start = nullptr, end = nullptr;
        std::string kernel;
    };
    std::vector<Timed> timed_;
    struct Mark {  // a section or part boundary on the queue
        hipEvent_t ev = nullptr;
        uint32_t layer = 0;
        int section = 0;
        std::string part;  // empty: the section itself
    };
    std::vector<Mark> marks_;
    std::vector<SectionTime> sections_;
    std::vector<KernelTime> parts_;
    bool part_timing_ = false;
    struct PendingProbe {
        std::string name;
        int layer = 0;
        float* host = nullptr;  // pinned
        size_t n = 0, cap = 0;
    };
    Probe probe_;
    std::vector<PendingProbe> pending_probes_;
    std::vector<std::pair<float*, size_t>> spare_host_;  // pinned buffers (values) for later probes
    RepeatSpec repeat_;
    std::vector<hipEvent_t> spare_events_;
    std::vector<KernelTime> kernels_;
    std::chrono::steady_clock::time_point step_start_;
    bool encoding_ = false;
    hipEvent_t event();
    void end_marks(Encoder* enc);  // closes an open section or part with an end mark (section -1)
    void resolve_times();
    void resolve_sections();
};

}  // namespace mako::gpu
