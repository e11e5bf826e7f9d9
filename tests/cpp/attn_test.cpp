// Dense and decode attention through TransformerRuntime against the CPU oracle:
// * attention() with the reference's own arguments and defaults (f16 tiles in, f32 rows out): causal GQA at
//   batch 1, 16 query heads over 8 kv heads, D 128, S 512 (the call QwenText::encode makes,
//   src/models/qwen_text.cpp:311), every row;
// * the same call with AttnOptions: bf16 in and out and an LSE, bidirectional (block 0, the call H3::block makes,
//   src/models/h3.cpp:364);
// * attention_decode: 4 sequences of different contexts, GQA 4;
// * the refusal of a head width the reference refuses (src/models/runtime.cpp:266-267);
// * heads_partial with the call H3::block makes (src/models/h3.cpp:348: heads of 128, the first 96 values
//   rotated, RMS norm, the cube row map), heads() with rotation and the padding cleared
//   (src/models/qwen_text.cpp:308), and the refusal of heads_partial's odd rotation (src/models/runtime.cpp:249);
// * proj() with BF16 weights after attention (src/models/qwen_text.cpp:312): f32 rows, the bf16 split the Qwen
//   encoders turn on (src/models/qwen_text.cpp:271), bf16 rows, a y row stride, and the refusal of k = 96
//   (src/gpu/runtime.cpp:179-180); within the f32 summation bound 2 k 2^-24 sum|terms| (4 k with the split);
// * the probe hook (src/gpu/runtime.cpp:502-524): the attention output probed after attention(), whole and a slice
//   at an offset, comes back bit-equal to o, with its name and layer; layer / part timing at the layers level
//   (src/gpu/runtime.hpp:137-152): two sections and three named parts, each timed; MAKO_REPEAT=flash_fwd:3 runs
//   attention three times inside one timed launch and leaves its output bit-equal;
// * kda_scan with the arguments QwenText::linear_layer passes (src/models/qwen_text.cpp:374-382: {128, T, vw, vw, VH,
//   0}, the state zeroed), 4 heads over 100 tokens; within 2e-5 + 1e-4 |ref| of the oracle.
// Tolerance: every element within 2e-3 + 1e-2 |ref|; LSE within 1e-3; head tiles within one f16 ulp.
//   attn_test
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "attn_oracle.h"
#include "transformer_runtime.hpp"

namespace {

class Harness final : public mako::models::TransformerRuntime {
public:
    explicit Harness(mako::gpu::Telemetry t = mako::gpu::Telemetry::kernels) : TransformerRuntime(t) {}
    using TransformerRuntime::attention;
    using TransformerRuntime::attention_rows;
    using TransformerRuntime::attention_decode;
    using TransformerRuntime::attention_sparse;
    using TransformerRuntime::heads;
    using TransformerRuntime::heads_partial;
    using TransformerRuntime::proj;
    using TransformerRuntime::kda_scan;
    using TransformerRuntime::Weight;
    using TransformerRuntime::bf16_split_;
    using TransformerRuntime::encoder;
    using TransformerRuntime::finish;
    using TransformerRuntime::scratch;
    using TransformerRuntime::probe;
    using TransformerRuntime::section;
    using TransformerRuntime::part;
    using TransformerRuntime::enable_part_timing;
    using TransformerRuntime::submit;
    using TransformerRuntime::commit_ahead;

    int committed = 0, completed = 0;
    bool ahead_ok = true;
    void on_committed(mako::gpu::Encoder*) override { ++committed; }
    void on_completed() override { ++completed; }
    bool commit_ahead_ok() const override { return ahead_ok; }
};

int failures = 0;
void check(bool ok, const std::string& what)
{
    std::printf("  %s  %s\n", ok ? "ok  " : "FAIL", what.c_str());
    failures += !ok;
}

uint64_t rng_state = 12345;
double normal()
{
    auto next = [] {
        uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    };
    const double u1 = ((next() >> 11) + 0.5) * 0x1.0p-53, u2 = (next() >> 11) * 0x1.0p-53;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(2 * M_PI * u2);
}

std::vector<uint16_t> random_tile(size_t n, int dtype)
{
    std::vector<uint16_t> v(n);
    for (auto& x : v)
        x = dtype == ORACLE_F16 ? oracle_f32_to_f16(float(normal())) : oracle_f32_to_bf16(float(normal()));
    return v;
}

template <class T>
mako::gpu::Buffer* put(Harness& h, const std::string& name, const std::vector<T>& v)
{
    auto* b = h.scratch(name, v.size() * sizeof(T));
    if (hipMemcpy(b->ptr, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return b;
}

template <class T>
std::vector<T> get(const mako::gpu::Buffer* b, size_t n)
{
    std::vector<T> v(n);
    if (hipMemcpy(v.data(), b->ptr, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return v;
}

float widen(uint16_t b, bool bf16)
{
    if (!bf16)
        return oracle_f16_to_f32(b);
    const uint32_t u = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Elements past 2e-3 + 1e-2 |ref| and the largest LSE error.
uint64_t bad_elems(const std::vector<float>& got, const std::vector<double>& want)
{
    uint64_t bad = 0;
    for (size_t i = 0; i < want.size(); ++i)
        bad += !(std::fabs(got[i] - want[i]) <= 2e-3 + 1e-2 * std::fabs(want[i]));
    return bad;
}

double lse_err(const std::vector<float>& got, const std::vector<double>& want)
{
    double e = 0;
    for (size_t i = 0; i < want.size(); ++i)
        e = std::max(e, std::isinf(want[i]) ? (got[i] == want[i] ? 0.0 : 1.0) : std::fabs(got[i] - want[i]));
    return e;
}

}  // namespace

int main()
{
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    Harness h;
    // Causal GQA, f16 in, f32 out: the reference's call and defaults.
    {
        const uint32_t heads = 16, kv = 8, D = 128, S = 512;
        const auto q = random_tile(size_t(heads) * S * D, ORACLE_F16), k = random_tile(size_t(kv) * S * D, ORACLE_F16),
                   v = random_tile(size_t(kv) * S * D, ORACLE_F16);
        auto qb = put(h, "q", q), kb = put(h, "k", k), vb = put(h, "v", v);
        auto ob = h.scratch("o", size_t(S) * heads * D * 4);
        auto* enc = h.encoder();
        h.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX);
        h.finish(enc);
        const oracle_attn_args a{S, S, S, S, heads, kv, 0, UINT32_MAX, heads * D, 1.0f / std::sqrt(float(D))};
        std::vector<double> want(size_t(S) * heads * D);
        oracle_attn_dense(&a, D, ORACLE_F16, q.data(), k.data(), v.data(), want.data(), nullptr, 0);
        const uint64_t bad = bad_elems(get<float>(ob, want.size()), want);
        check(bad == 0, "attention, causal GQA S512 f16 -> f32: " + std::to_string(bad) + " elements out of tolerance");
    }
    // Bidirectional, bf16 in and out, with the LSE.
    {
        const uint32_t heads = 4, kv = 4, D = 128, S = 300, q_pad = 320, k_pad = 384;
        const auto q = random_tile(size_t(heads) * q_pad * D, ORACLE_BF16),
                   k = random_tile(size_t(kv) * k_pad * D, ORACLE_BF16),
                   v = random_tile(size_t(kv) * k_pad * D, ORACLE_BF16);
        auto qb = put(h, "q", q), kb = put(h, "k", k), vb = put(h, "v", v);
        auto ob = h.scratch("o", size_t(S) * heads * D * 2);
        auto lb = h.scratch("lse", size_t(heads) * S * 4);
        mako::models::AttnOptions opt;
        opt.in = MAKO_BF16;
        opt.out = MAKO_BF16;
        opt.lse = lb;
        auto* enc = h.encoder();
        h.attention(enc, qb, kb, vb, ob, S, q_pad, S, k_pad, heads, kv, 0, 0, D, opt);
        h.finish(enc);
        const oracle_attn_args a{S, q_pad, S, k_pad, heads, kv, 0, 0, heads * D, 1.0f / std::sqrt(float(D))};
        std::vector<double> want(size_t(S) * heads * D), want_l(size_t(heads) * S);
        oracle_attn_dense(&a, D, ORACLE_BF16, q.data(), k.data(), v.data(), want.data(), want_l.data(), 0);
        const auto ob16 = get<uint16_t>(ob, want.size());
        std::vector<float> got(ob16.size());
        for (size_t i = 0; i < got.size(); ++i)
            got[i] = widen(ob16[i], true);
        const uint64_t bad = bad_elems(got, want);
        const double le = lse_err(get<float>(lb, want_l.size()), want_l);
        check(bad == 0 && le <= 1e-3, "attention, bidirectional S300 bf16 -> bf16 + LSE: " + std::to_string(bad) +
                                          " elements out of tolerance, LSE error " + std::to_string(le));
    }
    // Decode: 4 sequences, 32 query heads over 8 kv heads.
    {
        const uint32_t batch = 4, heads = 32, kv = 8, D = 128, cap = 3000;
        const std::vector<uint32_t> ctx{1, 700, 2048, 3000};
        const auto q = random_tile(size_t(batch) * heads * D, ORACLE_F16),
                   k = random_tile(size_t(batch) * kv * cap * D, ORACLE_F16),
                   v = random_tile(size_t(batch) * kv * cap * D, ORACLE_F16);
        auto qb = put(h, "q", q), kb = put(h, "k", k), vb = put(h, "v", v), cb = put(h, "ctx", ctx);
        auto ob = h.scratch("o", size_t(batch) * heads * D * 4);
        auto lb = h.scratch("lse", size_t(batch) * heads * 4);
        mako::models::AttnOptions opt;
        opt.lse = lb;
        auto* enc = h.encoder();
        h.attention_decode(enc, qb, kb, vb, cb, ob, batch, heads, kv, cap, cap, opt);
        h.finish(enc);
        std::vector<double> want(size_t(batch) * heads * D), want_l(size_t(batch) * heads);
        oracle_attn_decode(batch, heads, kv, D, cap, 1.0f / std::sqrt(float(D)), ORACLE_F16, q.data(), k.data(),
                           v.data(), ctx.data(), want.data(), want_l.data(), 0);
        const uint64_t bad = bad_elems(get<float>(ob, want.size()), want);
        const double le = lse_err(get<float>(lb, want_l.size()), want_l);
        check(bad == 0 && le <= 1e-3, "attention_decode, 4 sequences: " + std::to_string(bad) +
                                          " elements out of tolerance, LSE error " + std::to_string(le));
    }
    // The probe hook: attention's output probed whole and as one head of one row (at a byte offset).
    {
        const uint32_t heads = 8, kv = 2, D = 128, S = 256;
        const auto q = random_tile(size_t(heads) * S * D, ORACLE_F16), k = random_tile(size_t(kv) * S * D, ORACLE_F16),
                   v = random_tile(size_t(kv) * S * D, ORACLE_F16);
        auto qb = put(h, "q", q), kb = put(h, "k", k), vb = put(h, "v", v);
        const size_t n = size_t(S) * heads * D;
        auto ob = h.scratch("o", n * 4);
        std::vector<std::tuple<std::string, int, std::vector<float>>> got;
        h.set_probe([&](const std::string& name, int layer, const float* data, size_t cnt) {
            got.emplace_back(name, layer, std::vector<float>(data, data + cnt));
        });
        auto* enc = h.encoder();
        h.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX);
        h.probe(enc, "attn_out", 7, ob, n);
        const uint64_t off = (5ull * heads * D + 2 * D) * 4;  // row 5, head 2
        h.probe(enc, "attn_row5_head2", 7, ob, D, off);
        h.finish(enc);
        h.set_probe(nullptr);
        const auto o = get<float>(ob, n);
        bool same = got.size() == 2 && std::get<0>(got[0]) == "attn_out" && std::get<1>(got[0]) == 7 &&
                    std::get<2>(got[0]).size() == n && std::get<0>(got[1]) == "attn_row5_head2" &&
                    std::get<2>(got[1]).size() == D;
        same = same && std::memcmp(std::get<2>(got[0]).data(), o.data(), n * 4) == 0 &&
               std::memcmp(std::get<2>(got[1]).data(), o.data() + off / 4, size_t(D) * 4) == 0;
        check(same, "probe after attention: the f32 rows come back bit-equal to o, with name and layer");
    }
    // Layer / part timing at the layers level, and MAKO_REPEAT.
    {
        const uint32_t heads = 8, kv = 2, D = 128, S = 512;
        const auto q = random_tile(size_t(heads) * S * D, ORACLE_BF16),
                   k = random_tile(size_t(kv) * S * D, ORACLE_BF16), v = random_tile(size_t(kv) * S * D, ORACLE_BF16);
        mako::models::AttnOptions opt;
        opt.in = MAKO_BF16;
        const size_t n = size_t(S) * heads * D;
        std::vector<float> once;
        {
            Harness ht(mako::gpu::Telemetry::layers);
            auto qb = put(ht, "q", q), kb = put(ht, "k", k), vb = put(ht, "v", v);
            auto ob = ht.scratch("o", n * 4);
            ht.enable_part_timing(true);
            auto* enc = ht.encoder();
            ht.section(enc, 3, 0);
            ht.part(enc, "attention causal");
            ht.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX, D, opt);
            ht.part(enc, "attention bidirectional");
            ht.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, 0, D, opt);
            ht.section(enc, 4, 1);
            ht.part(enc, "attention causal");
            ht.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX, D, opt);
            ht.finish(enc);
            once = get<float>(ob, n);
            const auto secs = ht.section_times();
            const auto parts = ht.part_times();
            bool ok = secs.size() == 2 && secs[0].layer == 3 && secs[0].section == 0 && secs[1].layer == 4 &&
                      secs[1].section == 1 && secs[0].ms > 0 && secs[1].ms > 0;
            double causal = 0, bidir = 0;
            uint32_t causal_n = 0;
            for (const auto& p : parts) {
                if (p.kernel == "attention causal") {
                    causal = p.ms;
                    causal_n = p.count;
                } else if (p.kernel == "attention bidirectional") {
                    bidir = p.ms;
                }
            }
            ok = ok && parts.size() == 2 && causal_n == 2 && causal > 0 && bidir > 0 &&
                 secs[0].ms + 1e-6 >= bidir && ht.section_times().empty();
            check(ok, "layers timing: 2 sections (" + std::to_string(secs.size()) + "), parts causal x" +
                          std::to_string(causal_n) + " and bidirectional, each timed");
        }
        {
            setenv("MAKO_REPEAT", "flash_fwd:3", 1);
            Harness hr;
            unsetenv("MAKO_REPEAT");
            auto qb = put(hr, "q", q), kb = put(hr, "k", k), vb = put(hr, "v", v);
            auto ob = hr.scratch("o", n * 4);
            auto* enc = hr.encoder();
            hr.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX, D, opt);
            hr.finish(enc);
            const auto kt = hr.kernel_times();
            const auto o = get<float>(ob, n);
            check(hr.repeats("flash_fwd_128") == 3 && hr.repeats("proj BF16") == 1 && kt.size() == 1 &&
                      kt[0].count == 1 && std::memcmp(o.data(), once.data(), n * 4) == 0,
                  "MAKO_REPEAT=flash_fwd:3: attention repeated inside one timed launch, output bit-equal");
        }
        // commit_ahead ends a timed section without waiting; submit finishes and starts the next step.
        {
            Harness hs(mako::gpu::Telemetry::layers);
            auto qb = put(hs, "q", q), kb = put(hs, "k", k), vb = put(hs, "v", v);
            auto ob = hs.scratch("o", n * 4), ob2 = hs.scratch("o2", n * 4);
            auto* enc = hs.encoder();
            hs.section(enc, 1, 0);
            hs.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX, D, opt);
            hs.commit_ahead(enc);  // section (1, 0) ends here
            hs.attention(enc, qb, kb, vb, ob2, S, S, S, S, heads, kv, 0, 0, D, opt);  // untimed
            hs.ahead_ok = false;
            hs.commit_ahead(enc);  // refused by the hook: no effect
            hs.section(enc, 2, 0);
            hs.attention(enc, qb, kb, vb, ob, S, S, S, S, heads, kv, 0, UINT32_MAX, D, opt);
            const int committed_before = hs.committed;
            hs.submit(enc);
            const bool hooks_once = committed_before == 0 && hs.committed == 1 && hs.completed == 1;
            const auto secs = hs.section_times();
            const auto o = get<float>(ob, n);
            hs.attention(enc, qb, kb, vb, ob2, S, S, S, S, heads, kv, 0, UINT32_MAX, D, opt);
            hs.finish(enc);
            const auto o2 = get<float>(ob2, n);
            const bool ok = hooks_once && hs.committed == 2 && hs.completed == 2 && hs.stats().commits_ahead == 1 &&
                            secs.size() == 2 && secs[0].layer == 1 && secs[0].section == 0 && secs[0].ms > 0 &&
                            secs[1].layer == 2 && secs[1].section == 0 && secs[1].ms > 0 &&
                            std::memcmp(o.data(), once.data(), n * 4) == 0 &&
                            std::memcmp(o2.data(), once.data(), n * 4) == 0 && hs.section_times().empty();
            check(ok, "commit_ahead ends section (1, 0) without a wait, a refused commit_ahead does nothing, submit "
                      "finishes once (hooks " + std::to_string(hs.committed) + "/" + std::to_string(hs.completed) +
                      ", sections " + std::to_string(secs.size()) + "), outputs bit-equal");
        }
        {
            using mako::gpu::RepeatSpec;
            const RepeatSpec a = RepeatSpec::parse("flash,,cube:select:4");
            const RepeatSpec b = RepeatSpec::parse("attn:-2");
            const RepeatSpec c = RepeatSpec::parse(":x");
            bool threw = false;
            try {
                (void)RepeatSpec::parse("flash_fwd");
            } catch (const std::runtime_error&) {
                threw = true;
            }
            check(a.times == 4 && a.labels == std::vector<std::string>{"flash", "cube:select"} &&
                      a.matches("flash_fwd_128") && a.matches("cube:select") && !a.matches("cube_select") &&
                      b.times == 0 && c.times == 0 && c.labels.empty() && !c.matches("x") && threw &&
                      mako::gpu::parse_telemetry("layers") == mako::gpu::Telemetry::layers &&
                      !mako::gpu::parse_telemetry("Layers"),
                  "MAKO_REPEAT parse: comma-separated labels split at the last ':', counts clamped at 0, no ':' "
                  "throws; telemetry names exact");
        }
    }
    // A head width the reference refuses.
    {
        auto* enc = h.encoder();
        auto* b = h.scratch("q", 16);
        bool threw = false;
        try {
            h.attention(enc, b, b, b, b, 1, 64, 1, 128, 1, 1, 0, 0, 96);
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()) == "attention: heads of 96";
        }
        check(threw, "attention refuses heads of 96");
        h.finish(enc);
    }
    // Head tiles through heads_partial (norm, 96 of 128 rotated, a row map) and heads (rotation, padding cleared).
    {
        const uint32_t T = 300, H = 4, D = 128, ld = 3 * H * D, n_pad = 320, rot = 96;
        std::vector<float> x(size_t(T) * ld), cs(size_t(T) * D), w(D);
        for (auto& e : x)
            e = float(normal());
        for (size_t i = 0; i < cs.size() / 2; ++i) {
            const double a = 3.0 * normal();
            cs[2 * i] = float(std::cos(a));
            cs[2 * i + 1] = float(std::sin(a));
        }
        for (auto& e : w)
            e = float(1.0 + 0.25 * normal());
        std::vector<int32_t> map(T);
        for (uint32_t t = 0; t < T; ++t)
            map[t] = t % 7 == 3 ? -1 : int32_t((t * 37) % T);
        auto xb = put(h, "x", x), cb = put(h, "cs", cs), wb = put(h, "w", w), mb = put(h, "map", map);
        auto yb = h.scratch("y", size_t(H) * n_pad * D * 2);
        auto within_ulp = [&](const std::vector<uint16_t>& got, const std::vector<uint16_t>& want) {
            uint64_t bad = 0;
            for (size_t i = 0; i < want.size(); ++i) {
                const double g = oracle_f16_to_f32(got[i]), r = oracle_f16_to_f32(want[i]);
                bad += !(std::fabs(g - r) <= std::fabs(r) * 0x1p-10 + 0x1p-24);
            }
            return bad;
        };
        auto* enc = h.encoder();
        h.heads_partial(enc, xb, ld, 0, D, D, rot, H, T, n_pad, cb, wb, 1e-6f, yb, mb);
        h.finish(enc);
        const oracle_heads_args pa{T, ld, 0, D, D, H, n_pad, 0, 1, rot, 1e-6f, 0};
        std::vector<uint16_t> want(size_t(H) * n_pad * D, 0), got = get<uint16_t>(yb, want.size());
        oracle_heads(&pa, ORACLE_F16, x.data(), cs.data(), w.data(), map.data(), want.data());
        for (uint32_t hh = 0; hh < H; ++hh)  // rows past T are not the call's: compare the first T of each head
            for (uint32_t t = T; t < n_pad; ++t)
                for (uint32_t i = 0; i < D; ++i)
                    got[(size_t(hh) * n_pad + t) * D + i] = 0;
        uint64_t bad = within_ulp(got, want);
        check(bad == 0, "heads_partial (norm, 96 rotated, row map): " + std::to_string(bad) + " values past one ulp");

        enc = h.encoder();
        h.heads(enc, xb, ld, H * D, H, T, n_pad, cb, 1, yb);
        h.finish(enc);
        const oracle_heads_args ha{T, ld, H * D, D, D, H, n_pad, 0, 1, D, 0.0f, 1};
        std::fill(want.begin(), want.end(), 0x7777);
        oracle_heads(&ha, ORACLE_F16, x.data(), cs.data(), nullptr, nullptr, want.data());
        bad = within_ulp(get<uint16_t>(yb, want.size()), want);
        check(bad == 0, "heads (rope 1, padding cleared): " + std::to_string(bad) + " values past one ulp");

        bool threw = false;
        try {
            h.heads_partial(enc, xb, ld, 0, D, D, 95, H, T, n_pad, cb, wb, 1e-6f, yb);
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()) == "heads_partial: heads of 128 with 95 rotated";
        }
        check(threw, "heads_partial refuses an odd rotation");
    }
    // attention_rows(): the producers and attention in one call, against heads_partial x 3 + attention() through
    // the same runtime, bit for bit (32 / 8 heads of 128 over 300 tokens, q and k normed and rotated, bf16 tiles).
    {
        const uint32_t T = 300, H = 32, KV = 8, D = 128;
        std::vector<float> xq(size_t(T) * H * D), xk(size_t(T) * KV * D), xv(xk.size()), cs(size_t(T) * D);
        std::vector<float> wq(D), wk(D);
        for (auto* v : {&xq, &xk, &xv})
            for (auto& x : *v)
                x = float(2 * normal());
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t i = 0; i < D / 2; ++i) {
                const double ang = 0.001 * (t + 1) * (i + 1);
                cs[(size_t(t) * D / 2 + i) * 2] = float(std::cos(ang));
                cs[(size_t(t) * D / 2 + i) * 2 + 1] = float(std::sin(ang));
            }
        for (uint32_t i = 0; i < D; ++i) {
            wq[i] = float(0.5 + 0.004 * i);
            wk[i] = float(1.5 - 0.004 * i);
        }
        auto qx = put(h, "rq", xq), kx = put(h, "rk", xk), vx = put(h, "rv", xv), cb = put(h, "rcs", cs);
        auto wqb = put(h, "rwq", wq), wkb = put(h, "rwk", wk);
        auto o1 = h.scratch("ro1", size_t(T) * H * D * 4), o2 = h.scratch("ro2", size_t(T) * H * D * 4);
        auto qt = h.scratch("rqt", size_t(H) * T * D * 2), kt = h.scratch("rkt", size_t(KV) * T * D * 2);
        auto vt = h.scratch("rvt", size_t(KV) * T * D * 2);
        mako::models::AttnOptions opt;
        opt.in = MAKO_BF16;
        auto* enc = h.encoder();
        h.attention_rows(enc, qx, H * D, kx, vx, KV * D, cb, D, wqb, wkb, 1e-6f, o1, T, T, H, KV, 0, UINT32_MAX, D,
                         opt);
        h.heads_partial(enc, qx, H * D, 0, D, D, D, H, T, T, cb, wqb, 1e-6f, qt, nullptr, MAKO_BF16);
        h.heads_partial(enc, kx, KV * D, 0, D, D, D, KV, T, T, cb, wkb, 1e-6f, kt, nullptr, MAKO_BF16);
        h.heads_partial(enc, vx, KV * D, 0, D, D, 0, KV, T, T, nullptr, nullptr, 0.0f, vt, nullptr, MAKO_BF16);
        h.attention(enc, qt, kt, vt, o2, T, T, T, T, H, KV, 0, UINT32_MAX, D, opt);
        h.finish(enc);
        const auto a = get<uint32_t>(o1, size_t(T) * H * D), b = get<uint32_t>(o2, a.size());
        check(a == b, "attention_rows equals heads_partial x 3 + attention() bit for bit");
    }
    // The output projection after attention: proj() with BF16 weights (f32 rows, the split, bf16 rows).
    {
        const uint32_t T = 200, K = 512, N = 384, ldy = 400;
        std::vector<uint16_t> w(size_t(N) * K), xb16(size_t(T) * K);
        std::vector<float> x(size_t(T) * K), xa(x.size());
        std::vector<uint16_t> wa(w.size()), xba(xb16.size());
        for (size_t i = 0; i < w.size(); ++i) {
            w[i] = oracle_f32_to_bf16(float(0.05 * normal()));
            wa[i] = w[i] & 0x7fff;
        }
        for (size_t i = 0; i < x.size(); ++i) {
            x[i] = float(3.0 * normal());
            xa[i] = std::fabs(x[i]);
            xb16[i] = oracle_f32_to_bf16(x[i]);
            xba[i] = xb16[i] & 0x7fff;
        }
        auto wb = put(h, "w", w), xf = put(h, "x", x), xh = put(h, "xb", xb16);
        auto yb = h.scratch("y", size_t(T) * ldy * 4);
        const Harness::Weight W{wb, 0, K, N};
        auto run = [&](bool split, bool bf16_in, const char* what) {
            h.bf16_split_ = split;
            auto* enc = h.encoder();
            h.proj(enc, W, bf16_in ? xh : xf, 0, yb, 0, T, ldy, bf16_in);
            h.finish(enc);
            h.bf16_split_ = false;
            std::vector<double> want(size_t(T) * ldy, 0.0), mag(size_t(T) * ldy, 0.0);
            const int dt = bf16_in ? ORACLE_BF16 : ORACLE_F32;
            oracle_proj_bf16(T, K, N, K, ldy, dt, split, w.data(), bf16_in ? (const void*)xb16.data() : x.data(),
                             want.data());
            oracle_proj_bf16(T, K, N, K, ldy, dt, split, wa.data(), bf16_in ? (const void*)xba.data() : xa.data(),
                             mag.data());
            const std::vector<float> got = get<float>(yb, want.size());
            uint64_t bad = 0;
            for (uint32_t t = 0; t < T; ++t)
                for (uint32_t c = 0; c < N; ++c) {
                    const size_t i = size_t(t) * ldy + c;
                    bad += !(std::fabs(got[i] - want[i]) <= (split ? 4.0 : 2.0) * K * 0x1p-24 * mag[i] + 1e-30);
                }
            check(bad == 0, std::string(what) + ": " + std::to_string(bad) + " elements past the summation bound");
        };
        run(false, false, "proj, f32 rows");
        run(true, false, "proj, f32 rows with the bf16 split");
        run(false, true, "proj, bf16 rows");
        bool threw = false;
        auto* enc = h.encoder();
        try {
            h.proj(enc, Harness::Weight{wb, 0, 96, N}, xf, 0, yb, 0, T);
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()) == "BF16 96x384: k must be a multiple of 64";
        }
        h.finish(enc);
        check(threw, "proj refuses k = 96");
    }
    // The gated delta rule as the linear-attention layer calls it.
    {
        const uint32_t T = 100, VH = 4, D = 128, vw = VH * D;
        std::vector<float> q(size_t(T) * vw), k(q.size()), v(q.size()), g(q.size()), beta(size_t(T) * VH);
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t hh = 0; hh < VH; ++hh) {
                double nq = 0, nk = 0;
                float* qr = &q[size_t(t) * vw + hh * D];
                float* kr = &k[size_t(t) * vw + hh * D];
                for (uint32_t i = 0; i < D; ++i) {
                    qr[i] = float(normal());
                    kr[i] = float(normal());
                    nq += double(qr[i]) * qr[i];
                    nk += double(kr[i]) * kr[i];
                }
                for (uint32_t i = 0; i < D; ++i) {  // unit q and k per head, as the layer's L2 norm gives them
                    qr[i] = float(qr[i] / std::sqrt(nq));
                    kr[i] = float(kr[i] / std::sqrt(nk));
                }
                beta[size_t(t) * VH + hh] = float(0.5 + 0.4 * std::tanh(normal()));
            }
        for (size_t i = 0; i < v.size(); ++i) {
            v[i] = float(normal());
            g[i] = float(-0.25 * std::fabs(normal()));
        }
        std::vector<float> zero(size_t(VH) * D * D, 0.0f);
        auto qb = put(h, "kq", q), kb = put(h, "kk", k), vb = put(h, "kv", v), gb = put(h, "kg", g);
        auto bb = put(h, "kbeta", beta), sb = put(h, "kstate", zero);
        auto ob = h.scratch("ko", q.size() * 4);
        auto* enc = h.encoder();
        h.kda_scan(enc, qb, kb, vb, gb, bb, sb, ob, T, vw, vw, VH);
        h.finish(enc);
        std::vector<double> want_o(q.size()), want_s(zero.size(), 0.0);
        oracle_kda_scan(D, T, vw, vw, VH, 0, q.data(), k.data(), v.data(), g.data(), beta.data(), want_s.data(),
                        want_o.data(), nullptr);
        const std::vector<float> got_o = get<float>(ob, want_o.size()), got_s = get<float>(sb, want_s.size());
        uint64_t bad = 0;
        for (size_t i = 0; i < want_o.size(); ++i)
            bad += !(std::fabs(got_o[i] - want_o[i]) <= 2e-5 + 1e-4 * std::fabs(want_o[i]));
        for (size_t i = 0; i < want_s.size(); ++i)
            bad += !(std::fabs(got_s[i] - want_s[i]) <= 2e-5 + 1e-4 * std::fabs(want_s[i]));
        check(bad == 0, "kda_scan, 4 heads over 100 tokens: " + std::to_string(bad) + " values out of tolerance");
    }
    // Runtime-owned scratch: every workspace the attention calls need is the Runtime's named scratch (the
    // reference's Runtime owns its scratch, src/gpu/runtime.cpp:117-125): after a warm-up, repeated calls allocate
    // nothing (scratch_bytes() stable), and the library holds no buffer of its own.
    {
        const uint32_t H = 32, KV = 8, D = 128, S = 1024;
        const auto q = random_tile(size_t(H) * S * D, ORACLE_BF16), k = random_tile(size_t(KV) * S * D, ORACLE_BF16);
        auto qb = put(h, "wq", q), kb = put(h, "wk", k), vb = put(h, "wv", k);
        auto ob = h.scratch("wo", size_t(S) * H * D * 4);
        mako::models::AttnOptions opt;
        opt.in = MAKO_BF16;
        const uint32_t D2 = 256, H2 = 4, KV2 = 2, S2 = 200;
        const auto q2 = random_tile(size_t(H2) * 256 * D2, ORACLE_BF16);
        auto q2b = put(h, "wq2", q2), k2b = put(h, "wk2", q2);
        // the sparse r64 route: lists per kv head, 4 query heads each; every cube sees itself
        const uint32_t cubes = S / 64;
        std::vector<uint16_t> sel(size_t(KV) * cubes), nsel(size_t(KV) * cubes, 1);
        for (uint32_t i = 0; i < KV * cubes; ++i)
            sel[i] = uint16_t(i % cubes);
        std::vector<uint8_t> valid(S, 1);
        std::vector<int32_t> map(S);
        for (uint32_t i = 0; i < S; ++i)
            map[i] = int32_t(i);
        auto selb = put(h, "wsel", sel), nselb = put(h, "wnsel", nsel), validb = put(h, "wvalid", valid);
        auto mapb = put(h, "wmap", map);
        mako::models::AttnOptions sopt = opt;
        sopt.sel_per_kv_head = true;
        uint64_t bytes[3] = {0, 0, 0};
        for (int round = 0; round < 3; ++round) {
            auto* enc = h.encoder();
            h.attention(enc, qb, kb, vb, ob, 2, 64, S, S, H, KV, S - 2, UINT32_MAX, D, opt);   // split-K partials
            h.attention(enc, q2b, k2b, k2b, ob, S2, 256, S2, 256, H2, KV2, 0, UINT32_MAX, D2, opt);  // none (r32)
            h.attention_sparse(enc, qb, kb, vb, ob, S, S, S, S, H, KV, H * D, cubes, 1, S, S, selb, nselb, validb,
                               mapb, sopt);                                                       // pass table
            h.finish(enc);
            bytes[round] = h.scratch_bytes();
        }
        check(bytes[1] == bytes[0] && bytes[2] == bytes[0] && mako_attn_held_bytes() == 0,
              "Runtime-owned scratch: scratch bytes " + std::to_string(bytes[0]) + " / " + std::to_string(bytes[1]) +
                  " / " + std::to_string(bytes[2]) + ", library-held " + std::to_string(mako_attn_held_bytes()));
    }
    for (const auto& kt : h.kernel_times())
        std::printf("  %-20s %3u launches %8.3f ms\n", kt.kernel.c_str(), kt.count, kt.ms);
    std::printf("%s\n", failures ? "FAILED" : "all passed");
    return failures ? 1 : 0;
}
