// Block-sparse attention through TransformerRuntime against the CPU oracle, as the reference's own test does it
// (tests/sparse_attn_test.cpp:41-211): cube_select's pooled scores and top-k, then attention_sparse over 6 cubes
// (one with padding rows) and 60 dense rows, each cube's queries over its selected cubes and the dense rows, the
// dense rows' queries over everything; rows mapped back through an identity map with the padding dropped.
// Checks: the selection equals the CPU's exactly; the worst row's relative L2 error < 5e-3; padding and
// out-of-range rows keep the sentinel; with local = 3, stride 1, each cube and its neighbours lead the selection
// without duplicates. Inputs: seeded N(0, 1) from splitmix64 + Box-Muller (the reference's mt19937 +
// std::normal_distribution is implementation-defined), rounded to f16; invalid rows zero.
//   sparse_attn_test
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "attn_oracle.h"
#include "transformer_runtime.hpp"

namespace {

class Harness final : public mako::models::TransformerRuntime {
public:
    Harness() : TransformerRuntime(mako::gpu::Telemetry::kernels) {}
    const char* name() const override { return "sparse attention test"; }
    using TransformerRuntime::attention_sparse;
    using TransformerRuntime::cube_select;
    using TransformerRuntime::encoder;
    using TransformerRuntime::finish;
    using TransformerRuntime::scratch;
};

int failures = 0;
void check(bool ok, const std::string& what)
{
    std::printf("  %s  %s\n", ok ? "ok  " : "FAIL", what.c_str());
    failures += !ok;
}

struct Normal {  // splitmix64 + Box-Muller
    uint64_t s;
    bool have = false;
    double spare = 0;
    uint64_t next()
    {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double operator()()
    {
        if (have) {
            have = false;
            return spare;
        }
        const double u1 = ((next() >> 11) + 0.5) * 0x1.0p-53, u2 = (next() >> 11) * 0x1.0p-53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        spare = r * std::sin(2 * M_PI * u2);
        have = true;
        return r * std::cos(2 * M_PI * u2);
    }
};

template <class T>
void upload(Harness& h, mako::gpu::Buffer* b, const std::vector<T>& v)
{
    if (hipMemcpy(b->ptr, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    (void)h;
}

template <class T>
std::vector<T> download(const mako::gpu::Buffer* b, size_t n)
{
    std::vector<T> v(n);
    if (hipMemcpy(v.data(), b->ptr, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return v;
}

}  // namespace

int main()
{
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    Harness h;
    constexpr uint32_t D = 128, heads = 2, cubes = 6, dense = 60, topk = 3;  // 444 rows: q padded to 448, k to 512
    const uint32_t cnt[cubes] = {64, 64, 64, 64, 64, 20};
    const uint32_t n = cubes * 64 + dense, q_pad = (n + 63) / 64 * 64, k_pad = (n + 127) / 128 * 128;
    const uint32_t dense0 = cubes * 64, dense1 = n;
    std::vector<uint8_t> valid(k_pad, 0);
    std::vector<int32_t> map(q_pad, -1);
    for (uint32_t c = 0; c < cubes; ++c)
        for (uint32_t r = 0; r < cnt[c]; ++r)
            valid[c * 64 + r] = 1;
    for (uint32_t r = dense0; r < dense1; ++r)
        valid[r] = 1;
    for (uint32_t r = 0; r < n; ++r)
        if (valid[r])
            map[r] = int32_t(r);
    Normal nd{7};
    std::vector<uint16_t> qh(size_t(heads) * q_pad * D), kh(size_t(heads) * k_pad * D), vh(kh.size());
    for (auto [t, pad] : {std::pair{&qh, q_pad}, std::pair{&kh, k_pad}, std::pair{&vh, k_pad}})
        for (uint32_t hh = 0; hh < heads; ++hh)
            for (uint32_t r = 0; r < pad; ++r)
                for (uint32_t d = 0; d < D; ++d)
                    (*t)[(size_t(hh) * pad + r) * D + d] = oracle_f32_to_f16(valid[r] ? float(nd()) : 0.0f);
    auto qb = h.scratch("t_q", qh.size() * 2), kb = h.scratch("t_k", kh.size() * 2), vb = h.scratch("t_v", vh.size() * 2);
    upload(h, qb, qh);
    upload(h, kb, kh);
    upload(h, vb, vh);
    auto cntb = h.scratch("t_cnt", sizeof(cnt));
    upload(h, cntb, std::vector<uint32_t>(cnt, cnt + cubes));
    auto validb = h.scratch("t_valid", k_pad);
    upload(h, validb, valid);
    auto mapb = h.scratch("t_map", q_pad * 4);
    upload(h, mapb, map);
    auto ob = h.scratch("t_o", uint64_t(q_pad) * heads * D * 4);
    upload(h, ob, std::vector<float>(size_t(q_pad) * heads * D, 12345.0f));
    mako::gpu::Buffer *sel = nullptr, *nsel = nullptr;
    {
        auto* enc = h.encoder();
        h.cube_select(enc, qb, kb, heads, q_pad, k_pad, cubes, cntb, topk, sel, nsel);
        h.attention_sparse(enc, qb, kb, vb, ob, n, q_pad, n, k_pad, heads, heads, heads * D, cubes, topk, dense0, dense1,
                           sel, nsel, validb, mapb);
        h.finish(enc);
    }
    // The selection against the CPU's.
    const auto gsel = download<uint16_t>(sel, size_t(heads) * cubes * topk);
    const auto gnsel = download<uint16_t>(nsel, size_t(heads) * cubes);
    std::vector<uint16_t> csel(gsel.size()), cnsel(gnsel.size());
    oracle_cube_select(heads, D, ORACLE_F16, qh.data(), q_pad, kh.data(), k_pad, cubes, cnt, topk, 0, 0, csel.data(),
                       cnsel.data(), nullptr, nullptr, nullptr);
    uint32_t sel_bad = 0;
    for (uint32_t i = 0; i < heads * cubes; ++i)
        sel_bad += !std::equal(gsel.begin() + i * topk, gsel.begin() + (i + 1) * topk, csel.begin() + i * topk) ||
                   gnsel[i] != topk;
    check(sel_bad == 0, std::to_string(sel_bad) + " of " + std::to_string(heads * cubes) +
                            " selections differ from the CPU's");
    // The attention against the CPU's, over the GPU's selection.
    const auto of = download<float>(ob, size_t(q_pad) * heads * D);
    const oracle_sparse_args a{n, q_pad, n, k_pad, heads, heads, heads * D, 1.0f / std::sqrt(float(D)), cubes, topk,
                               dense0, dense1, 0, heads};
    std::vector<double> ref(size_t(q_pad) * heads * D, 12345.0);
    oracle_attn_sparse(&a, ORACLE_F16, qh.data(), kh.data(), vh.data(), gsel.data(), gnsel.data(), valid.data(),
                       map.data(), ref.data(), q_pad, nullptr, 0);
    double worst = 0;
    uint64_t untouched_bad = 0, elem_bad = 0;
    for (uint32_t r = 0; r < q_pad; ++r)
        for (uint32_t hh = 0; hh < heads; ++hh) {
            const float* out = &of[(size_t(r) * heads + hh) * D];
            const double* want = &ref[(size_t(r) * heads + hh) * D];
            if (r >= n || !valid[r]) {
                for (uint32_t d = 0; d < D; ++d)
                    untouched_bad += out[d] != 12345.0f;
                continue;
            }
            double e = 0, nrm = 0;
            for (uint32_t d = 0; d < D; ++d) {
                const double diff = out[d] - want[d];
                e += diff * diff;
                nrm += want[d] * want[d];
                elem_bad += std::fabs(diff) > 2e-3 + 1e-2 * std::fabs(want[d]);
            }
            worst = std::max(worst, std::sqrt(e / std::max(nrm, 1e-30)));
        }
    char msg[128];
    std::snprintf(msg, sizeof(msg), "attention_sparse: worst row rel error %.2e", worst);
    check(worst < 5e-3, msg);
    check(elem_bad == 0, "attention_sparse: " + std::to_string(elem_bad) + " elements past 2e-3 + 1e-2 |ref|");
    check(untouched_bad == 0, "padding and out-of-range rows left alone (" + std::to_string(untouched_bad) +
                                  " values written)");
    // The local option: the query cube and its neighbours (stride 1) lead the selection, the rest by score.
    {
        auto* enc = h.encoder();
        h.cube_select(enc, qb, kb, heads, q_pad, k_pad, cubes, cntb, 4, sel, nsel, 3, 1);
        h.finish(enc);
        const auto s4 = download<uint16_t>(sel, size_t(heads) * cubes * 4);
        uint32_t bad = 0;
        for (uint32_t hh = 0; hh < heads; ++hh)
            for (uint32_t qc = 0; qc < cubes; ++qc) {
                const uint16_t* e = &s4[(size_t(hh) * cubes + qc) * 4];
                std::vector<uint32_t> want{qc};
                if (qc >= 1)
                    want.push_back(qc - 1);
                if (qc + 1 < cubes)
                    want.push_back(qc + 1);
                for (size_t i = 0; i < want.size(); ++i)
                    bad += e[i] != want[i];
                for (uint32_t i = 0; i < 4; ++i)  // no cube twice
                    for (uint32_t j = i + 1; j < 4; ++j)
                        bad += e[i] == e[j];
            }
        check(bad == 0, "cube_select with local cubes: " + std::to_string(bad) + " entries off");
    }
    // The refusals the reference's host code makes.
    {
        auto* enc = h.encoder();
        bool threw = false;
        try {
            h.attention_sparse(enc, qb, kb, vb, ob, n, q_pad + 1, n, k_pad, heads, heads, heads * D, cubes, topk,
                               dense0, dense1, sel, nsel, validb, mapb);
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()).find("q_pad a multiple of 64") != std::string::npos;
        }
        check(threw, "attention_sparse refuses a q_pad that is not a multiple of 64");
        threw = false;
        try {
            h.cube_select(enc, qb, kb, heads, q_pad, k_pad, cubes, cntb, 0, sel, nsel);
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()).find("top 0") != std::string::npos;
        }
        check(threw, "cube_select refuses topk 0");
        h.finish(enc);
    }
    for (const auto& kt : h.kernel_times())
        std::printf("  %-20s %3u launches %8.3f ms\n", kt.kernel.c_str(), kt.count, kt.ms);
    std::printf("%s\n", failures ? "FAILED" : "all passed");
    return failures ? 1 : 0;
}
