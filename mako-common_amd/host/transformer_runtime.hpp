// The attention calls of the reference's TransformerRuntime (src/models/runtime.hpp:90-111) with their parameter
// lists kept, over HIP: `MTL::ComputeCommandEncoder*&` becomes the launch queue (gpu::Encoder*&) and
// `MTL::Buffer*` a device buffer (gpu::Buffer*). Each call checks its arguments (throwing what the reference
// throws, src/models/runtime.cpp:266-267, 290-291, 311-312), then enqueues through the C ABI of
// include/mako_attn.h; results are visible after finish().
//
// Defaults keep the reference's behaviour: f16 tiles in, f32 rows out, no LSE. AttnOptions (a trailing
// argument the reference's call sites never pass) selects bf16 inputs, a bf16 / f16 output, an LSE buffer, and,
// for the sparse call, the causal flag and lists shared by a kv head's query heads.
#pragma once

#include <cstdint>

#include "gpu_runtime.hpp"
#include "mako_attn.h"

namespace mako::models {

struct AttnOptions {
    mako_dtype in = MAKO_F16;
    mako_dtype out = MAKO_F32;
    gpu::Buffer* lse = nullptr;  // float [heads][n_q] (sparse: [heads][q_pad])
    bool causal = false;         // attention_sparse: key j seen by tile row r only when j <= r
    bool sel_per_kv_head = false;  // attention_sparse: sel / nsel hold one list per kv head
};

class TransformerRuntime : public gpu::Runtime {
public:
    virtual const char* name() const { return "model"; }

protected:
    explicit TransformerRuntime(gpu::Telemetry telemetry, int device = 0) : gpu::Runtime(telemetry, device) {}

    static constexpr uint32_t kHeadDim = 128;
    static constexpr uint32_t kAttnRows = 64;  // query rows of a tile: q_pad is a multiple of it
    static uint32_t round_up(uint32_t x, uint32_t m) { return (x + m - 1) / m * m; }

    // Head tiles from fp32 rows (src/models/runtime.hpp:78-89): head h of token t, x[t][col0 + h * dim ..], into
    // y [heads][n_pad][dim] (f16, as the reference's half tiles, or bf16 by `out`). heads(): dim 128, rotated by
    // cs [T][64] (cos, sin) pairs when rope is 1 (value i with i + 64) or 2 (2i with 2i + 1), rows [T, n_pad)
    // zeroed. heads_norm(): each head RMS-normed first (times w [128]), written from y row row0, the rows past T
    // left as they are; cs_off is a byte offset into cs. heads_partial(): heads of dim (a multiple of 32, at most
    // 256) `stride` apart, the first rot values rotated (i with i + rot / 2, cs [T][rot / 2]), the norm when w is
    // given, and through the row map when given (y row t from x row map[t], a zero row where map[t] < 0).
    void heads(gpu::Encoder*& enc, gpu::Buffer* x, uint32_t ld, uint32_t col0, uint32_t heads, uint32_t T,
               uint32_t n_pad, gpu::Buffer* cs, uint32_t rope, gpu::Buffer* y, mako_dtype out = MAKO_F16);
    void heads_norm(gpu::Encoder*& enc, gpu::Buffer* x, uint32_t ld, uint32_t col0, uint32_t heads, uint32_t T,
                    uint32_t n_pad, gpu::Buffer* cs, uint64_t cs_off, uint32_t rope, gpu::Buffer* w, float eps,
                    uint32_t row0, gpu::Buffer* y, mako_dtype out = MAKO_F16);
    void heads_partial(gpu::Encoder*& enc, gpu::Buffer* x, uint32_t ld, uint32_t col0, uint32_t stride, uint32_t dim,
                       uint32_t rot, uint32_t heads, uint32_t T, uint32_t n_pad, gpu::Buffer* cs, gpu::Buffer* w,
                       float eps, gpu::Buffer* y, gpu::Buffer* map = nullptr, mako_dtype out = MAKO_F16);
    // Flash attention over tiles q [heads][q_pad][dim], k and v [kv_heads][k_pad][dim] into o [n_q][heads * dim].
    // block: positions from here on see each other both ways; below it, causal (0: all both ways). dim 64, 128
    // or 256.
    void attention(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* o, uint32_t n_q,
                   uint32_t q_pad, uint32_t n_k, uint32_t k_pad, uint32_t heads, uint32_t kv_heads, uint32_t q_pos0,
                   uint32_t block, uint32_t dim = kHeadDim, const AttnOptions& opt = {});
    // Attention straight from fp32 projection rows (no counterpart in the reference, whose prefill steps call the
    // producers and then attention): query heads of dim `dim` side by side in xq rows of ld_q, key and value heads
    // in xk / xv rows of ld_kv; q and k RMS-normed when wq / wk are given (eps) and their first rot values rotated
    // by cs [T][rot / 2] (i with i + rot / 2) as heads_partial does, v sliced; then attention() over them. The
    // same results as those calls, in two launches where the fused kernels apply (mako_attn_fwd_rows).
    void attention_rows(gpu::Encoder*& enc, gpu::Buffer* xq, uint32_t ld_q, gpu::Buffer* xk, gpu::Buffer* xv,
                        uint32_t ld_kv, gpu::Buffer* cs, uint32_t rot, gpu::Buffer* wq, gpu::Buffer* wk, float eps,
                        gpu::Buffer* o, uint32_t n_q, uint32_t n_k, uint32_t heads, uint32_t kv_heads,
                        uint32_t q_pos0, uint32_t block, uint32_t dim = kHeadDim, const AttnOptions& opt = {});
    // Per head and query cube, the `topk` key cubes by the dot product of the cubes' mean q and k, into the
    // Runtime-owned scratch sel [heads][n_cubes][min(topk, n_cubes)] and nsel [heads][n_cubes] (returned by
    // reference, valid until the next call). local: 0 by score alone, 1 the query cube first, 3 also the cubes
    // `stride` before and after.
    void cube_select(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, uint32_t heads, uint32_t q_pad, uint32_t k_pad,
                     uint32_t n_cubes, gpu::Buffer* cnt, uint32_t topk, gpu::Buffer*& sel, gpu::Buffer*& nsel,
                     uint32_t local = 0, uint32_t stride = 0, mako_dtype in = MAKO_F16);
    // Each cube's queries over its selected cubes and the dense rows [dense0, dense1), the later rows' queries
    // over everything; query row r's output to o row map[r] (dropped when negative).
    void attention_sparse(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* o,
                          uint32_t n_q, uint32_t q_pad, uint32_t n_k, uint32_t k_pad, uint32_t heads, uint32_t kv_heads,
                          uint32_t width, uint32_t n_cubes, uint32_t topk, uint32_t dense0, uint32_t dense1,
                          gpu::Buffer* sel, gpu::Buffer* nsel, gpu::Buffer* valid, gpu::Buffer* map,
                          const AttnOptions& opt = {});
    // The gated delta rule of the linear-attention layers (the reference dispatches kda_scan by name in
    // QwenText::linear_layer, src/models/qwen_text.cpp:374-382, with ScanArgs {128, T, vw, vw, VH, 0}): q, k, v rows
    // qkv_stride floats apart, g and o rows `inner` apart, beta [T][heads], state [heads][128][128] (transposed,
    // updated in place), snap_state the state after `snap` tokens when snap is nonzero.
    void kda_scan(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* g,
                  gpu::Buffer* beta, gpu::Buffer* state, gpu::Buffer* o, uint32_t T, uint32_t qkv_stride,
                  uint32_t inner, uint32_t heads, uint32_t snap = 0, gpu::Buffer* snap_state = nullptr);
    // One new token for each of `batch` sequences against a contiguous cache: q [batch][heads][128],
    // k and v [batch][kv_heads][cap][128], ctx_len u32 [batch] (device), o [batch][heads * 128]; split-K with the
    // partials in the Runtime-owned scratch "attn_decode". No counterpart in the reference (it decodes one sequence
    // at a time through attention() with n_q = 1).
    void attention_decode(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* ctx_len,
                          gpu::Buffer* o, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t cap,
                          uint32_t max_ctx, const AttnOptions& opt = {});
};

}  // namespace mako::models
