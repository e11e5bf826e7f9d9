#include "transformer_runtime.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>

namespace mako::models {

namespace {

template <class... A>
std::string fmt(const char* f, A... a)
{
    char buf[256];
    std::snprintf(buf, sizeof(buf), f, a...);
    return buf;
}

}  // namespace

void TransformerRuntime::heads(gpu::Encoder*& enc, gpu::Buffer* x, uint32_t ld, uint32_t col0, uint32_t n_heads,
                               uint32_t T, uint32_t n_pad, gpu::Buffer* cs, uint32_t rope, gpu::Buffer* y,
                               mako_dtype out)
{
    const mako_heads_args a{T, ld, col0, kHeadDim, kHeadDim, n_heads, n_pad, 0, rope, rope ? kHeadDim : 0u, 0.0f,
                            1};
    before(enc);
    for (int r = repeats("heads"); r > 0; --r)
        check(mako_heads(&a, out, static_cast<const float*>(x->ptr), cs ? static_cast<const float*>(cs->ptr) : nullptr,
                         nullptr, nullptr, y->ptr, enc->stream));
    after(enc, "heads");
}

void TransformerRuntime::heads_norm(gpu::Encoder*& enc, gpu::Buffer* x, uint32_t ld, uint32_t col0, uint32_t n_heads,
                                    uint32_t T, uint32_t n_pad, gpu::Buffer* cs, uint64_t cs_off, uint32_t rope,
                                    gpu::Buffer* w, float eps, uint32_t row0, gpu::Buffer* y, mako_dtype out)
{
    const mako_heads_args a{T, ld, col0, kHeadDim, kHeadDim, n_heads, n_pad, row0, rope, rope ? kHeadDim : 0u, eps,
                            0};
    const float* c = cs ? reinterpret_cast<const float*>(static_cast<const char*>(cs->ptr) + cs_off) : nullptr;
    before(enc);
    for (int r = repeats("heads_norm"); r > 0; --r)
        check(mako_heads(&a, out, static_cast<const float*>(x->ptr), c, static_cast<const float*>(w->ptr), nullptr,
                         y->ptr, enc->stream));
    after(enc, "heads_norm");
}

void TransformerRuntime::heads_partial(gpu::Encoder*& enc, gpu::Buffer* x, uint32_t ld, uint32_t col0,
                                       uint32_t stride, uint32_t dim, uint32_t rot, uint32_t n_heads, uint32_t T,
                                       uint32_t n_pad, gpu::Buffer* cs, gpu::Buffer* w, float eps, gpu::Buffer* y,
                                       gpu::Buffer* map, mako_dtype out)
{
    if (dim > 256 || dim % 32 || rot % 2)
        throw std::runtime_error(fmt("heads_partial: heads of %u with %u rotated", dim, rot));
    const mako_heads_args a{T, ld, col0, stride, dim, n_heads, n_pad, 0, rot ? 1u : 0u, rot, w ? eps : 0.0f, 0};
    before(enc);
    for (int r = repeats("heads_partial"); r > 0; --r)
        check(mako_heads(&a, out, static_cast<const float*>(x->ptr), cs ? static_cast<const float*>(cs->ptr) : nullptr,
                         w ? static_cast<const float*>(w->ptr) : nullptr,
                         map ? static_cast<const int32_t*>(map->ptr) : nullptr, y->ptr, enc->stream));
    after(enc, "heads_partial");
}

void TransformerRuntime::kda_scan(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* g,
                                  gpu::Buffer* beta, gpu::Buffer* state, gpu::Buffer* o, uint32_t T,
                                  uint32_t qkv_stride, uint32_t inner, uint32_t n_heads, uint32_t snap,
                                  gpu::Buffer* snap_state)
{
    const mako_scan_args a{kHeadDim, T, qkv_stride, inner, n_heads, snap};
    auto f = [](gpu::Buffer* b) { return b ? static_cast<float*>(b->ptr) : nullptr; };
    before(enc);
    for (int r = repeats("kda_scan"); r > 0; --r)
        check(mako_kda_scan(&a, f(q), f(k), f(v), f(g), f(beta), f(state), f(o), f(snap_state), enc->stream));
    after(enc, "kda_scan");
}

void TransformerRuntime::attention(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* o,
                                   uint32_t n_q, uint32_t q_pad, uint32_t n_k, uint32_t k_pad, uint32_t n_heads,
                                   uint32_t kv_heads, uint32_t q_pos0, uint32_t block, uint32_t dim,
                                   const AttnOptions& opt)
{
    if (dim != 64 && dim != 128 && dim != 256)
        throw std::runtime_error(fmt("attention: heads of %u", dim));
    const mako_attn_args a{n_q, q_pad, n_k, k_pad, n_heads, kv_heads, q_pos0, block, n_heads * dim,
                           1.0f / std::sqrt(float(dim))};
    const char* label = dim == 64 ? "flash_fwd_64" : dim == 128 ? "flash_fwd_128" : "flash_fwd_256";
    // the split-K partials (a few rows) or the V^T images (heads of 256) live in Runtime-owned scratch
    const size_t need = mako_attn_fwd_workspace(&a, dim);
    gpu::Buffer* ws = need ? scratch("attn_fwd", need) : nullptr;
    before(enc);
    for (int r = repeats(label); r > 0; --r)
        check(mako_attn_fwd_ws(&a, dim, opt.in, opt.out, q->ptr, k->ptr, v->ptr, o->ptr,
                               opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr, ws ? ws->ptr : nullptr,
                               ws ? ws->bytes : 0, enc->stream));
    after(enc, label);
}

void TransformerRuntime::attention_rows(gpu::Encoder*& enc, gpu::Buffer* xq, uint32_t ld_q, gpu::Buffer* xk,
                                        gpu::Buffer* xv, uint32_t ld_kv, gpu::Buffer* cs, uint32_t rot,
                                        gpu::Buffer* wq, gpu::Buffer* wk, float eps, gpu::Buffer* o, uint32_t n_q,
                                        uint32_t n_k, uint32_t n_heads, uint32_t kv_heads, uint32_t q_pos0,
                                        uint32_t block, uint32_t dim, const AttnOptions& opt)
{
    if (dim != 64 && dim != 128 && dim != 256)
        throw std::runtime_error(fmt("attention: heads of %u", dim));
    if (rot % 2 || rot > dim)
        throw std::runtime_error(fmt("heads_partial: heads of %u with %u rotated", dim, rot));
    const uint32_t rope = rot ? 1u : 0u;
    const mako_heads_args hq{n_q, ld_q, 0, dim, dim, n_heads, n_q, 0, rope, rot, wq ? eps : 0.0f, 0};
    const mako_heads_args hk{n_k, ld_kv, 0, dim, dim, kv_heads, n_k, 0, rope, rot, wk ? eps : 0.0f, 0};
    const mako_heads_args hv{n_k, ld_kv, 0, dim, dim, kv_heads, n_k, 0, 0, 0, 0.0f, 0};
    const mako_attn_args a{n_q, 0, n_k, 0, n_heads, kv_heads, q_pos0, block, n_heads * dim,
                           1.0f / std::sqrt(float(dim))};
    const auto f = [](gpu::Buffer* b) { return b ? static_cast<const float*>(b->ptr) : nullptr; };
    const size_t need = mako_attn_fwd_rows_workspace(&a, dim);
    gpu::Buffer* ws = need ? scratch("attn_rows", need) : nullptr;
    before(enc);
    for (int r = repeats("attention_rows"); r > 0; --r)
        check(mako_attn_fwd_rows_ws(&a, &hq, &hk, &hv, opt.in, opt.out, f(xq), f(xk), f(xv), f(cs), f(wq), f(wk),
                                    o->ptr, opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr,
                                    ws ? ws->ptr : nullptr, ws ? ws->bytes : 0, enc->stream));
    after(enc, "attention_rows");
}

void TransformerRuntime::cube_select(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, uint32_t heads, uint32_t q_pad,
                                     uint32_t k_pad, uint32_t n_cubes, gpu::Buffer* cnt, uint32_t topk,
                                     gpu::Buffer*& sel, gpu::Buffer*& nsel, uint32_t local, uint32_t stride,
                                     mako_dtype in)
{
    if (n_cubes > 4096 || !topk || (local != 0 && local != 1 && local != 3))
        throw std::runtime_error(fmt("cube_select: %u cubes, top %u, local %u", n_cubes, topk, local));
    const uint32_t kk = std::min(topk, n_cubes);
    gpu::Buffer* ws = scratch("c_work", mako_cube_select_workspace(heads, n_cubes));
    sel = scratch("c_sel", uint64_t(heads) * n_cubes * kk * 2);
    nsel = scratch("c_nsel", uint64_t(heads) * n_cubes * 2);
    before(enc);
    for (int r = repeats("cube_select"); r > 0; --r)
        check(mako_cube_select(heads, q_pad, k_pad, n_cubes, topk, local, stride, in, q->ptr, k->ptr,
                               static_cast<const uint32_t*>(cnt->ptr), static_cast<uint16_t*>(sel->ptr),
                               static_cast<uint16_t*>(nsel->ptr), ws->ptr, ws->bytes, enc->stream));
    after(enc, "cube_select");
}

void TransformerRuntime::attention_sparse(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v,
                                          gpu::Buffer* o, uint32_t n_q, uint32_t q_pad, uint32_t n_k, uint32_t k_pad,
                                          uint32_t heads, uint32_t kv_heads, uint32_t width, uint32_t n_cubes,
                                          uint32_t topk, uint32_t dense0, uint32_t dense1, gpu::Buffer* sel,
                                          gpu::Buffer* nsel, gpu::Buffer* valid, gpu::Buffer* map,
                                          const AttnOptions& opt)
{
    if (q_pad % kAttnRows || k_pad % 128 || dense0 % 32)
        throw std::runtime_error(
            "attention_sparse: q_pad a multiple of 64, k_pad of 128, the dense rows from a multiple of 32");
    const mako_sparse_args a{n_q, q_pad, n_k, k_pad, heads, kv_heads, width, 1.0f / std::sqrt(float(kHeadDim)),
                             n_cubes, std::min(topk, n_cubes), dense0, dense1, opt.causal ? 1u : 0u,
                             opt.sel_per_kv_head ? kv_heads : heads};
    const size_t need = mako_attn_sparse_workspace(&a);
    gpu::Buffer* ws = need ? scratch("attn_sparse", need) : nullptr;
    before(enc);
    for (int r = repeats("flash_sparse_128"); r > 0; --r)
        check(mako_attn_sparse_ws(&a, opt.in, opt.out, q->ptr, k->ptr, v->ptr, o->ptr,
                                  sel ? static_cast<const uint16_t*>(sel->ptr) : nullptr,
                                  nsel ? static_cast<const uint16_t*>(nsel->ptr) : nullptr,
                                  static_cast<const uint8_t*>(valid->ptr), static_cast<const int32_t*>(map->ptr),
                                  opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr, ws ? ws->ptr : nullptr,
                                  ws ? ws->bytes : 0, enc->stream));
    after(enc, "flash_sparse_128");
}

void TransformerRuntime::attention_decode(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v,
                                          gpu::Buffer* ctx_len, gpu::Buffer* o, uint32_t batch, uint32_t heads,
                                          uint32_t kv_heads, uint32_t cap, uint32_t max_ctx, const AttnOptions& opt)
{
    const mako_decode_args a{batch, heads, kv_heads, kHeadDim, cap, max_ctx, 0, 1.0f / std::sqrt(float(kHeadDim))};
    const size_t need = mako_attn_decode_workspace(&a);
    if (!need)
        throw std::runtime_error(fmt("attention_decode: %u heads over %u kv heads", heads, kv_heads));
    gpu::Buffer* ws = scratch("attn_decode", need);
    before(enc);
    for (int r = repeats("attn_decode"); r > 0; --r)
        check(mako_attn_decode(&a, opt.in, opt.out, q->ptr, k->ptr, v->ptr, static_cast<const uint32_t*>(ctx_len->ptr),
                               o->ptr, opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr, ws->ptr, ws->bytes,
                               enc->stream));
    after(enc, "attn_decode");
}

}  // namespace mako::models
