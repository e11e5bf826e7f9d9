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

void TransformerRuntime::attention(gpu::Encoder*& enc, gpu::Buffer* q, gpu::Buffer* k, gpu::Buffer* v, gpu::Buffer* o,
                                   uint32_t n_q, uint32_t q_pad, uint32_t n_k, uint32_t k_pad, uint32_t n_heads,
                                   uint32_t kv_heads, uint32_t q_pos0, uint32_t block, uint32_t dim,
                                   const AttnOptions& opt)
{
    if (dim != 64 && dim != 128 && dim != 256)
        throw std::runtime_error(fmt("attention: heads of %u", dim));
    const mako_attn_args a{n_q, q_pad, n_k, k_pad, n_heads, kv_heads, q_pos0, block, n_heads * dim,
                           1.0f / std::sqrt(float(dim))};
    before(enc);
    check(mako_attn_fwd(&a, dim, opt.in, opt.out, q->ptr, k->ptr, v->ptr, o->ptr,
                        opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr, enc->stream));
    after(enc, dim == 64 ? "flash_fwd_64" : dim == 128 ? "flash_fwd_128" : "flash_fwd_256");
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
    before(enc);
    check(mako_attn_sparse(&a, opt.in, opt.out, q->ptr, k->ptr, v->ptr, o->ptr,
                           sel ? static_cast<const uint16_t*>(sel->ptr) : nullptr,
                           nsel ? static_cast<const uint16_t*>(nsel->ptr) : nullptr,
                           static_cast<const uint8_t*>(valid->ptr), static_cast<const int32_t*>(map->ptr),
                           opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr, enc->stream));
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
    check(mako_attn_decode(&a, opt.in, opt.out, q->ptr, k->ptr, v->ptr, static_cast<const uint32_t*>(ctx_len->ptr),
                           o->ptr, opt.lse ? static_cast<float*>(opt.lse->ptr) : nullptr, ws->ptr, ws->bytes,
                           enc->stream));
    after(enc, "attn_decode");
}

}  // namespace mako::models
