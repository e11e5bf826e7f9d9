// Attention from fp32 projection rows: the prefill step's head producers and attention (the reference's
// heads / heads_norm / heads_partial dispatches followed by attention: src/models/qwen_text.cpp:308-311 and
// :414-418, src/models/h3_vae.cpp:219) as two launches instead of four.
//
// qkv_prep, one launch, three kinds of workgroup:
//   * the value tiles as mako_heads writes them (heads_vec_item; flash_fwd_r64 and flash_fwd_r32 stage V from its
//     rows), or, for heads of 256 past flash_fwd_r32's offsets, the V^T tile images flash_fwd_d256 stages from,
//     written straight from the value rows (vt_rows_tiles): the value tiles are then never written, nor read back by
//     vt_image;
//   * the key tiles, normed and rotated as mako_heads writes them (heads_vec_item);
//   * the query tiles, the same.
// Then the attention kernel over those tiles (launch_fwd64, launch_fwd_r32; launch_fwd_d256 with the images ready),
// the one mako_attn_fwd takes. Every value is rounded as the separate launches round it, so both give the same bits.
//
// Bound: HBM for qkv_prep (4 bytes read a value, 2 written), then the attention kernel's MFMA bound.
#include "fwd64_common.hpp"
#include "heads_common.hpp"

namespace mako {

int attn_check(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q, const void* k,
               const void* v, const void* o);
bool splitk_takes(const mako_attn_args* a, uint32_t dim);
template <int D>
bool fwd64_fits(const mako_attn_args* a, uint32_t out_bytes);
bool d256_fits(const mako_attn_args* a);
bool r32_fits(const mako_attn_args* a, uint32_t out_bytes);
template <class T, class TO>
int launch_fwd_r32(const mako_attn_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                   float* lse, hipStream_t s);
template <class T, class TO, int D>
int launch_fwd64(const mako_attn_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                 float* lse, hipStream_t s);
template <class T, class TO>
int launch_fwd_d256(const mako_attn_args* a, float scale_log2, const void* q, const void* k, const void* v, void* o,
                    float* lse, hipStream_t s, const void* vt_ready, const Workspace* work);
size_t d256_workspace(const mako_attn_args* a);
size_t attn_fwd_workspace(const mako_attn_args* a, uint32_t dim);
int attn_fwd_core(const mako_attn_args* a, uint32_t dim, mako_dtype in, mako_dtype out, const void* q, const void* k,
                  const void* v, void* o, float* lse, const Workspace& work, void* stream);

namespace {

struct VtRowsParams {
    const float* x;
    uint32_t* img;
    uint32_t ld, col0, stride, n_k, n_vt;
    uint32_t nbx;  // workgroups a kv head (256 / D tiles each)
};

// Workgroups [0, nbv): value tiles (value items; heads of 256 for flash_fwd_d256: V^T images of kv head b / nbx);
// then nbk of key items; then the query items.
template <class T, int D>
__global__ __launch_bounds__(256) void qkv_prep(const HeadsParams pq, const HeadsParams pk, const HeadsParams pvt,
                                                const VtRowsParams pv, uint32_t nbv, uint32_t nbk)
{
    uint32_t b = blockIdx.x;
    const uint32_t w = threadIdx.x >> 6;
    if (b < nbv) {
        if (D == 256 && pv.img)
            vt_rows_tiles<T, D>(pv.x, pv.ld, pv.col0, pv.stride, pv.img, pv.n_k, pv.n_vt, b % pv.nbx, b / pv.nbx);
        else
            heads_vec_item<T, D / 4>(pvt, (uint64_t)b * kItems + w);
        return;
    }
    b -= nbv;
    if (b < nbk) {
        heads_vec_item<T, D / 4>(pk, (uint64_t)b * kItems + w);
        return;
    }
    b -= nbk;
    heads_vec_item<T, D / 4>(pq, (uint64_t)b * kItems + w);
}

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// The fused route for heads of D: qkv_prep, then the attention kernel. pvt: the value producer (its tiles at pvt.y,
// the V the attention kernel reads); heads of 256 past flash_fwd_r32's offsets write flash_fwd_d256's V^T images
// instead, into images (d256_workspace bytes). The kernel is the one mako_attn_fwd takes for the same call, so the
// fused route gives the separate launches' bits.
template <class T, class TO, int D>
int launch_rows(const mako_attn_args* t, const HeadsParams& pq, const HeadsParams& pk, const HeadsParams& pvt,
                const mako_heads_args* hv, const float* xv, void* o, float* lse, hipStream_t s,
                const Workspace& images)
{
    using L = R64<D>;
    const uint32_t n_vt = (t->n_k + 63) / 64, nbx = (n_vt + 256 / D - 1) / (256 / D);
    const bool images_route = D == 256 && !r32_fits(t, sizeof(TO));
    void* vt = nullptr;
    if (images_route) {
        const size_t vt_bytes = (size_t)t->kv_heads * n_vt * L::kVTile;
        if (vt_bytes && !(vt = images.get(vt_bytes, s)))
            return last_code();
    }
    const VtRowsParams pv{xv, static_cast<uint32_t*>(vt), hv->ld, hv->col0, hv->stride, t->n_k, n_vt, nbx};
    const uint64_t nbv = images_route ? (uint64_t)nbx * t->kv_heads : (pvt.n_items + kItems - 1) / kItems,
                   nbk = (pk.n_items + kItems - 1) / kItems, nbq = (pq.n_items + kItems - 1) / kItems;
    if (nbv + nbk + nbq > 0x7fffffffu)
        return fail(MAKO_EINVAL, "attention from rows: %llu workgroups exceed the grid",
                    (unsigned long long)(nbv + nbk + nbq));
    if (nbv + nbk + nbq)
        hipLaunchKernelGGL((qkv_prep<T, D>), dim3((uint32_t)(nbv + nbk + nbq)), dim3(256), 0, s, pq, pk, pvt, pv,
                           (uint32_t)nbv, (uint32_t)nbk);
    const float sl2 = t->scale * 1.4426950408889634f;
    int r;
    if (images_route)
        r = launch_fwd_d256<T, TO>(t, sl2, pq.y, pk.y, pk.y, o, lse, s, vt, &images);
    else if constexpr (D == 256)
        r = launch_fwd_r32<T, TO>(t, sl2, pq.y, pk.y, pvt.y, o, lse, s);
    else
        r = launch_fwd64<T, TO, D>(t, sl2, pq.y, pk.y, pvt.y, o, lse, s);
    if (r <= 0)  // (the route was chosen where the kernel fits and its images are given)
        return fail(MAKO_EHIP, "attention from rows: the attention kernel refused a checked call");
    return check_launch("attention from rows");
}

template <class T, class TO>
int launch_rows_dim(uint32_t dim, const mako_attn_args* t, const HeadsParams& pq, const HeadsParams& pk,
                    const HeadsParams& pvt, const mako_heads_args* hv, const float* xv, void* o, float* lse,
                    hipStream_t s, const Workspace& images)
{
    return dim == 128  ? launch_rows<T, TO, 128>(t, pq, pk, pvt, hv, xv, o, lse, s, images)
           : dim == 64 ? launch_rows<T, TO, 64>(t, pq, pk, pvt, hv, xv, o, lse, s, images)
                       : launch_rows<T, TO, 256>(t, pq, pk, pvt, hv, xv, o, lse, s, images);
}

// The call as mako_attn_fwd reads it (q_pad = n_q, k_pad = n_k), and the head tiles' bytes.
mako_attn_args tiles_call(const mako_attn_args* a)
{
    mako_attn_args t = *a;
    t.q_pad = a->n_q;
    t.k_pad = a->n_k;
    return t;
}

size_t tiles_bytes(const mako_attn_args* a, uint32_t dim)
{
    return round256((size_t)a->heads * a->n_q * dim * 2) + 2 * round256((size_t)a->kv_heads * a->n_k * dim * 2) + 256;
}

}  // namespace
}  // namespace mako

using namespace mako;

namespace {

// tiles: the head tiles' workspace (tiles_bytes); rest: the attention's (the fused route's V^T images for heads of
// 256, else what mako_attn_fwd needs for the tiles).
int rows_core(const mako_attn_args* a, const mako_heads_args* hq, const mako_heads_args* hk,
              const mako_heads_args* hv, mako_dtype in, mako_dtype out, const float* xq, const float* xk,
              const float* xv, const float* cs, const float* wq, const float* wk, void* o, float* lse,
              const Workspace& tiles, const Workspace& rest, void* stream)
{
    if (!a || !hq || !hk || !hv || !o)
        return fail(MAKO_EINVAL, "attention from rows: a null argument");
    const uint32_t dim = hq->dim;
    if (hk->dim != dim || hv->dim != dim)
        return fail(MAKO_EINVAL, "attention from rows: heads of %u, %u and %u", dim, hk->dim, hv->dim);
    if (hq->heads != a->heads || hk->heads != a->kv_heads || hv->heads != a->kv_heads)
        return fail(MAKO_EINVAL, "attention from rows: %u / %u / %u heads produced for %u over %u", hq->heads,
                    hk->heads, hv->heads, a->heads, a->kv_heads);
    if (hq->rows != a->n_q || hk->rows != a->n_k || hv->rows != a->n_k)
        return fail(MAKO_EINVAL, "attention from rows: %u / %u / %u rows produced for %u queries and %u keys",
                    hq->rows, hk->rows, hv->rows, a->n_q, a->n_k);
    // The producers write tiles [heads][rows][dim] with nothing cleared; attention reads them as q_pad = n_q and
    // k_pad = n_k. o stands in for the tiles (workspace, 256-byte aligned) in the checks.
    mako_heads_args tq = *hq, tk = *hk, tv = *hv;
    for (mako_heads_args* h : {&tq, &tk, &tv}) {
        h->n_pad = h->rows;
        h->row0 = 0;
        h->clear = 0;
    }
    mako_attn_args t = *a;
    t.q_pad = a->n_q;
    t.k_pad = a->n_k;
    if (const int e = attn_check(&t, dim, in, out, o, o, o, o))
        return e;
    // The angle table holds one row a key position (0 .. n_k - 1, the key producer's rows); query row t sits at
    // position q_pos0 + t and takes that row. With no keys every row is fully masked and the queries are never
    // used, so they are not rotated (no angle is read).
    if (a->n_k == 0)
        tq.rope = 0;
    if (tq.rope && (uint64_t)a->q_pos0 + a->n_q > a->n_k)
        return fail(MAKO_EINVAL,
                    "attention from rows: rotated queries at positions %u .. %llu past the %u angle rows", a->q_pos0,
                    (unsigned long long)a->q_pos0 + a->n_q - 1, a->n_k);
    const float* csq = cs && tq.rope ? cs + (size_t)a->q_pos0 * hq->rot : cs;
    if (const int e = heads_check(&tq, in, xq, csq, wq, o))
        return e;
    if (const int e = heads_check(&tk, in, xk, cs, wk, o))
        return e;
    if (const int e = heads_check(&tv, in, xv, cs, nullptr, o))
        return e;
    if (a->n_q == 0)
        return ok();
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t q_bytes = round256((size_t)a->heads * a->n_q * dim * 2),
                 k_bytes = round256((size_t)a->kv_heads * a->n_k * dim * 2);
    const uint32_t osz = out == MAKO_F32 ? 4u : 2u;
    const bool fits = dim == 256   ? r32_fits(&t, osz) || d256_fits(&t)
                      : dim == 128 ? fwd64_fits<128>(&t, osz)
                                   : fwd64_fits<64>(&t, osz);
    const bool fused = fits && !splitk_takes(&t, dim) && heads_vec_takes(&tq, xq, csq, wq, o) &&
                       heads_vec_takes(&tk, xk, cs, wk, o) && tv.rope == 0 && tv.eps == 0.0f &&
                       heads_vec_takes(&tv, xv, nullptr, nullptr, o);
    char* ws = static_cast<char*>(tiles.get(tiles_bytes(&t, dim), s));
    if (!ws)
        return last_code();
    void *qt = ws, *kt = ws + q_bytes, *vt = ws + q_bytes + k_bytes;
    if (!fused) {
        // The producers and attention as separate launches (the same results).
        int e = mako_heads(&tq, in, xq, csq, wq, nullptr, qt, stream);
        if (!e)
            e = mako_heads(&tk, in, xk, cs, wk, nullptr, kt, stream);
        if (!e)
            e = mako_heads(&tv, in, xv, cs, nullptr, nullptr, vt, stream);
        return e ? e : attn_fwd_core(&t, dim, in, out, qt, kt, vt, o, lse, rest, stream);
    }
    const HeadsParams pq = heads_params(&tq, xq, csq, wq, nullptr, qt, true);
    const HeadsParams pk = heads_params(&tk, xk, cs, wk, nullptr, kt, true);
    const HeadsParams pvt = heads_params(&tv, xv, nullptr, nullptr, nullptr, vt, true);
    if (in == MAKO_BF16)
        return out == MAKO_F32 ? launch_rows_dim<__bf16, float>(dim, &t, pq, pk, pvt, &tv, xv, o, lse, s, rest)
                               : launch_rows_dim<__bf16, __bf16>(dim, &t, pq, pk, pvt, &tv, xv, o, lse, s, rest);
    return out == MAKO_F32 ? launch_rows_dim<_Float16, float>(dim, &t, pq, pk, pvt, &tv, xv, o, lse, s, rest)
                           : launch_rows_dim<_Float16, _Float16>(dim, &t, pq, pk, pvt, &tv, xv, o, lse, s, rest);
}

}  // namespace

extern "C" size_t mako_attn_fwd_rows_workspace(const mako_attn_args* a, uint32_t dim)
{
    if (!a || (dim != 64 && dim != 128 && dim != 256))
        return 0;
    const mako_attn_args t = tiles_call(a);
    // the fused route's images (heads of 256 past flash_fwd_r32's offsets, sized for an f32 output, the larger) or
    // the separate calls' attention, whichever the call takes: the larger
    const size_t images = dim == 256 && !r32_fits(&t, 4) ? d256_workspace(&t) : 0;
    return tiles_bytes(&t, dim) + std::max(images, attn_fwd_workspace(&t, dim));
}

extern "C" int mako_attn_fwd_rows(const mako_attn_args* a, const mako_heads_args* hq, const mako_heads_args* hk,
                                  const mako_heads_args* hv, mako_dtype in, mako_dtype out, const float* xq,
                                  const float* xk, const float* xv, const float* cs, const float* wq,
                                  const float* wk, void* o, float* lse, void* stream)
{
    const uint32_t dim = hq ? hq->dim : 0;
    return rows_core(a, hq, hk, hv, in, out, xq, xk, xv, cs, wq, wk, o, lse,
                     library_workspace(kWsRowTiles, "attention from rows"),
                     library_workspace(dim == 128 ? kWsSplitK : kWsVtImages, "attention from rows"), stream);
}

extern "C" int mako_attn_fwd_rows_ws(const mako_attn_args* a, const mako_heads_args* hq, const mako_heads_args* hk,
                                     const mako_heads_args* hv, mako_dtype in, mako_dtype out, const float* xq,
                                     const float* xk, const float* xv, const float* cs, const float* wq,
                                     const float* wk, void* o, float* lse, void* workspace, size_t workspace_bytes,
                                     void* stream)
{
    const Workspace w = caller_workspace(workspace, workspace_bytes, "attention from rows");
    const size_t tb = a && hq ? tiles_bytes(a, hq->dim) : 0;
    return rows_core(a, hq, hk, hv, in, out, xq, xk, xv, cs, wq, wk, o, lse, w, w.at(tb), stream);
}
