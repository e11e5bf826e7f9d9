"""Attention from projection rows (mako_attn_fwd_rows) on the GPU: the prefill step of the reference's models
(heads / heads_norm / heads_partial for q, k and v, then attention: src/models/qwen_text.cpp:308-311 and 414-418,
src/models/h3_vae.cpp:219) in one entry point.

Each case is checked two ways:
  * bit for bit against the same call made as four launches (mako_heads three times into tiles, then
    mako_attn_fwd), which the other GPU tests check against the oracle: the fused route rounds every value as those
    launches do, so any difference is a fault of the fused route (a V^T image from the rows that differs from
    vt_image's, a tile item out of place);
  * against the oracle's composition (oracle heads, then oracle attention) within the attention tolerance.
Cases: the Qwen3-8B shape (32 / 8 heads of 128, q and k normed and rotated, rope 1), a query offset with fewer
queries than keys, heads of 64 bidirectional (the H3 VAE's attention, rope 2), heads of 256 with partial rotation
(Qwen3.5's gated attention), f16 and bf16 tiles with f32 and same-type outputs, and calls the fused route does not
take (unaligned columns, the split-K row count, a normed value head refused) which run the separate launches.
At full size: the Qwen3-8B prefill step at S4096, bit for bit against the four launches.
"""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402

U32 = 0xFFFFFFFF


def make(rng, *, T_q, T_k, heads, kv, dim, rope, rot, eps_q, eps_k, pad=0):
    """fp32 projection rows of q [T_q][heads dim + pad], k / v [T_k][kv dim + pad] (pad shifts col0), the angle
    table for max(T_q, T_k) rows, and the norm weights. Rows are of unit scale, and of twice that where the head is
    normed (so that the norm's division shows); un-normed q and k of scale 2 would make scores of deviation 4, a
    softmax that sits on a few keys, whose bf16 probabilities test_gpu_fwd.py's peaked case checks."""
    xq = rng.standard_normal((T_q, heads * dim + pad)).astype(np.float32) * (2 if eps_q else 1)
    xk = rng.standard_normal((T_k, kv * dim + pad)).astype(np.float32) * (2 if eps_k else 1)
    xv = rng.standard_normal((T_k, kv * dim + pad)).astype(np.float32)
    ang = rng.uniform(-np.pi, np.pi, (max(T_q, T_k, 1), max(rot // 2, 1)))
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    wq = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    wk = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    common = dict(dim=dim, rope=rope, rot=rot if rope else 0, stride=dim, col0=pad)
    hq = dict(rows=T_q, ld=heads * dim + pad, heads=heads, eps=eps_q, **common)
    hk = dict(rows=T_k, ld=kv * dim + pad, heads=kv, eps=eps_k, **common)
    hv = dict(rows=T_k, ld=kv * dim + pad, heads=kv, dim=dim, stride=dim, col0=pad)
    return (xq, xk, xv, cs, wq, wk), (hq, hk, hv)


def dev(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def run_rows(host, hs, *, n_q, n_k, heads, kv, q_pos0, block, dt, out):
    xq, xk, xv, cs, wq, wk = (dev(a) for a in host)
    hq, hk, hv = hs
    odt = torch.float32 if out == "f32" else G.TORCH[dt]
    o = torch.full((n_q, heads * hq["dim"]), float("nan"), dtype=odt, device="cuda")
    lse = torch.full((heads, max(n_q, 1)), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_fwd_rows(xq, xk, xv, o, hq, hk, hv, n_q=n_q, n_k=n_k, heads=heads, kv_heads=kv, q_pos0=q_pos0,
                    block=block, in_dtype=dt, cs=cs if hq["rope"] or hk["rope"] else None,
                    wq=wq if hq["eps"] else None, wk=wk if hk["eps"] else None, lse=lse)
    torch.cuda.synchronize()
    return o, lse


def run_separate(host, hs, *, n_q, n_k, heads, kv, q_pos0, block, dt, out):
    """The same call as mako_heads x 3 into tiles, then mako_attn_fwd."""
    xq, xk, xv, cs, wq, wk = (dev(a) for a in host)
    hq, hk, hv = hs
    dim = hq["dim"]
    tdt = G.TORCH[dt]
    qt = torch.zeros((heads, max(n_q, 1), dim), dtype=tdt, device="cuda")
    kt = torch.zeros((kv, max(n_k, 1), dim), dtype=tdt, device="cuda")
    vt = torch.zeros((kv, max(n_k, 1), dim), dtype=tdt, device="cuda")
    csq = cs[q_pos0:] if cs is not None else None  # query row t sits at position q_pos0 + t
    for x, h, y, w, c in ((xq, hq, qt, wq, csq), (xk, hk, kt, wk, cs), (xv, hv, vt, None, cs)):
        if h["rows"]:
            M.heads(x, y, n_pad=y.shape[1], cs=c if h.get("rope") else None, w=w if h.get("eps") else None, **h)
    odt = torch.float32 if out == "f32" else tdt
    o = torch.full((n_q, heads * dim), float("nan"), dtype=odt, device="cuda")
    lse = torch.full((heads, max(n_q, 1)), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_fwd(qt, kt, vt, o, n_q=n_q, q_pad=qt.shape[1], n_k=n_k, k_pad=kt.shape[1], heads=heads, kv_heads=kv,
               q_pos0=q_pos0, block=block, dim=dim, lse=lse)
    torch.cuda.synchronize()
    return o, lse


def oracle(host, hs, *, n_q, n_k, heads, kv, q_pos0, block, dt):
    xq, xk, xv, cs, wq, wk = host
    hq, hk, hv = hs
    dim = hq["dim"]
    tiles = []
    csq = cs[q_pos0:q_pos0 + n_q]  # the angles of positions q_pos0 .. q_pos0 + n_q - 1
    for x, h, w, rows, c in ((xq, hq, wq, n_q, csq), (xk, hk, wk, n_k, cs), (xv, hv, None, n_k, cs)):
        a = dict(h, n_pad=max(rows, 1))
        tiles.append(O.heads(x, c if a.get("rope") else None, w if a.get("eps") else None, None, out=dt, **a))
    return O.attn_dense(*tiles, n_q=n_q, q_pad=max(n_q, 1), n_k=n_k, k_pad=max(n_k, 1), heads=heads,
                        kv_heads=kv, q_pos0=q_pos0, block=block, dim=dim, dtype=dt)


def bits(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).cpu().numpy()


# (name, T_q, T_k, heads, kv, dim, rope, rot, eps_q, eps_k, q_pos0, block, dtype, out, pad)
CASES = [
    ("qwen3_gqa4_causal", 300, 300, 32, 8, 128, 1, 128, 1e-6, 1e-6, 0, U32, O.BF16, "f32", 0),
    ("qwen3_gqa4_causal_same", 257, 257, 32, 8, 128, 1, 128, 1e-6, 1e-6, 0, U32, O.BF16, "same", 0),
    ("offset_fewer_queries", 100, 300, 8, 2, 128, 1, 128, 1e-6, 0.0, 200, U32, O.F16, "f32", 0),
    ("d64_bidirectional_rope2", 200, 200, 8, 8, 64, 2, 64, 0.0, 0.0, 0, 0, O.BF16, "same", 0),
    ("d64_prefix_causal", 150, 150, 4, 2, 64, 1, 32, 1e-5, 1e-5, 0, 77, O.F16, "f32", 0),
    ("d256_partial_rot", 130, 130, 16, 2, 256, 1, 64, 1e-6, 1e-6, 0, U32, O.BF16, "f32", 0),
    ("d256_f16_same", 96, 96, 4, 4, 256, 2, 256, 0.0, 1e-6, 0, U32, O.F16, "same", 0),
    ("no_keys", 70, 0, 4, 2, 128, 1, 128, 0.0, 0.0, 0, U32, O.BF16, "f32", 0),
    # not fused: columns not 16-byte aligned (mako_heads' per-value path), then the split-K row count
    ("unaligned_columns", 120, 120, 8, 2, 128, 1, 128, 1e-6, 1e-6, 0, U32, O.BF16, "f32", 2),
    ("few_rows_splitk", 4, 2000, 32, 8, 128, 1, 128, 1e-6, 1e-6, 1996, U32, O.BF16, "f32", 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_rows_against_separate_launches_and_oracle(case):
    name, T_q, T_k, heads, kv, dim, rope, rot, eps_q, eps_k, q_pos0, block, dt, out, pad = case
    print(f"rows case {case}", flush=True)
    rng = np.random.default_rng(sum(map(ord, name)))
    host, hs = make(rng, T_q=T_q, T_k=T_k, heads=heads, kv=kv, dim=dim, rope=rope, rot=rot, eps_q=eps_q,
                    eps_k=eps_k, pad=pad)
    kw = dict(n_q=T_q, n_k=T_k, heads=heads, kv=kv, q_pos0=q_pos0, block=block, dt=dt, out=out)
    o, lse = run_rows(host, hs, **kw)
    o2, lse2 = run_separate(host, hs, **kw)
    assert np.array_equal(bits(o), bits(o2)), "the fused route's output differs from the separate launches'"
    assert np.array_equal(bits(lse), bits(lse2)), "the fused route's lse differs from the separate launches'"
    want_o, want_l = oracle(host, hs, n_q=T_q, n_k=T_k, heads=heads, kv=kv, q_pos0=q_pos0, block=block, dt=dt)
    got_o = G.to_host(o)
    G.assert_attn_close(got_o, want_o, "output")
    G.assert_lse_close(lse.cpu().numpy().astype(np.float64)[:, :T_q], want_l, "lse")


def test_offset_queries_equal_the_last_rows_of_the_whole_prefill():
    """Rotated queries at q_pos0 > 0 take the angles of their positions: 100 queries at positions 200 .. 299 over
    300 keys give the same rows (within the attention tolerance) as rows 200 .. 299 of the whole 300-row prefill
    whose query rows 200 .. 299 are the same projection rows. A query rotated by the angle of its row index instead
    of its position would score every key at the wrong relative position."""
    rng = np.random.default_rng(17)
    T, off, heads, kv, dim = 300, 200, 8, 2, 128
    host, (hq, hk, hv) = make(rng, T_q=T, T_k=T, heads=heads, kv=kv, dim=dim, rope=1, rot=128, eps_q=1e-6,
                              eps_k=1e-6)
    xq, xk, xv, cs, wq, wk = host
    kw = dict(n_k=T, heads=heads, kv=kv, block=U32, dt=O.BF16, out="f32")
    whole, wl = run_rows(host, (hq, hk, hv), n_q=T, q_pos0=0, **kw)
    part_host = (np.ascontiguousarray(xq[off:]), xk, xv, cs, wq, wk)
    part, pl = run_rows(part_host, (dict(hq, rows=T - off), hk, hv), n_q=T - off, q_pos0=off, **kw)
    G.assert_attn_close(G.to_host(part), G.to_host(whole)[off:], "offset rows")
    G.assert_lse_close(pl.cpu().numpy().astype(np.float64)[:, :T - off], wl.cpu().numpy()[:, off:], "offset lse")


def test_rows_refuses_query_angles_past_the_table():
    rng = np.random.default_rng(5)
    host, (hq, hk, hv) = make(rng, T_q=64, T_k=100, heads=4, kv=2, dim=128, rope=1, rot=128, eps_q=0.0, eps_k=0.0)
    with pytest.raises(M.MakoError, match="angle rows"):
        run_rows(host, (hq, hk, hv), n_q=64, n_k=100, heads=4, kv=2, q_pos0=50, block=U32, dt=O.BF16, out="f32")


def test_rows_refuses_a_normed_value_head():
    rng = np.random.default_rng(3)
    host, (hq, hk, hv) = make(rng, T_q=64, T_k=64, heads=4, kv=2, dim=128, rope=1, rot=128, eps_q=0.0, eps_k=0.0)
    hv = dict(hv, eps=1e-6)  # the value producer takes no weight
    with pytest.raises(M.MakoError, match="eps"):
        run_rows(host, (hq, hk, hv), n_q=64, n_k=64, heads=4, kv=2, q_pos0=0, block=U32, dt=O.BF16, out="f32")


def test_qwen3_8b_prefill_step_s4096_bit_for_bit():
    """The Qwen3-8B prefill step at S4096 (32 / 8 heads of 128, q and k normed and rotated), fused against the four
    separate launches, every output bit and every lse, plus 200 rows against the oracle's composition."""
    rng = np.random.default_rng(4096)
    S, heads, kv, dim = 4096, 32, 8, 128
    host, hs = make(rng, T_q=S, T_k=S, heads=heads, kv=kv, dim=dim, rope=1, rot=128, eps_q=1e-6, eps_k=1e-6)
    kw = dict(n_q=S, n_k=S, heads=heads, kv=kv, q_pos0=0, block=U32, dt=O.BF16, out="same")
    o, lse = run_rows(host, hs, **kw)
    o2, lse2 = run_separate(host, hs, **kw)
    assert np.array_equal(bits(o), bits(o2))
    assert np.array_equal(bits(lse), bits(lse2))
    # sampled rows against the oracle: tiles from the oracle's producers, then its attention on those rows
    xq, xk, xv, cs, wq, wk = host
    hq, hk, hv = hs
    tiles = [O.heads(x, cs if h.get("rope") else None, w if h.get("eps") else None, None, out=O.BF16,
                     **dict(h, n_pad=S)) for x, h, w in ((xq, hq, wq), (xk, hk, wk), (xv, hv, None))]
    rows = np.concatenate([[0, 1, 63, 64, S - 1], rng.integers(0, S, 195)])
    hr = np.stack([rng.integers(0, heads, len(rows)), rows], 1).astype(np.uint32)
    want_o, want_l = O.attn_dense_rows(*tiles, hr, n_q=S, q_pad=S, n_k=S, k_pad=S, heads=heads, kv_heads=kv,
                                       q_pos0=0, block=U32, dim=dim, dtype=O.BF16)
    got = G.to_host(o)
    got_o = np.stack([got[r, h * dim:(h + 1) * dim] for h, r in hr])
    G.assert_attn_close(got_o, want_o, "sampled output")
    got_l = lse.cpu().numpy()
    G.assert_lse_close(np.array([got_l[h, r] for h, r in hr], np.float64), want_l, "sampled lse")
