"""Block-sparse attention and cube selection on the GPU against the CPU oracle: the golden fixtures; the
reference's own test case restated (tests/sparse_attn_test.cpp:41-211: 2 heads, D 128, 6 cubes one with 20 valid
rows, 60 dense rows, top 3: the selection equal to the CPU's, worst row relative L2 < 5e-3, rows past n_q and
padding rows untouched, local = 3 neighbours first without duplicates); invariants (every cube selected equals
dense attention over the valid keys; causal lists of every earlier block equal causal dense attention); and the
S16384 window + random causal configuration on sampled rows."""
import numpy as np
import pytest

import oracle as O
from conftest import golden_files, load_golden

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402

SENTINEL = 12288.0  # exact in f16, bf16 and f32


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda")


def dev(a, _=None):
    """A numpy array (uint8 flags, int32 map) on cuda:0 as it is."""
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def run_sparse(q, k, v, sel, nsel, valid, map_, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, n_cubes, max_sel,
               dense0, dense1, causal=0, sel_heads=None, out=torch.float32, o_rows=None):
    o_rows = q_pad if o_rows is None else o_rows
    o = torch.full((o_rows, heads * 128), SENTINEL, dtype=out, device="cuda")
    lse = torch.full((heads, q_pad), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_sparse(q, k, v, o, sel, nsel, valid, map_, n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads,
                  kv_heads=kv_heads, n_cubes=n_cubes, max_sel=max_sel, dense0=dense0, dense1=dense1, causal=causal,
                  sel_heads=sel_heads, lse=lse)
    torch.cuda.synchronize()
    return G.to_host(o), lse.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("path", golden_files("sparse"), ids=lambda p: p.split("/")[-1][:-4])
def test_golden(path):
    g = load_golden(path)
    n_q, q_pad, n_k, k_pad, heads, kv, width, cubes, kk, d0, d1, causal, sh, topk, dt = [int(x) for x in g["args"]]
    args = dict(n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv, n_cubes=cubes, max_sel=kk,
                dense0=d0, dense1=d1, causal=causal, sel_heads=sh)
    for out in (torch.float32, G.TORCH[dt]):
        o, lse = run_sparse(G.to_dev(g["q"], dt), G.to_dev(g["k"], dt), G.to_dev(g["v"], dt), dev_u16(g["sel"]),
                            dev_u16(g["nsel"]), dev(g["valid"], None), dev(g["map"], None), out=out, **args)
        written = g["o"] != 12345.0
        G.assert_attn_close(o[written], g["o"][written], "output")
        assert np.all(o[~written] == SENTINEL), "rows outside the map were written"
        ok = ~np.isnan(g["lse"])
        G.assert_lse_close(lse[ok], g["lse"][ok], "lse")


def reference_case(seed=7, dtype=O.F16):
    """The shapes and layout of tests/sparse_attn_test.cpp:46-77 (inputs seeded here: the reference draws them
    from mt19937 + std::normal_distribution, whose values are implementation-defined)."""
    D, heads, cubes, dense, topk = 128, 2, 6, 60, 3
    cnt = np.array([64, 64, 64, 64, 64, 20], np.uint32)
    n = cubes * 64 + dense
    q_pad, k_pad = (n + 63) // 64 * 64, (n + 127) // 128 * 128
    valid = np.zeros(k_pad, np.uint8)
    for c in range(cubes):
        valid[c * 64:c * 64 + cnt[c]] = 1
    valid[cubes * 64:n] = 1
    map_ = np.full(q_pad, -1, np.int32)
    map_[:n][valid[:n] == 1] = np.nonzero(valid[:n])[0]
    rng = np.random.default_rng(seed)
    mk = lambda pad: G.bits(rng.standard_normal((heads, pad, D), dtype=np.float32) *  # noqa: E731
                            valid[:pad, None].astype(np.float32), dtype)
    qb, kb, vb = mk(q_pad), mk(k_pad), mk(k_pad)
    return dict(D=D, heads=heads, cubes=cubes, topk=topk, cnt=cnt, n=n, q_pad=q_pad, k_pad=k_pad, valid=valid,
                map=map_, q=qb, k=kb, v=vb, dense0=cubes * 64, dense1=n, dtype=dtype)


def gpu_cube_select(c, q, k, topk, local=0, stride=0):
    heads, cubes = c["heads"], c["cubes"]
    kk = min(topk, cubes)
    sel = torch.zeros((heads, cubes, kk), dtype=torch.int16, device="cuda")
    nsel = torch.zeros((heads, cubes), dtype=torch.int16, device="cuda")
    ws = torch.empty(M.cube_select_workspace(heads, cubes), dtype=torch.uint8, device="cuda")
    cnt = torch.from_numpy(c["cnt"].astype(np.int32)).to("cuda")
    M.cube_select(q, k, cnt, sel, nsel, ws, heads=heads, q_pad=c["q_pad"], k_pad=c["k_pad"], n_cubes=cubes,
                  topk=topk, local=local, stride=stride)
    torch.cuda.synchronize()
    return sel, nsel


def test_reference_sparse_attn_case():
    c = reference_case()
    dt = c["dtype"]
    q, k, v = G.to_dev(c["q"], dt), G.to_dev(c["k"], dt), G.to_dev(c["v"], dt)
    print("reference sparse case", flush=True)
    sel, nsel = gpu_cube_select(c, q, k, c["topk"])
    want_sel, want_nsel = O.cube_select(c["q"], c["k"], c["cnt"], heads=c["heads"], dim=128, q_pad=c["q_pad"],
                                        k_pad=c["k_pad"], n_cubes=c["cubes"], topk=c["topk"], dtype=dt)
    got_sel = sel.cpu().numpy().view(np.uint16)
    assert np.array_equal(got_sel, want_sel), "cube_select differs from the CPU's"
    assert np.all(nsel.cpu().numpy() == min(c["topk"], c["cubes"]))
    args = dict(n_q=c["n"], q_pad=c["q_pad"], n_k=c["n"], k_pad=c["k_pad"], heads=c["heads"], kv_heads=c["heads"],
                n_cubes=c["cubes"], max_sel=min(c["topk"], c["cubes"]), dense0=c["dense0"], dense1=c["dense1"])
    o, lse = run_sparse(q, k, v, sel, nsel, dev(c["valid"], None), dev(c["map"], None), **args)
    want_o, want_l = O.attn_sparse(c["q"], c["k"], c["v"], got_sel, nsel.cpu().numpy().view(np.uint16), c["valid"],
                                   c["map"], dtype=dt, o_fill=np.full((c["q_pad"], c["heads"] * 128), SENTINEL),
                                   **args)
    rows = c["map"][c["map"] >= 0]
    G.assert_attn_close(o[rows], want_o[rows], "output")
    G.assert_rows_l2(o[rows], want_o[rows], "output", 128)
    untouched = np.ones(c["q_pad"], bool)
    untouched[rows] = False
    assert np.all(o[untouched] == SENTINEL), "padding and out-of-range rows were written"
    ok = np.isfinite(want_l) & ~np.isnan(want_l)
    G.assert_lse_close(lse[ok], want_l[ok], "lse")
    # local = 3, stride 1: the cube and its neighbours lead the selection, no cube twice
    sel4, _ = gpu_cube_select(c, q, k, 4, local=3, stride=1)
    s4 = sel4.cpu().numpy().view(np.uint16)
    want4, _ = O.cube_select(c["q"], c["k"], c["cnt"], heads=c["heads"], dim=128, q_pad=c["q_pad"],
                             k_pad=c["k_pad"], n_cubes=c["cubes"], topk=4, local=3, stride=1, dtype=dt)
    assert np.array_equal(s4, want4)
    for h in range(c["heads"]):
        for qc in range(c["cubes"]):
            want = [qc] + ([qc - 1] if qc >= 1 else []) + ([qc + 1] if qc + 1 < c["cubes"] else [])
            assert list(s4[h, qc][:len(want)]) == want and len(set(s4[h, qc])) == 4


@pytest.mark.parametrize("n_cubes,topk,local,stride", [(37, 5, 0, 0), (37, 40, 1, 0), (300, 17, 3, 9), (4096, 3, 0, 0)])
def test_cube_select_sizes(n_cubes, topk, local, stride):
    heads = 2
    rng = np.random.default_rng(n_cubes)
    pad = n_cubes * 64
    cnt = rng.integers(1, 65, n_cubes).astype(np.uint32)
    cnt[::7] = 64
    rows = np.concatenate([np.arange(64) < ci for ci in cnt]).astype(np.float32)
    qb = G.bits(rng.standard_normal((heads, pad, 128), dtype=np.float32) * rows[None, :, None], O.BF16)
    kb = G.bits(rng.standard_normal((heads, pad, 128), dtype=np.float32) * rows[None, :, None], O.BF16)
    c = dict(heads=heads, cubes=n_cubes, q_pad=pad, k_pad=pad, cnt=cnt)
    sel, nsel = gpu_cube_select(c, G.to_dev(qb, O.BF16), G.to_dev(kb, O.BF16), topk, local, stride)
    want, want_n, _, _, _ = O.cube_select(qb, kb, cnt, heads=heads, dim=128, q_pad=pad, k_pad=pad,
                                           n_cubes=n_cubes, topk=topk, local=local, stride=stride, dtype=O.BF16,
                                           want_scores=True)
    got = sel.cpu().numpy().view(np.uint16)
    # index work is exact: the selection equals the double-precision check's everywhere
    # (tests/sparse_attn_test.cpp:98-129), and no cube appears twice
    assert np.array_equal(got, want), f"{(got != want).sum()} of {got.size} positions differ"
    assert all(len(set(r.tolist())) == len(r) for r in got.reshape(-1, got.shape[-1]))
    assert np.array_equal(nsel.cpu().numpy().view(np.uint16), want_n)


def test_all_cubes_equals_dense():
    """Every cube selected and no dense rows: the sparse kernel equals the dense kernel over the valid keys."""
    heads, kv, cubes = 4, 2, 6  # k_pad a multiple of 128, as the reference requires
    n = cubes * 64
    rng = np.random.default_rng(3)
    qb, kb, vb = (G.randn_bits(rng, (h, n, 128), O.BF16) for h in (heads, kv, kv))
    valid = np.ones(n, np.uint8)
    sel = np.tile(np.arange(cubes, dtype=np.uint16), (kv, cubes, 1))
    nsel = np.full((kv, cubes), cubes, np.uint16)
    map_ = np.arange(n, dtype=np.int32)
    q, k, v = G.to_dev(qb, O.BF16), G.to_dev(kb, O.BF16), G.to_dev(vb, O.BF16)
    o, lse = run_sparse(q, k, v, dev_u16(sel), dev_u16(nsel), dev(valid, None), dev(map_, None), n_q=n, q_pad=n,
                        n_k=n, k_pad=n, heads=heads, kv_heads=kv, n_cubes=cubes, max_sel=cubes, dense0=n, dense1=n,
                        sel_heads=kv)
    od = torch.empty((n, heads * 128), dtype=torch.float32, device="cuda")
    ld = torch.empty((heads, n), dtype=torch.float32, device="cuda")
    M.attn_fwd(q, k, v, od, n_q=n, q_pad=n, n_k=n, k_pad=n, heads=heads, kv_heads=kv, q_pos0=0, block=0, dim=128,
               lse=ld)
    torch.cuda.synchronize()
    # the two kernels visit the keys in other orders, so their running maxima, and with them the bf16 roundings of
    # P, differ: the outputs agree within the attention tolerance, the LSE (sums of unrounded exponentials) closer
    G.assert_attn_close(o, G.to_host(od), "sparse vs dense output")
    np.testing.assert_allclose(lse, ld.cpu().numpy(), atol=1e-4)


def test_causal_full_lists_equal_causal_dense():
    """Causal lists of every block up to the diagonal: the sparse kernel equals causal dense attention."""
    heads, kv, nb = 8, 2, 6
    n = nb * 64
    rng = np.random.default_rng(4)
    qb, kb, vb = (G.randn_bits(rng, (h, n, 128), O.F16) for h in (heads, kv, kv))
    sel = np.zeros((kv, nb, nb), np.uint16)
    nsel = np.zeros((kv, nb), np.uint16)
    for qbk in range(nb):
        sel[:, qbk, :qbk + 1] = rng.permutation(qbk + 1)  # any order
        nsel[:, qbk] = qbk + 1
    q, k, v = G.to_dev(qb, O.F16), G.to_dev(kb, O.F16), G.to_dev(vb, O.F16)
    o, _ = run_sparse(q, k, v, dev_u16(sel), dev_u16(nsel), dev(np.ones(n, np.uint8), None),
                      dev(np.arange(n, dtype=np.int32), None), n_q=n, q_pad=n, n_k=n, k_pad=n, heads=heads,
                      kv_heads=kv, n_cubes=nb, max_sel=nb, dense0=n, dense1=n, causal=1, sel_heads=kv)
    od = torch.empty((n, heads * 128), dtype=torch.float32, device="cuda")
    M.attn_fwd(q, k, v, od, n_q=n, q_pad=n, n_k=n, k_pad=n, heads=heads, kv_heads=kv, q_pos0=0, block=M.U32_MAX,
               dim=128)
    torch.cuda.synchronize()
    np.testing.assert_allclose(o, G.to_host(od), rtol=1e-2, atol=5e-4)


def test_window_random_s16384_sampled():
    """B1, 32 query heads over 8 kv heads, D 128, S 16384, 64x64 blocks, each block: the diagonal (causal), the 8
    before it and 8 random earlier ones (seed 16384, one list per kv head), bf16: one row of every (head, query tile)
    and sampled rows vs the oracle."""
    heads, kv, S = 32, 8, 16384
    nb = S // 64
    sel, nsel = M.window_random_blocks(nb, kv, seed=16384)
    gen = torch.Generator(device="cuda").manual_seed(16384)
    q = torch.randn((heads, S, 128), generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn((kv, S, 128), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((kv, S, 128), generator=gen, device="cuda").to(torch.bfloat16)
    valid = np.ones(S, np.uint8)
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=heads, kv_heads=kv, n_cubes=nb, max_sel=sel.shape[2],
                dense0=S, dense1=S, causal=1, sel_heads=kv)
    print("window + random S16384", flush=True)
    o, lse = run_sparse(q, k, v, dev_u16(sel), dev_u16(nsel), dev(valid, None), dev(np.arange(S, dtype=np.int32), None),
                        out=torch.bfloat16, **args)
    assert np.all(np.isfinite(o))
    rng = np.random.default_rng(2)
    rows = np.concatenate([[0, 1, 63, 64, 511, 512, S - 1], rng.integers(0, S, 150)])
    hr = np.stack([rng.integers(0, heads, len(rows)), rows], 1).astype(np.uint32)
    # and one random row of every (head, 64-row query tile): each workgroup item of the launch is compared
    h_, t_ = np.meshgrid(np.arange(heads), np.arange(nb), indexing="ij")
    hr = np.concatenate([hr, np.stack([h_.ravel(), t_.ravel() * 64 + rng.integers(0, 64, h_.size)], 1)]).astype(
        np.uint32)
    bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    want_o, want_l = O.attn_sparse_rows(bits(q), bits(k), bits(v), sel, nsel, valid, hr, dtype=O.BF16, **args)
    got = np.stack([o[r, h * 128:(h + 1) * 128] for h, r in hr])
    G.assert_attn_close(got, want_o, "sampled output")
    G.assert_rows_l2(got, want_o, "sampled output", 128)
    G.assert_lse_close(np.array([lse[h, r] for h, r in hr]), want_l, "sampled lse")


@pytest.mark.parametrize("heads,kv,causal,dt", [(8, 2, 0, O.BF16), (8, 2, 1, O.F16), (16, 2, 1, O.BF16),
                                                 (8, 1, 0, O.F16)])
def test_shared_lists_grouped(heads, kv, causal, dt):
    """Lists shared by a kv head's query heads in groups of 4 (the 8-wave path): random lists in random order,
    dense rows, a cube with invalid rows, rows past n_q, and a map that drops rows, against the oracle."""
    cubes, dense, topk = 5, 40, 3
    cnt = np.array([64, 64, 37, 64, 64], np.uint32)
    n = cubes * 64 + dense
    q_pad, k_pad = (n + 63) // 64 * 64, (n + 127) // 128 * 128
    n_q = n - 10
    valid = np.zeros(k_pad, np.uint8)
    for c in range(cubes):
        valid[c * 64:c * 64 + cnt[c]] = 1
    valid[cubes * 64:n] = 1
    map_ = np.full(q_pad, -1, np.int32)
    keep = np.nonzero(valid[:n_q])[0]
    map_[keep] = np.arange(len(keep), dtype=np.int32)
    map_[keep[::7]] = -1  # dropped rows stay untouched
    rng = np.random.default_rng(40 + heads + causal)
    sel = np.zeros((kv, cubes, topk), np.uint16)
    nsel = np.zeros((kv, cubes), np.uint16)
    for h in range(kv):
        for c in range(cubes):
            pool = np.arange(c + 1) if causal else np.arange(cubes)
            ch = rng.permutation(pool)[:topk]
            sel[h, c, :len(ch)] = ch
            nsel[h, c] = len(ch)
    qb, kb, vb = (G.randn_bits(rng, (hh, pad, 128), dt) for hh, pad in ((heads, q_pad), (kv, k_pad), (kv, k_pad)))
    args = dict(n_q=n_q, q_pad=q_pad, n_k=n, k_pad=k_pad, heads=heads, kv_heads=kv, n_cubes=cubes, max_sel=topk,
                dense0=cubes * 64, dense1=n, causal=causal, sel_heads=kv)
    print(f"shared lists heads {heads} kv {kv} causal {causal}", flush=True)
    want_o, want_l = O.attn_sparse(qb, kb, vb, sel, nsel, valid, map_, dtype=dt, o_fill=np.full((q_pad, heads * 128),
                                   SENTINEL), **args)
    for out in (torch.float32, G.TORCH[dt]):
        o, lse = run_sparse(G.to_dev(qb, dt), G.to_dev(kb, dt), G.to_dev(vb, dt), dev_u16(sel), dev_u16(nsel),
                            dev(valid), dev(map_), out=out, **args)
        written = np.zeros(q_pad, bool)
        written[map_[map_ >= 0]] = True
        G.assert_attn_close(o[written], want_o[written], "output")
        assert np.all(o[~written] == SENTINEL), "rows outside the map were written"
        rows = np.nonzero(map_ >= 0)[0]
        G.assert_lse_close(lse[:, rows], want_l[:, rows], "lse")


@pytest.mark.parametrize("heads,kv,causal,dt,cubes,dense,cut,topk", [
    (8, 8, 0, O.F16, 7, 70, 0, 4),     # MHA, heads a multiple of 8 (items dealt by XCD), dense rows past a 32 boundary
    (16, 4, 1, O.F16, 6, 45, 13, 4),   # GQA with a list per query head, causal, rows past n_q
    (3, 3, 0, O.F16, 5, 0, 0, 4),      # no dense rows, heads not a multiple of 8
    (2, 1, 0, O.BF16, 4, 33, 0, 4),    # bf16: the per-head route of the compiled kernel
    (1, 1, 0, O.F16, 72, 40, 0, 70),   # lists of up to 70 entries: more than 128 candidate tiles for one workgroup
    (2, 2, 1, O.F16, 7, 20, 0, 260),   # lists longer than the f16 route packs (max_sel 260): the compiled kernel
])
def test_per_head_lists(heads, kv, causal, dt, cubes, dense, cut, topk):
    """A list per query head (sel_heads == heads, as cube_select writes them and MiniMax-H3 calls it): random lists
    of random lengths (some empty), cubes with invalid rows and one with none past its first half, dense rows, query
    tiles past the cubes (every key), rows past n_q, and a map that permutes and drops rows, against the oracle in
    f32 and the input type out."""
    cnt = np.full(cubes, 64, np.uint32)
    cnt[1], cnt[-1] = 37, 20  # the last cube's second 32-key tile has no valid key
    n = cubes * 64 + dense
    q_pad, k_pad = (n + 63) // 64 * 64, (n + 127) // 128 * 128
    n_q = n - cut
    valid = np.zeros(k_pad, np.uint8)
    for c in range(cubes):
        valid[c * 64:c * 64 + cnt[c]] = 1
    valid[cubes * 64:n] = 1
    rng = np.random.default_rng(100 + heads + causal)
    keep = np.nonzero(valid[:n_q])[0]
    map_ = np.full(q_pad, -1, np.int32)
    map_[keep] = rng.permutation(len(keep)).astype(np.int32)
    map_[keep[::9]] = -1
    sel = np.zeros((heads, cubes, topk), np.uint16)
    nsel = np.zeros((heads, cubes), np.uint16)
    for h in range(heads):
        for c in range(cubes):
            pool = np.arange(c + 1) if causal else np.arange(cubes)
            ch = rng.permutation(pool)[:rng.integers(0, topk + 1)]
            sel[h, c, :len(ch)] = ch
            nsel[h, c] = len(ch)
    qb, kb, vb = (G.randn_bits(rng, (hh, pad, 128), dt) for hh, pad in ((heads, q_pad), (kv, k_pad), (kv, k_pad)))
    args = dict(n_q=n_q, q_pad=q_pad, n_k=n, k_pad=k_pad, heads=heads, kv_heads=kv, n_cubes=cubes, max_sel=topk,
                dense0=cubes * 64, dense1=n, causal=causal, sel_heads=heads)
    print(f"per-head lists heads {heads} kv {kv} causal {causal} dtype {dt}", flush=True)
    want_o, want_l = O.attn_sparse(qb, kb, vb, sel, nsel, valid, map_, dtype=dt, o_fill=np.full((q_pad, heads * 128),
                                   SENTINEL), **args)
    for out in (torch.float32, G.TORCH[dt]):
        o, lse = run_sparse(G.to_dev(qb, dt), G.to_dev(kb, dt), G.to_dev(vb, dt), dev_u16(sel), dev_u16(nsel),
                            dev(valid), dev(map_), out=out, **args)
        written = np.zeros(q_pad, bool)
        written[map_[map_ >= 0]] = True
        G.assert_attn_close(o[written], want_o[written], "output")
        G.assert_rows_l2(o[written], want_o[written], "output", 128)
        assert np.all(o[~written] == SENTINEL), "rows outside the map were written"
        rows = np.nonzero(map_ >= 0)[0]
        G.assert_lse_close(lse[:, rows], want_l[:, rows], "lse")
