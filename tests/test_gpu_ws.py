"""The workspace-taking entry points (mako_attn_fwd_ws, mako_attn_sparse_ws, mako_attn_fwd_rows_ws) on the GPU: with
exactly the workspace their queries report they give the bits of the entry points without one (which keep the
library's own), a workspace one byte short is refused with MAKO_EWORKSPACE, and mako_attn_release frees what the
library keeps for a stream. Routes: the prefill kernel (no workspace), the split-K route of a few rows (partials),
heads of 256 (V^T images), the block-sparse r64 route (pass table), attention from rows (tiles)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import mako_attn as M  # noqa: E402

U32 = 0xFFFFFFFF


def randn(g, shape, dt):
    return torch.randn(shape, generator=g, device="cuda").to(dt)


def bits(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).cpu().numpy()


def same(a, b):
    return np.array_equal(bits(a), bits(b))


def short(ws):
    return None if ws is None or ws.numel() <= 1 else ws[:-1]


DENSE = [
    # name, heads, kv, dim, n_q, n_k, q_pos0, block
    ("prefill", 8, 2, 128, 300, 300, 0, U32),
    ("split_k_rows", 32, 8, 128, 1, 3000, 2999, U32),
    ("split_k_4_rows", 32, 8, 128, 4, 700, 696, U32),
    ("d256", 4, 2, 256, 130, 130, 0, U32),   # flash_fwd_r32: no workspace (flash_fwd_d256's images past its offsets)
]
NO_WORKSPACE = ("prefill", "d256")


@pytest.mark.parametrize("case", DENSE, ids=lambda c: c[0])
def test_fwd_ws_matches_library_workspace(case):
    name, heads, kv, dim, n_q, n_k, q_pos0, block = case
    print(f"fwd ws {case}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    q_pad, k_pad = (n_q + 63) // 64 * 64, (n_k + 127) // 128 * 128
    q, k, v = randn(g, (heads, q_pad, dim), torch.bfloat16), randn(g, (kv, k_pad, dim), torch.bfloat16), \
        randn(g, (kv, k_pad, dim), torch.bfloat16)
    args = dict(n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=q_pos0, block=block,
                dim=dim)
    need = M.attn_fwd_workspace(**args)
    assert (need == 0) == (name in NO_WORKSPACE), need
    outs = []
    for ws in (M.LIBRARY, torch.empty(need, dtype=torch.uint8, device="cuda") if need else None):
        o = torch.full((n_q, heads * dim), float("nan"), dtype=torch.bfloat16, device="cuda")
        lse = torch.full((heads, n_q), float("nan"), dtype=torch.float32, device="cuda")
        M.attn_fwd(q, k, v, o, lse=lse, workspace=ws, **args)
        torch.cuda.synchronize()
        outs.append((o, lse))
    assert same(outs[0][0], outs[1][0]) and same(outs[0][1], outs[1][1])
    if need:
        o = torch.empty((n_q, heads * dim), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(M.MakoError) as e:
            M.attn_fwd(q, k, v, o, workspace=short(torch.empty(need, dtype=torch.uint8, device="cuda")), **args)
        assert e.value.code == M.EWORKSPACE


def test_sparse_ws_matches_library_workspace():
    """Lists shared by a kv head's 4 query heads (the r64 route and its pass table), causal."""
    heads, kv, cubes = 8, 2, 5
    n = cubes * 64
    g = torch.Generator(device="cuda").manual_seed(6)
    q, k, v = randn(g, (heads, n, 128), torch.bfloat16), randn(g, (kv, n + 64, 128), torch.bfloat16), \
        randn(g, (kv, n + 64, 128), torch.bfloat16)
    rng = np.random.default_rng(6)
    sel = np.zeros((kv, cubes, 3), np.uint16)
    nsel = np.zeros((kv, cubes), np.uint16)
    for h in range(kv):
        for c in range(cubes):
            ch = rng.permutation(c + 1)[:3]
            sel[h, c, :len(ch)] = ch
            nsel[h, c] = len(ch)
    sel_d = torch.from_numpy(sel.view(np.int16)).to("cuda")
    nsel_d = torch.from_numpy(nsel.view(np.int16)).to("cuda")
    valid = torch.ones(n + 64, dtype=torch.uint8, device="cuda")
    map_ = torch.arange(n, dtype=torch.int32, device="cuda")
    args = dict(n_q=n, q_pad=n, n_k=n, k_pad=n + 64, heads=heads, kv_heads=kv, n_cubes=cubes, max_sel=3,
                dense0=n, dense1=n, causal=1, sel_heads=kv)
    need = M.attn_sparse_workspace(**args)
    assert need > 0
    print(f"sparse ws: {need} bytes", flush=True)
    outs = []
    for ws in (M.LIBRARY, torch.empty(need, dtype=torch.uint8, device="cuda")):
        o = torch.full((n, heads * 128), float("nan"), dtype=torch.float32, device="cuda")
        M.attn_sparse(q, k, v, o, sel_d, nsel_d, valid, map_, workspace=ws, **args)
        torch.cuda.synchronize()
        outs.append(o)
    assert same(outs[0], outs[1])
    with pytest.raises(M.MakoError) as e:
        M.attn_sparse(q, k, v, outs[1], sel_d, nsel_d, valid, map_,
                      workspace=short(torch.empty(need, dtype=torch.uint8, device="cuda")), **args)
    assert e.value.code == M.EWORKSPACE


@pytest.mark.parametrize("dim,n_q,n_k,q_pos0", [(128, 200, 200, 0), (128, 2, 600, 598), (256, 70, 70, 0)],
                         ids=["fused", "split_k", "d256"])
def test_rows_ws_matches_library_workspace(dim, n_q, n_k, q_pos0):
    heads, kv = 8, 2
    rng = np.random.default_rng(dim + n_q)
    xq = torch.from_numpy(rng.standard_normal((n_q, heads * dim)).astype(np.float32)).to("cuda")
    xk = torch.from_numpy(rng.standard_normal((n_k, kv * dim)).astype(np.float32)).to("cuda")
    xv = torch.from_numpy(rng.standard_normal((n_k, kv * dim)).astype(np.float32)).to("cuda")
    hq = dict(rows=n_q, ld=heads * dim, col0=0, stride=dim, dim=dim, heads=heads)
    hk = dict(rows=n_k, ld=kv * dim, col0=0, stride=dim, dim=dim, heads=kv)
    hv = dict(hk)
    args = dict(n_q=n_q, n_k=n_k, heads=heads, kv_heads=kv, q_pos0=q_pos0, block=U32)
    need = M.attn_fwd_rows_workspace(dim=dim, **args)
    print(f"rows ws dim {dim}: {need} bytes", flush=True)
    outs = []
    for ws in (M.LIBRARY, torch.empty(need, dtype=torch.uint8, device="cuda")):
        o = torch.full((n_q, heads * dim), float("nan"), dtype=torch.bfloat16, device="cuda")
        M.attn_fwd_rows(xq, xk, xv, o, hq, hk, hv, in_dtype=M.BF16, workspace=ws, **args)
        torch.cuda.synchronize()
        outs.append(o)
    assert same(outs[0], outs[1])
    with pytest.raises(M.MakoError) as e:
        M.attn_fwd_rows(xq, xk, xv, outs[1], hq, hk, hv, in_dtype=M.BF16,
                        workspace=short(torch.empty(need, dtype=torch.uint8, device="cuda")), **args)
    assert e.value.code == M.EWORKSPACE


def test_release_frees_the_library_workspace():
    """A one-row call through mako_attn_fwd on a new stream leaves the library holding its partials for that stream;
    releasing the stream frees them (the others' stay), and the next call on it allocates again."""
    g = torch.Generator(device="cuda").manual_seed(7)
    q = randn(g, (32, 64, 128), torch.bfloat16)
    k, v = randn(g, (8, 2048, 128), torch.bfloat16), randn(g, (8, 2048, 128), torch.bfloat16)
    o = torch.empty((1, 32 * 128), dtype=torch.bfloat16, device="cuda")
    args = dict(n_q=1, q_pad=64, n_k=2048, k_pad=2048, heads=32, kv_heads=8, q_pos0=2047, block=U32, dim=128)
    torch.cuda.synchronize()
    before = M.held_bytes()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        M.attn_fwd(q, k, v, o, stream=s.cuda_stream, **args)
    s.synchronize()
    assert M.held_bytes() >= before + M.attn_fwd_workspace(**args) > before
    M.release(stream=s.cuda_stream)
    assert M.held_bytes() == before
    o2 = torch.empty_like(o)
    with torch.cuda.stream(s):
        M.attn_fwd(q, k, v, o2, stream=s.cuda_stream, **args)
    s.synchronize()
    assert same(o, o2)
    M.release(stream=s.cuda_stream)
