"""mako_attn_decode_noalloc (split-K partials in the library's static device scratch) against mako_attn_decode
(partials in a caller's workspace), through the C ABI: two calls in a row, the second smaller, each equal to the
workspace entry point's result bit for bit (the same split and kernels) and within the path's tolerance of the
oracle; a call whose partials exceed the static scratch is refused."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402


def _inputs(seed, batch, heads, kv, cap, ctx, dt):
    rng = np.random.default_rng(seed)
    qb = G.randn_bits(rng, (batch, heads, 128), dt)
    kb = G.randn_bits(rng, (batch, kv, cap, 128), dt)
    vb = G.randn_bits(rng, (batch, kv, cap, 128), dt)
    return qb, kb, vb, np.array(ctx, np.uint32)


def _both(qb, kb, vb, ctx, batch, heads, kv, cap, dt):
    q, k, v = G.to_dev(qb, dt), G.to_dev(kb, dt), G.to_dev(vb, dt)
    ctx_d = torch.from_numpy(ctx.astype(np.int32)).to("cuda")
    a = M.decode_args(batch=batch, heads=heads, kv_heads=kv, dim=128, cap=cap, max_ctx=int(ctx.max()))
    assert M.decode_workspace(a) <= M.DECODE_SCRATCH_BYTES
    ws = torch.empty(M.decode_workspace(a), dtype=torch.uint8, device="cuda")
    o_ws = torch.full((batch, heads * 128), float("nan"), dtype=torch.float32, device="cuda")
    l_ws = torch.full((batch, heads), float("nan"), dtype=torch.float32, device="cuda")
    o_na = torch.full_like(o_ws, float("nan"))
    l_na = torch.full_like(l_ws, float("nan"))
    M.attn_decode(a, q, k, v, ctx_d, o_ws, ws, lse=l_ws)
    M.attn_decode_noalloc(a, q, k, v, ctx_d, o_na, lse=l_na)
    torch.cuda.synchronize()
    return (o_ws.cpu().numpy(), l_ws.cpu().numpy()), (o_na.cpu().numpy(), l_na.cpu().numpy())


def test_noalloc_matches_workspace_entry_twice():
    cases = [
        # seed, batch, heads, kv, cap, contexts, dtype: the second call is smaller
        (101, 6, 32, 8, 5000, [4999, 1, 0, 2048, 3333, 4096], O.F16),
        (202, 2, 16, 4, 900, [777, 65], O.BF16),
    ]
    for seed, batch, heads, kv, cap, ctx, dt in cases:
        print(f"noalloc decode: batch {batch}, {heads}/{kv} heads, contexts {ctx}", flush=True)
        qb, kb, vb, ctx = _inputs(seed, batch, heads, kv, cap, ctx, dt)
        (o_ws, l_ws), (o_na, l_na) = _both(qb, kb, vb, ctx, batch, heads, kv, cap, dt)
        assert np.array_equal(o_na, o_ws, equal_nan=False), "output differs from mako_attn_decode"
        assert np.array_equal(l_na, l_ws), "lse differs from mako_attn_decode"
        want_o, want_l = O.attn_decode(qb, kb, vb, ctx, batch=batch, heads=heads, kv_heads=kv, dim=128, cap=cap,
                                       dtype=dt)
        G.assert_attn_close(o_na, want_o, "noalloc output")
        G.assert_lse_close(l_na, want_l, "noalloc lse")


def test_noalloc_refuses_partials_past_the_scratch():
    # group 32: the partials grow with the batch ((resident waves + pieces) x 32 heads x 520 bytes), so the batch
    # doubles until they exceed the static scratch on this GPU; the refusal comes before any launch.
    batch = 64
    while True:
        a = M.decode_args(batch=batch, heads=32, kv_heads=1, dim=128, cap=1024, max_ctx=1024)
        if M.decode_workspace(a) > M.DECODE_SCRATCH_BYTES:
            break
        batch *= 2
        assert batch <= 1 << 16, "the partials never exceed the static scratch"
    q = torch.zeros((batch, 32, 128), dtype=torch.float16, device="cuda")
    k = torch.zeros((batch, 1, 1024, 128), dtype=torch.float16, device="cuda")  # the full cache, in case of a launch
    ctx = torch.ones(batch, dtype=torch.int32, device="cuda")
    o = torch.empty((batch, 32 * 128), dtype=torch.float32, device="cuda")
    with pytest.raises(M.MakoError) as e:
        M.attn_decode_noalloc(a, q, k, k, ctx, o)
    assert e.value.code == M.EWORKSPACE and "static scratch" in str(e.value)
