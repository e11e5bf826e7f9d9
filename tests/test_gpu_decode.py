"""Batched split-K decode (mako_attn_decode) on the GPU against the CPU oracle: the golden fixture, a sweep of
ragged contexts and GQA groups (an empty context, contexts at and around split boundaries), invariance to the
split size, agreement with the dense kernel's row at q_pos0 = ctx - 1, and the batch-16 configuration (contexts
drawn from [1024, 32768]) on sampled (sequence, head) pairs."""
import numpy as np
import pytest

import oracle as O
from conftest import golden_files, load_golden

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402


def run_decode(q, k, v, ctx, *, batch, heads, kv_heads, cap, max_ctx=None, split=0, out=torch.float32):
    """q, k, v torch tensors on cuda; ctx a numpy u32 array. Returns (o, lse) as float64 numpy."""
    a = M.decode_args(batch=batch, heads=heads, kv_heads=kv_heads, dim=128, cap=cap,
                      max_ctx=int(ctx.max()) if max_ctx is None else max_ctx, split=split)
    ws = torch.empty(max(M.decode_workspace(a), 16), dtype=torch.uint8, device="cuda")
    ctx_d = torch.from_numpy(ctx.astype(np.int32)).to("cuda")
    o = torch.full((batch, heads * 128), float("nan"), dtype=out, device="cuda")
    lse = torch.full((batch, heads), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_decode(a, q, k, v, ctx_d, o, ws, lse=lse)
    torch.cuda.synchronize()
    return G.to_host(o), lse.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("path", golden_files("decode"), ids=lambda p: p.split("/")[-1][:-4])
def test_golden(path):
    g = load_golden(path)
    batch, heads, kv, dim, cap, dt = [int(x) for x in g["args"]]
    q, k, v = G.to_dev(g["q"], dt), G.to_dev(g["k"], dt), G.to_dev(g["v"], dt)
    for split in (0, 64):
        o, lse = run_decode(q, k, v, g["ctx"], batch=batch, heads=heads, kv_heads=kv, cap=cap, split=split)
        G.assert_attn_close(o, g["o"], f"output (split {split})")
        G.assert_lse_close(lse, g["lse"], f"lse (split {split})")


SWEEP = [
    # batch, heads, kv, cap, ctx, dtype, split
    (4, 32, 8, 1100, [1, 511, 512, 1025], O.F16, 0),
    (3, 8, 8, 700, [0, 64, 700], O.BF16, 64),        # an empty context: 0 and -inf
    (2, 16, 2, 3000, [2048, 2999], O.F16, 256),      # group 8
    (5, 4, 4, 300, [33, 31, 32, 100, 300], O.BF16, 128),
    (1, 32, 1, 4096, [4096], O.F16, 1024),           # group 32
]


@pytest.mark.parametrize("case", SWEEP, ids=lambda c: f"b{c[0]}h{c[1]}kv{c[2]}s{c[6]}")
def test_sweep(case):
    batch, heads, kv, cap, ctx, dt, split = case
    ctx = np.array(ctx, np.uint32)
    rng = np.random.default_rng(sum(ctx.tolist()) + heads)
    qb = G.randn_bits(rng, (batch, heads, 128), dt)
    kb = G.randn_bits(rng, (batch, kv, cap, 128), dt)
    vb = G.randn_bits(rng, (batch, kv, cap, 128), dt)
    print(f"decode sweep {case}", flush=True)
    for out in (torch.float32, G.TORCH[dt]):
        o, lse = run_decode(G.to_dev(qb, dt), G.to_dev(kb, dt), G.to_dev(vb, dt), ctx, batch=batch, heads=heads,
                            kv_heads=kv, cap=cap, max_ctx=cap, split=split, out=out)
        want_o, want_l = O.attn_decode(qb, kb, vb, ctx, batch=batch, heads=heads, kv_heads=kv, dim=128, cap=cap,
                                       dtype=dt)
        G.assert_attn_close(o, want_o, "output")
        G.assert_lse_close(lse, want_l, "lse")


def test_split_invariance_and_dense_agreement():
    """Splits of 64, 512 and 4096 keys agree to within P's f16 rounding (where the running maximum moves depends on
    the split, so P rounds against different maxima); each row equals mako_attn_fwd's single query at
    q_pos0 = ctx - 1 over the same cache (the reference's decode path). A dropped or doubled split would be off by
    the output's own size (~3e-2 here)."""
    batch, heads, kv, cap = 3, 16, 4, 5000
    ctx = np.array([4999, 1234, 77], np.uint32)
    gen = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((batch, heads, 128), generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn((batch, kv, cap, 128), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((batch, kv, cap, 128), generator=gen, device="cuda").to(torch.bfloat16)
    outs = [run_decode(q, k, v, ctx, batch=batch, heads=heads, kv_heads=kv, cap=cap, split=s)
            for s in (64, 512, 4096)]
    for o, lse in outs[1:]:
        np.testing.assert_allclose(o, outs[0][0], rtol=1e-2, atol=3e-4)
        np.testing.assert_allclose(lse, outs[0][1], rtol=0, atol=1e-4)
    for b in range(batch):
        qt = torch.zeros((heads, 64, 128), dtype=torch.bfloat16, device="cuda")
        qt[:, 0] = q[b]
        o = torch.empty((1, heads * 128), dtype=torch.float32, device="cuda")
        lse = torch.empty((heads, 1), dtype=torch.float32, device="cuda")
        M.attn_fwd(qt, k[b].contiguous(), v[b].contiguous(), o, n_q=1, q_pad=64, n_k=int(ctx[b]), k_pad=cap,
                   heads=heads, kv_heads=kv, q_pos0=int(ctx[b]) - 1, block=M.U32_MAX, dim=128, lse=lse)
        torch.cuda.synchronize()
        np.testing.assert_allclose(outs[1][0][b], G.to_host(o)[0], rtol=1e-2, atol=3e-4)
        np.testing.assert_allclose(outs[1][1][b], lse.cpu().numpy()[:, 0], rtol=0, atol=1e-4)


def test_batch16_contexts_1k_to_32k():
    """Batch 16, 32 query heads over 8 kv heads, D 128, contexts drawn uniformly from [1024, 32768] (seed 2026),
    f16 cache and query, f32 out: every (sequence, head) pair, all 512, against the oracle."""
    batch, heads, kv = 16, 32, 8
    ctx = np.random.default_rng(2026).integers(1024, 32769, batch).astype(np.uint32)
    cap = int(ctx.max())
    gen = torch.Generator(device="cuda").manual_seed(2026)
    q = torch.randn((batch, heads, 128), generator=gen, device="cuda").half()
    k = torch.randn((batch, kv, cap, 128), generator=gen, device="cuda").half()
    v = torch.randn((batch, kv, cap, 128), generator=gen, device="cuda").half()
    print("decode batch 16", flush=True)
    o, lse = run_decode(q, k, v, ctx, batch=batch, heads=heads, kv_heads=kv, cap=cap)
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(lse))
    pairs = np.stack(np.meshgrid(np.arange(batch), np.arange(heads), indexing="ij"), -1).reshape(-1, 2)
    pairs = pairs.astype(np.uint32)
    bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    want_o, want_l = O.attn_decode_rows(bits(q), bits(k), bits(v), ctx, pairs, batch=batch, heads=heads,
                                        kv_heads=kv, dim=128, cap=cap, dtype=O.F16)
    got_o = np.stack([o[b, h * 128:(h + 1) * 128] for b, h in pairs])
    G.assert_attn_close(got_o, want_o, "output")
    G.assert_rows_l2(got_o, want_o, "output", 128)
    G.assert_lse_close(np.array([lse[b, h] for b, h in pairs]), want_l, "lse")
