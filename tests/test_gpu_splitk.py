"""attention() with a few query rows (mako_attn_fwd, heads of 128): n_q rows x the GQA group <= 64 columns take the
split-K route (each kv head's keys cut over all CUs, a workgroup's waves combining their partials in LDS, the
pieces merged by LSE in a second launch) instead of the prefill kernels, which would leave the GPU nearly empty. Checked against the oracle on every row: the reference's decode shape
(attention(n_q, q_pos0 = ctx - n_q), ops.metal:289) at ctx 32768 with 32 query heads over 8 kv heads for n_q 1, 4
and 16, and the edges of the route: two column blocks (MHA with 64 rows, GQA 8 with 8 rows), rows whose keys stop
short of n_k, a prefix-causal block, n_k = 0, and a row count just past the route (prefill kernels)."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402

U32 = 0xFFFFFFFF

# (n_q, heads, kv_heads, n_k, q_pos0 or None for n_k - n_q, block, dtype, out)
CASES = [
    (1, 32, 8, 32768, None, U32, O.BF16, "same"),
    (4, 32, 8, 32768, None, U32, O.BF16, "f32"),
    (16, 32, 8, 32768, None, U32, O.F16, "same"),
    (64, 8, 8, 3000, None, U32, O.BF16, "f32"),     # MHA: 64 columns, two blocks
    (8, 16, 2, 4100, None, U32, O.F16, "f32"),      # GQA 8: 64 columns
    (3, 8, 4, 5000, 100, U32, O.BF16, "f32"),       # rows see keys [0, 101 .. 103) of 5000
    (5, 8, 2, 4000, 2500, 2000, O.BF16, "same"),    # prefix-causal, every row past the block: all keys
    (2, 8, 2, 3000, 1990, 2000, O.F16, "f32"),      # rows on both sides of the block
    (2, 8, 8, 0, 0, U32, O.BF16, "f32"),            # no keys: 0 and lse = -inf
    (17, 32, 8, 2048, None, U32, O.BF16, "f32"),    # 68 columns: the prefill kernels
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "q{}h{}kv{}k{}p{}b{}".format(
    c[0], c[1], c[2], c[3], "end" if c[4] is None else c[4], "c" if c[5] == U32 else c[5]))
def test_few_rows_against_oracle(case):
    n_q, heads, kv, n_k, q_pos0, block, dt, out = case
    q_pos0 = n_k - n_q if q_pos0 is None else q_pos0
    print(f"split-K case {case}", flush=True)
    rng = np.random.default_rng(n_q * 1000003 + n_k)
    q_pad, k_pad = max(n_q, 1), max(n_k, 64)
    qb = G.randn_bits(rng, (heads, q_pad, 128), dt)
    kb = G.randn_bits(rng, (kv, k_pad, 128), dt)
    vb = G.randn_bits(rng, (kv, k_pad, 128), dt)
    q, k, v = G.to_dev(qb, dt), G.to_dev(kb, dt), G.to_dev(vb, dt)
    odt = torch.float32 if out == "f32" else G.TORCH[dt]
    o = torch.full((n_q, heads * 128), float("nan"), dtype=odt, device="cuda")
    lse = torch.full((heads, n_q), float("nan"), dtype=torch.float32, device="cuda")
    args = dict(n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=q_pos0, block=block,
                dim=128)
    M.attn_fwd(q, k, v, o, lse=lse, **args)
    torch.cuda.synchronize()
    got_o, got_l = G.to_host(o), lse.cpu().numpy().astype(np.float64)
    want_o, want_l = O.attn_dense(qb, kb, vb, dtype=dt, **args)
    G.assert_attn_close(got_o, want_o, "output")
    G.assert_rows_l2(got_o, want_o, "output", 128)
    G.assert_lse_close(got_l, want_l, "lse")


def test_split_route_matches_prefill_kernel_rows():
    """The last 4 rows of a causal S2048 prefill (32 / 8 heads), asked for alone (split-K), equal the same rows of
    the whole prefill (the prefill kernels) to within the two kernels' rounding of P."""
    n, heads, kv = 2048, 32, 8
    rng = np.random.default_rng(77)
    qb, kb, vb = (G.randn_bits(rng, (h, n, 128), O.BF16) for h in (heads, kv, kv))
    q, k, v = G.to_dev(qb, O.BF16), G.to_dev(kb, O.BF16), G.to_dev(vb, O.BF16)
    full = torch.empty((n, heads * 128), dtype=torch.float32, device="cuda")
    lf = torch.empty((heads, n), dtype=torch.float32, device="cuda")
    M.attn_fwd(q, k, v, full, lse=lf, n_q=n, q_pad=n, n_k=n, k_pad=n, heads=heads, kv_heads=kv, q_pos0=0,
               block=U32, dim=128)
    tail = torch.empty((4, heads * 128), dtype=torch.float32, device="cuda")
    lt = torch.empty((heads, 4), dtype=torch.float32, device="cuda")
    qt = q[:, n - 4:].contiguous()
    M.attn_fwd(qt, k, v, tail, lse=lt, n_q=4, q_pad=4, n_k=n, k_pad=n, heads=heads, kv_heads=kv, q_pos0=n - 4,
               block=U32, dim=128)
    torch.cuda.synchronize()
    np.testing.assert_allclose(G.to_host(tail), G.to_host(full)[n - 4:], rtol=1e-2, atol=1e-3)
    np.testing.assert_allclose(lt.cpu().numpy(), lf.cpu().numpy()[:, n - 4:], rtol=0, atol=1e-4)


def test_repeated_calls_same_bits():
    """Calls in a row on one stream reuse its cached workspace: a repeat gives the same bits (the combine and merge
    orders are fixed), also after a call over other kv heads, rows and keys in the same workspace, which matches the
    oracle."""
    rng = np.random.default_rng(2027)

    def make(heads, kv, n_k, n_q):
        qb = G.randn_bits(rng, (heads, n_q, 128), O.BF16)
        kb = G.randn_bits(rng, (kv, n_k, 128), O.BF16)
        vb = G.randn_bits(rng, (kv, n_k, 128), O.BF16)
        args = dict(n_q=n_q, q_pad=n_q, n_k=n_k, k_pad=n_k, heads=heads, kv_heads=kv, q_pos0=n_k - n_q, block=U32,
                    dim=128)
        return (qb, kb, vb), tuple(G.to_dev(x, O.BF16) for x in (qb, kb, vb)), args

    def call(dev, args):
        o = torch.full((args["n_q"], args["heads"] * 128), float("nan"), dtype=torch.float32, device="cuda")
        lse = torch.full((args["heads"], args["n_q"]), float("nan"), dtype=torch.float32, device="cuda")
        M.attn_fwd(*dev, o, lse=lse, **args)
        torch.cuda.synchronize()
        return o.cpu().numpy(), lse.cpu().numpy()

    _, dev_a, args_a = make(32, 8, 9000, 2)
    host_b, dev_b, args_b = make(12, 4, 5000, 5)
    first = call(dev_a, args_a)
    assert np.isfinite(first[0]).all() and np.isfinite(first[1]).all()
    for _ in range(2):
        again = call(dev_a, args_a)
        assert np.array_equal(again[0], first[0]) and np.array_equal(again[1], first[1])
    got_o, got_l = call(dev_b, args_b)
    want_o, want_l = O.attn_dense(*host_b, dtype=O.BF16, **args_b)
    G.assert_attn_close(got_o, want_o, "output")
    G.assert_lse_close(got_l.astype(np.float64), want_l, "lse")
    again = call(dev_a, args_a)
    assert np.array_equal(again[0], first[0]) and np.array_equal(again[1], first[1])
