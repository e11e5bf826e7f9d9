"""Dense flash attention (mako_attn_fwd) on the GPU against the CPU oracle: the golden fixtures, the f16 S512
causal GQA case in full, a sweep of masks / head widths / GQA groups / ragged sizes, untouched rows past n_q,
and sampled rows of the Qwen3-8B-shape causal prefill (S4096) and the bidirectional S16384 case."""
import zlib

import numpy as np
import pytest

import oracle as O
from conftest import golden_files, load_golden

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402

U32 = 0xFFFFFFFF


def run_fwd(qb, kb, vb, dtype, out, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, dim, o_rows=None,
            fill=None):
    q, k, v = G.to_dev(qb, dtype), G.to_dev(kb, dtype), G.to_dev(vb, dtype)
    o_rows = n_q if o_rows is None else o_rows
    odt = torch.float32 if out == O.F32 else G.TORCH[dtype]
    o = torch.full((o_rows, heads * dim), float(fill) if fill is not None else float("nan"), dtype=odt,
                   device="cuda")
    lse = torch.full((heads, max(n_q, 1)), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_fwd(q, k, v, o, n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv_heads,
               q_pos0=q_pos0, block=block, dim=dim, lse=lse)
    torch.cuda.synchronize()
    return G.to_host(o), lse.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("path", golden_files("dense"), ids=lambda p: p.split("/")[-1][:-4])
@pytest.mark.parametrize("out", ["f32", "same"])
def test_golden(path, out):
    g = load_golden(path)
    n_q, q_pad, n_k, k_pad, heads, kv, q_pos0, block, width, dim, dt = [int(x) for x in g["args"]]
    print(f"golden {path.split('/')[-1]} out={out}", flush=True)
    o, lse = run_fwd(g["q"], g["k"], g["v"], dt, O.F32 if out == "f32" else dt, n_q=n_q, q_pad=q_pad, n_k=n_k,
                     k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=q_pos0, block=block, dim=dim)
    G.assert_attn_close(o, g["o"], "output")
    G.assert_lse_close(lse[:, :n_q], g["lse"], "lse")


def test_causal_gqa_s512_f16_full():
    """Batch 1, 16 query heads over 8 kv heads, D 128, S 512, f16 in, f32 out + LSE: every row."""
    rng = np.random.default_rng(1234)
    heads, kv, dim, S = 16, 8, 128, 512
    qb, kb, vb = (G.randn_bits(rng, (h, S, dim), O.F16) for h in (heads, kv, kv))
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=heads, kv_heads=kv, q_pos0=0, block=U32, dim=dim)
    print("causal S512 f16", flush=True)
    o, lse = run_fwd(qb, kb, vb, O.F16, O.F32, **args)
    want_o, want_l = O.attn_dense(qb, kb, vb, dtype=O.F16, **args)
    G.assert_attn_close(o, want_o, "output")
    G.assert_rows_l2(o, want_o, "output", dim)
    G.assert_lse_close(lse, want_l, "lse")


SWEEP = [
    # heads, kv, dim, n_q, n_k, q_pos0, block, dtype, out
    (4, 4, 128, 200, 200, 0, 0, O.BF16, "same"),        # bidirectional MHA, ragged
    (8, 2, 128, 257, 257, 0, U32, O.BF16, "f32"),       # causal, group 4, one row past a tile
    (6, 2, 128, 96, 96, 0, U32, O.F16, "same"),         # group 3 (hq 1)
    (4, 2, 128, 100, 300, 200, U32, O.F16, "f32"),      # chunked prefill: queries late in the keys
    (2, 1, 128, 150, 150, 0, 64, O.BF16, "f32"),        # prefix-causal
    (2, 1, 128, 150, 150, 0, 77, O.F16, "same"),        # prefix-causal, block inside a tile
    (16, 2, 64, 130, 130, 0, U32, O.F16, "f32"),        # D 64, group 8
    (4, 4, 64, 70, 333, 0, 0, O.BF16, "same"),          # D 64, more keys than queries
    (8, 8, 64, 300, 300, 0, 0, O.BF16, "same"),         # D 64, bidirectional MHA over five tiles (the H3 VAE's kind)
    (4, 2, 64, 100, 300, 200, U32, O.F16, "f32"),       # D 64, chunked prefill
    (2, 1, 64, 150, 150, 0, 77, O.BF16, "f32"),         # D 64, prefix-causal, block inside a tile
    (6, 2, 64, 96, 96, 0, U32, O.F16, "same"),          # D 64, group 3 (hq 1)
    (2, 2, 256, 80, 80, 0, U32, O.BF16, "f32"),         # D 256
    (4, 1, 256, 65, 129, 64, U32, O.F16, "same"),       # D 256, group 4, offset
    (4, 4, 256, 200, 200, 0, 0, O.BF16, "f32"),         # D 256, bidirectional MHA, ragged (hq 1)
    (16, 2, 256, 130, 300, 170, U32, O.BF16, "same"),   # D 256, group 8, chunked prefill
    (6, 2, 256, 96, 96, 0, 50, O.F16, "f32"),           # D 256, group 3, prefix-causal inside a tile
    (4, 2, 256, 40, 5, 0, U32, O.BF16, "f32"),          # D 256, fewer keys than queries
    (2, 1, 256, 3, 0, 0, U32, O.F16, "f32"),            # D 256, no keys: 0 and lse = -inf
    (2, 1, 64, 3, 0, 0, U32, O.BF16, "f32"),            # D 64, no keys
    (2, 1, 128, 100, 0, 0, U32, O.F16, "same"),         # no keys, rows enough for the prefill kernels
    (8, 2, 64, 1, 777, 776, U32, O.F16, "f32"),         # D 64, one query row
    (2, 2, 128, 1, 1000, 999, U32, O.BF16, "f32"),      # one query (decode through attention())
    (2, 1, 128, 40, 5, 0, U32, O.F16, "f32"),           # fewer keys than queries: later rows see n_k keys
]


@pytest.mark.parametrize("case", SWEEP, ids=lambda c: "h{}kv{}d{}q{}k{}p{}b{}".format(*c[:6], "c" if c[6] == U32
                                                                                      else c[6]))
def test_sweep(case):
    heads, kv, dim, n_q, n_k, q_pos0, block, dt, out = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))  # the same inputs in every process
    q_pad, k_pad = (n_q + 63) // 64 * 64, max(128, (n_k + 127) // 128 * 128)  # a buffer even for n_k = 0
    qb = G.randn_bits(rng, (heads, q_pad, dim), dt)
    kb = G.randn_bits(rng, (kv, k_pad, dim), dt)
    vb = G.randn_bits(rng, (kv, k_pad, dim), dt)
    # garbage past n_k: the kernel must mask, not rely on zero padding
    kb[:, n_k:] = G.bits(np.full((kv, k_pad - n_k, dim), 3e4, np.float32), dt)
    vb[:, n_k:] = G.bits(np.full((kv, k_pad - n_k, dim), np.nan, np.float32), dt)
    args = dict(n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=q_pos0, block=block,
                dim=dim)
    print(f"sweep {case}", flush=True)
    o, lse = run_fwd(qb, kb, vb, dt, O.F32 if out == "f32" else dt, o_rows=q_pad, fill=12288.0, **args)
    want_o, want_l = O.attn_dense(qb, kb, vb, dtype=dt, **args)
    G.assert_attn_close(o[:n_q], want_o, "output")
    G.assert_lse_close(lse, want_l, "lse")
    assert np.all(o[n_q:] == 12288.0), "rows past n_q were written"


@pytest.mark.parametrize("case", [c for c in SWEEP if not (c[2] == 128 and c[3] * (c[0] // c[1]) <= 64)],
                         ids=lambda c: "h{}kv{}d{}q{}k{}p{}b{}".format(*c[:6], "c" if c[6] == U32 else c[6]))
def test_sweep_fallback_kernels(case, monkeypatch):
    """The sweep through flash_fwd / flash_fwd_wide, which calls past the r64 / d256 kernels' 32-bit offsets take
    (MAKO_ATTN_FALLBACK=1 sends every call there; the split-K route of a few rows is not affected)."""
    monkeypatch.setenv("MAKO_ATTN_FALLBACK", "1")
    test_sweep(case)


def test_wide_output_rows_take_the_fallback_kernel():
    """o rows of 3.5M f32 (14 MB a row: 320 rows of o at this grid pass 2^32 bytes) leave flash_fwd_r64's 32-bit
    offsets, so the call takes flash_fwd by itself; sampled rows against the oracle, the columns past the heads
    untouched."""
    heads, kv, dim, S = 2, 2, 128, 100
    width = 3_500_000
    rng = np.random.default_rng(77)
    qb = G.randn_bits(rng, (heads, 128, dim), O.BF16)
    kb = G.randn_bits(rng, (kv, 128, dim), O.BF16)
    vb = G.randn_bits(rng, (kv, 128, dim), O.BF16)
    q, k, v = G.to_dev(qb, O.BF16), G.to_dev(kb, O.BF16), G.to_dev(vb, O.BF16)
    o = torch.full((S, width), 7.0, dtype=torch.float32, device="cuda")
    print("wide o rows (flash_fwd)", flush=True)
    M.attn_fwd(q, k, v, o, n_q=S, q_pad=128, n_k=S, k_pad=128, heads=heads, kv_heads=kv, q_pos0=0, block=U32,
               dim=dim, width=width)
    torch.cuda.synchronize()
    got = o[:, :heads * dim].cpu().numpy().astype(np.float64)
    assert bool((o[:, heads * dim:heads * dim + 1024] == 7.0).all())
    del o
    want, _ = O.attn_dense(qb, kb, vb, n_q=S, q_pad=128, n_k=S, k_pad=128, heads=heads, kv_heads=kv, q_pos0=0,
                           block=U32, dim=dim, dtype=O.BF16)
    G.assert_attn_close(got, want, "wide rows")


def every_tile(rng, heads, S):
    """One random row of every (head, 64-row query tile): each workgroup item of the launch is compared."""
    h, t = np.meshgrid(np.arange(heads), np.arange(S // 64), indexing="ij")
    return np.stack([h.ravel(), t.ravel() * 64 + rng.integers(0, 64, h.size)], 1).astype(np.uint32)


def _sampled(heads, kv, dim, S, block, dt, n_rows, seed):
    rng = np.random.default_rng(seed)
    qb, kb, vb = (G.randn_bits(rng, (h, S, dim), dt) for h in (heads, kv, kv))
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=heads, kv_heads=kv, q_pos0=0, block=block, dim=dim)
    o, lse = run_fwd(qb, kb, vb, dt, dt, **args)
    rows = np.concatenate([[0, 1, 31, 32, 63, 64, S - 1], rng.integers(0, S, n_rows)])
    hr = np.stack([rng.integers(0, heads, len(rows)), rows], 1).astype(np.uint32)
    hr = np.concatenate([hr, every_tile(rng, heads, S)])
    want_o, want_l = O.attn_dense_rows(qb, kb, vb, hr, dtype=dt, **args)
    got_o = np.stack([o[r, h * dim:(h + 1) * dim] for h, r in hr])
    got_l = np.array([lse[h, r] for h, r in hr])
    G.assert_attn_close(got_o, want_o, "sampled output")
    G.assert_rows_l2(got_o, want_o, "sampled output", dim)
    G.assert_lse_close(got_l, want_l, "sampled lse")
    return o


def test_qwen3_8b_causal_s4096_bf16_sampled():
    """32 query heads over 8 kv heads, D 128, S 4096, causal, bf16 in and out: one row of every (head, query tile)
    and sampled rows against the oracle."""
    print("causal S4096 bf16", flush=True)
    _sampled(32, 8, 128, 4096, U32, O.BF16, 300, 4096)


def test_bidirectional_s16384_bf16_sampled():
    """24 heads MHA, D 128, S 16384, bidirectional, bf16 in and out: one row of every (head, query tile) and
    sampled rows against the oracle."""
    print("bidirectional S16384 bf16", flush=True)
    _sampled(24, 24, 128, 16384, 0, O.BF16, 60, 16384)


def test_h3_vae_d64_bidirectional_s4096_bf16_sampled():
    """16 heads MHA, D 64, S 4096, bidirectional, bf16 in and out (the H3 VAE's attention shape, flash_fwd_r64 at
    heads of 64): one row of every (head, query tile) and sampled rows against the oracle."""
    print("bidirectional D64 S4096 bf16", flush=True)
    _sampled(16, 16, 64, 4096, 0, O.BF16, 200, 64)


def test_qwen35_d256_causal_s4096_bf16_sampled():
    """16 query heads over 2 kv heads, D 256, S 4096, causal, bf16 in and out (Qwen3.5 gated attention,
    flash_fwd_r32): one row of every (head, query tile) and sampled rows against the oracle."""
    print("causal D256 S4096 bf16", flush=True)
    _sampled(16, 2, 256, 4096, U32, O.BF16, 120, 256)


def test_d256_bidirectional_mha_s2048_f16_sampled():
    """Heads of 256 with one query head a kv head (a workgroup's waves hold rows 32 apart), bidirectional, f16 in
    and out, S 2048 (flash_fwd_r32): one row of every (head, query tile) and sampled rows against the oracle."""
    print("bidirectional D256 MHA S2048 f16", flush=True)
    _sampled(8, 8, 256, 2048, 0, O.F16, 80, 2562)


def test_d256_prefix_causal_gqa2_s3000_bf16_sampled():
    """Heads of 256, two query heads a kv head, prefix-causal (block 1000), ragged S 3000, bf16 (flash_fwd_r32):
    one row of every (head, query tile) and sampled rows against the oracle."""
    print("prefix-causal D256 GQA2 S3000 bf16", flush=True)
    _sampled(8, 4, 256, 3000, 1000, O.BF16, 80, 2563)


def test_deterministic_and_row_independent():
    """The same call twice gives identical bits; a row computed in a short call equals the same row in a long one
    (the reference's row-invariance style, tests/gemv_rows_test.cpp:1-2)."""
    rng = np.random.default_rng(7)
    heads, kv, dim, S = 8, 2, 128, 640
    qb, kb, vb = (G.randn_bits(rng, (h, S, dim), O.BF16) for h in (heads, kv, kv))
    args = dict(q_pad=S, k_pad=S, heads=heads, kv_heads=kv, q_pos0=0, block=0, dim=dim)
    o1, l1 = run_fwd(qb, kb, vb, O.BF16, O.F32, n_q=S, n_k=S, **args)
    o2, l2 = run_fwd(qb, kb, vb, O.BF16, O.F32, n_q=S, n_k=S, **args)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    o3, _ = run_fwd(qb, kb, vb, O.BF16, O.F32, n_q=33, n_k=S, **args)
    assert np.array_equal(o3, o1[:33])


@pytest.mark.parametrize("dim", [128, 64, 256])
def test_bf16_v_outside_the_f16_range(dim):
    """bf16 V is used as it is (P V runs in bf16 for bf16 inputs): head-dimension columns of V scaled from 1e-7 to
    1e5, beyond f16's range at both ends, come out with each column's relative L2 error (over all rows) within the
    reference's 5e-3, and every element within the tolerance at the column's scale."""
    rng = np.random.default_rng(100 + dim)
    heads, kv, S = 4, 2, 300
    scale = (10.0 ** np.linspace(-7, 5, dim)).astype(np.float32)
    qb = G.randn_bits(rng, (heads, S, dim), O.BF16)
    kb = G.randn_bits(rng, (kv, S, dim), O.BF16)
    vb = G.bits(rng.standard_normal((kv, S, dim)).astype(np.float32) * scale, O.BF16)
    args = dict(n_q=S, q_pad=(S + 63) // 64 * 64, n_k=S, k_pad=(S + 127) // 128 * 128, heads=heads, kv_heads=kv,
                q_pos0=0, block=U32, dim=dim)
    pad = lambda b, r: np.concatenate([b, np.zeros((b.shape[0], r - S, dim), b.dtype)], 1)
    qb, kb, vb = pad(qb, args["q_pad"]), pad(kb, args["k_pad"]), pad(vb, args["k_pad"])
    print(f"bf16 V over 1e-7 .. 1e5, D {dim}", flush=True)
    o, _ = run_fwd(qb, kb, vb, O.BF16, O.F32, **args)
    want, _ = O.attn_dense(qb, kb, vb, dtype=O.BF16, **args)
    got, want = o.reshape(S, heads, dim), want.reshape(S, heads, dim)
    rel = np.sqrt(((got - want) ** 2).sum((0, 1)) / (want ** 2).sum((0, 1)))
    assert rel.max() < G.ROW_L2, f"worst column relative L2 {rel.max():.2e} at scale {scale[rel.argmax()]:.1e}"
    G.assert_attn_close(got / scale, want / scale, "output at the column's scale")


def test_bf16_probabilities_on_peaked_rows():
    """P is rounded to the input type for P V: bf16 for bf16 inputs (8 significant bits, relative error <= 2^-8 a
    probability), f16 for f16 inputs (the reference's half P). Scores of deviation 4 put each row's softmax on a few
    keys, where those roundings do not average out: bf16 rows stay within the bound the rounding gives,
    2^-8 sum_j w_j |v_j| (w the softmax weights) plus 2e-4 for the rest of the arithmetic; the same values as f16
    inputs meet the element tolerance."""
    rng = np.random.default_rng(44)
    heads, kv, dim, S = 4, 2, 128, 256
    qf = rng.standard_normal((heads, S, dim)).astype(np.float32) * 2
    kf = rng.standard_normal((kv, S, dim)).astype(np.float32) * 2
    vf = rng.standard_normal((kv, S, dim)).astype(np.float32)
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=heads, kv_heads=kv, q_pos0=0, block=0, dim=dim)
    print("peaked rows, bf16 and f16", flush=True)
    qb, kb, vb = (G.bits(x, O.BF16) for x in (qf, kf, vf))
    o, _ = run_fwd(qb, kb, vb, O.BF16, O.F32, **args)
    want, _ = O.attn_dense(qb, kb, vb, dtype=O.BF16, **args)
    # the bound: w from the exact scores of the bf16 values
    q64 = O.bits_to_f32(qb, O.BF16).astype(np.float64)
    k64 = O.bits_to_f32(kb, O.BF16).astype(np.float64)
    v64 = O.bits_to_f32(vb, O.BF16).astype(np.float64)
    bound = np.empty((S, heads, dim))
    for h in range(heads):
        s = q64[h] @ k64[h // 2].T / np.sqrt(dim)
        w = np.exp(s - s.max(1, keepdims=True))
        w /= w.sum(1, keepdims=True)
        bound[:, h] = w @ np.abs(v64[h // 2])
    err = np.abs(o.reshape(S, heads, dim) - want.reshape(S, heads, dim))
    assert np.all(err <= 2.0 ** -8 * bound + 2e-4), f"max err over the bound {(err - 2.0 ** -8 * bound).max():.2e}"
    qh, kh, vh = (G.bits(x, O.F16) for x in (qf, kf, vf))
    o16, _ = run_fwd(qh, kh, vh, O.F16, O.F32, **args)
    want16, _ = O.attn_dense(qh, kh, vh, dtype=O.F16, **args)
    G.assert_attn_close(o16, want16, "f16 output")
