"""The output projection after attention (mako_proj_bf16: Runtime::proj with BF16 weights) on the GPU against the
CPU oracle: bf16 activations as the attention writes them, f32 activations rounded in the GEMM's loads, the bf16
split, tiles cut by t and n, strided x and y rows, and the Qwen3-8B o_proj shape (4096 tokens, 4096 -> 4096); and
the handoff itself: mako_attn_fwd writing bf16 rows [n_q][heads * D] that mako_proj_bf16 reads with no conversion.

Tolerance: bf16 times bf16 is exact in f32, so the only error is the f32 summation over k; every element must be
within 2 k 2^-24 sum|terms| of the oracle's double-precision sum (sum|terms| from the oracle on |x| and |w|; twice
that with the split's second product). Columns past n keep a sentinel.
"""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402

U = 2.0 ** -24
SENTINEL = 1234.5


def abs_bits(b):
    return np.asarray(b, np.uint16) & np.uint16(0x7FFF)


def run_proj(rng, t, k, n, x_dtype, split, ldx=0, ldy=0, scale=1.0):
    ldx_, ldy_ = ldx or k, ldy or n
    w = O.to_bf16_bits(rng.standard_normal((n, k)) * 0.05)
    xf = (rng.standard_normal((t, ldx_)) * scale).astype(np.float32)
    x = xf if x_dtype == O.F32 else O.to_bf16_bits(xf)
    wd = G.to_dev(w, O.BF16)
    xd = torch.from_numpy(x).to("cuda") if x_dtype == O.F32 else G.to_dev(x, O.BF16)
    y = torch.full((t, ldy_), SENTINEL, dtype=torch.float32, device="cuda")
    print(f"proj t={t} k={k} n={n} x={'f32' if x_dtype == O.F32 else 'bf16'} split={split} ldx={ldx} ldy={ldy}",
          flush=True)
    M.proj_bf16(wd, xd, y, t=t, k=k, n=n, ldx=ldx, ldy=ldy, split=split)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = O.proj_bf16(x, w, t=t, k=k, n=n, ldx=ldx, ldy=ldy, x_dtype=x_dtype, split=split,
                       y=np.full((t, ldy_), SENTINEL))
    xa = np.abs(x) if x_dtype == O.F32 else abs_bits(x)
    mag = O.proj_bf16(xa, abs_bits(w), t=t, k=k, n=n, ldx=ldx, ldy=ldy, x_dtype=x_dtype, split=split)
    return got, want, mag


def assert_sum_close(got, want, bound, what):
    err = np.abs(np.asarray(got, np.float64) - want)
    bad = err > bound + 1e-30
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements beyond the f32 summation bound, worst "
                           f"{err.max():.3e} at {np.unravel_index(np.argmax(err - bound), err.shape)}")


CASES = [
    # t, k, n, x dtype, split, ldx, ldy
    (300, 256, 320, O.BF16, 0, 0, 0),       # part tiles in both dimensions
    (256, 4096, 256, O.F32, 0, 0, 0),       # a long k
    (77, 128, 96, O.F32, 1, 0, 0),          # the split, one part tile
    (513, 1024, 1000, O.BF16, 0, 1032, 1010),  # strided x and y rows
    (1, 64, 1, O.F32, 0, 0, 0),
    (600, 512, 700, O.F32, 1, 520, 0),      # the split over several 128-row tiles
    (1100, 192, 2048, O.F32, 0, 0, 0),      # more tiles than the 8 XCDs take evenly
    # bf16 activations with 2, 4 and 6 chunks of 32 (each of the prologue's and the tail's DMA waits), part tiles
    (200, 64, 130, O.BF16, 0, 0, 0),
    (129, 128, 200, O.BF16, 0, 136, 0),
    (70, 192, 257, O.BF16, 0, 0, 260),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "t{}k{}n{}{}{}".format(
    *c[:3], "f32" if c[3] == O.F32 else "bf16", "s" if c[4] else ""))
def test_proj(case):
    t, k, n, xd, split, ldx, ldy = case
    rng = np.random.default_rng(t + k + n)
    got, want, mag = run_proj(rng, t, k, n, xd, split, ldx, ldy, scale=3.0)
    nn = n
    assert_sum_close(got[:, :nn], want[:, :nn], (4 if split else 2) * k * U * mag[:, :nn], "proj")
    assert (got[:, nn:] == SENTINEL).all(), "a column past n was written"


def test_qwen3_8b_o_proj():
    """Qwen3-8B's o_proj after a 4096-token prefill (src/models/qwen_text.cpp:312): 4096 x 4096 bf16 weights over
    bf16 attention rows; 64 sampled rows against the oracle."""
    rng = np.random.default_rng(8)
    t = k = n = 4096
    w = O.to_bf16_bits(rng.standard_normal((n, k)) * 0.02)
    x = O.to_bf16_bits(rng.standard_normal((t, k)))
    y = torch.empty((t, n), dtype=torch.float32, device="cuda")
    print("qwen3-8b o_proj", flush=True)
    M.proj_bf16(G.to_dev(w, O.BF16), G.to_dev(x, O.BF16), y, t=t, k=k, n=n)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(t, 64, replace=False))
    got = y.cpu().numpy()[rows]
    want = O.proj_bf16(x[rows], w, t=64, k=k, n=n, x_dtype=O.BF16)
    mag = O.proj_bf16(abs_bits(x[rows]), abs_bits(w), t=64, k=k, n=n, x_dtype=O.BF16)
    assert_sum_close(got, want, 2 * k * U * mag, "o_proj")


def test_attention_rows_feed_the_projection():
    """mako_attn_fwd with a bf16 output writes [n_q][heads * D] rows; mako_proj_bf16 reads them as x directly. The
    result equals the oracle's projection of exactly those bf16 rows (the attention itself is checked elsewhere)."""
    rng = np.random.default_rng(12)
    S, H, KV, D = 320, 8, 2, 128
    q = G.randn_bits(rng, (H, S, D), O.BF16)
    kk = G.randn_bits(rng, (KV, S, D), O.BF16)
    v = G.randn_bits(rng, (KV, S, D), O.BF16)
    o = torch.empty((S, H * D), dtype=torch.bfloat16, device="cuda")
    M.attn_fwd(G.to_dev(q, O.BF16), G.to_dev(kk, O.BF16), G.to_dev(v, O.BF16), o, n_q=S, q_pad=S, n_k=S, k_pad=S,
               heads=H, kv_heads=KV, q_pos0=0, block=M.U32_MAX, dim=D)
    n = 512
    w = O.to_bf16_bits(rng.standard_normal((n, H * D)) * 0.05)
    y = torch.empty((S, n), dtype=torch.float32, device="cuda")
    M.proj_bf16(G.to_dev(w, O.BF16), o, y, t=S, k=H * D, n=n)
    torch.cuda.synchronize()
    xb = o.view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.proj_bf16(xb, w, t=S, k=H * D, n=n, x_dtype=O.BF16)
    mag = O.proj_bf16(abs_bits(xb), abs_bits(w), t=S, k=H * D, n=n, x_dtype=O.BF16)
    assert_sum_close(y.cpu().numpy(), want, 2 * H * D * U * mag, "attention -> proj")
