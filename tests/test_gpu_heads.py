"""Head tiles (mako_heads) on the GPU against the CPU oracle: the reference's three producers (heads with and
without rotation and the padding cleared, heads_norm at a row offset, heads_partial with a head stride, partial
rotation, the optional norm and the row map), head widths 32 to 256, f16 and bf16 tiles, and the Qwen3-8B-shape
q / k / v tiles of a 4096-token prefill.

Tolerance: the plain slice is bit-exact (both round x to nearest even); with a norm or a rotation, each value within
one unit in the last place of the tile's type (2^-10 |ref| for f16, 2^-7 for bf16) of the oracle's double-precision
result rounded the same way, plus 2^-24 absolute for f16's subnormals. Rows the call does not own keep a sentinel.
"""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import gpu_util as G  # noqa: E402
import mako_attn as M  # noqa: E402

SENTINEL = 0x7777


def run(x, *, out, cs=None, w=None, map_=None, **a):
    heads, n_pad, dim = a["heads"], a["n_pad"], a["dim"]
    y = torch.from_numpy(np.full((heads, n_pad, dim), SENTINEL, np.uint16).view(np.int16)).to("cuda")
    y = y.view(G.TORCH[out])
    dev = lambda t, dt: None if t is None else torch.from_numpy(np.ascontiguousarray(t, dt)).to("cuda")
    M.heads(dev(x, np.float32), y, cs=dev(cs, np.float32), w=dev(w, np.float32), map_=dev(map_, np.int32), **a)
    torch.cuda.synchronize()
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.heads(x, cs, w, map_, out=out, y=np.full((heads, n_pad, dim), SENTINEL, np.uint16), **a)
    return got, want


def assert_tiles_close(got, want, out, exact=False):
    assert got.shape == want.shape
    untouched = want == SENTINEL
    assert np.array_equal(got[untouched], want[untouched]), "a row outside the call's rows was written"
    if exact:
        assert np.array_equal(got, want), f"{int(np.sum(got != want))} values differ from the oracle's rounding"
        return
    g, wv = O.bits_to_f32(got, out).astype(np.float64), O.bits_to_f32(want, out).astype(np.float64)
    ulp = 2.0 ** -10 if out == O.F16 else 2.0 ** -7
    err = np.abs(g - wv)
    bad = err > ulp * np.abs(wv) + 2.0 ** -24
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} values beyond one ulp, worst {err.max():.3e} at "
                           f"{np.unravel_index(np.argmax(err - ulp * np.abs(wv)), err.shape)}")


def angles(rng, rows, pairs):
    a = rng.uniform(-np.pi, np.pi, (rows, pairs))
    return np.stack([np.cos(a), np.sin(a)], -1).astype(np.float32)


@pytest.mark.parametrize("out", [O.F16, O.BF16], ids=["f16", "bf16"])
def test_plain_slice_exact_and_padding_cleared(out):
    rng = np.random.default_rng(5)
    T, H, D = 77, 8, 128
    x = rng.standard_normal((T, 3 * H * D)).astype(np.float32) * 4
    a = dict(rows=T, ld=3 * H * D, col0=H * D, stride=D, dim=D, heads=H, n_pad=128, clear=1)
    print(f"plain slice out={out}", flush=True)
    got, want = run(x, out=out, **a)
    assert_tiles_close(got, want, out, exact=True)
    assert (got[:, T:] == 0).all()


@pytest.mark.parametrize("rope", [1, 2])
def test_heads_rotated(rope):
    """TransformerRuntime::heads with rotation (qwen_text.cpp:308-309): full rotation over dim 128."""
    rng = np.random.default_rng(10 + rope)
    T, H, D = 200, 4, 128
    x = rng.standard_normal((T, H * D + 64)).astype(np.float32)
    a = dict(rows=T, ld=H * D + 64, col0=64, stride=D, dim=D, heads=H, n_pad=256, rope=rope, rot=D, clear=1)
    print(f"heads rope={rope}", flush=True)
    got, want = run(x, out=O.F16, cs=angles(rng, T, D // 2), **a)
    assert_tiles_close(got, want, O.F16)


def test_heads_norm_row_offset():
    """heads_norm: RMS norm times w, then the rotation, written from row0 on; rows past T left alone."""
    rng = np.random.default_rng(21)
    T, H, D = 90, 8, 128
    x = rng.standard_normal((T, H * D)).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    a = dict(rows=T, ld=H * D, col0=0, stride=D, dim=D, heads=H, n_pad=128, row0=17, rope=1, rot=D, eps=1e-6)
    print("heads_norm", flush=True)
    got, want = run(x, out=O.BF16, cs=angles(rng, T + 17, D // 2), w=w, **a)
    assert_tiles_close(got, want, O.BF16)


PARTIAL = [
    # dim, stride, rot, norm, mapped, out
    (128, 128, 96, True, True, O.F16),     # h3.cpp:348-351: 96 of 128 rotated, norm, the cube row map
    (128, 256, 128, True, False, O.BF16),  # qwen_text.cpp:415: q rows 2 D apart
    (128, 128, 0, False, True, O.F16),     # the value heads: no norm, no rotation
    (64, 192, 32, True, False, O.F16),     # h3_vae.cpp:210-211 shape: heads 3 D apart, partial rotation
    (256, 256, 64, True, False, O.BF16),   # the widest heads
    (32, 32, 32, False, False, O.F16),     # the narrowest
    (96, 96, 48, True, True, O.BF16),      # a width that is not a multiple of 64
]


@pytest.mark.parametrize("case", PARTIAL, ids=lambda c: "d{}s{}r{}{}{}".format(*c[:3], "n" if c[3] else "",
                                                                              "m" if c[4] else ""))
def test_heads_partial(case):
    dim, stride, rot, norm, mapped, out = case
    rng = np.random.default_rng(dim * 7 + rot)
    T, H = 150, 6
    ld = stride * H + 32
    x = rng.standard_normal((T, ld)).astype(np.float32) * 2
    w = rng.uniform(0.5, 1.5, dim).astype(np.float32) if norm else None
    mp = None
    if mapped:
        mp = rng.permutation(T).astype(np.int32)
        mp[rng.random(T) < 0.1] = -1
    a = dict(rows=T, ld=ld, col0=32, stride=stride, dim=dim, heads=H, n_pad=192, rope=1 if rot else 0, rot=rot,
             eps=1e-6 if norm else 0.0)
    print(f"heads_partial {case}", flush=True)
    got, want = run(x, out=out, cs=angles(rng, T, max(rot, 2) // 2), w=w, map_=mp, **a)
    assert_tiles_close(got, want, out)
    if mapped:
        assert (got[:, :T][:, mp < 0] == 0).all()


def test_qwen3_8b_prefill_tiles():
    """The q / k / v tiles of a 4096-token Qwen3-8B prefill (32 / 8 / 8 heads of 128, q and k RMS-normed and
    rotated over the full head, bf16 tiles): sampled rows against the oracle."""
    rng = np.random.default_rng(8)
    T, D = 4096, 128
    cs = angles(rng, T, D // 2)
    for name, H, norm, rope in (("q", 32, True, 1), ("k", 8, True, 1), ("v", 8, False, 0)):
        x = rng.standard_normal((T, H * D)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, D).astype(np.float32) if norm else None
        rows = np.sort(rng.choice(T, 64, replace=False))
        a = dict(rows=T, ld=H * D, col0=0, stride=D, dim=D, heads=H, n_pad=T, rope=rope, rot=D if rope else 0,
                 eps=1e-6 if norm else 0.0)
        print(f"qwen3-8b {name} tiles", flush=True)
        y = torch.empty((H, T, D), dtype=torch.bfloat16, device="cuda")
        dev = lambda t: None if t is None else torch.from_numpy(t).to("cuda")
        M.heads(dev(x), y, cs=dev(cs), w=dev(w), **a)
        torch.cuda.synchronize()
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)[:, rows]
        want = O.heads(x[rows], cs[rows], w, out=O.BF16, **dict(a, rows=len(rows), n_pad=len(rows)))
        assert_tiles_close(got, want, O.BF16)


@pytest.mark.parametrize("rope", [0, 1, 2])
def test_unaligned_rows_take_the_general_kernel(rope):
    """Rows whose head columns are not 16-byte aligned (col0 = 1) go through the general kernel: the same results."""
    rng = np.random.default_rng(40 + rope)
    T, H, D = 70, 4, 128
    x = rng.standard_normal((T, H * D + 3)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    a = dict(rows=T, ld=H * D + 3, col0=1, stride=D, dim=D, heads=H, n_pad=80, rope=rope, rot=D if rope else 0,
             eps=1e-6, clear=1)
    print(f"unaligned rope={rope}", flush=True)
    got, want = run(x, out=O.F16, cs=angles(rng, T, D // 2), w=w, **a)
    assert_tiles_close(got, want, O.F16)
