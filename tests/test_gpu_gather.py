"""The split-K and gathered latent-cache helpers (mako_attn_pv, mako_attn_gather_scores, mako_attn_gather_pv,
mako_idx_dots) on the GPU against the CPU oracle: ragged key counts and list counts (0, 1, part of a tile, the whole
list), head counts that fill part of a tile and, for attn_pv, more than one tile of heads, several splits, lists that
are not a multiple of the tile, and the shapes of a DeepSeek-style sparse latent decode (64 query heads, 512-wide
latent rows, lists of 2048 entries, the 128-dim float indexer over pooled keys).

Tolerance: f16 inputs give exact products in f32, so the only error is the f32 summation of n terms; every element
must be within 2 n 2^-24 sum|terms| of the oracle's double-precision sum (sum|terms| from the oracle on |p| and |kv|);
idx_dots multiplies f32 by f32, so 2 (n + 1) 2^-24 sum|terms|. Elements the call must not write keep a sentinel.
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


def dev(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x, dt)).to("cuda")


def dev_f16(bits):
    return G.to_dev(bits, O.F16)


def assert_sum_close(got, want, bound, what):
    got, want, bound = (np.asarray(x, np.float64) for x in (got, want, bound))
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    err = np.abs(got - want)
    bad = err > bound + 1e-30
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements beyond the f32 summation bound, "
                           f"worst {err.max():.3e} at {np.unravel_index(np.argmax(err - bound), err.shape)}")


PV = [
    # heads, dim, n_kv, keys_per_split
    (64, 512, 4096, 512),   # a 4096-key latent cache in 8 splits
    (16, 512, 1000, 256),   # ragged last split
    (128, 128, 777, 128),   # two tiles of heads (grid y = 2)
    (5, 64, 1, 64),         # one key, a part tile of heads
    (100, 192, 3 * 64 + 1, 64),
]


@pytest.mark.parametrize("case", PV, ids=lambda c: "h{}d{}n{}k{}".format(*c))
def test_attn_pv(case):
    heads, dim, n_kv, kps = case
    rng = np.random.default_rng(heads * 31 + n_kv)
    p = rng.uniform(0.0, 1.0, (heads, n_kv)).astype(np.float32) ** 4
    p[:, rng.random(n_kv) < 0.05] = 0.0
    kv = O.to_f16_bits(rng.standard_normal((n_kv, dim)))
    splits = -(-n_kv // kps)
    out = torch.full((splits, heads, dim), SENTINEL, dtype=torch.float32, device="cuda")
    print(f"attn_pv {case}", flush=True)
    M.attn_pv(dev(p, np.float32), dev_f16(kv), out, heads=heads, dim=dim, n_kv=n_kv, keys_per_split=kps)
    torch.cuda.synchronize()
    want = O.attn_pv(p, kv, heads=heads, dim=dim, n_kv=n_kv, keys_per_split=kps)
    mag = O.attn_pv(np.abs(p), O.to_f16_bits(np.abs(O.bits_to_f32(kv, O.F16))), heads=heads, dim=dim, n_kv=n_kv,
                    keys_per_split=kps)
    assert_sum_close(out.cpu().numpy(), want, 2 * kps * U * mag, "attn_pv")


def gathered_inputs(rng, tokens, heads, dim, stride, rows, counts):
    q = O.to_f16_bits(rng.standard_normal((tokens, heads, dim)) * 0.2)
    kv = O.to_f16_bits(rng.standard_normal((rows, dim)) * 0.2)
    lst = np.stack([rng.choice(rows, stride, replace=stride > rows) for _ in range(tokens)]).astype(np.int32)
    cnt = np.asarray(counts, np.int32)
    return q, kv, lst, cnt


GATHER = [
    # tokens, heads, dim, stride, rows, counts
    (4, 64, 512, 2048, 20000, [2048, 0, 1, 1500]),  # lists of 2048 over a 20000-row latent cache
    (2, 16, 256, 100, 300, [100, 37]),              # lists that are not a multiple of 64
    (3, 7, 768, 64, 64, [64, 63, 5]),
    (2, 64, 512, 192, 5000, [500, 191]),           # a count past the list's length reads only the list
]


@pytest.mark.parametrize("case", GATHER, ids=lambda c: "t{}h{}d{}s{}".format(*c[:4]))
def test_attn_gather_scores(case):
    tokens, heads, dim, stride, rows, counts = case
    rng = np.random.default_rng(stride + heads)
    q, kv, lst, cnt = gathered_inputs(rng, tokens, heads, dim, stride, rows, counts)
    out = torch.full((tokens, heads, stride), SENTINEL, dtype=torch.float32, device="cuda")
    print(f"attn_gather_scores {case[:5]}", flush=True)
    M.attn_gather_scores(dev_f16(q), dev_f16(kv), dev(lst, np.int32), dev(cnt, np.int32), out, heads=heads,
                         dim=dim, stride=stride, tokens=tokens)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = O.gather_scores(q, kv, lst, cnt, heads=heads, dim=dim, stride=stride, tokens=tokens)
    absb = lambda b: O.to_f16_bits(np.abs(O.bits_to_f32(b, O.F16)))
    mag = O.gather_scores(absb(q), absb(kv), lst, cnt, heads=heads, dim=dim, stride=stride, tokens=tokens)
    assert_sum_close(got, want, 2 * dim * U * mag, "attn_gather_scores")
    for t in range(tokens):
        assert (got[t, :, cnt[t]:] == 0).all(), "entries past count[t] must be 0"


@pytest.mark.parametrize("splits", [1, 3, 4])
@pytest.mark.parametrize("case", GATHER, ids=lambda c: "t{}h{}d{}s{}".format(*c[:4]))
def test_attn_gather_pv(case, splits):
    tokens, heads, dim, stride, rows, counts = case
    rng = np.random.default_rng(stride * 3 + splits)
    _, kv, lst, cnt = gathered_inputs(rng, tokens, heads, dim, stride, rows, counts)
    p = rng.uniform(0.0, 1.0, (tokens, heads, stride)).astype(np.float32) ** 4
    out = torch.full((splits, tokens, heads, dim), SENTINEL, dtype=torch.float32, device="cuda")
    print(f"attn_gather_pv {case[:5]} splits={splits}", flush=True)
    M.attn_gather_pv(dev(p, np.float32), dev_f16(kv), dev(lst, np.int32), dev(cnt, np.int32), out, heads=heads,
                     dim=dim, stride=stride, splits=splits, tokens=tokens)
    torch.cuda.synchronize()
    want = O.gather_pv(p, kv, lst, cnt, heads=heads, dim=dim, stride=stride, splits=splits, tokens=tokens)
    mag = O.gather_pv(p, O.to_f16_bits(np.abs(O.bits_to_f32(kv, O.F16))), lst, cnt, heads=heads, dim=dim,
                      stride=stride, splits=splits, tokens=tokens)
    per = -(-stride // (splits * 64)) * 64
    assert_sum_close(out.cpu().numpy(), want, 2 * per * U * mag, "attn_gather_pv")


IDX = [
    # tokens, heads, dim, pools, stride
    (4, 32, 128, 1000, 1024),  # the indexer: 32 heads of 128 over 1000 pooled keys
    (2, 7, 36, 300, 301),      # width a multiple of 4 but not of the 32-float chunk, a part pool tile
    (2, 32, 64, 129, 129),
    (3, 5, 33, 70, 80),        # odd width (one float a lane a step), part tiles of heads and pools
    (1, 1, 1, 1, 1),
    (3, 32, 128, 700, 700),    # an odd token count on the 16-byte path (token pairs: the last one alone)
    (1, 20, 128, 256, 260),
]


@pytest.mark.parametrize("case", IDX, ids=lambda c: "t{}h{}d{}p{}".format(*c[:4]))
def test_idx_dots(case):
    tokens, heads, dim, pools, stride = case
    rng = np.random.default_rng(pools + dim)
    q = rng.standard_normal((tokens, heads, dim)).astype(np.float32)
    pooled = rng.standard_normal((pools, dim)).astype(np.float32)
    # one more token's rows than the call covers: they must stay untouched
    out = torch.full((tokens + 1, heads, stride), SENTINEL, dtype=torch.float32, device="cuda")
    print(f"idx_dots {case}", flush=True)
    M.idx_dots(dev(q, np.float32), dev(pooled, np.float32), out, tokens=tokens, heads=heads, dim=dim, pools=pools,
               stride=stride)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert (got[tokens] == SENTINEL).all(), "idx_dots wrote past the last token"
    got = got[:tokens]
    want = O.idx_dots(q, pooled, heads=heads, dim=dim, pools=pools, stride=stride, tokens=tokens,
                      dots=np.full((tokens, heads, stride), SENTINEL))
    mag = O.idx_dots(np.abs(q), np.abs(pooled), heads=heads, dim=dim, pools=pools, stride=stride, tokens=tokens)
    assert_sum_close(got, want, 2 * (dim + 1) * U * mag, "idx_dots")


def test_gathered_decode_matches_dense_attention():
    """The three kernels composed as their caller composes them (scores, a softmax on the host side, split P V,
    the splits summed and normalised) give the attention of each query over its gathered rows, which is the dense
    oracle's attention over those rows laid out as a key / value cache (one kv head, keys = values = the rows)."""
    rng = np.random.default_rng(99)
    tokens, heads, dim, stride, rows = 2, 16, 256, 256, 4000
    q, kv, lst, cnt = gathered_inputs(rng, tokens, heads, dim, stride, rows, [256, 131])
    scale = 1.0 / np.sqrt(dim)
    s = torch.zeros((tokens, heads, stride), dtype=torch.float32, device="cuda")
    qd, kvd, ld, cd = dev_f16(q), dev_f16(kv), dev(lst, np.int32), dev(cnt, np.int32)
    M.attn_gather_scores(qd, kvd, ld, cd, s, heads=heads, dim=dim, stride=stride, tokens=tokens)
    mask = torch.arange(stride, device="cuda")[None, None, :] < cd.long()[:, None, None]
    p = torch.softmax((s * scale).masked_fill(~mask, float("-inf")), -1)
    part = torch.zeros((2, tokens, heads, dim), dtype=torch.float32, device="cuda")
    M.attn_gather_pv(p.contiguous(), kvd, ld, cd, part, heads=heads, dim=dim, stride=stride, splits=2,
                     tokens=tokens)
    got = part.sum(0).cpu().numpy()
    torch.cuda.synchronize()
    for t in range(tokens):
        n = int(cnt[t])
        keys = kv[lst[t, :n]]
        want = O.attn_dense(q[t][:, None, :], keys[None], keys[None], n_q=1, q_pad=1, n_k=n, k_pad=n, heads=heads,
                            kv_heads=1, q_pos0=0, block=0, dim=dim, dtype=O.F16, scale=scale)[0]
        G.assert_attn_close(got[t], want.reshape(heads, dim), f"gathered decode token {t}")
