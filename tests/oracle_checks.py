"""Checks that pin the CPU oracle (oracle/attn_oracle.c) to facts it does not compute itself.

Each check returns (ok, message) for a given oracle build (mutant=None is the real oracle; a mutant carries one
planted mistake), so the same checks both pass on the oracle and are shown to fail on every mutant:
  goldens        - the fixtures of tests/golden/ (explicit mask matrices + scipy softmax / logsumexp)
  closed forms   - q = 0 gives the mean of the visible values and lse = log(count); one visible key gives its
                   value row and lse = its score; no visible key gives 0 and lse = -inf
  invariants     - GQA equals MHA with the kv heads repeated; block = 0 is bidirectional (invariant to permuting
                   keys and values together); causal row i does not depend on keys past i
  sparse         - all cubes selected equals dense over the valid keys; rows with map < 0 stay untouched
  cube_select    - the order numpy's stable argsort of (-score) gives; local cubes lead without duplicates
  decode, merge  - decode equals the dense rule at q_pos0 = ctx - 1; merging splits equals the whole row
  heads          - the plain slice is numpy's f16 / bf16 rounding of x; padding rows zeroed, others untouched;
                   angle 0 is the identity and angle pi / 2 maps (u, v) to (-v, u); a rotation is the complex
                   product (u + i v)(c + i s); rope 2 pairs adjacent values; values past rot pass through; with w = 1
                   the normed head has unit mean square and is invariant to scaling x; a mapped row is the
                   unmapped row of its source, a negative map gives a zero row
  gather         - attn_pv summed over its splits is numpy's product of the half-rounded p and kv; a one-hot p
                   puts one kv row in exactly the split that owns its key; p = 1 + 2^-12 acts as 1 (half rounding);
                   scores with the identity list are numpy's q kv^T, a permuted list permutes the columns, entries
                   from count[t] on are 0; gather_pv with the identity list equals attn_pv at per keys a split, and
                   a one-hot p lands in split s // per; idx_dots is numpy's float64 q pooled^T, columns past pools
                   untouched
  proj           - y is torch's bf16 rounding of x times w^T (float64); w = I gives bf16(x) exactly, and with split
                   bf16(x) + bf16(x - bf16(x)); split brings y within 2^-15 sum|terms| of x w^T; bf16 input is
                   used as is; strided x and y rows, columns past n untouched
  kda_scan       - from a zero state one token gives o = (k.q) beta v / sqrt(D); with beta = 0 the state only decays
                   (numpy's exp of the summed g times the initial state, and o from it); orthonormal keys with g = 0,
                   beta = 1 are recalled exactly (delta rule), a key written twice keeps the second value; full decay
                   (g = -60) forgets the state before the token's read; two calls carrying the state equal one; the
                   snapshot equals the state of a call that stops there; heads in strided rows run independently
"""
import glob
import os

import numpy as np
from scipy.special import logsumexp, softmax

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
U32 = 0xFFFFFFFF


def _rng(seed):
    return np.random.default_rng(seed)


def _f16(x):
    return O.to_f16_bits(x)


def _close(a, b, tol=1e-9):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    same_inf = np.isinf(a) & np.isinf(b) & (np.sign(a) == np.sign(b))
    with np.errstate(invalid="ignore"):
        err = np.where(same_inf, 0.0, np.abs(a - b))
    return bool(np.all(err <= tol * (1.0 + np.abs(np.where(same_inf, 0.0, b)))))


def check_goldens(mutant=None):
    bad = []
    for f in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        with np.load(f) as z:
            g = {k: z[k] for k in z.files}
        kind = str(g["kind"])
        if kind == "dense":
            n_q, q_pad, n_k, k_pad, heads, kv, q_pos0, block, width, dim, dt = [int(x) for x in g["args"]]
            o, lse = O.attn_dense(g["q"], g["k"], g["v"], n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads,
                                  kv_heads=kv, q_pos0=q_pos0, block=block, dim=dim, dtype=dt, mutant=mutant)
        elif kind == "sparse":
            n_q, q_pad, n_k, k_pad, heads, kv, width, cubes, kk, d0, d1, causal, sh, topk, dt = \
                [int(x) for x in g["args"]]
            o, lse = O.attn_sparse(g["q"], g["k"], g["v"], g["sel"], g["nsel"], g["valid"], g["map"], n_q=n_q,
                                   q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv, n_cubes=cubes,
                                   max_sel=kk, dense0=d0, dense1=d1, causal=causal, sel_heads=sh, dtype=dt,
                                   o_fill=np.full((q_pad, width), 12345.0), mutant=mutant)
            lse = np.where(np.isnan(g["lse"]), np.nan, lse)
        else:
            batch, heads, kv, dim, cap, dt = [int(x) for x in g["args"]]
            o, lse = O.attn_decode(g["q"], g["k"], g["v"], g["ctx"], batch=batch, heads=heads, kv_heads=kv,
                                   dim=dim, cap=cap, dtype=dt, mutant=mutant)
        ok_o = _close(o, g["o"], 2e-6)
        gl = np.nan_to_num(g["lse"], nan=0.0)
        ml = np.nan_to_num(lse, nan=0.0)
        ok_l = _close(ml, gl, 2e-6)
        if not (ok_o and ok_l):
            bad.append(os.path.basename(f))
    return not bad, f"golden mismatches: {bad}"


def check_closed_forms(mutant=None):
    msgs = []
    rng = _rng(1)
    heads, kv, dim, n = 2, 1, 64, 20
    q_pad, k_pad = 64, 128
    qz = np.zeros((heads, q_pad, dim), np.uint16)  # q = 0: every visible key weighs the same
    k = _f16(rng.standard_normal((kv, k_pad, dim)))
    v = _f16(rng.standard_normal((kv, k_pad, dim)))
    vf = O.bits_to_f32(v, O.F16).astype(np.float64)
    o, lse = O.attn_dense(qz, k, v, n_q=n, q_pad=q_pad, n_k=n, k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=0,
                          block=U32, dim=dim, dtype=O.F16, mutant=mutant)
    want = np.stack([vf[0, :r + 1].mean(0) for r in range(n)])
    if not (_close(o[:, :dim], want) and _close(o[:, dim:], want)):
        msgs.append("q=0 causal: not the mean of the visible values")
    if not _close(lse, np.log(np.arange(1, n + 1))[None, :].repeat(heads, 0)):
        msgs.append("q=0 causal: lse is not log(count)")
    # one visible key: row 0 of a causal pass sees key 0 alone
    q = _f16(rng.standard_normal((heads, q_pad, dim)))
    qf = O.bits_to_f32(q, O.F16).astype(np.float64)
    kf = O.bits_to_f32(k, O.F16).astype(np.float64)
    o, lse = O.attn_dense(q, k, v, n_q=n, q_pad=q_pad, n_k=n, k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=0,
                          block=U32, dim=dim, dtype=O.F16, mutant=mutant)
    scale = float(np.float32(1 / np.sqrt(dim)))
    if not _close(o[0, :dim], vf[0, 0]):
        msgs.append("one visible key: output is not its value row")
    if not _close(lse[:, 0], [qf[h, 0] @ kf[0, 0] * scale for h in range(heads)]):
        msgs.append("one visible key: lse is not its score")
    # no visible key: n_k = 0
    o, lse = O.attn_dense(q, k, v, n_q=4, q_pad=q_pad, n_k=0, k_pad=k_pad, heads=heads, kv_heads=kv, q_pos0=0,
                          block=U32, dim=dim, dtype=O.F16, mutant=mutant)
    if not (np.all(o == 0) and np.all(np.isneginf(lse))):
        msgs.append("no visible key: not 0 and -inf")
    return not msgs, "; ".join(msgs)


def check_invariants(mutant=None):
    msgs = []
    rng = _rng(2)
    heads, kv, dim, n = 4, 2, 128, 70
    q_pad, k_pad = 128, 128
    q = _f16(rng.standard_normal((heads, q_pad, dim)))
    k = _f16(rng.standard_normal((kv, k_pad, dim)))
    v = _f16(rng.standard_normal((kv, k_pad, dim)))
    common = dict(n_q=n, q_pad=q_pad, n_k=n, k_pad=k_pad, dim=dim, dtype=O.F16, mutant=mutant)
    # GQA equals MHA over the kv heads repeated (head h reads kv head h / (heads / kv_heads))
    o_g, l_g = O.attn_dense(q, k, v, heads=heads, kv_heads=kv, q_pos0=0, block=U32, **common)
    kr, vr = np.repeat(k, heads // kv, axis=0), np.repeat(v, heads // kv, axis=0)
    o_m, l_m = O.attn_dense(q, kr, vr, heads=heads, kv_heads=heads, q_pos0=0, block=U32, **common)
    if not (_close(o_g, o_m) and _close(l_g, l_m)):
        msgs.append("GQA differs from MHA with the kv heads repeated")
    # block = 0: bidirectional, so permuting keys and values together changes nothing; and it matches scipy
    o_b, l_b = O.attn_dense(q, k, v, heads=heads, kv_heads=kv, q_pos0=0, block=0, **common)
    perm = np.concatenate([rng.permutation(n), np.arange(n, k_pad)])
    o_p, l_p = O.attn_dense(q, k[:, perm], v[:, perm], heads=heads, kv_heads=kv, q_pos0=0, block=0, **common)
    if not (_close(o_b, o_p) and _close(l_b, l_p)):
        msgs.append("bidirectional output changes when keys and values are permuted together")
    qf, kf, vf = (O.bits_to_f32(x, O.F16).astype(np.float64) for x in (q, k, v))
    s = qf[0, :n] @ kf[0, :n].T * float(np.float32(1 / np.sqrt(dim)))
    if not (_close(o_b[:, :dim], softmax(s, axis=1) @ vf[0, :n]) and _close(l_b[0], logsumexp(s, axis=1))):
        msgs.append("bidirectional head 0 differs from scipy's softmax")
    # causal: row i does not depend on keys and values past i
    k2, v2 = k.copy(), v.copy()
    cut = 30
    k2[:, cut + 1:n] = _f16(rng.standard_normal((kv, n - cut - 1, dim)))
    v2[:, cut + 1:n] = _f16(rng.standard_normal((kv, n - cut - 1, dim)))
    o_c2, _ = O.attn_dense(q, k2, v2, heads=heads, kv_heads=kv, q_pos0=0, block=U32, **common)
    if not _close(o_g[:cut + 1], o_c2[:cut + 1]):
        msgs.append("causal rows depend on later keys")
    if _close(o_g[cut + 1:], o_c2[cut + 1:]):
        msgs.append("causal rows past the cut ignore their own keys")
    # prefix-causal: rows >= block see all keys, rows below it are causal
    blk = 25
    o_x, _ = O.attn_dense(q, k, v, heads=heads, kv_heads=kv, q_pos0=0, block=blk, **common)
    if not (_close(o_x[blk:], o_b[blk:]) and _close(o_x[:blk], o_g[:blk])):
        msgs.append("prefix-causal rows differ from bidirectional / causal rows")
    return not msgs, "; ".join(msgs)


def check_sparse(mutant=None):
    msgs = []
    rng = _rng(3)
    heads, kv, cubes, D = 2, 1, 3, 128
    n = cubes * 64
    q_pad = k_pad = 256
    q = _f16(rng.standard_normal((heads, q_pad, D)))
    k = _f16(rng.standard_normal((kv, k_pad, D)))
    v = _f16(rng.standard_normal((kv, k_pad, D)))
    valid = np.zeros(k_pad, np.uint8)
    valid[:n] = 1
    valid[40:44] = 0  # a few invalid keys
    sel = np.tile(np.arange(cubes, dtype=np.uint16), (heads, cubes, 1))
    nsel = np.full((heads, cubes), cubes, np.uint16)
    map_ = np.where(np.arange(q_pad) < n, np.arange(q_pad), -1).astype(np.int32)
    map_[7] = -1
    fill = np.full((q_pad, heads * D), 12345.0)
    o, _ = O.attn_sparse(q, k, v, sel, nsel, valid, map_, n_q=n, q_pad=q_pad, n_k=n, k_pad=k_pad, heads=heads,
                         kv_heads=kv, n_cubes=cubes, max_sel=cubes, dense0=n, dense1=n, dtype=O.F16, o_fill=fill,
                         mutant=mutant)
    # dense bidirectional over the valid keys: mask invalid keys by zeroing them out of an explicit softmax
    qf, kf, vf = (O.bits_to_f32(x, O.F16).astype(np.float64) for x in (q, k, v))
    keys = np.nonzero(valid[:n])[0]
    scale = float(np.float32(1 / np.sqrt(D)))
    for h in range(heads):
        s = qf[h, :n] @ kf[0, keys].T * scale
        want = softmax(s, axis=1) @ vf[0, keys]
        rows = np.array([r for r in range(n) if map_[r] >= 0])
        if not _close(o[rows, h * D:(h + 1) * D], want[rows]):
            msgs.append(f"all cubes selected: head {h} differs from dense over the valid keys")
    if not np.all(o[7] == 12345.0) or not np.all(o[n:] == 12345.0):
        msgs.append("rows with map < 0 or past n_q were written")
    # dense rows respect validity too: a layout with dense rows, one of them invalid
    cubes2, dense = 2, 40
    n2 = cubes2 * 64 + dense
    valid2 = np.zeros(k_pad, np.uint8)
    valid2[:n2] = 1
    valid2[cubes2 * 64 + 5] = 0
    sel2 = np.tile(np.arange(cubes2, dtype=np.uint16), (heads, cubes2, 1))
    nsel2 = np.full((heads, cubes2), cubes2, np.uint16)
    map2 = np.where(np.arange(q_pad) < n2, np.arange(q_pad), -1).astype(np.int32)
    o2, _ = O.attn_sparse(q, k, v, sel2, nsel2, valid2, map2, n_q=n2, q_pad=q_pad, n_k=n2, k_pad=k_pad,
                          heads=heads, kv_heads=kv, n_cubes=cubes2, max_sel=cubes2, dense0=cubes2 * 64, dense1=n2,
                          dtype=O.F16, mutant=mutant)
    keys2 = np.nonzero(valid2[:n2])[0]
    s = qf[0, :n2] @ kf[0, keys2].T * scale
    if not _close(o2[:n2, :D], softmax(s, axis=1) @ vf[0, keys2]):
        msgs.append("cubes plus dense rows differ from dense over the valid keys")
    return not msgs, "; ".join(msgs)


def check_cube_select(mutant=None):
    msgs = []
    rng = _rng(4)
    heads, D, cubes = 2, 128, 7
    q_pad = k_pad = cubes * 64
    cnt = np.array([64, 64, 30, 64, 64, 1, 64], np.uint32)
    q = _f16(rng.standard_normal((heads, q_pad, D)))
    k = _f16(rng.standard_normal((heads, k_pad, D)))
    rowmask = np.concatenate([np.arange(64) < c for c in cnt]).astype(np.float32)
    q = _f16(O.bits_to_f32(q, O.F16) * rowmask[None, :, None])
    k = _f16(O.bits_to_f32(k, O.F16) * rowmask[None, :, None])
    for topk in (3, 9):
        sel, nsel = O.cube_select(q, k, cnt, heads=heads, dim=D, q_pad=q_pad, k_pad=k_pad, n_cubes=cubes, topk=topk,
                                  dtype=O.F16, mutant=mutant)
        qf, kf = O.bits_to_f32(q, O.F16).astype(np.float64), O.bits_to_f32(k, O.F16).astype(np.float64)
        kk = min(topk, cubes)
        for h in range(heads):
            qp = qf[h].reshape(cubes, 64, D).sum(1) / cnt[:, None]
            kp = kf[h].reshape(cubes, 64, D).sum(1) / cnt[:, None]
            sc = qp @ kp.T
            want = np.argsort(-sc, axis=1, kind="stable")[:, :kk]
            if not np.array_equal(sel[h], want) or not np.all(nsel[h] == kk):
                msgs.append(f"top {topk}: head {h} differs from the stable sort")
    # ties go to the smaller index: identical key cubes score the same
    k_t = k.copy()
    k_t[:, 3 * 64:4 * 64] = k_t[:, 1 * 64:2 * 64]
    cnt_t = cnt.copy()
    cnt_t[3] = cnt_t[1]
    sel, _ = O.cube_select(q, k_t, cnt_t, heads=heads, dim=D, q_pad=q_pad, k_pad=k_pad, n_cubes=cubes, topk=cubes,
                           dtype=O.F16, mutant=mutant)
    for h in range(heads):
        for qc in range(cubes):
            row = list(sel[h, qc])
            if row.index(1) > row.index(3):
                msgs.append("a tie went to the larger index")
                break
    # local = 3, stride 1: the cube and its neighbours lead, no cube twice (tests/sparse_attn_test.cpp:183-207)
    sel, _ = O.cube_select(q, k, cnt, heads=heads, dim=D, q_pad=q_pad, k_pad=k_pad, n_cubes=cubes, topk=4, local=3,
                           stride=1, dtype=O.F16, mutant=mutant)
    for h in range(heads):
        for qc in range(cubes):
            want = [qc] + ([qc - 1] if qc >= 1 else []) + ([qc + 1] if qc + 1 < cubes else [])
            row = list(sel[h, qc])
            if row[:len(want)] != want or len(set(row)) != len(row):
                msgs.append(f"local cubes: head {h} cube {qc} gives {row}")
    return not msgs, "; ".join(msgs)


def check_decode_and_merge(mutant=None):
    msgs = []
    rng = _rng(5)
    batch, heads, kv, dim, cap = 3, 4, 2, 128, 200
    ctx = np.array([1, 77, 200], np.uint32)
    q = _f16(rng.standard_normal((batch, heads, dim)))
    k = _f16(rng.standard_normal((batch, kv, cap, dim)))
    v = _f16(rng.standard_normal((batch, kv, cap, dim)))
    o, lse = O.attn_decode(q, k, v, ctx, batch=batch, heads=heads, kv_heads=kv, dim=dim, cap=cap, dtype=O.F16,
                           mutant=mutant)
    for b in range(batch):
        qt = np.zeros((heads, 64, dim), np.uint16)
        qt[:, 0] = q[b]
        od, ld = O.attn_dense(qt, k[b], v[b], n_q=1, q_pad=64, n_k=int(ctx[b]), k_pad=cap, heads=heads, kv_heads=kv,
                              q_pos0=int(ctx[b]) - 1, block=U32, dim=dim, dtype=O.F16, mutant=mutant)
        if not (_close(o[b], od[0]) and _close(lse[b], ld[:, 0])):
            msgs.append(f"decode of sequence {b} differs from the dense row at q_pos0 = ctx - 1")
    # merging splits of one row equals the whole row (scipy softmax over each split)
    qf = O.bits_to_f32(q, O.F16).astype(np.float64)[2, 0]
    kf = O.bits_to_f32(k, O.F16).astype(np.float64)[2, 0]
    vf = O.bits_to_f32(v, O.F16).astype(np.float64)[2, 0]
    s = kf @ qf * float(np.float32(1 / np.sqrt(dim)))
    parts = [(0, 64), (64, 150), (150, 200)]
    o_i = np.stack([softmax(s[a:b]) @ vf[a:b] for a, b in parts])
    l_i = np.array([logsumexp(s[a:b]) for a, b in parts])
    om, lm = O.lse_merge(o_i, l_i, mutant=mutant)
    if not (_close(om, softmax(s) @ vf) and _close(lm, logsumexp(s))):
        msgs.append("merging splits differs from the whole row")
    om, lm = O.lse_merge(np.stack([o_i[0], o_i[0]]), np.array([l_i[0], l_i[0]]), mutant=mutant)
    if not (_close(om, o_i[0]) and _close(lm, l_i[0] + np.log(2.0))):
        msgs.append("merging two equal partials is not the same row with lse + log 2")
    return not msgs, "; ".join(msgs)


def check_heads(mutant=None):
    msgs = []
    rng = _rng(31)
    T, H, D, ld = 6, 3, 128, 3 * 128 + 16
    x = rng.standard_normal((T, ld)).astype(np.float32)
    args = dict(rows=T, ld=ld, col0=8, stride=D, dim=D, heads=H, n_pad=9, mutant=mutant)
    heads3 = x[:, 8:8 + H * D].reshape(T, H, D).transpose(1, 0, 2)
    # the plain slice, rounded by numpy; padding zeroed with clear, left alone without
    for out, conv in ((O.F16, O.to_f16_bits), (O.BF16, O.to_bf16_bits)):
        y = O.heads(x, clear=1, out=out, y=np.full((H, 9, D), 0x7777, np.uint16), **args)
        if not (np.array_equal(y[:, :T], conv(heads3)) and (y[:, T:] == 0).all()):
            msgs.append(f"plain slice ({'f16' if out == O.F16 else 'bf16'}) is not numpy's rounding of x")
    y = O.heads(x, row0=2, y=np.full((H, 9, D), 0x7777, np.uint16), **args)
    if not ((y[:, :2] == 0x7777).all() and (y[:, 2 + T:] == 0x7777).all()):
        msgs.append("rows outside [row0, row0 + rows) were written without clear")

    def rot(rope, rr, ang, src=None):
        cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
        return O.bits_to_f32(O.heads(x, cs, rope=rope, rot=rr, **args), O.F16).astype(np.float64)[:, :T], cs
    ident, _ = rot(1, D, np.zeros((T, D // 2)))
    if not np.array_equal(ident, O.bits_to_f32(O.to_f16_bits(heads3), O.F16)):
        msgs.append("angle 0 is not the identity")
    q90, _ = rot(1, D, np.full((T, D // 2), np.pi / 2))
    if not (np.allclose(q90[..., :D // 2], -heads3[..., D // 2:], atol=2e-3, rtol=2e-3) and
            np.allclose(q90[..., D // 2:], heads3[..., :D // 2], atol=2e-3, rtol=2e-3)):
        msgs.append("angle pi / 2 does not map (u, v) to (-v, u)")
    for rope, rr in ((1, D), (1, 96), (2, D), (2, 64)):
        ang = rng.uniform(-np.pi, np.pi, (T, rr // 2))
        got, cs = rot(rope, rr, ang)
        c = cs[..., 0].astype(np.float64) + 1j * cs[..., 1].astype(np.float64)  # [T][rr / 2]
        xs = heads3.astype(np.float64)
        if rope == 1:
            z = (xs[..., :rr // 2] + 1j * xs[..., rr // 2:rr]) * c[None]
            want = np.concatenate([z.real, z.imag, xs[..., rr:]], -1)
        else:
            z = (xs[..., 0:rr:2] + 1j * xs[..., 1:rr:2]) * c[None]
            want = xs.copy()
            want[..., 0:rr:2], want[..., 1:rr:2] = z.real, z.imag
        if not np.allclose(got, want, atol=1e-3, rtol=2 ** -10):
            msgs.append(f"rope {rope} over {rr} is not the complex product (u + i v)(c + i s)")
    # the norm: unit mean square with w = 1, invariant to scaling x, the weight multiplies value-wise
    ones = np.ones(D, np.float32)
    yn = O.bits_to_f32(O.heads(x, w=ones, eps=1e-6, **args), O.F16).astype(np.float64)[:, :T]
    if not np.allclose((yn ** 2).mean(-1), 1.0, rtol=2e-3):
        msgs.append("a normed head with w = 1 does not have unit mean square")
    ys = O.bits_to_f32(O.heads(x * 8.0, w=ones, eps=1e-6, **args), O.F16).astype(np.float64)[:, :T]
    if not np.allclose(ys, yn, atol=2e-3, rtol=2e-3):
        msgs.append("the norm is not invariant to scaling x")
    wv = rng.uniform(0.5, 2.0, D).astype(np.float32)
    yw = O.bits_to_f32(O.heads(x, w=wv, eps=1e-6, **args), O.F16).astype(np.float64)[:, :T]
    if not np.allclose(yw, yn * wv, atol=2e-3, rtol=2e-3):
        msgs.append("the weight does not multiply the normed values")
    # the row map: row t from x row map[t] with that row's angles; a negative entry gives a zero row
    ang = rng.uniform(-np.pi, np.pi, (T, 48))
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    mp = np.array([3, -1, 0, 5, 5, 2], np.int32)
    full = O.heads(x, cs, w=wv, eps=1e-5, rope=1, rot=96, **args)
    mapped = O.heads(x, cs, wv, mp, eps=1e-5, rope=1, rot=96, **args)
    if not all(np.array_equal(mapped[:, t], full[:, mp[t]]) if mp[t] >= 0 else (mapped[:, t] == 0).all()
               for t in range(T)):
        msgs.append("a mapped row is not its source row's result (or a negative map is not a zero row)")
    return not msgs, "; ".join(msgs)


def check_gather(mutant=None):
    rng = _rng(77)
    msgs = []
    H, D, N, kps = 5, 64, 200, 64
    kv = _f16(rng.standard_normal((N, D)))
    kvf = O.bits_to_f32(kv, O.F16).astype(np.float64)
    p = rng.uniform(0.0, 1.0, (H, N)).astype(np.float32)
    ph = p.astype(np.float16).astype(np.float64)
    part = O.attn_pv(p, kv, heads=H, dim=D, n_kv=N, keys_per_split=kps, mutant=mutant)
    if part.shape != (4, H, D) or not _close(part.sum(0), ph @ kvf, 1e-12):
        msgs.append("attn_pv splits do not sum to p kv")
    onehot = np.zeros((H, N), np.float32)
    taus = [0, 63, 64, 150, 199]
    for h, tau in enumerate(taus):
        onehot[h, tau] = 1.0
    part = O.attn_pv(onehot, kv, heads=H, dim=D, n_kv=N, keys_per_split=kps, mutant=mutant)
    want = np.zeros_like(part)
    for h, tau in enumerate(taus):
        want[tau // kps, h] = kvf[tau]
    if not np.array_equal(part, want):
        msgs.append("attn_pv: a one-hot p does not give its kv row in its key's split")
    part = O.attn_pv(np.full((H, N), 1.0 + 2.0 ** -12, np.float32), kv, heads=H, dim=D, n_kv=N, keys_per_split=kps,
                     mutant=mutant)
    if not np.array_equal(part.sum(0)[0], kvf.sum(0)):
        msgs.append("attn_pv does not round p to half")

    # gathered scores: T tokens, lists of S entries, count[t] used
    T, S, R, DL = 3, 96, 300, 256
    kvl = _f16(rng.standard_normal((R, DL)) * 0.5)
    kvlf = O.bits_to_f32(kvl, O.F16).astype(np.float64)
    q = _f16(rng.standard_normal((T, H, DL)) * 0.5)
    qf = O.bits_to_f32(q, O.F16).astype(np.float64)
    ident = np.tile(np.arange(S, dtype=np.uint32), (T, 1))
    full = np.full(T, S, np.uint32)
    sc = O.gather_scores(q, kvl, ident, full, heads=H, dim=DL, stride=S, tokens=T, mutant=mutant)
    if not _close(sc, qf @ kvlf[:S].T, 1e-12):
        msgs.append("gather_scores with the identity list is not q kv^T")
    perm = np.stack([rng.permutation(R)[:S] for _ in range(T)]).astype(np.uint32)
    sc = O.gather_scores(q, kvl, perm, full, heads=H, dim=DL, stride=S, tokens=T, mutant=mutant)
    if not all(_close(sc[t], qf[t] @ kvlf[perm[t]].T, 1e-12) for t in range(T)):
        msgs.append("gather_scores with a permuted list does not permute the columns")
    cnt = np.array([0, 37, S], np.uint32)
    sc2 = O.gather_scores(q, kvl, perm, cnt, heads=H, dim=DL, stride=S, tokens=T, mutant=mutant)
    if not all(np.array_equal(sc2[t, :, :cnt[t]], sc[t, :, :cnt[t]]) and (sc2[t, :, cnt[t]:] == 0).all()
               for t in range(T)):
        msgs.append("gather_scores entries from count[t] on are not zero")

    # gathered P V
    pg = rng.uniform(0.0, 1.0, (T, H, S)).astype(np.float32)
    for splits in (1, 2, 3):
        per = -(-S // (splits * 64)) * 64
        gp = O.gather_pv(pg, kvl, ident, full, heads=H, dim=DL, stride=S, splits=splits, tokens=T, mutant=mutant)
        ok = True
        for t in range(T):
            ref = O.attn_pv(pg[t], kvl[:S], heads=H, dim=DL, n_kv=S, keys_per_split=per, mutant=mutant)
            want = np.zeros((splits, H, DL))  # ceil(S / per) <= splits: trailing splits are empty
            want[:len(ref)] = ref
            ok &= _close(gp[:, t], want, 1e-12)
        if not ok:
            msgs.append(f"gather_pv with the identity list differs from attn_pv at {per} keys a split")
    gp = O.gather_pv(pg, kvl, perm, cnt, heads=H, dim=DL, stride=S, splits=2, tokens=T, mutant=mutant)
    pgh = pg.astype(np.float16).astype(np.float64)
    if not all(_close(gp[:, t].sum(0), pgh[t, :, :cnt[t]] @ kvlf[perm[t, :cnt[t]]], 1e-12) for t in range(T)):
        msgs.append("gather_pv splits do not sum to p kv over the first count[t] entries")
    oh = np.zeros((T, H, S), np.float32)
    picks = [(0, 0, 5), (1, 2, 36), (2, 4, 64), (2, 1, 95)]
    for t, h, s_ in picks:
        oh[t, h, s_] = 1.0
    gp = O.gather_pv(oh, kvl, perm, full, heads=H, dim=DL, stride=S, splits=2, tokens=T, mutant=mutant)
    want = np.zeros_like(gp)
    for t, h, s_ in picks:
        want[s_ // 64, t, h] = kvlf[perm[t, s_]]
    if not np.array_equal(gp, want):
        msgs.append("gather_pv: a one-hot p does not land in split s // per")

    # idx_dots in float
    P, St = 45, 64
    qd = rng.standard_normal((T, H, 96)).astype(np.float32)
    pooled = rng.standard_normal((P, 96)).astype(np.float32)
    d = O.idx_dots(qd, pooled, heads=H, dim=96, pools=P, stride=St, tokens=T, dots=np.full((T, H, St), 7.0),
                   mutant=mutant)
    if not _close(d[:, :, :P], qd.astype(np.float64) @ pooled.astype(np.float64).T, 1e-12) or \
            not (d[:, :, P:] == 7.0).all():
        msgs.append("idx_dots is not q pooled^T on the first pools columns")
    return not msgs, "; ".join(msgs)


def check_proj(mutant=None):
    import torch

    rng = _rng(31)
    msgs = []
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()
    T, K, N = 5, 128, 96
    x = (rng.standard_normal((T, K)) * 3).astype(np.float32)
    w = O.to_bf16_bits(rng.standard_normal((N, K)) * 0.1)
    wf = O.bits_to_f32(w, O.BF16).astype(np.float64)
    y = O.proj_bf16(x, w, t=T, k=K, n=N, mutant=mutant)
    if not _close(y, bf(x).astype(np.float64) @ wf.T, 1e-12):
        msgs.append("proj is not bf16(x) w^T")
    eye = O.to_bf16_bits(np.eye(K))
    y = O.proj_bf16(x, eye, t=T, k=K, n=K, mutant=mutant)
    if not np.array_equal(y, bf(x).astype(np.float64)):
        msgs.append("proj with w = I is not bf16(x)")
    y = O.proj_bf16(x, eye, t=T, k=K, n=K, split=1, mutant=mutant)
    hi = bf(x)
    if not np.array_equal(y, hi.astype(np.float64) + bf(x - hi).astype(np.float64)):
        msgs.append("proj split with w = I is not bf16(x) + bf16(x - bf16(x))")
    exact = x.astype(np.float64) @ wf.T
    mag = np.abs(x).astype(np.float64) @ np.abs(wf).T
    y = O.proj_bf16(x, w, t=T, k=K, n=N, split=1, mutant=mutant)
    if not (np.abs(y - exact) <= 2.0 ** -15 * mag).all():
        msgs.append("proj split is not within 2^-15 of x w^T")
    xb = O.to_bf16_bits(x)
    y = O.proj_bf16(xb, w, t=T, k=K, n=N, x_dtype=O.BF16, mutant=mutant)
    if not _close(y, O.bits_to_f32(xb, O.BF16).astype(np.float64) @ wf.T, 1e-12):
        msgs.append("proj with bf16 x is not x w^T")
    xs = np.zeros((T, K + 64), np.float32)
    xs[:, :K] = x
    y = O.proj_bf16(xs, w, t=T, k=K, n=N, ldx=K + 64, ldy=N + 8, y=np.full((T, N + 8), 5.0), mutant=mutant)
    if not _close(y[:, :N], bf(x).astype(np.float64) @ wf.T, 1e-12) or not (y[:, N:] == 5.0).all():
        msgs.append("proj with strided rows reads or writes the wrong elements")
    return not msgs, "; ".join(msgs)


def check_kda(mutant=None):
    rng = _rng(459)
    msgs = []
    D = 128
    sq = np.sqrt(D)
    unit = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    # one token from a zero state
    q, k, v = rng.standard_normal((3, 1, D)).astype(np.float32)
    g = rng.uniform(-1, 0, (1, D)).astype(np.float32)
    beta = np.array([[0.7]], np.float32)
    o, st, _ = O.kda_scan(q, k, v, g, beta, tokens=1, heads=1, mutant=mutant)
    want = float(np.dot(k[0].astype(np.float64), q[0])) * float(beta[0, 0]) * v[0].astype(np.float64) / sq
    if not _close(o[0], want, 1e-9):
        msgs.append("kda one token from zero state is not (k.q) beta v / sqrt(D)")
    # beta = 0: pure decay of a given state
    T = 6
    S0 = rng.standard_normal((1, D, D))
    q = rng.standard_normal((T, D)).astype(np.float32)
    k = rng.standard_normal((T, D)).astype(np.float32)
    v = rng.standard_normal((T, D)).astype(np.float32)
    g = rng.uniform(-0.5, 0, (T, D)).astype(np.float32)
    o, st, _ = O.kda_scan(q, k, v, g, np.zeros((T, 1), np.float32), S0, tokens=T, heads=1, mutant=mutant)
    cum = np.cumsum(g.astype(np.float64), 0)
    ok = _close(st[0], S0[0] * np.exp(cum[-1])[None, :], 1e-9)
    for t in range(T):
        ok &= _close(o[t], (S0[0] * np.exp(cum[t])[None, :]) @ q[t].astype(np.float64) / sq, 1e-9)
    if not ok:
        msgs.append("kda with beta = 0 is not the decayed initial state")
    # exact recall of orthonormal keys (g = 0, beta = 1), then reads (beta = 0) with q = k_b
    n = 5
    Q, _ = np.linalg.qr(rng.standard_normal((D, D)))
    keys = Q[:n].astype(np.float32)
    vals = rng.standard_normal((n, D)).astype(np.float32)
    kk = np.concatenate([keys, np.zeros((n, D), np.float32)])
    qq = np.concatenate([np.zeros((n, D), np.float32), keys])
    vv = np.concatenate([vals, np.zeros((n, D), np.float32)])
    bb = np.concatenate([np.ones((n, 1)), np.zeros((n, 1))]).astype(np.float32)
    o, _, _ = O.kda_scan(qq, kk, vv, np.zeros((2 * n, D), np.float32), bb, tokens=2 * n, heads=1, mutant=mutant)
    if not _close(o[n:], vals.astype(np.float64) / sq, 1e-6):
        msgs.append("kda does not recall orthonormal keys exactly")
    # the same key twice: the second value replaces the first
    k1 = unit(rng.standard_normal(D)).astype(np.float32)
    v1, v2 = rng.standard_normal((2, D)).astype(np.float32)
    o, _, _ = O.kda_scan(np.stack([k1 * 0, k1 * 0, k1]), np.stack([k1, k1, k1 * 0]), np.stack([v1, v2, v1 * 0]),
                         np.zeros((3, D), np.float32), np.array([[1], [1], [0]], np.float32), tokens=3, heads=1,
                         mutant=mutant)
    if not _close(o[2], v2.astype(np.float64) / sq, 1e-6):
        msgs.append("kda does not overwrite a key written twice")
    # full decay: g = -60 forgets the state before the token's read
    o, _, _ = O.kda_scan(np.stack([k1 * 0, k1]), np.stack([k1, k1]), np.stack([v1, v2]),
                         np.stack([np.zeros(D), np.full(D, -60.0)]).astype(np.float32),
                         np.ones((2, 1), np.float32), tokens=2, heads=1, mutant=mutant)
    if not _close(o[1], float(np.dot(k1.astype(np.float64), k1)) * v2.astype(np.float64) / sq, 1e-6):
        msgs.append("kda full decay does not forget the state before the read")
    # two calls carrying the state equal one call; the snapshot equals the state of a call that stops there
    T, H = 12, 2
    q = unit(rng.standard_normal((T, H, D))).astype(np.float32).reshape(T, H * D)
    k = unit(rng.standard_normal((T, H, D))).astype(np.float32).reshape(T, H * D)
    v = rng.standard_normal((T, H * D)).astype(np.float32)
    g = rng.uniform(-0.3, 0, (T, H * D)).astype(np.float32)
    beta = rng.uniform(0, 1, (T, H)).astype(np.float32)
    o, st, snap = O.kda_scan(q, k, v, g, beta, tokens=T, heads=H, snap=5, mutant=mutant)
    o1, st1, _ = O.kda_scan(q[:5], k[:5], v[:5], g[:5], beta[:5], tokens=5, heads=H, mutant=mutant)
    o2, st2, _ = O.kda_scan(q[5:], k[5:], v[5:], g[5:], beta[5:], st1, tokens=T - 5, heads=H, mutant=mutant)
    if not (_close(np.concatenate([o1, o2]), o, 1e-12) and _close(st2, st, 1e-12) and _close(snap, st1, 1e-12)):
        msgs.append("kda split calls, or the snapshot, differ from one call")
    # heads in strided rows run independently
    ld = H * D + 64
    pad = lambda x: np.concatenate([x, np.zeros((T, 64), np.float32)], 1)
    oh, sth, _ = O.kda_scan(pad(q), pad(k), pad(v), pad(g), beta, tokens=T, heads=H, qkv_stride=ld, inner=ld,
                            mutant=mutant)
    ok = _close(oh[:, :H * D], o, 1e-12)
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        oo, ss, _ = O.kda_scan(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, h:h + 1], tokens=T, heads=1,
                               mutant=mutant)
        ok &= _close(oo, o[:, sl], 1e-12) and _close(ss[0], st[h], 1e-12)
    if not ok:
        msgs.append("kda heads are not independent of each other and of the row stride")
    return not msgs, "; ".join(msgs)


ALL_CHECKS = [check_goldens, check_closed_forms, check_invariants, check_sparse, check_cube_select,
              check_decode_and_merge, check_heads, check_gather, check_proj, check_kda]
