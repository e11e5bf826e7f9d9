"""Writes the small golden fixtures under tests/golden/ (run: python tests/golden/gen_golden.py).

The reference stores no vectors for its attention path (its only test draws inputs at run time from mt19937 and
std::normal_distribution, whose output is implementation-defined). These fixtures are computed here from the
mathematical definition, independently of the oracle's loops: explicit boolean visibility matrices built from
the reference's mask rule (src/kernels/ops.metal:289; GQA map :242; block-sparse pass list :1079-1098, validity
:1109, row map :1173-1184), scipy's softmax / logsumexp, and numpy's stable argsort for cube selection
(tests/sparse_attn_test.cpp:103-128). Inputs are seeded N(0,1), rounded to fp16 / bf16 (round to nearest even).
"""
import os

import numpy as np
from scipy.special import logsumexp, softmax

HERE = os.path.dirname(os.path.abspath(__file__))
F16, BF16 = 1, 2


def bits(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == F16:
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def widen(b, dtype):
    if dtype == F16:
        return b.view(np.float16).astype(np.float64)
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dense_case(name, *, heads, kv_heads, dim, n_q, n_k, q_pos0, block, dtype, seed, q_pad=None, k_pad=None):
    rng = np.random.default_rng(seed)
    q_pad = q_pad or (n_q + 63) // 64 * 64
    k_pad = k_pad or (n_k + 127) // 128 * 128
    qb = bits(rng.standard_normal((heads, q_pad, dim)), dtype)
    kb = bits(rng.standard_normal((kv_heads, k_pad, dim)), dtype)
    vb = bits(rng.standard_normal((kv_heads, k_pad, dim)), dtype)
    q, k, v = widen(qb, dtype), widen(kb, dtype), widen(vb, dtype)
    scale = float(np.float32(1.0 / np.sqrt(dim)))
    pos = q_pos0 + np.arange(n_q)[:, None]
    j = np.arange(n_k)[None, :]
    seen = (j <= pos) | ((pos >= block) & (j >= block))
    o = np.zeros((n_q, heads * dim))
    lse = np.zeros((heads, n_q))
    g = heads // kv_heads
    for h in range(heads):
        s = q[h, :n_q] @ k[h // g, :n_k].T * scale
        s = np.where(seen, s, -np.inf)
        any_seen = seen.any(axis=1)
        p = np.zeros_like(s)
        p[any_seen] = softmax(s[any_seen], axis=1)
        o[:, h * dim:(h + 1) * dim] = p @ v[h // g, :n_k]
        lse[h] = np.where(any_seen, logsumexp(np.where(seen, s, -np.inf), axis=1), -np.inf)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="dense", q=qb, k=kb, v=vb, o=o.astype(np.float32),
                        lse=lse.astype(np.float32),
                        args=np.array([n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, heads * dim, dim,
                                       dtype], np.int64), scale=np.float32(scale))


def sparse_case(name, *, heads, kv_heads, cnt, dense, topk, causal, dtype, seed, sel_shared=False):
    """A reference-test-like layout: len(cnt) cubes (cnt[c] valid rows each), then `dense` rows."""
    rng = np.random.default_rng(seed)
    D = 128
    cubes = len(cnt)
    n = cubes * 64 + dense
    q_pad, k_pad = (n + 63) // 64 * 64, (n + 127) // 128 * 128
    valid = np.zeros(k_pad, np.uint8)
    for c in range(cubes):
        valid[c * 64:c * 64 + cnt[c]] = 1
    valid[cubes * 64:n] = 1
    map_ = np.where(np.arange(q_pad) < n, np.arange(q_pad), -1).astype(np.int32)
    map_[valid[:q_pad] == 0] = -1
    qb = bits(rng.standard_normal((heads, q_pad, D)) * valid[:q_pad, None], dtype)
    kb = bits(rng.standard_normal((kv_heads, k_pad, D)) * valid[:, None], dtype)
    vb = bits(rng.standard_normal((kv_heads, k_pad, D)) * valid[:, None], dtype)
    q, k, v = widen(qb, dtype), widen(kb, dtype), widen(vb, dtype)
    # selection: pooled means over cnt, scored, sorted by (-score, index) - numpy's stable argsort
    sel_heads = kv_heads if sel_shared else heads
    kk = min(topk, cubes)
    sel = np.zeros((sel_heads, cubes, kk), np.uint16)
    nsel = np.full((sel_heads, cubes), kk, np.uint16)
    g = heads // kv_heads
    for sh in range(sel_heads):
        hq = sh * g if sel_shared else sh
        kvh = sh if sel_shared else sh // g
        qp = np.stack([q[hq, c * 64:c * 64 + 64].sum(0) / cnt[c] for c in range(cubes)])
        kp = np.stack([k[kvh, c * 64:c * 64 + 64].sum(0) / cnt[c] for c in range(cubes)])
        sc = qp @ kp.T
        for qc in range(cubes):
            sel[sh, qc] = np.argsort(-sc[qc], kind="stable")[:kk]
    dense0, dense1 = cubes * 64, n
    o = np.full((q_pad, heads * D), 12345.0)
    lse = np.full((heads, q_pad), np.nan)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    for h in range(heads):
        sh = h // g if sel_shared else h
        kvh = h // g
        for r in range(n):
            if map_[r] < 0:
                continue
            seen = np.zeros(k_pad, np.int64)  # multiplicity of each key
            if r // 64 < cubes:
                for c in sel[sh, r // 64, :nsel[sh, r // 64]]:
                    seen[c * 64:c * 64 + 64] += 1
                seen[dense0:dense1] += 1
            else:
                seen[:n] += 1
            seen *= valid
            if causal:
                seen[r + 1:] = 0
            keys = np.repeat(np.arange(k_pad), seen)
            s = k[kvh, keys] @ q[h, r] * scale
            o[map_[r], h * D:(h + 1) * D] = softmax(s) @ v[kvh, keys]
            lse[h, r] = logsumexp(s)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="sparse", q=qb, k=kb, v=vb, o=o.astype(np.float32),
                        lse=lse.astype(np.float32),
                        sel=sel, nsel=nsel, valid=valid, map=map_, cnt=np.array(cnt, np.uint32),
                        args=np.array([n, q_pad, n, k_pad, heads, kv_heads, heads * D, cubes, kk, dense0, dense1,
                                       causal, sel_heads, topk, dtype], np.int64), scale=np.float32(scale))


def decode_case(name, *, batch, heads, kv_heads, dim, cap, ctx, dtype, seed):
    rng = np.random.default_rng(seed)
    qb = bits(rng.standard_normal((batch, heads, dim)), dtype)
    kb = bits(rng.standard_normal((batch, kv_heads, cap, dim)), dtype)
    vb = bits(rng.standard_normal((batch, kv_heads, cap, dim)), dtype)
    q, k, v = widen(qb, dtype), widen(kb, dtype), widen(vb, dtype)
    scale = float(np.float32(1.0 / np.sqrt(dim)))
    o = np.zeros((batch, heads * dim))
    lse = np.zeros((batch, heads))
    g = heads // kv_heads
    for b in range(batch):
        for h in range(heads):
            n = ctx[b]
            if n == 0:
                lse[b, h] = -np.inf
                continue
            s = k[b, h // g, :n] @ q[b, h] * scale
            o[b, h * dim:(h + 1) * dim] = softmax(s) @ v[b, h // g, :n]
            lse[b, h] = logsumexp(s)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="decode", q=qb, k=kb, v=vb, o=o.astype(np.float32),
                        lse=lse.astype(np.float32),
                        ctx=np.array(ctx, np.uint32),
                        args=np.array([batch, heads, kv_heads, dim, cap, dtype], np.int64), scale=np.float32(scale))


def main():
    U = 0xFFFFFFFF
    dense_case("dense_causal_gqa_f16_d64", heads=4, kv_heads=2, dim=64, n_q=48, n_k=48, q_pos0=0, block=U,
               dtype=F16, seed=11)
    dense_case("dense_bidir_bf16_d128", heads=2, kv_heads=2, dim=128, n_q=40, n_k=40, q_pos0=0, block=0,
               dtype=BF16, seed=12)
    dense_case("dense_prefix_f16_d128", heads=2, kv_heads=1, dim=128, n_q=50, n_k=50, q_pos0=0, block=20,
               dtype=F16, seed=13)
    dense_case("dense_tail_bf16_d128", heads=4, kv_heads=1, dim=128, n_q=3, n_k=77, q_pos0=74, block=U,
               dtype=BF16, seed=14)
    dense_case("dense_causal_f16_d256", heads=2, kv_heads=1, dim=256, n_q=33, n_k=33, q_pos0=0, block=U,
               dtype=F16, seed=15)
    dense_case("dense_masked_rows_f16_d128", heads=1, kv_heads=1, dim=128, n_q=8, n_k=3, q_pos0=0, block=U,
               dtype=F16, seed=16, q_pad=64, k_pad=128)
    sparse_case("sparse_ref_like_f16", heads=2, kv_heads=2, cnt=[64, 64, 20], dense=30, topk=2, causal=0,
                dtype=F16, seed=21)
    sparse_case("sparse_causal_gqa_bf16", heads=4, kv_heads=2, cnt=[64, 64, 64], dense=0, topk=2, causal=1,
                dtype=BF16, seed=22, sel_shared=True)
    decode_case("decode_gqa_f16", batch=3, heads=4, kv_heads=2, dim=128, cap=160, ctx=[1, 100, 160], dtype=F16,
                seed=31)


if __name__ == "__main__":
    main()
