"""ctypes binding of the CPU oracle (oracle/attn_oracle.c): test infrastructure only.

Only the tests, the smoke check and the benchmark's CPU-baseline leg use this module, and only as the checker or
the timed CPU baseline. Inputs are numpy arrays of float32, or uint16 bit patterns of float16 / bfloat16; outputs
are float64.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32, F16, BF16 = 0, 1, 2


class AttnArgs(ctypes.Structure):
    """The reference's AttnArgs (src/kernels/ops.metal:54-64)."""

    _fields_ = [(n, ctypes.c_uint32) for n in ("n_q", "q_pad", "n_k", "k_pad", "heads", "kv_heads", "q_pos0",
                                               "block", "width")] + [("scale", ctypes.c_float)]


class SparseArgs(ctypes.Structure):
    """The reference's SparseAttnArgs (src/kernels/ops.metal:1029-1034) plus causal and sel_heads."""

    _fields_ = [(n, ctypes.c_uint32) for n in ("n_q", "q_pad", "n_k", "k_pad", "heads", "kv_heads", "width")] + \
        [("scale", ctypes.c_float)] + \
        [(n, ctypes.c_uint32) for n in ("n_cubes", "max_sel", "dense0", "dense1", "causal", "sel_heads")]


class HeadsArgs(ctypes.Structure):
    """HeadsArgs / HeadsNormArgs / HeadsPartialArgs (src/kernels/ops.metal:11-19, 371-374, 577-585) in one."""

    _fields_ = [(n, ctypes.c_uint32) for n in ("rows", "ld", "col0", "stride", "dim", "heads", "n_pad", "row0",
                                               "rope", "rot")] + [("eps", ctypes.c_float), ("clear", ctypes.c_uint32)]


def build(name="liboracle.so", mutant=None):
    """Builds the oracle library (or a mutant with one planted mistake) and returns its path."""
    target = name if mutant is None else f"liboracle_mutant{mutant}.so"
    subprocess.run(["make", "-s", "-C", HERE, target], check=True)
    return os.path.join(HERE, target)


_libs = {}


def lib(mutant=None):
    """The oracle library (built on first use when missing)."""
    if mutant not in _libs:
        path = os.path.join(HERE, "liboracle.so" if mutant is None else f"liboracle_mutant{mutant}.so")
        if not os.path.exists(path) or mutant is not None:
            path = build(mutant=mutant)
        L = ctypes.CDLL(path)
        P, U32, I, SZ, F = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
        L.oracle_attn_dense.argtypes = [ctypes.POINTER(AttnArgs), U32, I, P, P, P, P, P, I]
        L.oracle_attn_dense_rows.argtypes = [ctypes.POINTER(AttnArgs), U32, I, P, P, P, P, SZ, P, P, I]
        L.oracle_attn_sparse.argtypes = [ctypes.POINTER(SparseArgs), I, P, P, P, P, P, P, P, P, U32, P, I]
        L.oracle_attn_sparse_rows.argtypes = [ctypes.POINTER(SparseArgs), I, P, P, P, P, P, P, P, SZ, P, P, I]
        L.oracle_cube_select.argtypes = [U32, U32, I, P, U32, P, U32, U32, P, U32, U32, U32, P, P, P, P, P]
        L.oracle_attn_decode.argtypes = [U32, U32, U32, U32, U32, F, I, P, P, P, P, P, P, I]
        L.oracle_attn_decode_rows.argtypes = [U32, U32, U32, U32, U32, F, I, P, P, P, P, P, SZ, P, P, I]
        L.oracle_heads.argtypes = [ctypes.POINTER(HeadsArgs), I, P, P, P, P, P]
        L.oracle_attn_pv.argtypes = [U32, U32, U32, U32, P, P, P]
        L.oracle_gather_scores.argtypes = [U32, U32, U32, U32, P, P, P, P, P]
        L.oracle_gather_pv.argtypes = [U32, U32, U32, U32, U32, P, P, P, P, P]
        L.oracle_idx_dots.argtypes = [U32, U32, U32, U32, U32, P, P, P]
        L.oracle_proj_bf16.argtypes = [U32, U32, U32, U32, U32, I, I, P, P, P]
        L.oracle_kda_scan.argtypes = [U32, U32, U32, U32, U32, U32, P, P, P, P, P, P, P, P]
        L.oracle_lse_merge.argtypes = [U32, U32, P, P, P, P]
        L.oracle_lse_merge.restype = None
        L.oracle_f32_to_f16.argtypes = [F]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [F]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = F
        _libs[mutant] = L
    return _libs[mutant]


def _p(x):
    return None if x is None else x.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(x):
    if x.dtype == np.float32:
        return F32
    raise TypeError("pass float32 arrays, or uint16 bit patterns with an explicit dtype")


def _raw(x, dtype):
    x = np.ascontiguousarray(x)
    if dtype is None:
        return x, _dtype_code(x)
    assert x.dtype == np.uint16 and dtype in (F16, BF16)
    return x, dtype


def attn_dense(q, k, v, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, dim, scale=None, dtype=None,
               width=None, nthreads=0, mutant=None):
    """Dense attention: returns (o [n_q][width], lse [heads][n_q])."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    v, _ = _raw(v, dtype)
    width = heads * dim if width is None else width
    scale = np.float32(1.0 / np.sqrt(dim)) if scale is None else scale
    a = AttnArgs(n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block & 0xFFFFFFFF, width, scale)
    o = np.zeros((n_q, width), np.float64)
    lse = np.zeros((heads, n_q), np.float64)
    rc = lib(mutant).oracle_attn_dense(ctypes.byref(a), dim, code, _p(q), _p(k), _p(v), _p(o), _p(lse), nthreads)
    if rc:
        raise ValueError("oracle_attn_dense: shape refused")
    return o, lse


def attn_dense_rows(q, k, v, head_row, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, dim, scale=None,
                    dtype=None, nthreads=0, mutant=None):
    """Dense attention for (head, row) pairs: returns (o [n][dim], lse [n])."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    v, _ = _raw(v, dtype)
    hr = np.ascontiguousarray(head_row, np.uint32).reshape(-1, 2)
    scale = np.float32(1.0 / np.sqrt(dim)) if scale is None else scale
    a = AttnArgs(n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block & 0xFFFFFFFF, heads * dim, scale)
    o = np.zeros((len(hr), dim), np.float64)
    lse = np.zeros(len(hr), np.float64)
    rc = lib(mutant).oracle_attn_dense_rows(ctypes.byref(a), dim, code, _p(q), _p(k), _p(v), _p(hr), len(hr),
                                            _p(o), _p(lse), nthreads)
    if rc:
        raise ValueError("oracle_attn_dense_rows: shape refused")
    return o, lse


def attn_sparse(q, k, v, sel, nsel, valid, map_, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, n_cubes, max_sel,
                dense0, dense1, causal=0, sel_heads=None, o_rows=None, width=None, dtype=None, o_fill=None,
                nthreads=0, mutant=None):
    """Block-sparse attention: returns (o [o_rows][width], lse [heads][q_pad]); o starts as o_fill."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    v, _ = _raw(v, dtype)
    width = heads * 128 if width is None else width
    o_rows = q_pad if o_rows is None else o_rows
    sel_heads = heads if sel_heads is None else sel_heads
    a = SparseArgs(n_q, q_pad, n_k, k_pad, heads, kv_heads, width, np.float32(1.0 / np.sqrt(128.0)), n_cubes,
                   max_sel, dense0, dense1, causal, sel_heads)
    o = np.zeros((o_rows, width), np.float64) if o_fill is None else np.array(o_fill, np.float64)
    lse = np.full((heads, q_pad), np.nan, np.float64)
    sel = np.ascontiguousarray(sel, np.uint16)
    nsel = np.ascontiguousarray(nsel, np.uint16)
    valid = np.ascontiguousarray(valid, np.uint8)
    map_ = np.ascontiguousarray(map_, np.int32)
    rc = lib(mutant).oracle_attn_sparse(ctypes.byref(a), code, _p(q), _p(k), _p(v), _p(sel), _p(nsel), _p(valid),
                                        _p(map_), _p(o), o_rows, _p(lse), nthreads)
    if rc:
        raise ValueError("oracle_attn_sparse: shape refused")
    return o, lse


def attn_sparse_rows(q, k, v, sel, nsel, valid, head_row, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, n_cubes,
                     max_sel, dense0, dense1, causal=0, sel_heads=None, dtype=None, nthreads=0, mutant=None):
    """Block-sparse attention for (head, tile row) pairs: returns (o [n][128], lse [n])."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    v, _ = _raw(v, dtype)
    sel_heads = heads if sel_heads is None else sel_heads
    a = SparseArgs(n_q, q_pad, n_k, k_pad, heads, kv_heads, heads * 128, np.float32(1.0 / np.sqrt(128.0)),
                   n_cubes, max_sel, dense0, dense1, causal, sel_heads)
    hr = np.ascontiguousarray(head_row, np.uint32).reshape(-1, 2)
    o = np.zeros((len(hr), 128), np.float64)
    lse = np.zeros(len(hr), np.float64)
    sel = np.ascontiguousarray(sel, np.uint16)
    nsel = np.ascontiguousarray(nsel, np.uint16)
    valid = np.ascontiguousarray(valid, np.uint8)
    rc = lib(mutant).oracle_attn_sparse_rows(ctypes.byref(a), code, _p(q), _p(k), _p(v), _p(sel), _p(nsel),
                                             _p(valid), _p(hr), len(hr), _p(o), _p(lse), nthreads)
    if rc:
        raise ValueError("oracle_attn_sparse_rows: shape refused")
    return o, lse


def cube_select(q, k, cnt, *, heads, dim, q_pad, k_pad, n_cubes, topk, local=0, stride=0, dtype=None,
                mutant=None, want_scores=False):
    """cube_select: returns (sel [heads][n][kk] u16, nsel [heads][n] u16[, qp, kp, sc])."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    kk = min(topk, n_cubes)
    sel = np.zeros((heads, n_cubes, max(kk, 1)), np.uint16)
    nsel = np.zeros((heads, n_cubes), np.uint16)
    cnt = np.ascontiguousarray(cnt, np.uint32)
    qp = np.zeros((heads, n_cubes, dim)) if want_scores else None
    kp = np.zeros((heads, n_cubes, dim)) if want_scores else None
    sc = np.zeros((heads, n_cubes, n_cubes)) if want_scores else None
    rc = lib(mutant).oracle_cube_select(heads, dim, code, _p(q), q_pad, _p(k), k_pad, n_cubes, _p(cnt), topk, local,
                                        stride, _p(sel), _p(nsel), _p(qp), _p(kp), _p(sc))
    if rc:
        raise ValueError("cube_select: refused")
    if want_scores:
        return sel, nsel, qp, kp, sc
    return sel, nsel


def attn_decode(q, k, v, ctx, *, batch, heads, kv_heads, dim, cap, scale=None, dtype=None, nthreads=0,
                mutant=None):
    """Batched decode: returns (o [batch][heads*dim], lse [batch][heads])."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    v, _ = _raw(v, dtype)
    ctx = np.ascontiguousarray(ctx, np.uint32)
    scale = np.float32(1.0 / np.sqrt(dim)) if scale is None else scale
    o = np.zeros((batch, heads * dim), np.float64)
    lse = np.zeros((batch, heads), np.float64)
    rc = lib(mutant).oracle_attn_decode(batch, heads, kv_heads, dim, cap, scale, code, _p(q), _p(k), _p(v), _p(ctx),
                                        _p(o), _p(lse), nthreads)
    if rc:
        raise ValueError("oracle_attn_decode: refused")
    return o, lse


def attn_decode_rows(q, k, v, ctx, seq_head, *, batch, heads, kv_heads, dim, cap, scale=None, dtype=None,
                     nthreads=0, mutant=None):
    """Batched decode for (sequence, head) pairs: returns (o [n][dim], lse [n])."""
    q, code = _raw(q, dtype)
    k, _ = _raw(k, dtype)
    v, _ = _raw(v, dtype)
    ctx = np.ascontiguousarray(ctx, np.uint32)
    sh = np.ascontiguousarray(seq_head, np.uint32).reshape(-1, 2)
    scale = np.float32(1.0 / np.sqrt(dim)) if scale is None else scale
    o = np.zeros((len(sh), dim), np.float64)
    lse = np.zeros(len(sh), np.float64)
    rc = lib(mutant).oracle_attn_decode_rows(batch, heads, kv_heads, dim, cap, scale, code, _p(q), _p(k), _p(v),
                                             _p(ctx), _p(sh), len(sh), _p(o), _p(lse), nthreads)
    if rc:
        raise ValueError("oracle_attn_decode_rows: refused")
    return o, lse


def lse_merge(o_i, lse_i, mutant=None):
    """Merges partial rows (o_i [n][dim] normalised, lse_i [n]) into (o [dim], lse)."""
    o_i = np.ascontiguousarray(o_i, np.float64)
    lse_i = np.ascontiguousarray(lse_i, np.float64)
    n, dim = o_i.shape
    o = np.zeros(dim, np.float64)
    lse = np.zeros(1, np.float64)
    lib(mutant).oracle_lse_merge(n, dim, _p(o_i), _p(lse_i), _p(o), _p(lse))
    return o, float(lse[0])


def heads(x, cs=None, w=None, map_=None, *, rows, ld, col0, stride, dim, heads, n_pad, row0=0, rope=0, rot=0,
          eps=0.0, clear=0, out=F16, y=None, mutant=None):
    """Head tiles: x float32 [*][ld] rows, cs float32 [*][rot / 2][2], w float32 [dim], map_ int32 [rows].
    Returns y [heads][n_pad][dim] as uint16 bits of `out` (f16 or bf16); pass y to see which rows stay untouched."""
    x = np.ascontiguousarray(x, np.float32)
    cs = None if cs is None else np.ascontiguousarray(cs, np.float32)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    map_ = None if map_ is None else np.ascontiguousarray(map_, np.int32)
    if y is None:
        y = np.zeros((heads, n_pad, dim), np.uint16)
    assert y.dtype == np.uint16 and y.flags.c_contiguous and y.shape == (heads, n_pad, dim)
    a = HeadsArgs(rows, ld, col0, stride, dim, heads, n_pad, row0, rope, rot, eps, clear)
    rc = lib(mutant).oracle_heads(ctypes.byref(a), out, _p(x), _p(cs), _p(w), _p(map_), _p(y))
    if rc:
        raise ValueError("oracle_heads: bad arguments")
    return y


def _u32(x):
    return np.ascontiguousarray(x).astype(np.uint32, copy=False)


def attn_pv(p, kv, *, heads, dim, n_kv, keys_per_split, mutant=None):
    """attn_pv (src/kernels/gemm.metal:688-730): p float32 [heads][n_kv], kv float16 bits [n_kv][dim]. Returns
    partial float64 [ceil(n_kv / keys_per_split)][heads][dim]."""
    p = np.ascontiguousarray(p, np.float32)
    kv = np.ascontiguousarray(kv, np.uint16)
    assert p.size >= heads * n_kv and kv.size >= n_kv * dim
    splits = -(-n_kv // keys_per_split)
    out = np.zeros((splits, heads, dim), np.float64)
    if lib(mutant).oracle_attn_pv(heads, dim, n_kv, keys_per_split, _p(p), _p(kv), _p(out)):
        raise ValueError("oracle_attn_pv: bad arguments")
    return out


def gather_scores(q, kv, list_, count, *, heads, dim, stride, tokens, mutant=None):
    """attn_gather_scores (src/kernels/gemm.metal:743-786): q float16 bits [tokens][heads][dim], kv float16 bits
    [rows][dim], list_ [tokens][stride], count [tokens]. Returns scores float64 [tokens][heads][stride]."""
    q = np.ascontiguousarray(q, np.uint16)
    kv = np.ascontiguousarray(kv, np.uint16)
    list_, count = _u32(list_), _u32(count)
    assert q.size >= tokens * heads * dim and list_.size >= tokens * stride and count.size >= tokens
    rows = kv.size // dim
    for t in range(tokens):
        assert (list_.reshape(-1)[t * stride:t * stride + min(int(count[t]), stride)] < rows).all()
    out = np.zeros((tokens, heads, stride), np.float64)
    lib(mutant).oracle_gather_scores(heads, dim, stride, tokens, _p(q), _p(kv), _p(list_), _p(count), _p(out))
    return out


def gather_pv(p, kv, list_, count, *, heads, dim, stride, splits, tokens, mutant=None):
    """attn_gather_pv (src/kernels/gemm.metal:788-844): p float32 [tokens][heads][stride]. Returns partial float64
    [splits][tokens][heads][dim]."""
    p = np.ascontiguousarray(p, np.float32)
    kv = np.ascontiguousarray(kv, np.uint16)
    list_, count = _u32(list_), _u32(count)
    assert p.size >= tokens * heads * stride and list_.size >= tokens * stride and count.size >= tokens
    out = np.zeros((splits, tokens, heads, dim), np.float64)
    if lib(mutant).oracle_gather_pv(heads, dim, stride, splits, tokens, _p(p), _p(kv), _p(list_), _p(count),
                                    _p(out)):
        raise ValueError("oracle_gather_pv: bad arguments")
    return out


def idx_dots(q, pooled, *, heads, dim, pools, stride, tokens, dots=None, mutant=None):
    """idx_dots (src/kernels/gemm.metal:846-870): q float32 [tokens][heads][dim], pooled float32 [pools][dim].
    Returns dots float64 [tokens][heads][stride], columns from pools on as passed in (zeros by default)."""
    q = np.ascontiguousarray(q, np.float32)
    pooled = np.ascontiguousarray(pooled, np.float32)
    if dots is None:
        dots = np.zeros((tokens, heads, stride), np.float64)
    dots = np.ascontiguousarray(dots, np.float64)
    lib(mutant).oracle_idx_dots(heads, dim, pools, stride, tokens, _p(q), _p(pooled), _p(dots))
    return dots


def proj_bf16(x, w, *, t, k, n, ldx=0, ldy=0, x_dtype=F32, split=0, y=None, mutant=None):
    """Runtime::proj with BF16 weights (src/gpu/runtime.cpp:164-205): w bfloat16 bits [n][k], x float32 [t][ldx]
    (x_dtype F32) or bfloat16 bits (BF16). Returns y float64 [t][ldy]; columns past n as passed in (zeros)."""
    ldx, ldy = ldx or k, ldy or n
    x = np.ascontiguousarray(x, np.float32 if x_dtype == F32 else np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    assert x.size >= (t - 1) * ldx + k if t else True
    assert w.size >= n * k
    if y is None:
        y = np.zeros((t, ldy), np.float64)
    y = np.ascontiguousarray(y, np.float64)
    if lib(mutant).oracle_proj_bf16(t, k, n, ldx, ldy, x_dtype, split, _p(w), _p(x), _p(y)):
        raise ValueError("oracle_proj_bf16: bad arguments")
    return y


def kda_scan(q, k, v, g, beta, state=None, *, tokens, heads, qkv_stride=None, inner=None, snap=0, head_dim=128,
             o=None, mutant=None):
    """kda_scan (src/kernels/ops.metal:459-519): q, k, v float32 rows qkv_stride apart, g rows inner apart, beta
    [tokens][heads]; state float64 [heads][head_dim][head_dim] (transposed, zeros by default). Returns (o float64
    rows inner apart, the final state, the state after `snap` tokens or None)."""
    D = head_dim
    qkv_stride = qkv_stride or heads * D
    inner = inner or heads * D
    q, k, v, g, beta = (np.ascontiguousarray(a, np.float32) for a in (q, k, v, g, beta))
    for a_, ld in ((q, qkv_stride), (k, qkv_stride), (v, qkv_stride), (g, inner)):
        assert a_.size >= (tokens - 1) * ld + heads * D if tokens else True
    assert beta.size >= tokens * heads
    state = np.zeros((heads, D, D)) if state is None else np.array(state, np.float64, copy=True)
    state = np.ascontiguousarray(state, np.float64)
    if o is None:
        o = np.zeros((tokens, inner), np.float64)
    o = np.ascontiguousarray(o, np.float64)
    snap_state = np.zeros((heads, D, D)) if snap else None
    if lib(mutant).oracle_kda_scan(D, tokens, qkv_stride, inner, heads, snap, _p(q), _p(k), _p(v), _p(g), _p(beta),
                                   _p(state), _p(o), _p(snap_state)):
        raise ValueError("oracle_kda_scan: bad arguments")
    return o, state, snap_state


def to_f16_bits(x):
    """float32 array -> float16 bit patterns (round to nearest even), by numpy."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def to_bf16_bits(x):
    """float32 array -> bfloat16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bits_to_f32(bits, dtype):
    """float16 / bfloat16 bit patterns -> float32 (exact)."""
    bits = np.asarray(bits, np.uint16)
    if dtype == F16:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)
