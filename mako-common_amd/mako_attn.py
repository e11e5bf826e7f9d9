"""Python binding of the C ABI in include/mako_attn.h (lib/libmako_attn.so), for the tests and the benchmark.

Tensors are torch tensors on the GPU (torch supplies device memory and streams here: plumbing, not compute).
Every call goes through the HIP kernels of libmako_attn.so; there is no fallback: a missing library raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmako_attn.so")

F32, F16, BF16 = 0, 1, 2
OK, EINVAL, EUNSUPPORTED, EWORKSPACE, EHIP = 0, 1, 2, 3, 4
U32_MAX = 0xFFFFFFFF

# Every symbol include/mako_attn.h declares.
EXPORTS = ("mako_attn_abi_version", "mako_last_error", "mako_attn_fwd", "mako_cube_select_workspace",
           "mako_cube_select", "mako_attn_sparse", "mako_attn_decode_workspace", "mako_attn_decode",
           "mako_attn_decode_noalloc", "mako_heads", "mako_attn_fwd_rows",
           "mako_attn_pv", "mako_attn_gather_scores", "mako_attn_gather_pv", "mako_idx_dots", "mako_proj_bf16",
           "mako_kda_scan", "mako_attn_fwd_workspace", "mako_attn_fwd_ws", "mako_attn_sparse_workspace",
           "mako_attn_sparse_ws", "mako_attn_fwd_rows_workspace", "mako_attn_fwd_rows_ws", "mako_attn_release",
           "mako_attn_held_bytes")


class AttnArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("n_q", "q_pad", "n_k", "k_pad", "heads", "kv_heads", "q_pos0",
                                               "block", "width")] + [("scale", ctypes.c_float)]


class SparseArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("n_q", "q_pad", "n_k", "k_pad", "heads", "kv_heads", "width")] + \
        [("scale", ctypes.c_float)] + \
        [(n, ctypes.c_uint32) for n in ("n_cubes", "max_sel", "dense0", "dense1", "causal", "sel_heads")]


class DecodeArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("batch", "heads", "kv_heads", "dim", "cap", "max_ctx", "split")] + \
        [("scale", ctypes.c_float)]


class HeadsArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("rows", "ld", "col0", "stride", "dim", "heads", "n_pad", "row0",
                                               "rope", "rot")] + [("eps", ctypes.c_float), ("clear", ctypes.c_uint32)]


class PvArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("heads", "dim", "n_kv", "keys_per_split")]


class GatherArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("heads", "dim", "stride", "splits", "tokens")]


class IdxDotArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("heads", "dim", "pools", "stride")]


class GemmArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("t", "k", "n", "row_bytes", "ldy", "ldx")]


class ScanArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("head_dim", "tokens", "qkv_stride", "inner", "heads", "snap")]


class MakoError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def lib():
    """The loaded library; raises when it has not been built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(LIB_PATH)
        P, U32, I, SZ = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t
        L.mako_attn_abi_version.restype = I
        L.mako_last_error.restype = ctypes.c_char_p
        L.mako_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs), U32, I, I, P, P, P, P, P, P]
        L.mako_cube_select_workspace.argtypes = [U32, U32]
        L.mako_cube_select_workspace.restype = SZ
        L.mako_cube_select.argtypes = [U32, U32, U32, U32, U32, U32, U32, I, P, P, P, P, P, P, SZ, P]
        L.mako_attn_sparse.argtypes = [ctypes.POINTER(SparseArgs), I, I, P, P, P, P, P, P, P, P, P, P]
        L.mako_attn_decode_workspace.argtypes = [ctypes.POINTER(DecodeArgs)]
        L.mako_attn_decode_workspace.restype = SZ
        L.mako_attn_decode.argtypes = [ctypes.POINTER(DecodeArgs), I, I, P, P, P, P, P, P, P, SZ, P]
        L.mako_attn_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), I, I, P, P, P, P, P, P, P]
        L.mako_heads.argtypes = [ctypes.POINTER(HeadsArgs), I, P, P, P, P, P, P]
        L.mako_attn_fwd_rows.argtypes = [ctypes.POINTER(AttnArgs)] + [ctypes.POINTER(HeadsArgs)] * 3 + [I, I] + \
            [P] * 9
        L.mako_attn_pv.argtypes = [ctypes.POINTER(PvArgs), P, P, P, P]
        L.mako_attn_gather_scores.argtypes = [ctypes.POINTER(GatherArgs), P, P, P, P, P, P]
        L.mako_attn_gather_pv.argtypes = [ctypes.POINTER(GatherArgs), P, P, P, P, P, P]
        L.mako_idx_dots.argtypes = [ctypes.POINTER(IdxDotArgs), U32, P, P, P, P]
        L.mako_proj_bf16.argtypes = [ctypes.POINTER(GemmArgs), I, I, P, P, P, P]
        L.mako_kda_scan.argtypes = [ctypes.POINTER(ScanArgs)] + [P] * 9
        L.mako_attn_fwd_workspace.argtypes = [ctypes.POINTER(AttnArgs), U32]
        L.mako_attn_fwd_workspace.restype = SZ
        L.mako_attn_fwd_ws.argtypes = [ctypes.POINTER(AttnArgs), U32, I, I, P, P, P, P, P, P, SZ, P]
        L.mako_attn_sparse_workspace.argtypes = [ctypes.POINTER(SparseArgs)]
        L.mako_attn_sparse_workspace.restype = SZ
        L.mako_attn_sparse_ws.argtypes = [ctypes.POINTER(SparseArgs), I, I] + [P] * 10 + [SZ, P]
        L.mako_attn_fwd_rows_workspace.argtypes = [ctypes.POINTER(AttnArgs), U32]
        L.mako_attn_fwd_rows_workspace.restype = SZ
        L.mako_attn_fwd_rows_ws.argtypes = [ctypes.POINTER(AttnArgs)] + [ctypes.POINTER(HeadsArgs)] * 3 + \
            [I, I] + [P] * 9 + [SZ, P]
        L.mako_attn_release.argtypes = [P]
        L.mako_attn_held_bytes.argtypes = []
        L.mako_attn_held_bytes.restype = SZ
        for name in ("mako_attn_fwd", "mako_cube_select", "mako_attn_sparse", "mako_attn_decode",
                     "mako_attn_decode_noalloc", "mako_heads", "mako_attn_fwd_rows", "mako_attn_fwd_ws",
                     "mako_attn_sparse_ws", "mako_attn_fwd_rows_ws", "mako_attn_release",
                     "mako_attn_pv", "mako_attn_gather_scores", "mako_attn_gather_pv", "mako_idx_dots",
                     "mako_proj_bf16", "mako_kda_scan"):
            getattr(L, name).restype = I
        _lib = L
    return _lib


def _check(rc):
    if rc != OK:
        raise MakoError(rc, lib().mako_last_error().decode())


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(stream)


def dtype_code(t):
    import torch

    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]


LIBRARY = "library"  # workspace= default: the entry point without a workspace argument (the library keeps its own)


def _nbytes(t):
    return 0 if t is None else t.numel() * t.element_size()


def attn_args(*, n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, dim, scale=None, width=None):
    width = heads * dim if width is None else width
    scale = 1.0 / dim ** 0.5 if scale is None else scale
    return AttnArgs(n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block & U32_MAX, width, scale)


def attn_fwd_workspace(*, dim, **kw):
    """mako_attn_fwd_workspace for the call attn_fwd would make with these arguments."""
    return lib().mako_attn_fwd_workspace(ctypes.byref(attn_args(dim=dim, **kw)), dim)


def attn_fwd(q, k, v, o, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, q_pos0, block, dim, lse=None, scale=None,
             width=None, stream=None, workspace=LIBRARY):
    """mako_attn_fwd on torch tensors q [heads][q_pad][dim], k, v [kv_heads][k_pad][dim], o [n_q][width]; with
    workspace (a tensor, or None for none), mako_attn_fwd_ws."""
    a = attn_args(n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv_heads, q_pos0=q_pos0,
                  block=block, dim=dim, scale=scale, width=width)
    if isinstance(workspace, str):
        _check(lib().mako_attn_fwd(ctypes.byref(a), dim, dtype_code(q), dtype_code(o), _ptr(q), _ptr(k), _ptr(v),
                                   _ptr(o), _ptr(lse), _stream(stream)))
    else:
        _check(lib().mako_attn_fwd_ws(ctypes.byref(a), dim, dtype_code(q), dtype_code(o), _ptr(q), _ptr(k), _ptr(v),
                                      _ptr(o), _ptr(lse), _ptr(workspace), _nbytes(workspace), _stream(stream)))


def release(stream=None):
    """mako_attn_release: frees the workspaces the library keeps for the stream."""
    _check(lib().mako_attn_release(_stream(stream)))


def held_bytes():
    """mako_attn_held_bytes: bytes of the workspaces the library keeps on the current device."""
    return lib().mako_attn_held_bytes()


def cube_select_workspace(heads, n_cubes):
    return lib().mako_cube_select_workspace(heads, n_cubes)


def cube_select(q, k, cnt, sel, nsel, workspace, *, heads, q_pad, k_pad, n_cubes, topk, local=0, stride=0,
                stream=None):
    _check(lib().mako_cube_select(heads, q_pad, k_pad, n_cubes, topk, local, stride, dtype_code(q), _ptr(q), _ptr(k),
                                  _ptr(cnt), _ptr(sel), _ptr(nsel), _ptr(workspace),
                                  0 if workspace is None else workspace.numel() * workspace.element_size(),
                                  _stream(stream)))


def sparse_args(*, n_q, q_pad, n_k, k_pad, heads, kv_heads, n_cubes, max_sel, dense0, dense1, causal=0,
                sel_heads=None, width=None):
    width = heads * 128 if width is None else width
    sel_heads = heads if sel_heads is None else sel_heads
    return SparseArgs(n_q, q_pad, n_k, k_pad, heads, kv_heads, width, 1.0 / 128 ** 0.5, n_cubes, max_sel, dense0,
                      dense1, causal, sel_heads)


def attn_sparse_workspace(**kw):
    return lib().mako_attn_sparse_workspace(ctypes.byref(sparse_args(**kw)))


def attn_sparse(q, k, v, o, sel, nsel, valid, map_, *, n_q, q_pad, n_k, k_pad, heads, kv_heads, n_cubes, max_sel,
                dense0, dense1, causal=0, sel_heads=None, width=None, lse=None, stream=None, workspace=LIBRARY):
    a = sparse_args(n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad, heads=heads, kv_heads=kv_heads, n_cubes=n_cubes,
                    max_sel=max_sel, dense0=dense0, dense1=dense1, causal=causal, sel_heads=sel_heads, width=width)
    ptrs = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(sel), _ptr(nsel), _ptr(valid), _ptr(map_), _ptr(lse))
    if isinstance(workspace, str):
        _check(lib().mako_attn_sparse(ctypes.byref(a), dtype_code(q), dtype_code(o), *ptrs, _stream(stream)))
    else:
        _check(lib().mako_attn_sparse_ws(ctypes.byref(a), dtype_code(q), dtype_code(o), *ptrs, _ptr(workspace),
                                         _nbytes(workspace), _stream(stream)))


def decode_args(*, batch, heads, kv_heads, dim, cap, max_ctx, split=0, scale=None):
    scale = 1.0 / dim ** 0.5 if scale is None else scale
    return DecodeArgs(batch, heads, kv_heads, dim, cap, max_ctx, split, scale)


def decode_workspace(a):
    return lib().mako_attn_decode_workspace(ctypes.byref(a))


def attn_decode(a, q, k, v, ctx_len, o, workspace, *, lse=None, stream=None):
    _check(lib().mako_attn_decode(ctypes.byref(a), dtype_code(q), dtype_code(o), _ptr(q), _ptr(k), _ptr(v),
                                  _ptr(ctx_len), _ptr(o), _ptr(lse), _ptr(workspace),
                                  0 if workspace is None else workspace.numel() * workspace.element_size(),
                                  _stream(stream)))


def attn_decode_noalloc(a, q, k, v, ctx_len, o, *, lse=None, stream=None):
    """mako_attn_decode_noalloc: mako_attn_decode with the partials in the library's static device scratch."""
    _check(lib().mako_attn_decode_noalloc(ctypes.byref(a), dtype_code(q), dtype_code(o), _ptr(q), _ptr(k), _ptr(v),
                                          _ptr(ctx_len), _ptr(o), _ptr(lse), _stream(stream)))


DECODE_SCRATCH_BYTES = 16 << 20  # MAKO_DECODE_SCRATCH_BYTES


def window_random_blocks(n_blocks, lists, window=8, n_random=8, seed=0):
    """Block lists for causal block-sparse attention over n_blocks 64-row blocks: block qb attends itself (the
    diagonal, causally masked inside), the `window` blocks before it, and `n_random` distinct blocks drawn
    uniformly from the earlier ones (fewer when fewer exist), for each of `lists` lists (one per kv head).
    Returns (sel u16 [lists][n_blocks][1 + window + n_random], nsel u16 [lists][n_blocks]) as numpy arrays."""
    import numpy as np

    rng = np.random.default_rng(seed)
    width = 1 + window + n_random
    sel = np.zeros((lists, n_blocks, width), np.uint16)
    nsel = np.zeros((lists, n_blocks), np.uint16)
    for li in range(lists):
        for qb in range(n_blocks):
            picks = [qb] + list(range(qb - 1, max(qb - 1 - window, -1), -1))
            early = qb - window
            if early > 0:
                picks += sorted(rng.choice(early, size=min(n_random, early), replace=False).tolist())
            sel[li, qb, :len(picks)] = picks
            nsel[li, qb] = len(picks)
    return sel, nsel


def heads(x, y, *, rows, ld, col0, stride, dim, heads, n_pad, row0=0, rope=0, rot=0, eps=0.0, clear=0, cs=None,
          w=None, map_=None, stream=None):
    """mako_heads on torch tensors: x float32 rows, y [heads][n_pad][dim] f16 or bf16, cs float32 [*][rot / 2][2],
    w float32 [dim], map_ int32 [rows]."""
    a = HeadsArgs(rows, ld, col0, stride, dim, heads, n_pad, row0, rope, rot, eps, clear)
    _check(lib().mako_heads(ctypes.byref(a), dtype_code(y), _ptr(x), _ptr(cs), _ptr(w), _ptr(map_), _ptr(y),
                            _stream(stream)))


def attn_fwd_rows_workspace(*, n_q, n_k, heads, kv_heads, q_pos0, block, dim, scale=None, width=None):
    a = attn_args(n_q=n_q, q_pad=0, n_k=n_k, k_pad=0, heads=heads, kv_heads=kv_heads, q_pos0=q_pos0, block=block,
                  dim=dim, scale=scale, width=width)
    return lib().mako_attn_fwd_rows_workspace(ctypes.byref(a), dim)


def attn_fwd_rows(xq, xk, xv, o, hq, hk, hv, *, n_q, n_k, heads, kv_heads, q_pos0, block, in_dtype, cs=None,
                  wq=None, wk=None, lse=None, scale=None, width=None, stream=None, workspace=LIBRARY):
    """mako_attn_fwd_rows on torch tensors: xq, xk, xv float32 rows; hq, hk, hv dicts of mako_heads_args fields
    (rows, ld, col0, stride, dim, heads, rope, rot, eps); o [n_q][width] of float32 or in_dtype (F16 / BF16); with
    workspace (a tensor, or None), mako_attn_fwd_rows_ws."""
    dim = hq["dim"]
    a = attn_args(n_q=n_q, q_pad=0, n_k=n_k, k_pad=0, heads=heads, kv_heads=kv_heads, q_pos0=q_pos0, block=block,
                  dim=dim, scale=scale, width=width)
    fields = ("rows", "ld", "col0", "stride", "dim", "heads", "n_pad", "row0", "rope", "rot", "eps", "clear")
    hs = [HeadsArgs(*[h.get(f, 0) for f in fields]) for h in (hq, hk, hv)]
    args = [ctypes.byref(a), *[ctypes.byref(h) for h in hs], in_dtype, dtype_code(o), _ptr(xq), _ptr(xk), _ptr(xv),
            _ptr(cs), _ptr(wq), _ptr(wk), _ptr(o), _ptr(lse)]
    if isinstance(workspace, str):
        _check(lib().mako_attn_fwd_rows(*args, _stream(stream)))
    else:
        _check(lib().mako_attn_fwd_rows_ws(*args, _ptr(workspace), _nbytes(workspace), _stream(stream)))


def attn_pv(p, kv, partial, *, heads, dim, n_kv, keys_per_split, stream=None):
    """mako_attn_pv: p float32 [heads][n_kv], kv float16 [*][dim], partial float32 [splits][heads][dim]."""
    a = PvArgs(heads, dim, n_kv, keys_per_split)
    _check(lib().mako_attn_pv(ctypes.byref(a), _ptr(p), _ptr(kv), _ptr(partial), _stream(stream)))


def attn_gather_scores(q, kv, list_, count, scores, *, heads, dim, stride, tokens, splits=1, stream=None):
    """mako_attn_gather_scores: q float16 [tokens][heads][dim], list_ / count int32 (read as u32), scores float32
    [tokens][heads][stride]."""
    a = GatherArgs(heads, dim, stride, splits, tokens)
    _check(lib().mako_attn_gather_scores(ctypes.byref(a), _ptr(q), _ptr(kv), _ptr(list_), _ptr(count), _ptr(scores),
                                         _stream(stream)))


def attn_gather_pv(p, kv, list_, count, partial, *, heads, dim, stride, splits, tokens, stream=None):
    """mako_attn_gather_pv: p float32 [tokens][heads][stride], partial float32 [splits][tokens][heads][dim]."""
    a = GatherArgs(heads, dim, stride, splits, tokens)
    _check(lib().mako_attn_gather_pv(ctypes.byref(a), _ptr(p), _ptr(kv), _ptr(list_), _ptr(count), _ptr(partial),
                                     _stream(stream)))


def idx_dots(q, pooled, dots, *, tokens, heads, dim, pools, stride, stream=None):
    """mako_idx_dots: q float32 [tokens][heads][dim], pooled float32 [pools][dim], dots float32
    [tokens][heads][stride]."""
    a = IdxDotArgs(heads, dim, pools, stride)
    _check(lib().mako_idx_dots(ctypes.byref(a), tokens, _ptr(q), _ptr(pooled), _ptr(dots), _stream(stream)))


def proj_bf16(w, x, y, *, t, k, n, ldx=0, ldy=0, split=0, stream=None):
    """mako_proj_bf16: w bfloat16 [n][k], x float32 or bfloat16 [t][ldx], y float32 [t][ldy]."""
    a = GemmArgs(t, k, n, 2 * k, ldy, ldx)
    _check(lib().mako_proj_bf16(ctypes.byref(a), dtype_code(x), split, _ptr(w), _ptr(x), _ptr(y), _stream(stream)))


def kda_scan(q, k, v, g, beta, state, o, *, tokens, heads, qkv_stride=None, inner=None, snap=0, snap_state=None,
             head_dim=128, stream=None):
    """mako_kda_scan: float32 q, k, v rows qkv_stride apart, g and o rows inner apart, beta [tokens][heads], state
    [heads][head_dim][head_dim] (transposed, updated in place)."""
    a = ScanArgs(head_dim, tokens, qkv_stride or heads * head_dim, inner or heads * head_dim, heads, snap)
    _check(lib().mako_kda_scan(ctypes.byref(a), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(state), _ptr(o),
                               _ptr(snap_state), _stream(stream)))
