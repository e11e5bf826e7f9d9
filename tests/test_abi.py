"""The C ABI without a GPU: the library loads, exports every function include/mako_attn.h declares, reports its
ABI version, and refuses bad arguments (with the reference's messages) before touching the device."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

import mako_attn as M

HEADER = os.path.join(ROOT, "include", "mako_attn.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*)\s+(mako_\w+)\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared() == sorted(M.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = M.lib()
    for name in declared():
        assert hasattr(L, name), f"{name} is declared in include/mako_attn.h but not exported"
    assert L.mako_attn_abi_version() == 1


def test_host_library_loads():
    """The C++ host side (libmako_host.so) loads and resolves against libmako_attn.so."""
    path = os.path.join(ROOT, "mako-common_amd", "lib", "libmako_host.so")
    assert os.path.exists(path)
    ctypes.CDLL(path)


FAKE = ctypes.c_void_p(0x10000)  # aligned, never dereferenced: every call below fails validation first


def fwd_rc(**kw):
    a = dict(n_q=64, q_pad=64, n_k=64, k_pad=128, heads=4, kv_heads=2, q_pos0=0, block=0xFFFFFFFF, width=512,
             scale=0.088)
    a.update(kw.pop("args", {}))
    args = M.AttnArgs(*[a[f] for f, _ in M.AttnArgs._fields_])
    dim = kw.pop("dim", 128)
    i, o = kw.pop("in_", M.BF16), kw.pop("out", M.BF16)
    ptrs = [kw.pop(n, FAKE) for n in ("q", "k", "v", "o")]
    rc = M.lib().mako_attn_fwd(ctypes.byref(args), dim, i, o, *ptrs, None, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dim=96), M.EUNSUPPORTED, "attention: heads of 96"),
    (dict(in_=M.F32), M.EUNSUPPORTED, "input type"),
    (dict(out=M.F16), M.EUNSUPPORTED, "output type"),
    (dict(args=dict(heads=5)), M.EINVAL, "heads over"),
    (dict(args=dict(n_q=65)), M.EINVAL, "queries in"),
    (dict(args=dict(n_k=129)), M.EINVAL, "keys in"),
    (dict(args=dict(width=256)), M.EINVAL, "o rows"),
    (dict(q=None), M.EINVAL, "null"),
    (dict(k=ctypes.c_void_p(0x10002)), M.EINVAL, "aligned"),
    (dict(args=dict(scale=0.0)), M.EINVAL, "scale"),
    (dict(args=dict(scale=-0.088)), M.EINVAL, "scale"),
])
def test_fwd_refuses(kw, code, msg):
    rc, err = fwd_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def sparse_rc(**kw):
    a = dict(n_q=64, q_pad=64, n_k=128, k_pad=128, heads=4, kv_heads=2, width=512, scale=0.088, n_cubes=1, max_sel=1,
             dense0=0, dense1=0, causal=1, sel_heads=4)
    a.update(kw)
    args = M.SparseArgs(*[a[f] for f, _ in M.SparseArgs._fields_])
    rc = M.lib().mako_attn_sparse(ctypes.byref(args), M.BF16, M.BF16, *([FAKE] * 8), None, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(q_pad=65), M.EINVAL, "multiple of 64"),
    (dict(heads=3), M.EINVAL, "heads over"),
    (dict(sel_heads=3), M.EINVAL, "sel rows"),
    (dict(n_cubes=3), M.EINVAL, "cubes of"),
    (dict(width=100), M.EINVAL, "o rows"),
    (dict(scale=0.0), M.EINVAL, "scale"),
])
def test_sparse_refuses(kw, code, msg):
    rc, err = sparse_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def decode_rc(**kw):
    a = dict(batch=2, heads=8, kv_heads=2, dim=128, cap=256, max_ctx=256, split=0, scale=0.088)
    a.update(kw)
    args = M.DecodeArgs(*[a[f] for f, _ in M.DecodeArgs._fields_])
    rc = M.lib().mako_attn_decode(ctypes.byref(args), M.BF16, M.BF16, *([FAKE] * 6), FAKE, 1 << 20, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(dim=64), M.EUNSUPPORTED, "heads of 64"),
    (dict(heads=7), M.EINVAL, "kv heads"),
    (dict(max_ctx=512), M.EINVAL, "max_ctx"),
    (dict(split=100), M.EINVAL, "a split"),
    (dict(scale=float("inf")), M.EINVAL, "scale"),
])
def test_decode_refuses(kw, code, msg):
    rc, err = decode_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def heads_rc(**kw):
    a = dict(rows=64, ld=4096, col0=0, stride=128, dim=128, heads=32, n_pad=64, row0=0, rope=1, rot=128, eps=1e-6,
             clear=0)
    a.update(kw.pop("args", {}))
    args = M.HeadsArgs(*[a[f] for f, _ in M.HeadsArgs._fields_])
    out = kw.pop("out", M.BF16)
    ptrs = [kw.pop(n, FAKE) for n in ("x", "cs", "w")]
    rc = M.lib().mako_heads(ctypes.byref(args), out, *ptrs, None, FAKE, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(out=M.F32), M.EUNSUPPORTED, "output type"),
    (dict(args=dict(dim=288, ld=1 << 16)), M.EINVAL, "heads of 288"),   # the reference: dim > 256
    (dict(args=dict(dim=100)), M.EINVAL, "heads of 100"),               # the reference: dim % 32
    (dict(args=dict(rot=95)), M.EINVAL, "95 rotated"),                  # the reference: odd rot
    (dict(args=dict(rope=3)), M.EINVAL, "rope 3"),
    (dict(args=dict(rot=160)), M.EINVAL, "over 160"),
    (dict(cs=None), M.EINVAL, "angle table"),
    (dict(w=None), M.EINVAL, "without a weight"),
    (dict(args=dict(eps=-1.0)), M.EINVAL, "eps"),
    (dict(args=dict(row0=8)), M.EINVAL, "exceed 64"),
    (dict(args=dict(col0=1)), M.EINVAL, "exceed rows of 4096"),
    (dict(x=None), M.EINVAL, "null"),
])
def test_heads_refuses(kw, code, msg):
    rc, err = heads_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def rows_rc(**kw):
    """mako_attn_fwd_rows with the Qwen3-8B step's arguments (64 tokens) and fake device pointers, changed by kw."""
    a = dict(n_q=64, q_pad=0, n_k=64, k_pad=0, heads=32, kv_heads=8, q_pos0=0, block=0xFFFFFFFF, width=4096,
             scale=0.088)
    a.update(kw.pop("attn", {}))
    base = dict(rows=64, ld=4096, col0=0, stride=128, dim=128, heads=32, n_pad=0, row0=0, rope=1, rot=128, eps=1e-6,
                clear=0)
    hs = []
    for name, extra in (("hq", {}), ("hk", dict(ld=1024, heads=8)),
                        ("hv", dict(ld=1024, heads=8, rope=0, rot=0, eps=0.0))):
        h = dict(base, **extra)
        h.update(kw.pop(name, {}))
        hs.append(M.HeadsArgs(*[h[f] for f, _ in M.HeadsArgs._fields_]))
    args = M.AttnArgs(*[a[f] for f, _ in M.AttnArgs._fields_])
    ins, out = kw.pop("in_", M.BF16), kw.pop("out", M.F32)
    ptrs = [kw.pop(n, FAKE) for n in ("xq", "xk", "xv", "cs", "wq", "wk", "o")]
    rc = M.lib().mako_attn_fwd_rows(ctypes.byref(args), *[ctypes.byref(h) for h in hs], ins, out, *ptrs, None, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(o=None), M.EINVAL, "null"),
    (dict(hk=dict(dim=64)), M.EINVAL, "heads of 128, 64"),
    (dict(hq=dict(heads=16)), M.EINVAL, "16 / 8 / 8 heads produced for 32 over 8"),
    (dict(hv=dict(rows=60)), M.EINVAL, "64 / 64 / 60 rows produced"),
    (dict(in_=M.F32), M.EUNSUPPORTED, "input type"),
    (dict(attn=dict(scale=0.0)), M.EINVAL, "scale"),
    (dict(hq=dict(rot=130)), M.EINVAL, "over 130"),
    (dict(wk=None), M.EINVAL, "without a weight"),
    (dict(hv=dict(eps=1e-6)), M.EINVAL, "without a weight"),      # the value producer takes no weight
    (dict(hk=dict(col0=4)), M.EINVAL, "exceed rows of 1024"),
    (dict(xv=None), M.EINVAL, "null"),
])
def test_rows_refuses(kw, code, msg):
    """mako_attn_fwd_rows refuses what mako_heads and mako_attn_fwd refuse, and arguments that do not describe one
    step (heads, rows or widths that disagree), before touching the device."""
    rc, err = rows_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def gather_rc(fn, **kw):
    """Calls one of the four gathered decode helpers with valid arguments but for the overrides in kw."""
    if fn == "mako_attn_pv":
        a = dict(heads=64, dim=512, n_kv=4096, keys_per_split=256)
        a.update(kw.pop("args", {}))
        args = M.PvArgs(*[a[f] for f, _ in M.PvArgs._fields_])
        ptrs = [kw.pop(n, FAKE) for n in ("p", "kv", "partial")]
    elif fn == "mako_idx_dots":
        a = dict(heads=32, dim=128, pools=100, stride=128)
        a.update(kw.pop("args", {}))
        args = M.IdxDotArgs(*[a[f] for f, _ in M.IdxDotArgs._fields_])
        ptrs = [kw.pop("tokens", 4)] + [kw.pop(n, FAKE) for n in ("q", "pooled", "dots")]
    else:
        a = dict(heads=64, dim=512, stride=2048, splits=4, tokens=4)
        a.update(kw.pop("args", {}))
        args = M.GatherArgs(*[a[f] for f, _ in M.GatherArgs._fields_])
        ptrs = [kw.pop(n, FAKE) for n in ("x", "kv", "list", "count", "out")]
    rc = getattr(M.lib(), fn)(ctypes.byref(args), *ptrs, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("fn,kw,code,msg", [
    ("mako_attn_pv", dict(args=dict(dim=96)), M.EINVAL, "heads of 96"),            # gemm.metal: TN = 64 columns
    ("mako_attn_pv", dict(args=dict(keys_per_split=100)), M.EINVAL, "100 keys a split"),  # gemm.metal:685
    ("mako_attn_pv", dict(args=dict(keys_per_split=64, n_kv=1 << 31)), M.EINVAL, "exceed the grid"),
    ("mako_attn_pv", dict(kv=ctypes.c_void_p(FAKE.value + 2)), M.EINVAL, "aligned"),
    ("mako_attn_pv", dict(p=None), M.EINVAL, "null"),
    ("mako_attn_gather_scores", dict(args=dict(heads=65)), M.EINVAL, "65 heads"),  # gemm.metal:743 heads <= 64
    ("mako_attn_gather_scores", dict(args=dict(dim=384)), M.EINVAL, "of 384"),    # gemm.metal:737 dim % 256
    ("mako_attn_gather_scores", dict(args=dict(tokens=1 << 23)), M.EINVAL, "exceed the grid"),
    ("mako_attn_gather_scores", dict(count=None), M.EINVAL, "null"),
    ("mako_attn_gather_pv", dict(args=dict(dim=320)), M.EINVAL, "of 320"),        # gemm.metal:789 dim / 128
    ("mako_attn_gather_pv", dict(args=dict(splits=0)), M.EINVAL, "0 splits"),
    ("mako_attn_gather_pv", dict(args=dict(splits=4096, tokens=1024)), M.EINVAL, "exceed the grid"),
    ("mako_attn_gather_pv", dict(list=None), M.EINVAL, "null"),
    ("mako_idx_dots", dict(args=dict(heads=33)), M.EINVAL, "33 heads"),            # gemm.metal:850 heads <= 32
    ("mako_idx_dots", dict(args=dict(stride=64)), M.EINVAL, "rows of 64"),
    ("mako_idx_dots", dict(pooled=None), M.EINVAL, "null"),
])
def test_gather_helpers_refuse(fn, kw, code, msg):
    rc, err = gather_rc(fn, **kw)
    assert rc == code and msg in err, (rc, err)


@pytest.mark.parametrize("fn,kw", [("mako_attn_pv", dict(args=dict(n_kv=0))),
                                   ("mako_attn_gather_scores", dict(args=dict(tokens=0))),
                                   ("mako_attn_gather_pv", dict(args=dict(tokens=0))),
                                   ("mako_idx_dots", dict(tokens=0))])
def test_gather_helpers_empty_is_a_no_op(fn, kw):
    """No keys or no tokens: nothing to launch, the call succeeds (no GPU needed)."""
    rc, err = gather_rc(fn, **kw)
    assert rc == M.OK, err


def proj_rc(**kw):
    a = dict(t=4096, k=4096, n=4096, row_bytes=8192, ldy=0, ldx=0)
    a.update(kw.pop("args", {}))
    args = M.GemmArgs(*[a[f] for f, _ in M.GemmArgs._fields_])
    rc = M.lib().mako_proj_bf16(ctypes.byref(args), kw.pop("x_dtype", M.BF16), kw.pop("split", 0),
                                kw.pop("w", FAKE), kw.pop("x", FAKE), kw.pop("y", FAKE), None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(args=dict(k=4000, row_bytes=8000)), M.EINVAL, "BF16 4000x4096: k must be a multiple of 64"),  # runtime.cpp:180
    (dict(x_dtype=M.F16), M.EUNSUPPORTED, "activations of type 1"),
    (dict(args=dict(row_bytes=4096)), M.EINVAL, "not 4096"),
    (dict(split=1), M.EINVAL, "split needs f32"),
    (dict(args=dict(ldx=2048)), M.EINVAL, "shorter"),
    (dict(args=dict(ldx=4100)), M.EINVAL, "ldx a multiple of 8"),
    (dict(x=ctypes.c_void_p(FAKE.value + 8)), M.EINVAL, "16-byte aligned"),
    (dict(args=dict(t=1 << 20, ldx=8192)), M.EINVAL, "exceed 2^32"),
    (dict(args=dict(t=256, ldx=1 << 23)), M.EINVAL, "too long for 32-bit tile offsets"),
    (dict(w=None), M.EINVAL, "null"),
])
def test_proj_refuses(kw, code, msg):
    rc, err = proj_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def test_proj_no_rows_is_a_no_op():
    rc, err = proj_rc(args=dict(t=0))
    assert rc == M.OK, err


def scan_rc(**kw):
    a = dict(head_dim=128, tokens=4096, qkv_stride=4096, inner=4096, heads=32, snap=0)
    a.update(kw.pop("args", {}))
    args = M.ScanArgs(*[a[f] for f, _ in M.ScanArgs._fields_])
    ptrs = [kw.pop(n, FAKE) for n in ("q", "k", "v", "g", "beta", "state", "o", "snap_state")]
    rc = M.lib().mako_kda_scan(ctypes.byref(args), *ptrs, None)
    return rc, M.lib().mako_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(args=dict(head_dim=64)), M.EUNSUPPORTED, "head_dim 64"),      # ops.metal:481 "head_dim must be 128"
    (dict(args=dict(qkv_stride=2048)), M.EINVAL, "32 heads of 128"),
    (dict(args=dict(inner=4098)), M.EINVAL, "multiples of 4"),
    (dict(k=ctypes.c_void_p(FAKE.value + 4)), M.EINVAL, "16-byte aligned"),
    (dict(args=dict(snap=5000)), M.EINVAL, "5000 of 4096"),
    (dict(args=dict(snap=5), snap_state=None), M.EINVAL, "null"),
    (dict(beta=None), M.EINVAL, "null"),
])
def test_kda_scan_refuses(kw, code, msg):
    rc, err = scan_rc(**kw)
    assert rc == code and msg in err, (rc, err)


def test_workspace_entry_points_refuse_a_short_workspace():
    """The *_ws entry points validate before the workspace; a workspace smaller than the call's query is refused
    with MAKO_EWORKSPACE before any launch (the split-K route of a one-row call needs one)."""
    args = M.attn_args(n_q=1, q_pad=64, n_k=4096, k_pad=4096, heads=32, kv_heads=8, q_pos0=4095, block=M.U32_MAX,
                       dim=128)
    need = M.lib().mako_attn_fwd_workspace(ctypes.byref(args), 128)
    if need == 0:
        pytest.skip("no GPU to size the split-K route (the query needs the compute-unit count)")
    rc = M.lib().mako_attn_fwd_ws(ctypes.byref(args), 128, M.BF16, M.BF16, *([FAKE] * 4), None, FAKE, need - 1,
                                  None)
    assert rc == M.EWORKSPACE and "workspace" in M.lib().mako_last_error().decode()


def test_workspace_queries_without_a_device():
    """The prefill routes need no workspace: the queries say 0 for them (no device needed)."""
    args = M.attn_args(n_q=4096, q_pad=4096, n_k=4096, k_pad=4096, heads=32, kv_heads=8, q_pos0=0, block=M.U32_MAX,
                       dim=128)
    assert M.lib().mako_attn_fwd_workspace(ctypes.byref(args), 128) == 0
    assert M.lib().mako_attn_fwd_workspace(ctypes.byref(args), 64) == 0
    assert M.lib().mako_attn_held_bytes() == 0
