"""The gated delta rule (mako_kda_scan, the reference's kda_scan) on the GPU against the CPU oracle: the inputs the
linear-attention layers feed it (q and k L2-normalised per head, v normal, g a log-decay in [-0.5, 0], beta in
(0, 1)), a nonzero starting state, strided rows, the rollback snapshot (after the first token, the last, and at a
boundary of the kernel's 16-token batches), token counts one past and one short of a batch multiple, no tokens,
and the Qwen3.5 shape (32 heads of 128 over 4096 tokens, four heads checked).

Tolerance: the oracle runs in double; the kernel in f32 with a different summation order (8 values a lane, then a
16-lane tree) and the hardware exponential. Every output and state element within 2e-5 + 1e-4 |ref| (the f32
rounding of 128-term sums carried through the recurrence stays well inside it at these lengths).
"""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import mako_attn as M  # noqa: E402

ATOL, RTOL = 2e-5, 1e-4
D = 128


def inputs(rng, T, H, ld=None, scale_state=0.0):
    ld = ld or H * D
    unit = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)

    def rows(x):
        out = np.zeros((T, ld), np.float32)
        out[:, :H * D] = x.reshape(T, H * D)
        return out

    q = rows(unit(rng.standard_normal((T, H, D))))
    k = rows(unit(rng.standard_normal((T, H, D))))
    v = rows(rng.standard_normal((T, H, D)))
    g = rows(rng.uniform(-0.5, 0.0, (T, H, D)))
    beta = rng.uniform(0.05, 0.95, (T, H)).astype(np.float32)
    state = (rng.standard_normal((H, D, D)) * scale_state).astype(np.float32)
    return q, k, v, g, beta, state


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def assert_close(got, want, what):
    err = np.abs(np.asarray(got, np.float64) - want)
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} beyond tolerance, worst {err.max():.3e} at "
                           f"{np.unravel_index(np.argmax(err), err.shape)} (ref {want.flat[np.argmax(err)]:.4e})")


def run(q, k, v, g, beta, state, *, T, H, ld=None, snap=0):
    ld = ld or H * D
    o = torch.full((max(T, 1), ld), 7.0, dtype=torch.float32, device="cuda")
    st = dev(state)
    snap_d = torch.zeros((H, D, D), dtype=torch.float32, device="cuda") if snap else None
    print(f"kda_scan T={T} H={H} ld={ld} snap={snap}", flush=True)
    M.kda_scan(dev(q), dev(k), dev(v), dev(g), dev(beta), st, o, tokens=T, heads=H, qkv_stride=ld, inner=ld,
               snap=snap, snap_state=snap_d)
    torch.cuda.synchronize()
    return o.cpu().numpy(), st.cpu().numpy(), (snap_d.cpu().numpy() if snap else None)


@pytest.mark.parametrize("T,H,ld,snap", [(200, 4, 0, 0), (37, 2, 320, 20), (1, 1, 0, 1), (16, 3, 0, 16),
                                         (17, 2, 0, 17), (33, 1, 0, 32), (47, 3, 400, 1), (31, 2, 0, 0)],
                         ids=["t200h4", "t37h2_strided_snap20", "t1", "t16h3_snap16", "t17h2_snap_last",
                              "t33h1_snap_batch_edge", "t47h3_strided_snap_first", "t31h2"])
def test_kda_scan(T, H, ld, snap):
    rng = np.random.default_rng(T * 7 + H)
    q, k, v, g, beta, state = inputs(rng, T, H, ld or None, scale_state=0.3)
    o, st, sn = run(q, k, v, g, beta, state, T=T, H=H, ld=ld or None, snap=snap)
    ldx = ld or H * D
    want_o, want_st, want_sn = O.kda_scan(q, k, v, g, beta, state.astype(np.float64), tokens=T, heads=H,
                                          qkv_stride=ldx, inner=ldx, snap=snap, o=np.full((T, ldx), 7.0))
    assert_close(o[:T], want_o, "o")
    assert_close(st, want_st, "state")
    if snap:
        assert_close(sn, want_sn, "snapshot")


def test_strong_decays_and_growth():
    """Batches whose decays leave the kernel's rescaling range run unscaled: a channel decaying by -4 a token for a
    whole batch (-64 over it), single tokens at -50, a channel growing by +3 a token (+48), and weak batches between
    (rescaled); the last batch partial."""
    rng = np.random.default_rng(77)
    T, H = 91, 2
    q, k, v, g, beta, state = inputs(rng, T, H, scale_state=0.3)
    g[16:32, 5] = -4.0                   # batch 1: a channel at -64 over the batch
    g[40, D + 7] = -50.0                 # batch 2: one token, one channel
    g[70, :D] = -50.0                    # batch 4: one token, every channel of head 0
    g[48:64, D + 9] = 3.0                # batch 3: growth, +48 over the batch
    o, st, _ = run(q, k, v, g, beta, state, T=T, H=H)
    want_o, want_st, _ = O.kda_scan(q, k, v, g, beta, state.astype(np.float64), tokens=T, heads=H)
    assert_close(o[:T], want_o, "o")
    assert_close(st, want_st, "state")


def test_no_tokens_leaves_the_state():
    rng = np.random.default_rng(3)
    q, k, v, g, beta, state = inputs(rng, 1, 2, scale_state=1.0)
    _, st, _ = run(q, k, v, g, beta, state, T=0, H=2)
    assert np.array_equal(st, state)


def test_qwen35_linear_attention_shape():
    """32 heads of 128 over 4096 tokens (the linear-attention layers of Qwen3.5's encoder,
    src/models/qwen_text.cpp:374-382: qkv_stride = inner = 32 * 128, state zeroed): four heads against the oracle."""
    rng = np.random.default_rng(35)
    T, H = 4096, 32
    q, k, v, g, beta, state = inputs(rng, T, H)
    o, st, _ = run(q, k, v, g, beta, np.zeros_like(state), T=T, H=H)
    for h in (0, 9, 22, 31):
        sl = slice(h * D, (h + 1) * D)
        want_o, want_st, _ = O.kda_scan(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, h:h + 1], tokens=T, heads=1)
        assert_close(o[:, sl], want_o, f"o head {h}")
        assert_close(st[h], want_st[0], f"state head {h}")
