"""CPU checks of flash_fwd_r64's generated instruction stream (mako-common_amd/csrc/gen_attn_fwd64.py), for heads of
128 and of 64: every register it names is one its clobber list reserves; no gfx950 software hazard in any of its
type variants; and,
on an instruction-level emulator (tests/fwd64_emu.py), outputs and LSE within the attention tolerance of the oracle
with the LDS bank conflicts it allows (LDS_WORST): causal GQA with a query offset and ragged sizes, bidirectional over eleven tiles,
prefix-causal, f16 in and out, and inputs whose growing scores send most tiles down the exact path. Two planted
mistakes show the checks have teeth: a dropped wait state after an M0 write, and barriers that let V tiles be read
before their loads land. The V^T operands come from V's rows in LDS by transpose reads (ds_read_b64_tr_b16), whose
lane layout the emulator restates as measured on the GPU. The emulator also counts LDS reads that sample bytes an LDS
DMA load in flight has not yet written, and every case requires none: a K tile read early is otherwise healed in the
emulator (its garbage scores fail the row-sum check and the exact path recomputes the tile once it has landed), while
on the GPU it would read the buffer's previous tile. The MHA causal case has waves three tiles apart in a workgroup,
where a wave's last iteration must still stage its share of tile j + 3 for the others.
The block-sparse stream (flash_sparse_r64) gets the same register and hazard checks, and emulated shared-list cases
(invalid keys, dense rows, rows past n_q, a map that drops rows; causal and not) against the oracle through the pass
table restated in tests/sparse64_run.py, with a planted mistake in its validity masks."""
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "mako-common_amd", "csrc"))
import fwd64_emu as E  # noqa: E402
import fwd64_hazards as Hz  # noqa: E402
import fwd64_run as R  # noqa: E402
import gen_attn_fwd64 as G  # noqa: E402

U32 = 0xFFFFFFFF
VARIANTS = [("bf16", "f32"), ("bf16", "bf16"), ("f16", "f32"), ("f16", "f16")]


@pytest.mark.parametrize("ind,outd", VARIANTS)
def test_registers_and_hazards(ind, outd):
    lines = G.body(ind, outd)
    G.check_registers(lines)
    assert Hz.check(lines, f"{ind}->{outd}") == 0


# LDS bank-conflict multiplicities allowed (the emulator's model, which SQ_LDS_BANK_CONFLICT bears out): the
# epilogue's 8-byte writes (2-byte outputs) meet 2-way, sixteen lanes of one write covering rows with eight distinct
# chunk slots; the V^T transpose reads at 128 head dims 2-way, a 32-lane pass covering the 32 banks of half a row
# twice (v_unit; at 64 head dims two rows share the 64 banks and the pass covers them once). A layout without the
# conflict needs four read-address registers instead of two; on the heads-of-256 stream it measured under 1 %.
# Every other LDS access is conflict-free.
LDS_WORST = {"ds_write_b64": 2, "ds_read_b64_tr_b16": 2}

CASES = [
    dict(heads=8, kv=2, S_q=100, S_k=330, q_pos0=230, block=U32, seed=1),
    dict(heads=4, kv=1, S_q=64, S_k=700, q_pos0=0, block=0, seed=2),
    dict(heads=2, kv=1, S_q=130, S_k=300, q_pos0=150, block=250, seed=5),
    dict(heads=4, kv=4, S_q=70, S_k=300, q_pos0=200, block=U32, ind="f16", outd="f16", seed=3),
    dict(heads=4, kv=1, S_q=64, S_k=130, q_pos0=0, block=U32, ind="bf16", outd="bf16", seed=4),
    # growing scores: most tiles take the exact path. P is rounded to the input type, and with bf16's 8 significant
    # bits a softmax this peaked (a few keys of weight ~1 whose values cancel) leaves the tolerance at growth 0.8
    # and above (tests/test_gpu_fwd.py checks bf16 P against its rounding bound there); f16 P at the full growth
    dict(heads=4, kv=1, S_q=64, S_k=448, q_pos0=0, block=0, seed=7, kgrow=1.5, ind="f16"),
    dict(heads=4, kv=1, S_q=64, S_k=448, q_pos0=0, block=0, seed=7, kgrow=0.5),
    # one query head a kv head: a workgroup's four waves hold rows 64 apart, so their last tiles differ by up to three
    dict(heads=1, kv=1, S_q=512, S_k=512, q_pos0=0, block=U32, seed=3),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_stream_matches_oracle(case):
    taken = E.EXACT_COUNT[0]
    r = R.run(**case, verbose=False)
    assert r["out_bad"] == 0 and r["lse_bad"] == 0 and r["early_reads"] == 0, r
    assert all(m <= LDS_WORST.get(op, 1) for op, m in r["lds_worst"].items()), r["lds_worst"]
    if case.get("kgrow"):
        assert E.EXACT_COUNT[0] > taken  # the exact path ran


@pytest.mark.parametrize("ind,outd", VARIANTS)
def test_d64_registers_and_hazards(ind, outd):
    lines = G.body(ind, outd, d=64)
    G.check_registers(lines)
    assert Hz.check(lines, f"d64 {ind}->{outd}") == 0


# heads of 64: the same stream with half the head dimensions (9 KiB K images, 8 KiB V^T images, 32 MFMAs a tile)
CASES_D64 = [
    dict(heads=4, kv=1, S_q=64, S_k=300, q_pos0=0, block=0, seed=2),
    dict(heads=8, kv=2, S_q=100, S_k=330, q_pos0=230, block=U32, seed=1),
    dict(heads=4, kv=4, S_q=70, S_k=300, q_pos0=200, block=U32, ind="f16", outd="f16", seed=3),
    dict(heads=2, kv=1, S_q=130, S_k=300, q_pos0=150, block=250, ind="bf16", outd="bf16", seed=5),
    dict(heads=4, kv=1, S_q=64, S_k=448, q_pos0=0, block=0, seed=7, kgrow=1.5, ind="f16"),
    dict(heads=4, kv=1, S_q=64, S_k=448, q_pos0=0, block=0, seed=7, kgrow=0.5),
    dict(heads=2, kv=1, S_q=3, S_k=0, q_pos0=0, block=U32, seed=8),       # no keys: 0 and lse = -inf
    dict(heads=8, kv=2, S_q=40, S_k=5, q_pos0=0, block=U32, seed=9),      # fewer keys than queries
]


@pytest.mark.parametrize("case", CASES_D64, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_d64_stream_matches_oracle(case):
    taken = E.EXACT_COUNT[0]
    r = R.run(**case, d=64, verbose=False)
    assert r["out_bad"] == 0 and r["lse_bad"] == 0 and r["early_reads"] == 0, r
    assert all(m <= (1 if op == "ds_read_b64_tr_b16" else LDS_WORST.get(op, 1)) for op, m in r["lds_worst"].items()), \
        r["lds_worst"]
    if case.get("kgrow"):
        assert E.EXACT_COUNT[0] > taken  # the exact path ran


def test_planted_missing_wait_state_is_found():
    lines = G.body("bf16", "f32")
    i = next(i for i, ln in enumerate(lines) if ln.startswith("s_mov_b32 m0"))
    assert lines[i + 1] == "s_nop 0"
    assert Hz.check(lines[:i + 1] + lines[i + 2:], "planted") > 0


def test_planted_barrier_without_lds_wait_is_found(monkeypatch):
    """Phase PV's barrier must follow the landing of its V^T reads: without the lgkmcnt(0), another wave's staging
    after the barrier overwrites the buffer those reads still sample."""
    monkeypatch.setattr(G, "barrier", lambda: [f"s_waitcnt vmcnt({G.DMA_PER_TILE})", "s_barrier"])
    r = R.run(4, 1, 64, 448, 0, 0, seed=9, verbose=False)
    assert r["out_bad"] > 0


def test_planted_short_barrier_wait_is_found(monkeypatch):
    monkeypatch.setattr(G, "barrier", lambda: [f"s_waitcnt vmcnt({3 * G.DMA_PER_TILE}) lgkmcnt(0)", "s_barrier"])
    r = R.run(4, 1, 64, 448, 0, 0, seed=9, verbose=False)
    assert r["out_bad"] > 0 and r["early_reads"] > 0


def test_planted_last_iteration_without_staging_is_found(monkeypatch):
    """A wave whose last iteration leaves out its share of tile j + 3 (staging then falls a barrier behind) lets the
    longer waves of an MHA workgroup read K tiles before they land: counted as early reads."""
    monkeypatch.setattr(G, "iteration_last_staging", lambda: [])
    r = R.run(heads=1, kv=1, S_q=512, S_k=512, q_pos0=0, block=U32, seed=3, verbose=False)
    assert r["early_reads"] > 0


# ---- the block-sparse stream (flash_sparse_r64: tiles, masks and output rows from the pass table and the row map) ----

@pytest.mark.parametrize("ind,outd", VARIANTS)
def test_sparse_registers_and_hazards(ind, outd):
    lines = G.body(ind, outd, sparse=True)
    G.check_registers(lines, sparse=True)
    assert Hz.check(lines, f"sparse {ind}->{outd}") == 0


def shared_lists_case(causal, seed):
    """8 query heads over 2 kv heads, 5 cubes (one with 37 valid rows), 40 dense rows, rows past n_q and a map that
    drops rows (tests/test_gpu_sparse.py's shared-lists case at its small size)."""
    import numpy as np

    heads, kv, cubes, dense, topk = 8, 2, 5, 40, 3
    cnt = np.array([64, 64, 37, 64, 64])
    n = cubes * 64 + dense
    q_pad, k_pad = (n + 63) // 64 * 64, (n + 127) // 128 * 128
    n_q = n - 10
    valid = np.zeros(k_pad, np.uint8)
    for c in range(cubes):
        valid[c * 64:c * 64 + cnt[c]] = 1
    valid[cubes * 64:n] = 1
    map_ = np.full(q_pad, -1, np.int32)
    keep = np.nonzero(valid[:n_q])[0]
    map_[keep] = np.arange(len(keep), dtype=np.int32)
    map_[keep[::7]] = -1
    rng = np.random.default_rng(seed)
    sel = np.zeros((kv, cubes, topk), np.uint16)
    nsel = np.zeros((kv, cubes), np.uint16)
    for h in range(kv):
        for c in range(cubes):
            ch = rng.permutation(np.arange(c + 1) if causal else np.arange(cubes))[:topk]
            sel[h, c, :len(ch)] = ch
            nsel[h, c] = len(ch)
    return (heads, kv, sel, nsel, valid, map_), dict(n_q=n_q, q_pad=q_pad, n_k=n, k_pad=k_pad, n_cubes=cubes,
                                                     max_sel=topk, dense0=cubes * 64, dense1=n, causal=causal)


@pytest.mark.parametrize("causal,ind,outd", [(0, "bf16", "f32"), (1, "f16", "f16")])
def test_sparse_stream_matches_oracle(causal, ind, outd):
    import sparse64_run as SR

    args, kw = shared_lists_case(causal, 41 + causal)
    r = SR.run(*args, **kw, ind=ind, outd=outd, verbose=False)
    assert r == dict(out_bad=0, lse_bad=0, untouched=0, early_reads=0), r


def test_sparse_planted_mask_shift_is_found(monkeypatch):
    """Validity words shifted by a wrong amount (another operand's register in place of 32 g) mask the wrong keys."""
    import sparse64_run as SR

    monkeypatch.setattr(G, "mask_general", lambda sbuf, j0, w, f=G.mask_general: [
        op.replace("%[g32]", "%[mo]") for op in f(sbuf, j0, w)])
    args, kw = shared_lists_case(0, 41)
    r = SR.run(*args, **kw, verbose=False)
    assert r["out_bad"] > 0


def test_planted_missing_low_part_pass_is_found(monkeypatch):
    """bf16 P alone leaves rows that see a handful of keys outside the tolerance (errors of ~2^-9 |v| on small
    outputs); the low-part pass over tile 0 is what keeps them within it."""
    monkeypatch.setattr(G, "low_part_pass", lambda e: None)
    r = R.run(heads=8, kv=2, S_q=40, S_k=5, q_pos0=0, block=U32, seed=9, d=64, verbose=False)
    assert r["out_bad"] > 0


def test_planted_missing_q_wait_is_found(monkeypatch):
    """Tile 0's score MFMAs start while Q is still arriving: without the per-pair waits they read Q registers whose
    loads have not landed."""
    monkeypatch.setattr(G, "q_waits", lambda mfmas, n_groups: {})
    r = R.run(4, 1, 64, 200, 0, 0, seed=9, verbose=False)
    assert r["out_bad"] > 0


def test_planted_q_waits_that_miscount_the_early_dma_are_found(monkeypatch):
    """Tiles 1 and 2 are staged between tile 0's score MFMAs, so a Q wait counts only the DMA loads issued before
    it. Waits that count all of them (as when both tiles went out ahead of Q) let MFMAs read Q before it lands."""
    monkeypatch.setattr(G, "q_waits", lambda mfmas, n_groups: {
        2 * kk: [f"s_waitcnt vmcnt({2 * (G.NKK - 1 - kk) + n_groups})"] for kk in range(G.NKK)})
    r = R.run(4, 1, 64, 200, 0, 0, seed=9, verbose=False)
    assert r["out_bad"] > 0
