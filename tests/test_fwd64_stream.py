"""CPU checks of flash_fwd_r64's generated instruction stream (mako-common_amd/csrc/gen_attn_fwd64.py): every
register it names is one its clobber list reserves; no gfx950 software hazard in any of its four type variants; and,
on an instruction-level emulator (tests/fwd64_emu.py), outputs and LSE within the attention tolerance of the oracle
with conflict-free LDS access: causal GQA with a query offset and ragged sizes, bidirectional over eleven tiles,
prefix-causal, f16 in and out, and inputs whose growing scores send most tiles down the exact path. Two planted
mistakes show the checks have teeth: a dropped wait state after an M0 write, and barriers that let V^T tiles be read
before their loads land. (Barriers that let only K tiles be read early are healed by the design: the garbage
scores fail the row-sum check, and the exact path recomputes the tile after the next barrier, when it has landed.)"""
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


CASES = [
    dict(heads=8, kv=2, S_q=100, S_k=330, q_pos0=230, block=U32, seed=1),
    dict(heads=4, kv=1, S_q=64, S_k=700, q_pos0=0, block=0, seed=2),
    dict(heads=2, kv=1, S_q=130, S_k=300, q_pos0=150, block=250, seed=5),
    dict(heads=4, kv=4, S_q=70, S_k=300, q_pos0=200, block=U32, ind="f16", outd="f16", seed=3),
    dict(heads=4, kv=1, S_q=64, S_k=130, q_pos0=0, block=U32, ind="bf16", outd="bf16", seed=4),
    dict(heads=4, kv=1, S_q=64, S_k=448, q_pos0=0, block=0, seed=7, kgrow=1.5),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_stream_matches_oracle(case):
    taken = E.EXACT_COUNT[0]
    r = R.run(**case, verbose=False)
    assert r["out_bad"] == 0 and r["lse_bad"] == 0, r
    # the epilogue's 8-byte writes (2-byte outputs) meet 2-way: sixteen lanes of one write cover rows with eight
    # distinct chunk slots; every other LDS access is conflict-free
    assert all(m == (2 if op == "ds_write_b64" else 1) or m == 1 for op, m in r["lds_worst"].items()), r["lds_worst"]
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
    if G.STAGING != "dma":
        pytest.skip("the staging in use has no DMA wait")
    monkeypatch.setattr(G, "barrier", lambda: [f"s_waitcnt vmcnt({G.DMA_PER_TILE})", "s_barrier"])
    r = R.run(4, 1, 64, 448, 0, 0, seed=9, verbose=False)
    assert r["out_bad"] > 0


def test_planted_short_barrier_wait_is_found(monkeypatch):
    if G.STAGING != "dma":
        pytest.skip("the staging in use has no DMA wait")
    monkeypatch.setattr(G, "barrier", lambda: [f"s_waitcnt vmcnt({3 * G.DMA_PER_TILE}) lgkmcnt(0)", "s_barrier"])
    r = R.run(4, 1, 64, 448, 0, 0, seed=9, verbose=False)
    assert r["out_bad"] > 0
