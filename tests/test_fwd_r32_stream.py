"""CPU checks of flash_fwd_r32's generated instruction stream (mako-common_amd/csrc/gen_attn_fwd_r32.py, heads of
256, 32 rows a wave): every register it names is one its clobber list reserves; no gfx950 software hazard in any of its
type variants; and, on the instruction-level emulator (tests/fwd64_emu.py), outputs and LSE within the attention
tolerance of the oracle, conflict-free LDS access and no LDS read of bytes whose DMA load has not landed: causal GQA
with a query offset and ragged sizes, bidirectional, prefix-causal, f16 in and out, bf16 out, one head a kv head (a
workgroup's waves 32 rows apart), no keys, fewer keys than queries, and growing scores that send tiles down the exact
path (which here works from the raw scores kept in registers). Planted mistakes show the checks have teeth: V pieces
staged with the lane offsets of the wrong row parity, an exact path that forgets to rescale the outputs, and a
barrier that does not wait for the staging."""
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "mako-common_amd", "csrc"))
import fwd64_emu as E  # noqa: E402
import fwd64_hazards as Hz  # noqa: E402
import fwd_r32_run as R  # noqa: E402
import gen_attn_fwd_r32 as G  # noqa: E402

U32 = 0xFFFFFFFF
VARIANTS = [("bf16", "f32"), ("bf16", "bf16"), ("f16", "f32"), ("f16", "f16")]


@pytest.mark.parametrize("ind,outd", VARIANTS)
def test_registers_and_hazards(ind, outd):
    lines = G.body(ind, outd)
    G.check_registers(lines)
    assert Hz.check(lines, f"r32 {ind}->{outd}") == 0


CASES = [
    dict(heads=8, kv=2, S_q=100, S_k=330, q_pos0=230, block=U32, seed=1),
    dict(heads=4, kv=1, S_q=64, S_k=200, q_pos0=0, block=0, seed=2),
    dict(heads=2, kv=1, S_q=130, S_k=300, q_pos0=150, block=250, seed=5),
    dict(heads=4, kv=4, S_q=70, S_k=300, q_pos0=200, block=U32, ind="f16", outd="f16", seed=3),
    dict(heads=4, kv=1, S_q=64, S_k=130, q_pos0=0, block=U32, ind="bf16", outd="bf16", seed=4),
    # growing scores: most tiles take the exact path (bf16 P at a milder growth: a softmax this peaked leaves the
    # tolerance with bf16's 8 significant bits, as in every bf16 flash attention; f16 P at the full growth)
    dict(heads=4, kv=1, S_q=32, S_k=448, q_pos0=0, block=0, seed=7, kgrow=1.5, ind="f16"),
    dict(heads=4, kv=1, S_q=32, S_k=448, q_pos0=0, block=0, seed=7, kgrow=0.3),
    dict(heads=1, kv=1, S_q=256, S_k=256, q_pos0=0, block=U32, seed=3),
    dict(heads=2, kv=1, S_q=3, S_k=0, q_pos0=0, block=U32, seed=8),       # no keys: 0 and lse = -inf
    dict(heads=8, kv=2, S_q=40, S_k=5, q_pos0=0, block=U32, seed=9),      # fewer keys than queries
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_stream_matches_oracle(case):
    taken = E.EXACT_COUNT[0]
    r = R.run(**case, verbose=False)
    assert r["out_bad"] == 0 and r["lse_bad"] == 0 and r["early_reads"] == 0, r
    # the epilogue's 8-byte writes (2-byte outputs) meet 2-way; every other LDS access is conflict-free
    assert all(m == (2 if op == "ds_write_b64" else 1) or m == 1 for op, m in r["lds_worst"].items()), r["lds_worst"]
    if case.get("kgrow"):
        assert E.EXACT_COUNT[0] > taken  # the exact path ran


def test_planted_wrong_v_parity_is_found(monkeypatch):
    """V pieces whose rows start at 2 mod 4 need the other lane offsets (the units are permuted by the row mod 4)."""
    src = G.dma_v
    monkeypatch.setattr(G, "dma_v", lambda: tuple(
        [[op.replace("%[vdo", "%[vd") for op in grp] for grp in part] if i == 0 else part
        for i, part in enumerate(src())))
    r = R.run(heads=4, kv=1, S_q=64, S_k=200, q_pos0=0, block=0, seed=2, verbose=False)
    assert r["out_bad"] > 0


def test_planted_exact_path_without_rescale_is_found(monkeypatch):
    src = G.exact
    monkeypatch.setattr(G, "exact", lambda e, dtype, par, first=False: src(e, dtype, par, first=True))
    r = R.run(heads=4, kv=1, S_q=32, S_k=448, q_pos0=0, block=0, seed=7, kgrow=1.5, ind="f16", verbose=False)
    assert r["out_bad"] > 0


def test_planted_barrier_without_dma_wait_is_found(monkeypatch):
    monkeypatch.setattr(G, "barrier", lambda: ["s_waitcnt lgkmcnt(0)", "s_barrier"])
    r = R.run(heads=4, kv=1, S_q=64, S_k=330, q_pos0=0, block=0, seed=2, verbose=False)
    assert r["early_reads"] > 0
