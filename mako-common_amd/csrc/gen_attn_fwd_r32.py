#!/usr/bin/env python3
"""Writes attn_fwd_r32_asm.inc: the instruction stream of flash_fwd_r32 (attn_fwd64.hip), dense attention for heads of
256 with 32 query rows a wave.

It is flash_fwd_r64's design (gen_attn_fwd64.py, whose primitives it reuses: the operand ring, the phase scheduler,
the fragment reads) at the other corner of the same register budget. At 256 head dims a 32-row O block is 128
accumulator registers and its Q 64, exactly what r64 spends on 64 rows at 128, so one wave a SIMD again holds O, Q and
an 8-slot operand ring in the accumulator registers, and a tile of 64 keys is again 32 score MFMAs (16 head-dim steps
x 2 key halves) and 32 P V MFMAs (8 output blocks x 4 key chunks). Each K / V^T operand read now feeds one MFMA.

What differs from r64:
  * A K image (64 rows of 528 bytes) and a V image (64 rows of 512) take 65 KiB a tile, so four tile buffers do not
    fit the 160 KiB of LDS. K and V go through rings of two buffers each (130 KiB): iteration j reads K(j + 1) and
    V(j), and stages K(j + 2) and V(j + 1) (the buffers of K(j) and V(j - 1), free since barrier j - 1), which
    barrier j waits for in full. The prologue stages K(0) and V(0), and K(1) between tile 0's score MFMAs.
  * K(j) is overwritten during iteration j, so the exact path cannot recompute tile j's scores from LDS as r64's
    does. The raw (masked) scores stay in registers instead: two raw sets alternate (tile j's, checked after phase
    QK j, and tile j + 1's, written by it), and the exponentials go to a third set E, which phase QK packs into P.
    The exact path therefore reads no LDS and re-issues no operand reads.
  * One row block: the mask, exponentials, sums, checks and epilogue cover 32 rows.
  * V's 32-byte units are placed so that each 32-lane pass of the transpose reads covers the 64 LDS banks once
    (v_unit), which takes four V^T read-address registers (one for each db % 4) instead of r64's two.
  * The grid is persistent, as r64's; the C++ side (attn_fwd_r32.hip) walks the items.

Iteration j (RAW(j) masked raw scores of tile j, E its exponentials against the running maximum):
  phase QK: 32 MFMAs, RAW(j + 1) = K(j + 1) Q^T, beside the staging of K(j + 2) and V(j + 1), P = E rounded to the
            input type and the row sums of E; its last fragments' time reads the first V^T(j) operands. Then the
            check (some lane's sum over its 32 keys above 256, or not a number): the exact path takes RAW(j)'s
            maximum, moves the running maximum by the reference's rule, rescales O and the sums, and makes E, P and
            the sums again.
  phase PV: 32 MFMAs, O += V^T(j) P^T, beside the mask of RAW(j + 1) and E = its exponentials. Barrier j sits after
            fragment BAR_AT (every V^T(j) read issued by then): past it K(j + 2) and V(j + 1) are in LDS, the first
            K(j + 2) reads of the next phase QK go out, and K(j)'s and V(j)'s buffers are free.

Register map: a0..a127 O[db], a128..a191 Q[kk], a192..a223 the operand ring; v0..v63 the two raw score sets, v64..v95
E, v96..v127 the low-part pass's P and temporaries, v128..v143 P, v160..v183 softmax state and temporaries, s60..s99
scalars; the C++ operands sit in the registers the clobber list leaves free.

Run: python3 gen_attn_fwd_r32.py  (writes attn_fwd_r32_asm.inc beside this file; the Makefile reruns it)
"""
import contextlib
import os

import gen_attn_fwd64 as G

HERE = os.path.dirname(os.path.abspath(__file__))

D = 256
K_ROW, V_ROW = 2 * D + 16, 2 * D
K_TILE, V_TILE = 64 * K_ROW, 64 * V_ROW        # 33 KiB, 32 KiB
NKK, NDB = D // 16, D // 32
NKP = (K_TILE // 1024 - 1) // 4                 # K pieces a wave DMAs (w + 4 m), plus the last piece (every wave)
NVP = V_TILE // 4096                            # V KiB a wave DMAs (rows 16 w .. 16 w + 15)
DMA_K = NKP + 1
DMA_V = NVP
RING = 8                                        # operand ring slots (4 accumulator registers each, from a192)
AHEAD = 6                                       # operand reads in flight ahead of their MFMAs
BAR_AT = 32 - AHEAD                             # phase PV's fragment after which the barrier sits: every V^T read
                                                # of the phase (fragment f's goes out after fragment f - AHEAD) is
                                                # issued before it
LDS_BYTES = 2 * (K_TILE + V_TILE)

NEGMU, LSUM, MAXV, NINF, ZERO, TMP = G.NEGMU[0], G.LSUM[0], G.MAXV[0], G.NINF, G.ZERO, G.TMP
SJ, S256 = G.SJ, G.S256
SKRT = "s61"      # +-K_TILE: moves the K read address to the other K buffer
SVRT = "s62"      # +-V_TILE: moves the V^T read addresses to the other V buffer
SKT = "s63"       # +-K_TILE: moves the K DMA destination to the other K buffer
SVT = "s65"       # +-V_TILE: moves the V DMA destination to the other V buffer
SKW, SKWW, SVWW = G.SKW, G.SKWW, G.SVWW
KRS, VRS, ST, SCMP, SJ0, SM0, SMASK = G.KRS, G.VRS, G.ST, G.SCMP, G.SJ0, G.SM0, G.SMASK

CLOBBER_V = 184
CLOBBER_A = 192 + 4 * RING
CLOBBER_S = (60, 100)


@contextlib.contextmanager
def shapes():
    """r64's fragment readers, ring and register helpers at 256 head dims (they read the generator's shape globals)."""
    names = ("D", "K_ROW", "V_ROW", "K_TILE", "V_TILE", "NKK", "NDB", "RING", "AHEAD", "N_K_AHEAD")
    saved = {n: getattr(G, n) for n in names}
    for n in names:
        setattr(G, n, globals()[n] if n != "N_K_AHEAD" else AHEAD)
    try:
        yield
    finally:
        for n, v in saved.items():
            setattr(G, n, v)


def RAW(par, t, r=None):
    """Raw score set par (0, 1), key half t; register r holds key 32 t + 16 (r / 8) + 8 g + r % 8 of row c32."""
    base = 32 * par + 16 * t
    return f"v{base + r}" if r is not None else f"v[{base}:{base + 15}]"


def E(t, r):
    return f"v{64 + 16 * t + r}"


def P(cc, i=None):
    """Probabilities in the input type, 16-key chunk cc: dword i holds keys 16 cc + 8 g + 2 i, + 1."""
    base = 128 + 4 * cc
    return f"v{base + i}" if i is not None else f"v[{base}:{base + 3}]"


def v_unit(u, k):
    """Where 32-byte unit u (head dims 16 u .. 16 u + 15) of V row k sits in the row's LDS image: u ^ (k % 4) ^
    4 (u % 2), a bijection of each aligned group of 8 units (256 bytes, the 64 banks). A transpose read's 32-lane pass
    addresses units 2 db and 2 db + 1 of four rows k % 4 = 0 .. 3 (one a 4-lane group): the XOR with k % 4 spreads the
    rows over four units and the 4 (u % 2) term puts the odd unit's four in the other half of the 256 bytes, so the
    pass covers the 64 banks once (r64's v_unit covers the 32 banks of one half twice: a 2-way conflict)."""
    return u ^ (k & 3) ^ (4 * (u & 1))


def v_reads():
    """LDS transpose reads of V^T fragment f = (cc, db) = (f // NDB, f % NDB), the A operand of O^T += V^T P^T: lane
    l = 32 g + 16 h + i receives head dim 32 db + 16 h + i of keys 16 cc + 8 g .. + 7, in two ds_read_b64_tr_b16 of
    four keys ({lo}: keys + 0 .. 3, {hi}: + 4 .. 7). In a read, lane i of the group addresses key 16 cc + 8 g + 4 r +
    i / 4, head dims 16 (2 db + h) + 4 (i % 4) .. + 3: unit v_unit(2 db + h, i / 4) of that row, whose place in the
    row's 256-byte half depends on db % 4 and the lane, so %[vr0] .. %[vr3] hold the lane's address for db % 4 = 0 ..
    3; db / 4 adds 256 bytes, cc and r add whole rows."""
    out = []
    for f in range(4 * NDB):
        cc, db = f // NDB, f % NDB
        base = 16 * cc * V_ROW + 256 * (db >> 2)
        out.append([f"ds_read_b64_tr_b16 {{{half}}}, %[vr{db & 3}] offset:{base + 4 * r * V_ROW}"
                    for r, half in ((0, "lo"), (1, "hi"))])
    return out


def VALS(par):
    return [RAW(par, t, r) for t in range(2) for r in range(16)]


# ---- staging ------------------------------------------------------------------------------------------------------

def dma_k():
    """LDS DMA of the next K tile into the K buffer at SKW (lane l of a load writes 16 bytes at M0 + 16 l): pieces
    w + 4 m (m < NKP) of the 33 KiB image at SKWW + 4 KiB m, and piece 4 NKP (every wave; the same bytes to the same
    place); then the source moves on by a tile (the record count shrinks and stops at zero: later tiles load zeros)
    and the destination to the other K buffer. Returns (groups, tail): a group a load, with the M0 write it needs."""
    groups = []
    for m in range(NKP):
        groups.append([f"s_add_u32 m0, {SKWW}, {4096 * m}" if m else f"s_mov_b32 m0, {SKWW}", "s_nop 0",
                       f"buffer_load_dwordx4 %[kd{m}], {G.quad(KRS)}, 0 offen lds"])
    groups.append([f"s_add_u32 m0, {SKW}, {4 * NKP * 1024}", "s_nop 0",
                   f"buffer_load_dwordx4 %[kd{NKP}], {G.quad(KRS)}, 0 offen lds"])
    step = 128 * D
    tail = [f"s_add_u32 {KRS[0]}, {KRS[0]}, {step:#x}", f"s_addc_u32 {KRS[1]}, {KRS[1]}, 0",
            f"s_sub_u32 {KRS[2]}, {KRS[2]}, {step:#x}", f"s_cselect_b32 {KRS[2]}, 0, {KRS[2]}",
            f"s_add_u32 {SKW}, {SKW}, {SKT}", f"s_add_u32 {SKWW}, {SKWW}, {SKT}", f"s_sub_u32 {SKT}, 0, {SKT}"]
    return groups, tail


def dma_v():
    """LDS DMA of the next V tile into the V buffer at SVWW (this wave's 8 KiB: rows 16 w .. 16 w + 15), eight 1 KiB
    loads of two rows each, the instruction offset (1 KiB (k % 4)) moving source and destination alike. A lane's
    source offset picks the 16 bytes its LDS slot holds, which depend on the rows' index mod 4 (v_unit): %[vd] for
    pieces starting on a multiple of 4 rows, %[vdo] for the others, and both + 4 KiB (%[vd2], %[vdo2]) for the second
    4 KiB. Then the source moves on by a tile and the destination to the other buffer."""
    groups = []
    for k in range(NVP):
        half, odd = k // 4, k % 2
        reg = "vd" + ("o" if odd else "") + ("2" if half else "")
        # every load sets M0 itself: the K loads interleaved with these set it too
        pre = [f"s_mov_b32 m0, {SVWW}" if half == 0 else f"s_add_u32 m0, {SVWW}, 4096", "s_nop 0"]
        groups.append(pre + [f"buffer_load_dwordx4 %[{reg}], {G.quad(VRS)}, 0 offen offset:{1024 * (k % 4)} lds"])
    step = 128 * D
    tail = [f"s_add_u32 {VRS[0]}, {VRS[0]}, {step:#x}", f"s_addc_u32 {VRS[1]}, {VRS[1]}, 0",
            f"s_sub_u32 {VRS[2]}, {VRS[2]}, {step:#x}", f"s_cselect_b32 {VRS[2]}, 0, {VRS[2]}",
            f"s_add_u32 {SVWW}, {SVWW}, {SVT}", f"s_sub_u32 {SVT}, 0, {SVT}"]
    return groups, tail


def unit_groups():
    """The staging of an iteration (K(j + 2) and V(j + 1)) as one (groups, tail)."""
    gk, tk = dma_k()
    gv, tv = dma_v()
    # interleave K and V loads so both streams start early; each group keeps its own M0 write
    groups = []
    for i in range(max(len(gk), len(gv))):
        if i < len(gk):
            groups.append(gk[i])
        if i < len(gv):
            groups.append(gv[i])
    return groups, tk + tv


def flat(gt):
    groups, tail = gt
    return sum(groups, []) + tail


def staging():
    return flat(unit_groups())


def barrier():
    """Every load this wave has issued has landed (the iteration's staging is what the next iteration reads) and its
    LDS reads are done (the buffers read last are overwritten after the barrier); then the barrier."""
    return ["s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier"]


# ---- the softmax pieces -------------------------------------------------------------------------------------------

def mask(par, j0):
    """Keys a row does not see become -inf: key (tile first key) + C is seen when C < %[lim0] - j0 (%[lim0]: the row's
    limit less 8 g)."""
    ops = [f"v_sub_u32 {TMP[0]}, %[lim0], {j0}"]
    elems = [(t, r) for t in range(2) for r in range(16)]
    cmp = [f"v_cmp_lt_i32 {SMASK[i % 4]}, {32 * t + 16 * (r >> 3) + (r & 7)}, {TMP[0]}"
           for i, (t, r) in enumerate(elems)]
    cnd = [f"v_cndmask_b32 {RAW(par, t, r)}, {NINF}, {RAW(par, t, r)}, {SMASK[i % 4]}"
           for i, (t, r) in enumerate(elems)]
    # a compare's mask is read three instructions later (a VALU-written lane mask needs two wait states)
    ops += cmp[:2]
    for i in range(len(elems)):
        if i + 2 < len(elems):
            ops.append(cmp[i + 2])
        ops.append(cnd[i])
    return ops


def exps(par):
    """E = exp2(s c - m) of raw set par."""
    ops = []
    for t in range(2):
        for r in range(16):
            ops.append(f"v_fma_f32 {E(t, r)}, {RAW(par, t, r)}, %[c], {NEGMU}")
            ops.append(f"v_exp_f32 {E(t, r)}, {E(t, r)}")
    return ops


def pack_and_sum(dtype):
    """P = pairs of E rounded to the input type (to nearest even), and the row sum of the f32 exponentials (as the
    reference sums them, ops.metal:326-331) into TMP[0], by four interleaved chains of adds."""
    cvt = f"v_cvt_pk_{dtype}_f32"
    ops = []
    for cc in range(4):
        t, r0 = cc // 2, 8 * (cc % 2)
        for i in range(4):
            ops.append(f"{cvt} {P(cc, i)}, {E(t, r0 + 2 * i)}, {E(t, r0 + 2 * i + 1)}")
    vals = [E(t, r) for t in range(2) for r in range(16)]
    for k in range(1, 8):
        for c in range(4):
            first = vals[c] if k == 1 else TMP[c]
            ops.append(f"v_add_f32 {TMP[c]}, {first}, {vals[4 * k + c]}")
    ops += [f"v_add_f32 {TMP[0]}, {TMP[0]}, {TMP[1]}", f"v_add_f32 {TMP[2]}, {TMP[2]}, {TMP[3]}",
            f"v_add_f32 {TMP[0]}, {TMP[0]}, {TMP[2]}"]
    return ops


def exact(e, dtype, par, first=False):
    """The exact path for the tile in raw set par (masked): each row's maximum, the reference's rule for moving the
    running maximum (outputs and sums rescaled when it moves, not for the first tile), then E, P and the sum
    (TMP[0])."""
    mx = TMP[2]
    vals = VALS(par)
    e(f"v_max3_f32 {mx}, {vals[0]}, {vals[1]}, {vals[2]}")
    rest = vals[3:]
    while len(rest) >= 2:
        e(f"v_max3_f32 {mx}, {mx}, {rest[0]}, {rest[1]}")
        rest = rest[2:]
    if rest:
        e(f"v_max_f32 {mx}, {mx}, {rest[0]}")
    # the row's maximum over both halves of the wave (lane l ^ 32), to base 2 (c > 0)
    e("s_waitcnt lgkmcnt(0)")
    e(f"ds_bpermute_b32 {TMP[4]}, %[swp], {mx}")
    e("s_waitcnt lgkmcnt(0)")
    f = TMP[8]
    e(f"v_max_f32 {mx}, {mx}, {TMP[4]}")
    e(f"v_mul_f32 {mx}, %[c], {mx}")
    # up = mx > m + 8 (m = -inf: up for any finite mx); when up, f = exp2(-negmu - mx), m = mx, negmu = -mx
    e(f"v_add_f32 {TMP[6]}, 0x41000000, {MAXV}")
    e(f"v_cmp_gt_f32 vcc, {mx}, {TMP[6]}")
    e(f"v_add_f32 {TMP[7]}, {NEGMU}, {mx}")
    e(f"v_exp_f32 {TMP[7]}, -{TMP[7]}")
    e("s_nop 1")  # the exponential's result, and vcc, read next
    e(f"v_cndmask_b32 {f}, 1.0, {TMP[7]}, vcc")
    e(f"v_cndmask_b32 {MAXV}, {MAXV}, {mx}, vcc")
    e(f"v_sub_f32 {TMP[7]}, 0, {mx}")
    e(f"v_cndmask_b32 {NEGMU}, {NEGMU}, {TMP[7]}, vcc")
    if not first:
        e(f"v_mul_f32 {LSUM}, {LSUM}, {f}")
        # rescale the outputs (the MFMAs that wrote them were issued before the last barrier)
        for op in G.wait_mfma():
            e(op)
        for i in range(16 * NDB):
            a, tv = f"a{i}", TMP[10 + (i % 4)]
            e(f"v_accvgpr_read_b32 {tv}, {a}")
            e(f"v_mul_f32 {tv}, {tv}, {f}")
            e(f"v_accvgpr_write_b32 {a}, {tv}")
    for op in exps(par) + pack_and_sum(dtype):
        e(op)


# ---- phases -------------------------------------------------------------------------------------------------------

def qk_mfmas(dtype, par):
    mf = f"v_mfma_f32_32x32x16_{dtype}"
    out = []
    for f in range(2 * NKK):
        kk, t = f // 2, f % 2
        src_c = "0" if kk == 0 else RAW(par, t)
        out.append((f, f"{mf} {RAW(par, t)}, {{ring}}, {G.Q(0, kk)}, {src_c}"))
    return out


def pv_mfmas(dtype, pbase=None):
    out = []
    for f in range(4 * NDB):
        cc, db = f // NDB, f % NDB
        pp = P(cc) if pbase is None else f"v[{pbase + 4 * cc}:{pbase + 4 * cc + 3}]"
        out.append((f, f"v_mfma_f32_32x32x16_{dtype} {G.O(0, db)}, {{ring}}, {pp}, {G.O(0, db)}"))
    return out


def q_waits(mfmas, n_groups):
    """Tile 0's score MFMAs wait for the Q step they use: fragment 2 kk's MFMAs read Q(kk), the kk-th of NKK loads
    after K(0) and V(0); behind it are the later Q loads and the DMA loads of K(1) this phase has issued before the
    fragment's first MFMA (group i after MFMA i * n / n_groups)."""
    n = len(mfmas)
    out = {}
    for kk in range(NKK):
        first = next(i for i, (f, _) in enumerate(mfmas) if f == 2 * kk)
        issued = sum(1 for g in range(n_groups) if g * n // n_groups < first)
        out[2 * kk] = [f"s_waitcnt vmcnt({NKK - 1 - kk + issued})"]
    return out


def toggle_k():
    return [f"v_add_u32 %[kr], {SKRT}, %[kr]", f"s_sub_u32 {SKRT}, 0, {SKRT}"]


def toggle_v():
    return [f"v_add_u32 %[vr{i}], {SVRT}, %[vr{i}]" for i in range(4)] + [f"s_sub_u32 {SVRT}, 0, {SVRT}"]


def low_part_pass(e):
    """bf16 inputs: tile 0's P V once more with P_lo = bf16(p - P) of tile 0's f32 exponentials, when the wave's first
    row sees fewer than 64 keys (such rows see only tile 0's keys, too few to average bf16 P's rounding away; see
    gen_attn_fwd64.low_part_pass). Runs before iteration 0 from V(0)'s buffer, P_lo in v96..v111."""
    e("s_cmp_ge_u32 %[lmin], 64")
    e(f"s_cbranch_scc1 {G.lbl('L_nolo')}")
    ops_a, ops_b, ops_c = [], [], []
    for cc in range(4):
        t, r0 = cc // 2, 8 * (cc % 2)
        for i in range(4):
            k = 4 * cc + i
            hi, lr, tr = P(cc, i), f"v{96 + k}", f"v{112 + k}"
            a, b = E(t, r0 + 2 * i), E(t, r0 + 2 * i + 1)
            ops_a += [f"v_lshlrev_b32 {lr}, 16, {hi}", f"v_and_b32 {tr}, 0xffff0000, {hi}"]
            ops_b += [f"v_sub_f32 {lr}, {a}, {lr}", f"v_sub_f32 {tr}, {b}, {tr}"]
            ops_c.append(f"v_cvt_pk_bf16_f32 {lr}, {lr}, {tr}")
    for op in ops_a + ops_b + ops_c:
        e(op)
    G.interleave(e, v_reads(), pv_mfmas("bf16", pbase=96), [])
    e.label("L_nolo")


def epilogue(e, out_dtype):
    """Normalise and store this wave's 32 rows of O, then the LSE, through LDS as gen_attn_fwd64.epilogue: each lane
    writes its 4-dim pieces of row c32 into the wave's region (row-major, 16-byte chunk c of row R at c ^ (R % 8)),
    then reads back whole-row chunks, so each global store writes 1 KiB of contiguous row segments. Rows past n_q fall
    outside the output buffer and are dropped; LSE offsets of rows past n_q are outside its buffer."""
    e("s_waitcnt vmcnt(0) lgkmcnt(0)")
    e("s_barrier")
    for op in G.wait_mfma():
        e(op)
    sz = {"f32": 4, "bf16": 2, "f16": 2}[out_dtype]
    row = D * sz
    inv, lt = TMP[1], TMP[0]
    e(f"ds_bpermute_b32 {lt}, %[swp], {LSUM}")
    e("s_waitcnt lgkmcnt(0)")
    e(f"v_add_f32 {lt}, {lt}, {LSUM}")
    e(f"v_rcp_f32 {inv}, {lt}")
    e(f"v_cmp_lt_f32 vcc, 0, {lt}")
    e("s_nop 1")
    e(f"v_cndmask_b32 {inv}, {ZERO}, {inv}, vcc")
    # lse = (m + log2 l) ln 2 with m the maximum the exponentials are relative to (-negmu); -inf when l = 0
    e("s_cmp_eq_u32 %[has_lse], 0")
    e(f"s_cbranch_scc1 {G.lbl('L_nolse')}")
    e(f"v_log_f32 {TMP[3]}, {lt}")
    e("s_nop 1")
    e(f"v_sub_f32 {TMP[3]}, {TMP[3]}, {NEGMU}")
    e(f"v_mul_f32 {TMP[3]}, 0x3f317218, {TMP[3]}")
    e(f"v_cndmask_b32 {TMP[3]}, {NINF}, {TMP[3]}, vcc")
    e(f"buffer_store_dword {TMP[3]}, %[lo0], %[lrs], 0 offen")
    e.label("L_nolse")
    # writes: piece (db, r4) is head dims 32 db + 8 r4 + 4 g .. + 3 of row c32; its address is %[ew] ^ (16 x its chunk
    # without the lane's part), %[ew] holding the row, the lane's part and the swizzle
    n = 0
    for db in range(NDB):
        for r4 in range(4):
            vals = [f"v{4 * n + i}" for i in range(4)]
            addr = f"v{128 + n}"
            for i in range(4):
                e(f"v_accvgpr_read_b32 {vals[i]}, {G.O(0, db, 4 * r4 + i)}")
            for i in range(4):
                e(f"v_mul_f32 {vals[i]}, {vals[i]}, {inv}")
            chunk = 4 * db + r4 if sz == 2 else 8 * db + 2 * r4
            e(f"v_xor_b32 {addr}, {16 * chunk}, %[ew]")
            if sz == 4:
                e(f"ds_write_b128 {addr}, v[{4 * n}:{4 * n + 3}]")
            else:
                cvt = "v_cvt_pk_bf16_f32" if out_dtype == "bf16" else "v_cvt_pk_f16_f32"
                e(f"{cvt} {vals[0]}, {vals[0]}, {vals[1]}")
                e(f"{cvt} {vals[1]}, {vals[2]}, {vals[3]}")
                e(f"ds_write_b64 {addr}, v[{4 * n}:{4 * n + 1}]")
            n += 1
    e("s_waitcnt lgkmcnt(0)")
    # reads: load i covers rows (rows_i of them) rows_i i .. of the wave's 32; the lane's chunk swizzle depends on the
    # row through i, folded in by an xor of %[er]
    rows_i = 1024 // row
    n_ld = 32 // rows_i
    for i in range(n_ld):
        swz = ((rows_i * i) & 7) * 16
        addr = f"v{128 + i}"
        e(f"v_xor_b32 {addr}, {swz}, %[er]")
        e(f"ds_read_b128 v[{4 * i}:{4 * i + 3}], {addr} offset:{1024 * i}")
    ga = (TMP[4], TMP[5])
    e(f"v_mov_b32 {ga[0]}, %[og]")
    e(f"v_add_u32 {ga[1]}, %[ogs], %[og]")
    e(f"s_lshl_b32 {ST[0]}, %[ogs], 1")
    e("s_waitcnt lgkmcnt(0)")
    for i in range(n_ld):
        a = ga[i % 2]
        e(f"buffer_store_dwordx4 v[{4 * i}:{4 * i + 3}], {a}, %[ors], 0 offen nt")
        if i + 2 < n_ld:
            e("s_nop 1")
            e(f"v_add_u32 {a}, {ST[0]}, {a}")


# ---- the kernel body ----------------------------------------------------------------------------------------------

def body(in_dtype, out_dtype):
    with shapes():
        return body_of(in_dtype, out_dtype)


def body_of(in_dtype, out_dtype):
    e = G.Emit()
    e(f"s_mov_b32 {S256}, 0x43800000")
    for r in TMP[8:12]:   # zeros for the MFMAs that clear the outputs
        e(f"v_mov_b32 {r}, 0")
    e(f"v_mov_b32 {NINF}, 0xff800000")
    e(f"v_mov_b32 {ZERO}, 0")
    e(f"v_mov_b32 {NEGMU}, 0")
    e(f"v_mov_b32 {LSUM}, 0")
    e(f"v_mov_b32 {MAXV}, {NINF}")
    for r, pre in ((KRS, "k"), (VRS, "v")):
        e(f"s_mov_b32 {r[0]}, %[{pre}b0]")
        e(f"s_mov_b32 {r[1]}, %[{pre}b1]")
        e(f"s_mov_b32 {r[2]}, %[{pre}n]")
        e(f"s_mov_b32 {r[3]}, 0x20000")
    for r, v in ((SKRT, K_TILE), (SVRT, V_TILE), (SKT, K_TILE), (SVT, V_TILE)):
        e(f"s_mov_b32 {r}, {v:#x}")
    # M0 is the compiler's: kept in SM0 while the stream uses it, restored at the end
    e(f"s_mov_b32 {SM0}, m0")
    e(f"s_mov_b32 {SKW}, %[skw]")
    e(f"s_mov_b32 {SKWW}, %[skww]")
    e(f"s_mov_b32 {SVWW}, %[svww]")
    # K(0) and V(0) into buffers 0, then Q into the accumulator registers (rows past n_q load as zeros); the outputs
    # cleared meanwhile; K(1) goes into K buffer 1 between tile 0's score MFMAs. Loads retire in order: the first
    # barrier waits for K(0) and V(0), tile 0's score MFMAs each wait for the Q step they use (q_waits), and the
    # barrier after tile 0 for K(1).
    for op in flat(dma_k()) + flat(dma_v()):
        e(op)
    for kk in range(NKK):
        e(f"buffer_load_dwordx4 {G.Q(0, kk)}, %[qo], %[qrs], 0 offen offset:{32 * kk}")
    z = f"v[{TMP[8][1:]}:{TMP[11][1:]}]"
    for i in range(NDB):
        e(f"v_mfma_f32_32x32x16_{in_dtype} a[{16 * i}:{16 * i + 15}], {z}, {z}, 0")
    body_rest(e, in_dtype, out_dtype)
    return e.out


def body_rest(e, in_dtype, out_dtype):
    e(f"s_mov_b32 {SJ}, 0")
    e(f"s_waitcnt vmcnt({NKK}) lgkmcnt(0)")
    e("s_barrier")
    e("s_cmp_eq_u32 %[ntw], 0")
    e(f"s_cbranch_scc0 {G.lbl('L_live')}")
    # a wave with no rows: its share of K(1), the barrier after tile 0 as the others, then the load-only loop
    for op in flat(dma_k()) + barrier():
        e(op)
    e(f"s_branch {G.lbl('L_tail')}")
    e.label("L_live")
    # tile 0: scores into raw set 0 (K(1) staged between the MFMAs), masked, then the exact path
    mfmas = qk_mfmas(in_dtype, 0)
    early = dma_k()
    G.phase(e, "X", G.k_reads("%[kr]"), mfmas, [], fwait=q_waits(mfmas, len(early[0])), dma=early)
    for op in G.wait_mfma() + mask(0, 0):
        e(op)
    exact(e, in_dtype, 0, first=True)
    e(f"v_add_f32 {LSUM}, {LSUM}, {TMP[0]}")
    if in_dtype == "bf16":
        low_part_pass(e)
    for op in barrier():   # every wave's loads of K(1) have landed, and none reads K(0)'s buffer any more
        e(op)

    exact_tags = []

    def iteration(par, variant, masked_next=False):
        """Iteration j with RAW(par) tile j's masked scores and RAW(1 - par) receiving tile j + 1's. variant:
        'plain' (tile j + 1 fully seen by the wave's rows), 'masked', 'last' (no tile j + 1), 'first' (j = 0: tile
        0's P and sums came from its exact path; masked_next: tile 1 needs the mask)."""
        cur, nxt = par, 1 - par
        tag = f"{variant}{par}"
        valu = [] if variant == "first" else pack_and_sum(in_dtype)
        n_v = 0
        if variant != "last":
            n_v = G.phase(e, "K", G.k_reads("%[kr]"), qk_mfmas(in_dtype, nxt), valu,
                          pre=0 if variant == "first" else G.N_K_AHEAD, nxt=("V", v_reads()), dma=unit_groups())
        else:
            # the wave's last tile; the workgroup's other waves still read what this iteration stages
            for op in valu + staging():
                e(op)
        if variant != "first":
            e(f"v_cmp_nle_f32 {SCMP[0]}, {TMP[0]}, {S256}")
            e("s_nop 1")
            e(f"s_or_b64 vcc, {SCMP[0]}, {SCMP[0]}")
            e(f"s_cbranch_vccnz {G.lbl('L_exact_' + tag)}")
            e(f"v_add_f32 {LSUM}, {LSUM}, {TMP[0]}")
            e.label(f"L_back_{tag}")
            exact_tags.append((tag, cur))
        if variant != "last":
            for op in toggle_k():
                e(op)
        valu = []
        if variant != "last":
            kind = masked_next or variant
            m = mask(nxt, SJ0) if kind == "masked" else []
            valu = ["s_nop 7", "s_nop 7"] + m + exps(nxt)
        n_k = G.phase(e, "V", v_reads(), pv_mfmas(in_dtype), valu, pre=n_v,
                      nxt=None if variant == "last" else ("K", G.k_reads("%[kr]")), gate_at=BAR_AT, gate=barrier())
        assert variant == "last" or n_k == G.N_K_AHEAD
        for op in toggle_v():
            e(op)

    def exact_block(tag, par):
        e.label(f"L_exact_{tag}")
        for op in G.wait_mfma():
            e(op)
        exact(e, in_dtype, par)
        e(f"v_add_f32 {LSUM}, {LSUM}, {TMP[0]}")
        e(f"s_branch {G.lbl('L_back_' + tag)}")

    def dispatch(par, first=False):
        name = "first" if first else f"iter{par}"
        e.label(f"L_{name}")
        e(f"s_add_u32 {ST[1]}, {SJ}, 1")
        e(f"s_cmp_ge_u32 {ST[1]}, %[ntw]")
        e(f"s_cbranch_scc1 {G.lbl(f'L_last_{name}')}")
        e(f"s_lshl_b32 {SJ0}, {ST[1]}, 6")
        e(f"s_add_u32 {ST[2]}, {SJ0}, 64")
        e(f"s_cmp_le_u32 {ST[2]}, %[lmin]")
        e(f"s_cbranch_scc0 {G.lbl(f'L_masked_{name}')}")
        iteration(par, "first" if first else "plain")
        e(f"s_branch {G.lbl(f'L_next_{name}')}")
        e.label(f"L_masked_{name}")
        if first:
            iteration(0, "first", masked_next="masked")
        else:
            iteration(par, "masked")
        e.label(f"L_next_{name}")
        e(f"s_add_u32 {SJ}, {SJ}, 1")

    for op in toggle_k():
        e(op)
    dispatch(0, first=True)
    dispatch(1)
    dispatch(0)
    e(f"s_branch {G.lbl('L_iter1')}")
    # the last iteration of the wave, by entry point
    e.label("L_last_first")
    for op in staging():
        e(op)
    G.phase(e, "V", v_reads(), pv_mfmas(in_dtype), [], gate_at=BAR_AT, gate=barrier())
    for op in toggle_v():
        e(op)
    e(f"s_add_u32 {SJ}, {SJ}, 1")
    e(f"s_branch {G.lbl('L_tail')}")
    for par in (1, 0):
        e.label(f"L_last_iter{par}")
        iteration(par, "last")
        e(f"s_add_u32 {SJ}, {SJ}, 1")
        e(f"s_branch {G.lbl('L_tail')}")
    for tag, par in exact_tags:
        exact_block(tag, par)
    # load-only iterations for the tiles the workgroup's other waves still compute: the staging of iteration SJ,
    # then its barrier
    e.label("L_tail")
    e(f"s_cmp_ge_u32 {SJ}, %[nt]")
    e(f"s_cbranch_scc1 {G.lbl('L_epi')}")
    for op in staging() + barrier():
        e(op)
    e(f"s_add_u32 {SJ}, {SJ}, 1")
    e(f"s_branch {G.lbl('L_tail')}")
    e.label("L_epi")
    epilogue(e, out_dtype)
    e(f"s_mov_b32 m0, {SM0}")


def clobbers():
    regs = [f'"v{i}"' for i in range(CLOBBER_V)]
    regs += [f'"a{i}"' for i in range(CLOBBER_A)]
    regs += [f'"s{i}"' for i in range(*CLOBBER_S)]
    return ", ".join(regs)


def check_registers(lines):
    """Every register the stream names must be one the clobber list reserves."""
    import re
    for ln in lines:
        for kind, one, lo, hi in re.findall(r"\b([vas])(?:(\d+)|\[(\d+):(\d+)\])", ln.split(";")[0]):
            top = int(one) if one else int(hi)
            bot = int(one) if one else int(lo)
            limit = {"v": (0, CLOBBER_V), "a": (0, CLOBBER_A), "s": CLOBBER_S}[kind]
            assert limit[0] <= bot and top < limit[1], f"{kind}{bot}..{top} outside the reserved registers: {ln}"
            assert one or bot % 2 == 0, f"{kind}[{bot}:{top}]: a register tuple must start on an even register: {ln}"


def main():
    out = ["// Generated by gen_attn_fwd_r32.py (the instruction stream of flash_fwd_r32; the design is described there).",
           "// Do not edit: change the generator and run it.", "#pragma once", ""]
    for ind in ("bf16", "f16"):
        for outd in ("f32", ind):
            lines = body(ind, outd)
            check_registers(lines)
            name = f"MAKO_FWD_R32_ASM_{ind.upper()}_{outd.upper()}"
            out.append(f"#define {name} \\")
            for ln in lines:
                out.append(f'    "{ln}\\n" \\')
            out.append('    ""')
            out.append("")
    out.append(f"#define MAKO_FWD_R32_CLOBBERS {clobbers()}")
    out.append("")
    with open(os.path.join(HERE, "attn_fwd_r32_asm.inc"), "w") as f:
        f.write("\n".join(out))


if __name__ == "__main__":
    main()
