#!/usr/bin/env python3
"""Writes attn_fwd64_asm.inc: the instruction stream of flash_fwd_r64 (attn_fwd64.hip), the dense attention kernel for
heads of 128 that gives each wave 64 query rows.

Why a generated stream: the kernel keeps the output accumulators (128 registers) and Q (64) in the accumulator
registers and two score tiles (128) in the vector registers, one wave per SIMD, and interleaves the softmax with the
MFMAs instruction by instruction. hipcc does not allocate that working set without spills or accumulator copies,
so the stream is emitted here with fixed registers and placed in one inline-asm statement; the C++ side computes the
per-lane addresses and passes them in as operands.

Per wave: rows q0 .. q0 + 63 as two 32-row blocks (rb 0, 1). Scores are S^T = K Q^T on v_mfma_f32_32x32x16 (K from
LDS as the A operand, Q from the accumulator registers as B), so each lane holds one query row's scores for 16 keys
of each 32-key half; P V is O^T += V^T P^T with V^T from LDS (f16) and the f16 probabilities as B. Every K / V^T
operand read from LDS feeds both row blocks' MFMAs. Keys go by tiles of 64 through three LDS buffers: tile j + 2 is
written while tiles j and j + 1 are read, one workgroup barrier a tile.

Iteration j, with S_cur holding tile j's exponentials (f32, made against the running maximum known when they were
made) and S_nxt receiving tile j + 1's scores:
  phase QK: 32 MFMAs, S_nxt = K(j + 1) Q^T, beside the vector work: the staging of tile j + 2 (K as loaded, V
            converted to f16 and transposed), P = f16(S_cur), the row sums of those f16 values (v_dot2), and the
            loads of tile j + 3. Then the check: when some lane's sum over its 32 keys exceeds 256 (a score above the
            running maximum by more than 8, base 2) or is not a number, the wave takes the exact path, which
            recomputes tile j's scores from LDS, masks them, moves the running maximum by the reference's rule (only
            when a score passes it by more than 8), rescales the outputs and sums, and makes the exponentials, P and
            sums again. Tile 0 always takes that path.
  phase PV: 32 MFMAs, O += V^T(j) P^T, beside the exponentials of tile j + 1 (masked first when some row of the
            wave does not see all of its keys).
The loop is unrolled twice so that S_cur and S_nxt swap registers statically.

Register map: a0..a127 the outputs O[rb][db] (32 head dims a block), a128..a191 Q[rb][kk], a192..a207 the LDS
operand ring; v0..v127 the two score tiles, v128..v159 P[rb], v160..v207 staging, v208..v231 softmax state and
temporaries; s60..s91 scalars. The C++ operands sit in the registers the clobber list leaves free.

Run: python3 gen_attn_fwd64.py  (writes attn_fwd64_asm.inc beside this file; the Makefile reruns it when it changes)
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))

K_ROW = 272             # LDS bytes of a K row (256 + 16 of padding: 16-byte reads down a column are conflict-free)
K_TILE = 64 * K_ROW     # 17408
V_TILE = 128 * 64 * 2   # 16384: V^T, 128 head dims x 64 keys in f16
RING = 8                # LDS operand ring slots
AHEAD = 6               # operand reads in flight ahead of their MFMAs (a slot is refilled two fragments after its
                        # last MFMA was issued)

# ---- registers ---------------------------------------------------------------------------------------------------


def S(buf, rb, t, r=None):
    """Score tile buf (0, 1), row block rb, key half t; register r holds key 32 t + 16 (r / 8) + 8 g + r % 8."""
    base = 64 * buf + 32 * rb + 16 * t
    return f"v{base + r}" if r is not None else f"v[{base}:{base + 15}]"


def P(rb, cc, i=None):
    """f16 probabilities, 16-key chunk cc: dword i holds keys 16 cc + 8 g + 2 i, + 1 (the B operand of P V)."""
    base = 128 + 16 * rb + 4 * cc
    return f"v{base + i}" if i is not None else f"v[{base}:{base + 3}]"


def O(rb, db, r=None):
    """Output block: register r holds head dim 32 db + 8 (r / 4) + 4 g + r % 4 of query row c32."""
    base = 64 * rb + 16 * db
    return f"a{base + r}" if r is not None else f"a[{base}:{base + 15}]"


def Q(rb, kk):
    base = 128 + 32 * rb + 4 * kk
    return f"a[{base}:{base + 3}]"


def RINGR(s):
    return f"a[{192 + 4 * s}:{192 + 4 * s + 3}]"


# Two staging sets (tiles alternate between them, so a tile's loads are issued two tiles ahead of its LDS writes):
# K rows as loaded in the accumulator registers, V rows in vector registers.
def KST(i, st):         # staged K of set st, key i of the thread's four
    b = 224 + 16 * st + 4 * i
    return f"a[{b}:{b + 3}]"


def VST(i, p, st):      # staged V of set st, key i, dword p (head dims 2p, 2p + 1 of the thread's 8)
    return f"v{176 + 16 * st + 4 * i + p}"


def VSTQ(i, st):
    b = 176 + 16 * st + 4 * i
    return f"v[{b}:{b + 3}]"


def VTO(e, half):       # transposed V, head dim e of the thread's 8: keys (0, 1) in half 0, (2, 3) in half 1
    return f"v{160 + 2 * e + half}"


def VTO2(e):
    return f"v[{160 + 2 * e}:{161 + 2 * e}]"


NEGMU = ("v208", "v209")   # -(running maximum) of the lane's row, 0 while it is -inf
LSUM = ("v210", "v211")    # row sum over this lane's keys
MAXV = ("v212", "v213")    # running maximum (base 2), -inf until a key was seen
NINF = "v214"              # -inf
ZERO = "v215"              # 0
TMP = [f"v{216 + i}" for i in range(16)]   # v216 .. v231

SJ = "s60"        # j
SBK = "s61"       # buffer of the tile whose K is read next
SBV = "s62"       # buffer of the tile whose V^T is read next
SBW = "s63"       # buffer written next
S256 = "s64"      # 256.0f
SONES = "s65"     # f16 pair (1, 1)
SHIMASK = "s66"   # 0xffff0000
SPLO = "s67"      # v_perm selector: the low halves of two dwords
SPHI = "s68"      # v_perm selector: the high halves
SJ0 = "s69"       # first key of the next tile (its mask)
SJX = "s70"       # first key of the tile on the exact path
SROT = {"w": ("s72", "s73"), "k": ("s74",), "v": ("s75",)}   # rotation increments, by role
ST = ["s76", "s77", "s78", "s79"]
SCMP = ("s[80:81]", "s[82:83]")
SMASK = ("s[88:89]", "s[90:91]", "s[92:93]", "s[94:95]")  # lane masks of the key mask, in rotation
SINC = {K_TILE: ("s84", "s85"), V_TILE: ("s86", "s87")}   # (step, wrap) of a buffer rotation, by stride

CLOBBER_V = 232
CLOBBER_A = 256
CLOBBER_S = (60, 96)


class Emit:
    def __init__(self):
        self.out = []

    def __call__(self, line):
        self.out.append(line)

    def label(self, name):
        self.out.append(f"{name}_%=:")


def lbl(name):
    return f"{name}_%="


# ---- pieces (each returns a list of instructions) -----------------------------------------------------------------

def rotate(sidx, role, regs):
    """Moves the LDS addresses `regs` ((register, buffer stride) pairs) to the next of the three buffers; sidx holds
    the current buffer index. The increments go through role-specific scalars, so rotations can be queued."""
    tmps = SROT[role]
    strides = sorted({st for _, st in regs})
    tmp = dict(zip(strides, tmps))
    ops = [f"s_cmp_eq_u32 {sidx}, 2"]
    for st in strides:
        ops.append(f"s_cselect_b32 {tmp[st]}, {SINC[st][1]}, {SINC[st][0]}")
    ops += [f"v_add_u32 {r}, {tmp[st]}, {r}" for r, st in regs]
    ops += [f"s_add_u32 {sidx}, {sidx}, 1", f"s_cmp_eq_u32 {sidx}, 3", f"s_cselect_b32 {sidx}, 0, {sidx}"]
    return ops


WREGS = [("%[kw]", K_TILE), ("%[vwx]", V_TILE)]
KREGS = [("%[kr]", K_TILE)]
VREGS = [(f"%[vr{i}]", V_TILE) for i in range(4)]


def stage_loads(st):
    """Staging set st gets the thread's four K rows (voffset %[st]) and four V rows (%[stv]), 16 bytes each, of the
    next tile to load; both offsets then move on by a tile. Rows past the workgroup's keys lie outside the buffers
    and load as zeros."""
    ops = [f"buffer_load_dwordx4 {KST(i, st)}, %[st], %[krs], 0 offen offset:{256 * i}" for i in range(4)]
    ops += [f"buffer_load_dwordx4 {VSTQ(i, st)}, %[stv], %[vrs], 0 offen offset:{256 * i}" for i in range(4)]
    ops += ["v_add_u32 %[st], 0x4000, %[st]", "v_add_u32 %[stv], 0x4000, %[stv]"]
    return ops


def stage_convert(bf16, st):
    """V of keys 0..3 (dword p: head dims 2p, 2p + 1) into f16 pairs of consecutive keys for each head dim
    (bf16 -> f16 rounds toward zero, as the C++ kernels' staging does)."""
    ops = []
    for p in range(4):
        for lohi in range(2):
            e = 2 * p + lohi
            for half in range(2):
                a, b = VST(2 * half, p, st), VST(2 * half + 1, p, st)
                dst = VTO(e, half)
                if bf16:
                    if lohi == 0:
                        ops += [f"v_lshlrev_b32 {TMP[12]}, 16, {a}", f"v_lshlrev_b32 {TMP[13]}, 16, {b}"]
                    else:
                        ops += [f"v_and_b32 {TMP[12]}, {SHIMASK}, {a}", f"v_and_b32 {TMP[13]}, {SHIMASK}, {b}"]
                    ops.append(f"v_cvt_pkrtz_f16_f32 {dst}, {TMP[12]}, {TMP[13]}")
                else:
                    ops.append(f"v_perm_b32 {dst}, {b}, {a}, {SPHI if lohi else SPLO}")
    return ops


def stage_writes(st):
    """K rows to their LDS rows; V^T: head dim 8 c + e of the thread's keys at %[vwx] ^ 16 e (the chunk swizzle of
    row d is (d % 8) ^ (d / 8 % 4), here e ^ a per-lane constant folded into %[vwx]) plus the row, 128 e."""
    ops = [f"ds_write_b128 %[kw], {KST(i, st)} offset:{K_ROW * i}" for i in range(4)]
    for e in range(8):
        t = TMP[8 + (e % 4)]
        ops.append(f"v_xor_b32 {t}, {16 * e}, %[vwx]")
        ops.append(f"ds_write_b64 {t}, {VTO2(e)} offset:{128 * e}")
    return ops


def staging(bf16, st):
    """A tile's staging in the loop (staging set st): wait for its loads (the next tile's stay in flight), convert,
    write to LDS and rotate the write addresses; then load the tile two ahead into the same set."""
    return (["s_waitcnt vmcnt(8)"] + stage_convert(bf16, st) + stage_writes(st) + rotate(SBW, "w", WREGS))


def k_reads(addr):
    """LDS reads of K fragment f = (kk, t) = (f // 2, f % 2): rows 32 t + c32 (slot order), head dims 16 kk + 8 g."""
    return [f"ds_read_b128 {{ring}}, {addr} offset:{8704 * (f % 2) + 32 * (f // 2)}" for f in range(16)]


def qk_mfmas(dtype, sbuf):
    mf = f"v_mfma_f32_32x32x16_{dtype}"
    out = []
    for f in range(16):
        kk, t = f // 2, f % 2
        for rb in range(2):
            src_c = "0" if kk == 0 else S(sbuf, rb, t)
            out.append((f, f"{mf} {S(sbuf, rb, t)}, {{ring}}, {Q(rb, kk)}, {src_c}"))
    return out


def v_reads():
    """LDS reads of V^T fragment f = (cc, db) = (f // 4, f % 4): head dims 32 db + c32, keys 16 cc + 8 g .. + 7."""
    return [f"ds_read_b128 {{ring}}, %[vr{f // 4}] offset:{4096 * (f % 4)}" for f in range(16)]


def pv_mfmas():
    out = []
    for f in range(16):
        cc, db = f // 4, f % 4
        for rb in range(2):
            out.append((f, f"v_mfma_f32_32x32x16_f16 {O(rb, db)}, {{ring}}, {P(rb, cc)}, {O(rb, db)}"))
    return out


def interleave(e, reads, mfmas, valu):
    """Emits the MFMAs, each tagged with the fragment it reads, fed by a ring of RING LDS reads (a fragment is read
    into its slot once the previous occupant's last MFMA is issued), with the instructions of `valu` spread evenly
    between them. LDS instructions inside `valu` are counted for the lgkmcnt waits (LDS returns in order)."""
    issued = []
    slot = {}

    def issue(f):
        slot[f] = f % RING
        e(reads[f].format(ring=RINGR(slot[f])))
        issued.append(f"R{f}")

    nxt = 0
    while nxt < min(AHEAD, len(reads)):
        issue(nxt)
        nxt += 1
    n = len(mfmas)
    per = [0] * n
    for i in range(len(valu)):
        per[min(n - 1, i * n // len(valu))] += 1
    vi = 0
    for i, (f, text) in enumerate(mfmas):
        if i == 0 or mfmas[i - 1][0] != f:
            after = len(issued) - 1 - issued.index(f"R{f}")
            e(f"s_waitcnt lgkmcnt({min(after, 15)})")
        e(text.format(ring=RINGR(slot[f])))
        if (i + 1 == n or mfmas[i + 1][0] != f) and nxt < len(reads):
            issue(nxt)
            nxt += 1
        for _ in range(per[i]):
            op = valu[vi]
            vi += 1
            e(op)
            if op.startswith("ds_"):
                issued.append("W")
    assert vi == len(valu)


def mask(sbuf, j0):
    """Keys a row does not see become -inf: key (tile first key) + C is seen by a lane when C < its limit - 8 g - j0
    (the limit: the reference's visibility rule collapsed to `key < lim` for the lane's row)."""
    ops = [f"v_sub_u32 {TMP[rb]}, %[lim{rb}], {j0}" for rb in range(2)]
    elems = [(rb, t, r) for rb in range(2) for t in range(2) for r in range(16)]
    cmp = [f"v_cmp_lt_i32 {SMASK[i % 4]}, {32 * t + 16 * (r >> 3) + (r & 7)}, {TMP[rb]}"
           for i, (rb, t, r) in enumerate(elems)]
    cnd = [f"v_cndmask_b32 {S(sbuf, rb, t, r)}, {NINF}, {S(sbuf, rb, t, r)}, {SMASK[i % 4]}"
           for i, (rb, t, r) in enumerate(elems)]
    # a compare's mask is read three instructions later (a VALU-written lane mask needs two wait states)
    ops += cmp[:2]
    for i in range(len(elems)):
        if i + 2 < len(elems):
            ops.append(cmp[i + 2])
        ops.append(cnd[i])
    return ops


def exps(sbuf):
    """Exponentials in place: exp2(s c - m)."""
    ops = []
    for rb in range(2):
        for t in range(2):
            for r in range(16):
                ops.append(f"v_fma_f32 {S(sbuf, rb, t, r)}, {S(sbuf, rb, t, r)}, %[c], {NEGMU[rb]}")
                ops.append(f"v_exp_f32 {S(sbuf, rb, t, r)}, {S(sbuf, rb, t, r)}")
    return ops


def pack_and_sum(sbuf):
    """P[rb] = f16 pairs of tile S(sbuf)'s exponentials, and the sum a row block of the f16 values (v_dot2 against
    (1, 1), four chains) into TMP[0] (rb 0) and TMP[4] (rb 1)."""
    ops = [f"v_mov_b32 {TMP[q]}, 0" for q in range(8)]
    for rb in range(2):
        for cc in range(4):
            t, r0 = cc // 2, 8 * (cc % 2)
            for i in range(4):
                ops.append(f"v_cvt_pk_f16_f32 {P(rb, cc, i)}, {S(sbuf, rb, t, r0 + 2 * i)}, "
                           f"{S(sbuf, rb, t, r0 + 2 * i + 1)}")
    for cc in range(4):
        for rb in range(2):
            for i in range(4):
                acc = TMP[4 * rb + i]
                ops.append(f"v_dot2_f32_f16 {acc}, {P(rb, cc, i)}, {SONES}, {acc}")
    for rb in range(2):
        a = TMP[4 * rb: 4 * rb + 4]
        ops += [f"v_add_f32 {a[0]}, {a[0]}, {a[1]}", f"v_add_f32 {a[2]}, {a[2]}, {a[3]}",
                f"v_add_f32 {a[0]}, {a[0]}, {a[2]}"]
    return ops


def wait_mfma():
    """Independent instructions between MFMAs and the vector unit's access to their results."""
    return ["s_nop 7", "s_nop 7", "s_nop 4"]


def exact_tile(e, dtype, sbuf, kaddr, j0):
    """The exact path for a tile (K at LDS address kaddr, first key in scalar j0): its raw scores into S(sbuf), the
    mask, each row's maximum, the reference's rule for moving the running maximum (outputs and sums rescaled when it
    moves), the exponentials, P and the sums (TMP[0], TMP[4])."""
    interleave(e, k_reads(kaddr), qk_mfmas(dtype, sbuf), [])
    for op in wait_mfma() + mask(sbuf, j0):
        e(op)
    for rb in range(2):
        mx = TMP[2 + rb]
        vals = [S(sbuf, rb, t, r) for t in range(2) for r in range(16)]
        e(f"v_max3_f32 {mx}, {vals[0]}, {vals[1]}, {vals[2]}")
        rest = vals[3:]
        while len(rest) >= 2:
            e(f"v_max3_f32 {mx}, {mx}, {rest[0]}, {rest[1]}")
            rest = rest[2:]
        if rest:
            e(f"v_max_f32 {mx}, {mx}, {rest[0]}")
    # the row's maximum over both halves of the wave (lane l ^ 32), to base 2 (c > 0)
    e("s_waitcnt lgkmcnt(0)")
    for rb in range(2):
        e(f"ds_bpermute_b32 {TMP[4 + rb]}, %[swp], {TMP[2 + rb]}")
    e("s_waitcnt lgkmcnt(0)")
    for rb in range(2):
        mx, other, f = TMP[2 + rb], TMP[4 + rb], TMP[8 + rb]
        e(f"v_max_f32 {mx}, {mx}, {other}")
        e(f"v_mul_f32 {mx}, %[c], {mx}")
        # up = mx > m + 8 (m = -inf: up for any finite mx); when up, f = exp2(-negmu - mx), m = mx, negmu = -mx
        e(f"v_add_f32 {TMP[6]}, 0x41000000, {MAXV[rb]}")
        e(f"v_cmp_gt_f32 vcc, {mx}, {TMP[6]}")
        e(f"v_add_f32 {TMP[7]}, {NEGMU[rb]}, {mx}")
        e(f"v_exp_f32 {TMP[7]}, -{TMP[7]}")
        e("s_nop 1")  # the exponential's result, and vcc, read next
        e(f"v_cndmask_b32 {f}, 1.0, {TMP[7]}, vcc")
        e(f"v_cndmask_b32 {MAXV[rb]}, {MAXV[rb]}, {mx}, vcc")
        e(f"v_sub_f32 {TMP[7]}, 0, {mx}")
        e(f"v_cndmask_b32 {NEGMU[rb]}, {NEGMU[rb]}, {TMP[7]}, vcc")
        e(f"v_mul_f32 {LSUM[rb]}, {LSUM[rb]}, {f}")
    # rescale the outputs (the MFMAs that wrote them were issued before the last barrier)
    for rb in range(2):
        f = TMP[8 + rb]
        for i in range(64):
            a, tv = f"a{64 * rb + i}", TMP[10 + (i % 4)]
            e(f"v_accvgpr_read_b32 {tv}, {a}")
            e(f"v_mul_f32 {tv}, {tv}, {f}")
            e(f"v_accvgpr_write_b32 {a}, {tv}")
    for op in exps(sbuf) + pack_and_sum(sbuf):
        e(op)


def epilogue(e, out_dtype):
    """Normalise and store this wave's rows of O (rows past n_q fall outside the output buffer and are dropped),
    then the LSE (offsets of rows past n_q are outside its buffer)."""
    e("s_waitcnt vmcnt(0) lgkmcnt(0)")
    for op in wait_mfma():
        e(op)
    sz = {"f32": 4, "bf16": 2, "f16": 2}[out_dtype]
    for rb in range(2):
        lt, inv, addr = TMP[0], TMP[1], TMP[2]
        e(f"ds_bpermute_b32 {lt}, %[swp], {LSUM[rb]}")
        e("s_waitcnt lgkmcnt(0)")
        e(f"v_add_f32 {lt}, {lt}, {LSUM[rb]}")
        e(f"v_rcp_f32 {inv}, {lt}")
        e(f"v_cmp_lt_f32 vcc, 0, {lt}")
        e("s_nop 1")
        e(f"v_cndmask_b32 {inv}, {ZERO}, {inv}, vcc")
        if rb == 0:
            e(f"v_mov_b32 {addr}, %[oo]")
        else:
            e(f"v_add_u32 {addr}, %[so1], %[oo]")
        # store data alternates between two register sets: a store of more than 8 bytes reads its data after
        # issue, so the next group must not overwrite it right away
        for db in range(4):
            for r4 in range(4):
                alt = 4 * ((4 * db + r4) % 2)
                vals = [TMP[4 + alt + i] for i in range(4)]  # v220..v223 or v224..v227
                for i in range(4):
                    e(f"v_accvgpr_read_b32 {vals[i]}, {O(rb, db, 4 * r4 + i)}")
                for i in range(4):
                    e(f"v_mul_f32 {vals[i]}, {vals[i]}, {inv}")
                off = (32 * db + 8 * r4) * sz
                first = int(vals[0][1:])
                if out_dtype == "f32":
                    e(f"buffer_store_dwordx4 v[{first}:{first + 3}], {addr}, %[ors], 0 offen offset:{off}")
                else:
                    cvt = "v_cvt_pk_bf16_f32" if out_dtype == "bf16" else "v_cvt_pk_f16_f32"
                    e(f"{cvt} {vals[0]}, {vals[0]}, {vals[1]}")
                    e(f"{cvt} {vals[1]}, {vals[2]}, {vals[3]}")
                    e(f"buffer_store_dwordx2 v[{first}:{first + 1}], {addr}, %[ors], 0 offen offset:{off}")
        e("s_nop 1")
        # lse = (m + log2 l) ln 2 with m the maximum the exponentials are relative to (-negmu); -inf when l = 0
        e("s_cmp_eq_u32 %[has_lse], 0")
        e(f"s_cbranch_scc1 {lbl(f'L_nolse{rb}')}")
        e(f"v_log_f32 {TMP[3]}, {lt}")
        e("s_nop 1")
        e(f"v_sub_f32 {TMP[3]}, {TMP[3]}, {NEGMU[rb]}")
        e(f"v_mul_f32 {TMP[3]}, 0x3f317218, {TMP[3]}")
        e(f"v_cndmask_b32 {TMP[3]}, {NINF}, {TMP[3]}, vcc")
        e(f"buffer_store_dword {TMP[3]}, %[lo{rb}], %[lrs], 0 offen")
        e.label(f"L_nolse{rb}")


# ---- the kernel body ----------------------------------------------------------------------------------------------

def body(in_dtype, out_dtype):
    bf16 = in_dtype == "bf16"
    e = Emit()
    e(f"s_mov_b32 {S256}, 0x43800000")
    e(f"s_mov_b32 {SONES}, 0x3c003c00")
    e(f"s_mov_b32 {SHIMASK}, 0xffff0000")
    e(f"s_mov_b32 {SPLO}, 0x05040100")
    e(f"s_mov_b32 {SPHI}, 0x07060302")
    for st, (step, wrap) in SINC.items():
        e(f"s_mov_b32 {step}, {st:#x}")
        e(f"s_mov_b32 {wrap}, {(-2 * st) & 0xFFFFFFFF:#x}")
    e(f"v_mov_b32 {NINF}, 0xff800000")
    e(f"v_mov_b32 {ZERO}, 0")
    for rb in range(2):
        e(f"v_mov_b32 {NEGMU[rb]}, 0")
        e(f"v_mov_b32 {LSUM[rb]}, 0")
        e(f"v_mov_b32 {MAXV[rb]}, {NINF}")
    # Q into the accumulator registers (rows past n_q load as zeros); outputs zeroed
    e(f"v_add_u32 {TMP[0]}, 0x2000, %[qo]")
    for rb in range(2):
        for kk in range(8):
            e(f"buffer_load_dwordx4 {Q(rb, kk)}, {'%[qo]' if rb == 0 else TMP[0]}, %[qrs], 0 offen offset:{32 * kk}")
    # tiles 0 and 1 through the two staging sets, then tiles 2 and 3 in flight
    for op in stage_loads(0) + stage_loads(1):
        e(op)
    for i in range(128):
        e(f"v_accvgpr_write_b32 a{i}, 0")
    e(f"s_mov_b32 {SBW}, 0")
    e("s_waitcnt vmcnt(0)")
    for op in stage_convert(bf16, 0) + stage_writes(0) + rotate(SBW, "w", WREGS):
        e(op)
    for op in stage_convert(bf16, 1) + stage_writes(1) + rotate(SBW, "w", WREGS):
        e(op)
    for op in stage_loads(0) + stage_loads(1):
        e(op)
    e(f"s_mov_b32 {SJ}, 0")
    e(f"s_mov_b32 {SBK}, 0")
    e(f"s_mov_b32 {SBV}, 0")
    e("s_waitcnt lgkmcnt(0)")
    e("s_barrier")
    e("s_cmp_eq_u32 %[ntw], 0")
    e(f"s_cbranch_scc1 {lbl('L_tail')}")
    # tile 0 by the exact path
    e(f"s_mov_b32 {SJX}, 0")
    exact_tile(e, in_dtype, 0, "%[kr]", SJX)
    e(f"v_add_f32 {LSUM[0]}, {LSUM[0]}, {TMP[0]}")
    e(f"v_add_f32 {LSUM[1]}, {LSUM[1]}, {TMP[4]}")

    def iteration(par, variant):
        """Iteration j with S_cur = S(par), S_nxt = S(1 - par). variant: 'plain' (tile j + 1 fully seen by the
        wave's rows), 'masked', 'last' (no tile j + 1), 'first' (j = 0: tile 0's P and sums came from the exact
        path)."""
        cur, nxt = par, 1 - par
        tag = f"{variant}{par}"
        # phase QK (tile j's staging set is j % 2 = par)
        valu = staging(bf16, par)
        if variant != "first":
            valu += pack_and_sum(cur)
        valu += stage_loads(par)
        if variant != "last":
            interleave(e, k_reads("%[kr]"), qk_mfmas(in_dtype, nxt), valu)
        else:
            for op in valu:
                e(op)
        if variant != "first":
            e(f"v_cmp_nle_f32 {SCMP[0]}, {TMP[0]}, {S256}")
            e(f"v_cmp_nle_f32 {SCMP[1]}, {TMP[4]}, {S256}")
            e("s_nop 1")
            e(f"s_or_b64 vcc, {SCMP[0]}, {SCMP[1]}")
            e(f"s_cbranch_vccnz {lbl('L_exact_' + tag)}")
            e(f"v_add_f32 {LSUM[0]}, {LSUM[0]}, {TMP[0]}")
            e(f"v_add_f32 {LSUM[1]}, {LSUM[1]}, {TMP[4]}")
            e.label(f"L_back_{tag}")
        if variant != "last":
            for op in rotate(SBK, "k", KREGS):
                e(op)
        # phase PV
        valu = []
        if variant != "last":
            valu = ["s_nop 7", "s_nop 7"] + (mask(nxt, SJ0) if variant == "masked" else []) + exps(nxt)
        interleave(e, v_reads(), pv_mfmas(), valu)
        for op in rotate(SBV, "v", VREGS):
            e(op)

    def exact_block(par, variant):
        tag = f"{variant}{par}"
        e.label(f"L_exact_{tag}")
        # K of tile j is in buffer SBV (the buffer whose V^T is read next)
        e(f"s_mul_i32 {ST[0]}, {SBV}, {K_TILE}")
        e(f"v_add_u32 {TMP[15]}, {ST[0]}, %[kr0]")
        e(f"s_lshl_b32 {SJX}, {SJ}, 6")
        exact_tile(e, in_dtype, par, TMP[15], SJX)
        e(f"v_add_f32 {LSUM[0]}, {LSUM[0]}, {TMP[0]}")
        e(f"v_add_f32 {LSUM[1]}, {LSUM[1]}, {TMP[4]}")
        e(f"s_branch {lbl('L_back_' + tag)}")

    def dispatch(par, first=False):
        """Barrier, then the variant of iteration SJ: this wave's last, one whose next tile needs the mask, plain."""
        name = "first" if first else f"iter{par}"
        e.label(f"L_{name}")
        e("s_waitcnt lgkmcnt(0)")
        e("s_barrier")
        e(f"s_add_u32 {ST[1]}, {SJ}, 1")
        e(f"s_cmp_ge_u32 {ST[1]}, %[ntw]")
        e(f"s_cbranch_scc1 {lbl(f'L_last_{name}')}")
        e(f"s_lshl_b32 {SJ0}, {ST[1]}, 6")
        e(f"s_add_u32 {ST[2]}, {SJ0}, 64")
        e(f"s_cmp_le_u32 {ST[2]}, %[lmin]")
        e(f"s_cbranch_scc0 {lbl(f'L_masked_{name}')}")
        iteration(par, "first" if first else "plain")
        e(f"s_branch {lbl(f'L_next_{name}')}")
        e.label(f"L_masked_{name}")
        if first:
            iteration_first_masked()
        else:
            iteration(par, "masked")
        e.label(f"L_next_{name}")
        e(f"s_add_u32 {SJ}, {SJ}, 1")

    def iteration_first_masked():
        # as iteration(0, 'first') with the next tile masked
        valu = staging(bf16, 0) + stage_loads(0)
        interleave(e, k_reads("%[kr]"), qk_mfmas(in_dtype, 1), valu)
        for op in rotate(SBK, "k", KREGS):
            e(op)
        valu = ["s_nop 7", "s_nop 7"] + mask(1, SJ0) + exps(1)
        interleave(e, v_reads(), pv_mfmas(), valu)
        for op in rotate(SBV, "v", VREGS):
            e(op)

    for op in rotate(SBK, "k", KREGS):
        e(op)
    dispatch(0, first=True)
    dispatch(1)
    dispatch(0)
    e(f"s_branch {lbl('L_iter1')}")
    # the last iteration of the wave, by entry point
    e.label("L_last_first")
    valu = staging(bf16, 0) + stage_loads(0)
    for op in valu:
        e(op)
    interleave(e, v_reads(), pv_mfmas(), [])
    for op in rotate(SBV, "v", VREGS):
        e(op)
    e(f"s_add_u32 {SJ}, {SJ}, 1")
    e(f"s_branch {lbl('L_tail')}")
    for par in (1, 0):
        e.label(f"L_last_iter{par}")
        iteration(par, "last")
        e(f"s_add_u32 {SJ}, {SJ}, 1")
        e(f"s_branch {lbl('L_tail')}")
    for par in (0, 1):
        for variant in ("plain", "masked", "last"):
            exact_block(par, variant)
    # staging-only iterations for the tiles the workgroup's other waves still compute (staging set j % 2)
    e.label("L_tail")
    e(f"s_and_b32 {ST[3]}, {SJ}, 1")
    e(f"s_cmp_eq_u32 {ST[3]}, 1")
    e(f"s_cbranch_scc1 {lbl('L_tail1')}")
    for par in (0, 1):
        e.label(f"L_tail{par}")
        e("s_cmp_ge_u32 %s, %%[nt]" % SJ)
        e(f"s_cbranch_scc1 {lbl('L_epi')}")
        e("s_waitcnt lgkmcnt(0)")
        e("s_barrier")
        for op in staging(bf16, par) + stage_loads(par):
            e(op)
        e(f"s_add_u32 {SJ}, {SJ}, 1")
    e(f"s_branch {lbl('L_tail0')}")
    e.label("L_epi")
    epilogue(e, out_dtype)
    return e.out


def clobbers():
    regs = [f'"v{i}"' for i in range(CLOBBER_V)] + [f'"a{i}"' for i in range(CLOBBER_A)]
    regs += [f'"s{i}"' for i in range(*CLOBBER_S)]
    return ", ".join(regs)


def check_registers(lines):
    """Every register the stream names must be one the clobber list reserves (the wave is only given those)."""
    import re
    for ln in lines:
        for kind, one, lo, hi in re.findall(r"\b([vas])(?:(\d+)|\[(\d+):(\d+)\])", ln.split(";")[0]):
            top = int(one) if one else int(hi)
            bot = int(one) if one else int(lo)
            limit = {"v": (0, CLOBBER_V), "a": (0, CLOBBER_A), "s": CLOBBER_S}[kind]
            assert limit[0] <= bot and top < limit[1], f"{kind}{bot}..{top} outside the reserved registers: {ln}"


def main():
    out = ["// Generated by gen_attn_fwd64.py (the instruction stream of flash_fwd_r64; the design is described there).",
           "// Do not edit: change the generator and run it.", "#pragma once", ""]
    for ind in ("bf16", "f16"):
        for outd in ("f32", ind):
            lines = body(ind, outd)
            check_registers(lines)
            name = f"MAKO_FWD64_ASM_{ind.upper()}_{outd.upper()}"
            out.append(f"#define {name} \\")
            for ln in lines:
                out.append(f'    "{ln}\\n" \\')
            out.append('    ""')
            out.append("")
    out.append(f"#define MAKO_FWD64_CLOBBERS {clobbers()}")
    out.append("")
    with open(os.path.join(HERE, "attn_fwd64_asm.inc"), "w") as f:
        f.write("\n".join(out))


if __name__ == "__main__":
    main()
