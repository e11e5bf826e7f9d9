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
of each 32-key half; P V is O^T += V^T P^T with V^T read from V's rows in LDS by transpose reads
(ds_read_b64_tr_b16) and the probabilities, rounded to the input type (f16 or bf16), as B. Every K / V^T operand
read from LDS feeds both row blocks' MFMAs.

Keys go by tiles of 64 through four LDS buffers (a K image and a V image each). Staging is straight copies by LDS DMA,
16 bytes a lane, with no conversion, from K and V as they lie in memory: the K image (five 1 KiB pieces a wave) has
rows padded to an odd number of 16-byte chunks, the V image (four 1 KiB pieces a wave) keeps 2 d-byte rows with
their 32-byte units permuted by row (v_unit), each lane loading the 16 bytes its LDS slot holds. Iteration j loads
tile j + 3 into the buffer of tile j - 1. Loads past the workgroup's keys lie outside the buffer descriptors and load
zeros.

ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane i receives element i % 4 of the 8 bytes that lanes
i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4 address, in that order (checked on the GPU). So when lanes 4 y .. 4 y + 3
of a group address the 16 head dims of one key row (8 bytes each), lane i receives head dim i of four keys: a column
of V, which is what the MFMA's A operand holds (eight keys of one head dim a lane, two reads).

Iteration j, with S_cur holding tile j's exponentials (f32, made against the running maximum known when they were
made) and S_nxt receiving tile j + 1's scores:
  phase QK: 32 MFMAs, S_nxt = K(j + 1) Q^T, beside the staging of tile j + 3, P = f16(S_cur) and the row sums
            of S_cur (f32, as the reference sums them); its last fragments' time reads the first V^T(j) operands.
            Then the check: when some lane's sum over its 32 keys exceeds 256 (a score above the running maximum by
            more than 8, base 2) or is not a number, the wave takes the exact path, which recomputes tile j's scores
            from LDS, masks them, moves the running maximum by the reference's rule (only when a score passes it by
            more than 8), rescales the outputs and sums, and makes the exponentials, P and sums again. Tile 0 always
            takes that path.
  phase PV: 32 MFMAs, O += V^T(j) P^T, beside the exponentials of tile j + 1 (masked first when some row of the
            wave does not see all of its keys). Barrier j sits after its fragment BAR_AT, once the wave's V^T(j)
            reads have landed: past it, every wave's loads of tile j + 2 are in LDS (so the first K(j + 2) operands
            of the next phase QK are read from there on) and no wave reads the buffer of tile j any more (so the
            next iteration's staging may overwrite it).
Operand reads thus run across the phase boundaries, and no MFMA waits for an LDS read issued at its phase's start.
The loop is unrolled twice so that S_cur and S_nxt swap registers statically.

Register map: a0..a127 the outputs O[rb][db] (32 head dims a block), a128..a191 Q[rb][kk], a192..a223 the LDS
operand ring; v0..v127 the two score tiles, v128..v159 P[rb], v160..v183 softmax state and temporaries,
s60..s99 scalars. The C++ operands sit in the registers the clobber list leaves free.

Run: python3 gen_attn_fwd64.py  (writes attn_fwd64_asm.inc beside this file; the Makefile reruns it when it changes)
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))

NBUF = 4                # LDS tile buffers
RING = 8                # LDS operand ring slots
AHEAD = 6               # operand reads in flight ahead of their MFMAs (a slot is refilled two fragments after its
                        # last MFMA was issued)
N_K_AHEAD = 6           # K reads of the next phase QK that go out in phase PV's tail, after the barrier


def set_dim(d):
    """The head width's constants (128, or 64: the same stream with half the head dimensions):
    K_ROW   LDS bytes of a K row: 2 d + 16 of padding (an odd number of 16-byte chunks, so 16-byte reads down a column
            are conflict-free);
    K_TILE  the padded K image of a 64-key tile (17 or 9 pieces of 1 KiB: a wave DMAs pieces w + 4 m, m < NKP, and
            every wave the last, piece 4 NKP);
    V_ROW   LDS bytes of a V row: 2 d, its 32-byte units permuted by row (v_unit);
    V_TILE  the V image of a tile, 64 rows (a wave DMAs NVP KiB of it);
    NKK, NDB  16-wide head-dimension steps of Q K^T, 32-wide output blocks;
    BAR_AT  phase PV's fragment (of 4 NDB) after whose MFMAs the tile's barrier sits."""
    global D, K_ROW, V_ROW, K_TILE, V_TILE, NKK, NDB, NKP, NVP, DMA_PER_TILE, BAR_AT
    assert d in (64, 128)
    D = d
    K_ROW = 2 * d + 16
    V_ROW = 2 * d
    K_TILE = 64 * K_ROW
    V_TILE = d * 64 * 2
    NKK, NDB = d // 16, d // 32
    NKP = (K_TILE // 1024 - 1) // 4
    NVP = V_TILE // 4096
    DMA_PER_TILE = NKP + 1 + NVP   # LDS DMA loads a wave issues a tile (9 at d 128, 5 at 64)
    BAR_AT = 12 if d == 128 else 6


set_dim(128)

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
    base = 16 * NDB * rb + 16 * db
    return f"a{base + r}" if r is not None else f"a[{base}:{base + 15}]"


def Q(rb, kk):
    base = 128 + 4 * NKK * rb + 4 * kk
    return f"a[{base}:{base + 3}]"


def RINGR(s):
    return f"a[{192 + 4 * s}:{192 + 4 * s + 3}]"


def ring_fmt(text, s):
    """An operand read's text with ring slot s filled in: {ring} the slot, {lo} / {hi} its halves."""
    b = 192 + 4 * s
    return text.format(ring=RINGR(s), lo=f"a[{b}:{b + 1}]", hi=f"a[{b + 2}:{b + 3}]")


NEGMU = ("v160", "v161")   # -(running maximum) of the lane's row, 0 while it is -inf
LSUM = ("v162", "v163")    # row sum over this lane's keys
MAXV = ("v164", "v165")    # running maximum (base 2), -inf until a key was seen
NINF = "v166"              # -inf
ZERO = "v167"              # 0
TMP = [f"v{168 + i}" for i in range(16)]   # v168 .. v183

SJ = "s60"        # j
SBK = "s61"       # buffer of the tile whose K is read next
SBV = "s62"       # buffer of the tile whose V^T is read next
SBW = "s63"       # buffer written next
S256 = "s64"      # 256.0f
KRS = ("s68", "s69", "s70", "s71")   # buffer descriptor of K from the tile loaded next (4-aligned)
VRS = ("s72", "s73", "s74", "s75")   # buffer descriptor of the V^T tile images from the tile loaded next
ST = ["s76", "s77", "s78", "s79"]
SCMP = ("s[80:81]", "s[82:83]")
SJ0 = "s85"       # first key of the next tile (its mask)
SJX = "s86"       # first key of the tile on the exact path
SMASK = ("s[88:89]", "s[90:91]", "s[92:93]", "s[94:95]")  # lane masks of the key mask, in rotation
SROT = {"k": "s96", "v": "s97", "wk": "s98", "wv": "s99"}   # rotation increments, by role
SKW = "s66"       # DMA: LDS address of the K image of buffer SBW
SKWW = "s67"      # DMA: SKW + 1 KiB x (wave index), this wave's first K piece
SVWW = "s84"      # DMA: LDS address of this wave's 4 KiB of the V image of buffer SBW
SM0 = "s87"       # DMA: the compiler's M0, restored at the end

# The block-sparse stream (body(..., sparse=True)): each tile's first key, and the validity of its keys, come from the
# item's pass table (%[ent]: 16 bytes an entry, {first key or -1 for none, 0, W0, W1}; bit 16 t + r of W_g: key
# 32 t + 16 (r / 8) + 8 g + r % 8 of the tile may be seen), read with scalar loads an iteration ahead.
SPARSE = False
SD = "s65"              # first key of the tile the next staging loads (-1: none, loads zeros)
SEJ = "s86"             # first key of the tile the next phase PV masks (the exact path's is ST[0])
SEW = "s[94:95]"        # that tile's validity words (the exact path's are s[78:79]); the fourth lane-mask pair,
SEW_LO, SEW_HI = "s94", "s95"   # which the sparse stream's masks leave alone
MAPV = "v184"           # the output row map[q0 + lane] (-1: dropped)


def quad(r):
    return f"s[{r[0][1:]}:{r[3][1:]}]"


CLOBBER_V = 184
CLOBBER_A = 224
CLOBBER_S = (60, 100)
CLOBBER_V_SPARSE = 185     # + MAPV
CLOBBER_S_SPARSE = (60, 100)


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

def rotate(sidx, role, regs, stride):
    """Moves the LDS addresses `regs` to the next of the NBUF buffers (buffers are `stride` bytes apart); sidx holds
    the current buffer index."""
    t = SROT[role]
    ops = [f"s_cmp_eq_u32 {sidx}, {NBUF - 1}", f"s_cselect_b32 {t}, {(-NBUF * stride) & 0xFFFFFFFF:#x}, 0",
           f"s_add_u32 {t}, {t}, {stride:#x}"]
    ops += [f"v_add_u32 {r}, {t}, {r}" for r in regs]
    ops += [f"s_add_u32 {sidx}, {sidx}, 1", f"s_cmp_eq_u32 {sidx}, {NBUF}", f"s_cselect_b32 {sidx}, 0, {sidx}"]
    return ops


KREGS = ["%[kr]"]
VREGS = ["%[vr0]", "%[vr1]"]


def dma_issue():
    """The LDS DMA loads of the next tile, flat (dma_groups() in order)."""
    groups, tail = dma_groups()
    return sum(groups, []) + tail


def dma_groups():
    """LDS DMA loads of the next tile into buffer SBW (lane l of a load writes 16 bytes at M0 + offset + 16 l), then
    the sources move on by a tile and the destinations to the next buffer. K: pieces w, w + 4, w + 8, w + 12 of the
    17 KiB image at M0 = their LDS address, and piece 16 (every wave; the same bytes to the same place). V: the
    wave's 4 KiB of the tile image (rows 16 w .. 16 w + 15), as four 1 KiB loads whose offset moves source and
    destination alike (%[vd]: the byte of V a lane's LDS slot holds, relative to the piece). A write of M0 is read by
    an LDS load after one wait state. Record counts shrink by a tile and stop at zero. Sparse: the sources are set
    from SD, the tile's first key (K and V rows are both 256 bytes a key), one tile long, or empty when SD is -1.
    Returns (groups, tail): a group per load (with the M0 write it needs), and the scalar work after the last load.
    A phase spreads the groups evenly between its MFMAs: a burst of these loads holds up the wave's vector and matrix
    instructions behind it (a timing probe of the plain iteration on one CU: 2654 cycles a tile with the loads at
    the phase's start, 2536 spread one every few MFMAs)."""
    groups = []
    pre = []
    if SPARSE:
        t = SROT["k"]
        pre = [f"s_lshl_b32 {t}, {SD}, 8",
               f"s_add_u32 {KRS[0]}, %[kb0], {t}", f"s_addc_u32 {KRS[1]}, %[kb1], 0",
               f"s_add_u32 {VRS[0]}, %[vb0], {t}", f"s_addc_u32 {VRS[1]}, %[vb1], 0",
               f"s_cmp_eq_u32 {SD}, -1", f"s_cselect_b32 {KRS[2]}, 0, 0x4000", f"s_mov_b32 {VRS[2]}, {KRS[2]}"]
    for m in range(NKP):
        groups.append([f"s_add_u32 m0, {SKWW}, {4096 * m}" if m else f"s_mov_b32 m0, {SKWW}", "s_nop 0",
                       f"buffer_load_dwordx4 %[kd{m}], {quad(KRS)}, 0 offen lds"])
    groups.append([f"s_add_u32 m0, {SKW}, {4 * NKP * 1024}", "s_nop 0",
                   f"buffer_load_dwordx4 %[kd4], {quad(KRS)}, 0 offen lds"])
    for i in range(NVP):
        groups.append(([f"s_mov_b32 m0, {SVWW}", "s_nop 0"] if i == 0 else []) +
                      [f"buffer_load_dwordx4 %[vd], {quad(VRS)}, 0 offen offset:{1024 * i} lds"])
    groups[0] = pre + groups[0]
    ops = []
    step = 128 * D   # K and V rows: 2 d bytes a key, 64 keys a tile
    for r in (KRS, VRS) if not SPARSE else ():
        ops += [f"s_add_u32 {r[0]}, {r[0]}, {step:#x}", f"s_addc_u32 {r[1]}, {r[1]}, 0",
                f"s_sub_u32 {r[2]}, {r[2]}, {step:#x}", f"s_cselect_b32 {r[2]}, 0, {r[2]}"]
    wk, wv = SROT["wk"], SROT["wv"]
    ops += [f"s_cmp_eq_u32 {SBW}, {NBUF - 1}",
            f"s_cselect_b32 {wk}, {(-NBUF * K_TILE) & 0xFFFFFFFF:#x}, 0",
            f"s_cselect_b32 {wv}, {(-NBUF * V_TILE) & 0xFFFFFFFF:#x}, 0",
            f"s_add_u32 {wk}, {wk}, {K_TILE:#x}", f"s_add_u32 {wv}, {wv}, {V_TILE:#x}",
            f"s_add_u32 {SKW}, {SKW}, {wk}", f"s_add_u32 {SKWW}, {SKWW}, {wk}", f"s_add_u32 {SVWW}, {SVWW}, {wv}",
            f"s_add_u32 {SBW}, {SBW}, 1", f"s_cmp_eq_u32 {SBW}, {NBUF}", f"s_cselect_b32 {SBW}, 0, {SBW}"]
    return groups, ops


def staging():
    """A tile's staging in the loop: load tile j + 3 (waited for before barrier j + 2)."""
    return dma_issue()


def iteration_last_staging():
    """A wave's last iteration stages its share of tile j + 3 as the others do: the workgroup's longer waves (rows up
    to three tiles later) read it after barrier j + 1."""
    return staging()


def barrier():
    """The wave's staging of the tile before the last is in LDS and its LDS reads are done (the buffer it read last
    is written after the barrier); then the barrier."""
    return [f"s_waitcnt vmcnt({DMA_PER_TILE}) lgkmcnt(0)", "s_barrier"]


def k_reads(addr):
    """LDS reads of K fragment f = (kk, t) = (f // 2, f % 2): rows 32 t + c32 (slot order), head dims 16 kk + 8 g.
    Each fragment's reads are a list of instruction texts ({ring} the ring slot, {lo} / {hi} its halves)."""
    return [[f"ds_read_b128 {{ring}}, {addr} offset:{32 * K_ROW * (f % 2) + 32 * (f // 2)}"] for f in range(2 * NKK)]


def qk_mfmas(dtype, sbuf):
    mf = f"v_mfma_f32_32x32x16_{dtype}"
    out = []
    for f in range(2 * NKK):
        kk, t = f // 2, f % 2
        for rb in range(2):
            src_c = "0" if kk == 0 else S(sbuf, rb, t)
            out.append((f, f"{mf} {S(sbuf, rb, t)}, {{ring}}, {Q(rb, kk)}, {src_c}"))
    return out


def v_unit(u, k):
    """Where 32-byte unit u (head dims 16 u .. 16 u + 15) of V row k sits in the row's LDS image: the unit's low two
    bits XOR the row's. The four rows a transpose read's 16-lane group addresses (k % 4 = 0 .. 3, one unit each) then
    cover the 128 bytes of banks once."""
    return (u & ~3) | ((u & 3) ^ (k & 3))


def v_reads():
    """LDS transpose reads of V^T fragment f = (cc, db) = (f // NDB, f % NDB), the A operand of O^T += V^T P^T: lane
    l = 32 g + 16 h + i receives head dim 32 db + 16 h + i of keys 16 cc + 8 g .. + 7, in two ds_read_b64_tr_b16 of
    four keys ({lo}: keys + 0 .. 3, {hi}: + 4 .. 7). In a read, lane i of the group addresses key 16 cc + 8 g + 4 r +
    i / 4, head dims 16 (2 db + h) + 4 (i % 4) .. + 3: unit v_unit(2 db + h, i / 4) of that row. %[vr0] holds the
    lane's address for even db (unit h ^ (i / 4)), %[vr1] for odd db (unit (2 + h) ^ (i / 4)); db / 2 adds 128
    bytes, cc and r add whole rows."""
    out = []
    for f in range(4 * NDB):
        cc, db = f // NDB, f % NDB
        base = 16 * cc * V_ROW + 128 * (db >> 1)
        out.append([f"ds_read_b64_tr_b16 {{{half}}}, %[vr{db & 1}] offset:{base + 4 * r * V_ROW}"
                    for r, half in ((0, "lo"), (1, "hi"))])
    return out


def pv_mfmas(dtype):
    out = []
    for f in range(4 * NDB):
        cc, db = f // NDB, f % NDB
        for rb in range(2):
            out.append((f, f"v_mfma_f32_32x32x16_{dtype} {O(rb, db)}, {{ring}}, {P(rb, cc)}, {O(rb, db)}"))
    return out


def phase(e, kind, reads, mfmas, valu, pre=0, nxt=None, gate_at=None, gate=(), dma=None, fwait=None):
    """Emits the MFMAs of a phase, each tagged with the fragment it reads, fed by a ring of RING LDS reads, with the
    instructions of `valu` spread evenly between them. Fragment f lives in ring slot f % RING; its read goes out AHEAD
    fragments before its MFMAs (a slot is refilled two fragments after its previous occupant's last MFMA). The first
    `pre` reads were issued before the phase began, as the last LDS instructions before it. nxt = (kind, reads) of
    the next phase: its read m goes out after fragment len(reads) + m - AHEAD of this phase, and not before `gate`,
    the instructions emitted after fragment gate_at's MFMAs. dma = (groups, tail) of dma_groups(): group i after
    MFMA i * n / len(groups) (after that MFMA's share of `valu`), the tail after the last MFMA's. fwait: {fragment:
    instructions} emitted before that fragment's first MFMA.
    Returns how many of the next phase's reads went out.
    LDS returns in order, so the wait for a read is lgkmcnt(LDS instructions issued after it); LDS instructions inside
    `valu` are counted too. A fragment's reads may be several instructions; its MFMAs wait for the last."""
    issued = [(kind, f) for f in range(pre) for _ in reads[f]]
    nfr = len(reads)

    def issue(k, f, texts):
        for text in texts:
            e(ring_fmt(text, f % RING))
            issued.append((k, f))

    after = {}
    for f in range(max(pre, AHEAD), nfr):
        after.setdefault(f - AHEAD, []).append((kind, f, reads[f]))
    n_next = 0
    if nxt:
        nkind, nreads = nxt
        for m in range(len(nreads)):
            at = nfr + m - AHEAD
            if at > nfr - 1:
                break
            if gate_at is not None:
                at = max(at, gate_at)
            after.setdefault(at, []).append((nkind, m, nreads[m]))
            n_next += 1
    for f in range(pre, min(AHEAD, nfr)):
        issue(kind, f, reads[f])
    n = len(mfmas)
    per = [0] * n
    for i in range(len(valu)):
        per[min(n - 1, i * n // len(valu))] += 1
    dslot = [[] for _ in range(n)]
    if dma:
        groups, tail = dma
        for i, grp in enumerate(groups):
            dslot[i * n // len(groups)] += grp
        dslot[n - 1] += tail
    vi = 0
    for i, (f, text) in enumerate(mfmas):
        if i == 0 or mfmas[i - 1][0] != f:
            pos = len(issued) - 1 - issued[::-1].index((kind, f))
            e(f"s_waitcnt lgkmcnt({min(len(issued) - 1 - pos, 15)})")
            for op in (fwait or {}).get(f, []):
                e(op)
        e(ring_fmt(text, f % RING))
        if i + 1 == n or mfmas[i + 1][0] != f:
            if gate_at == f:
                for op in gate:
                    e(op)
            for k, g, t in after.get(f, []):
                issue(k, g, t)
        for _ in range(per[i]):
            op = valu[vi]
            vi += 1
            e(op)
            if op.startswith("ds_"):
                issued.append(None)
        for op in dslot[i]:
            e(op)
    assert vi == len(valu)
    assert gate_at is None or gate_at in {f for f, _ in mfmas}
    return n_next


def interleave(e, reads, mfmas, valu):
    """A phase with nothing in flight before it and nothing read ahead for the next."""
    phase(e, "X", reads, mfmas, valu)


def mask(sbuf, j0):
    """Keys a row does not see become -inf: key (tile first key) + C is seen by a lane when C < its limit - 8 g - j0
    (the limit: the reference's visibility rule collapsed to `key < lim` for the lane's row)."""
    ops = [f"v_sub_u32 {TMP[rb]}, %[lim{rb}], {j0}" for rb in range(2)]
    elems = [(rb, t, r) for rb in range(2) for t in range(2) for r in range(16)]
    nm = 3 if SPARSE else 4   # the sparse stream keeps the fourth pair for SEW
    cmp = [f"v_cmp_lt_i32 {SMASK[i % nm]}, {32 * t + 16 * (r >> 3) + (r & 7)}, {TMP[rb]}"
           for i, (rb, t, r) in enumerate(elems)]
    cnd = [f"v_cndmask_b32 {S(sbuf, rb, t, r)}, {NINF}, {S(sbuf, rb, t, r)}, {SMASK[i % nm]}"
           for i, (rb, t, r) in enumerate(elems)]
    # a compare's mask is read three instructions later (a VALU-written lane mask needs two wait states)
    ops += cmp[:2]
    for i in range(len(elems)):
        if i + 2 < len(elems):
            ops.append(cmp[i + 2])
        ops.append(cnd[i])
    return ops


def mask_general(sbuf, j0, w):
    """Sparse masking of a tile (first key in scalar j0, validity words in the SGPR pair w): the row limit as mask(),
    then the keys whose validity bit is clear. The lane's word W_g is w shifted right by 32 g (%[g32])."""
    ops = [f"v_sub_u32 {TMP[rb]}, %[lim{rb}], {j0}" for rb in range(2)]
    wlo = int(TMP[2][1:])
    ops.append(f"v_lshrrev_b64 v[{wlo}:{wlo + 1}], %[g32], {w}")
    for t in range(2):
        for r in range(16):
            key = 32 * t + 16 * (r >> 3) + (r & 7)
            ops += [f"v_cmp_lt_i32 {SMASK[0]}, {key}, {TMP[0]}",
                    f"v_cmp_lt_i32 {SMASK[1]}, {key}, {TMP[1]}",
                    f"v_bfe_u32 {TMP[4]}, {TMP[2]}, {16 * t + r}, 1",
                    f"v_cmp_ne_u32 {SMASK[2]}, 0, {TMP[4]}",
                    f"v_cndmask_b32 {S(sbuf, 0, t, r)}, {NINF}, {S(sbuf, 0, t, r)}, {SMASK[0]}",
                    f"v_cndmask_b32 {S(sbuf, 1, t, r)}, {NINF}, {S(sbuf, 1, t, r)}, {SMASK[1]}",
                    f"v_cndmask_b32 {S(sbuf, 0, t, r)}, {NINF}, {S(sbuf, 0, t, r)}, {SMASK[2]}",
                    f"v_cndmask_b32 {S(sbuf, 1, t, r)}, {NINF}, {S(sbuf, 1, t, r)}, {SMASK[2]}"]
    return ops


def entry_loads():
    """Sparse: the scalar loads for iteration SJ + 1, issued in phase PV of iteration SJ (before its barrier, whose
    lgkmcnt(0) retires them): entry SJ + 2 (the tile it masks) into SEJ / SEW, and the first key of tile SJ + 4 (the
    tile it stages) into SD."""
    t = ST[0]
    return [f"s_lshl_b32 {t}, {SJ}, 4", f"s_add_u32 {t}, {t}, 32", f"s_load_dword {SEJ}, %[ent], {t}",
            f"s_add_u32 {t}, {t}, 8", f"s_load_dwordx2 {SEW}, %[ent], {t}",
            f"s_add_u32 {t}, {t}, 24", f"s_load_dword {SD}, %[ent], {t}"]


def exps(sbuf):
    """Exponentials in place: exp2(s c - m)."""
    ops = []
    for rb in range(2):
        for t in range(2):
            for r in range(16):
                ops.append(f"v_fma_f32 {S(sbuf, rb, t, r)}, {S(sbuf, rb, t, r)}, %[c], {NEGMU[rb]}")
                ops.append(f"v_exp_f32 {S(sbuf, rb, t, r)}, {S(sbuf, rb, t, r)}")
    return ops


def pack_and_sum(sbuf, dtype):
    """P[rb] = pairs of tile S(sbuf)'s exponentials rounded to the input type dtype (to nearest even), and the sum a
    row block of the f32 exponentials (as the reference sums them, ops.metal:326-331; P V multiplies their roundings)
    into TMP[0] (rb 0) and TMP[4] (rb 1): four chains of adds a row block, interleaved, so no add waits on the one
    before it."""
    cvt = f"v_cvt_pk_{dtype}_f32"
    ops = []
    for rb in range(2):
        for cc in range(4):
            t, r0 = cc // 2, 8 * (cc % 2)
            for i in range(4):
                ops.append(f"{cvt} {P(rb, cc, i)}, {S(sbuf, rb, t, r0 + 2 * i)}, "
                           f"{S(sbuf, rb, t, r0 + 2 * i + 1)}")
    vals = {rb: [S(sbuf, rb, t, r) for t in range(2) for r in range(16)] for rb in range(2)}
    for k in range(1, 8):       # chain c of row block rb sums values c, c + 4, c + 8, ...
        for rb in range(2):
            for c in range(4):
                acc = TMP[4 * rb + c]
                first = vals[rb][c] if k == 1 else acc
                ops.append(f"v_add_f32 {acc}, {first}, {vals[rb][4 * k + c]}")
    for rb in range(2):
        a = TMP[4 * rb: 4 * rb + 4]
        ops += [f"v_add_f32 {a[0]}, {a[0]}, {a[1]}", f"v_add_f32 {a[2]}, {a[2]}, {a[3]}",
                f"v_add_f32 {a[0]}, {a[0]}, {a[2]}"]
    return ops


def wait_mfma():
    """Independent instructions between MFMAs and the vector unit's access to their results."""
    return ["s_nop 7", "s_nop 7", "s_nop 4"]


def q_waits(mfmas, n_groups):
    """Tile 0's score MFMAs wait for the Q pair (both row blocks of a 16-dim step) they use: fragment 2 kk's MFMAs
    read Q(., kk), loaded kk-th after tile 0. Behind Q are the loads still to come of later Q pairs and the LDS DMA
    loads of tiles 1 and 2 that this phase has issued before the fragment's first MFMA: n_groups loads (one a group),
    group i after MFMA i * n / n_groups (phase's placement)."""
    n = len(mfmas)
    out = {}
    for kk in range(NKK):
        first = next(i for i, (f, _) in enumerate(mfmas) if f == 2 * kk)
        issued = sum(1 for g in range(n_groups) if g * n // n_groups < first)
        out[2 * kk] = [f"s_waitcnt vmcnt({2 * (NKK - 1 - kk) + issued})"]
    return out


def early_dma():
    """The LDS DMA loads of tiles 1 and 2 as one (groups, tail) for tile 0's exact path: they are not needed before
    the first iteration, so they go out between tile 0's score MFMAs instead of ahead of them (issuing them held the
    prologue for ~4000 cycles). Sparse: each tile's first key (SD) from the pass table's entries 1 and 2, then entry
    3's for the loop's first staging."""
    g1, t1 = dma_groups()
    g2, t2 = dma_groups()
    if SPARSE:
        g1 = [["s_mov_b32 %s, s89" % SD] + g1[0]] + g1[1:]
        g2 = [["s_mov_b32 %s, s90" % SD] + g2[0]] + g2[1:]
        t2 = t2 + ["s_mov_b32 %s, s91" % SD]
    return g1 + [t1 + g2[0]] + g2[1:], t2


def exact_tile(e, dtype, sbuf, kaddr, j0, first=False, w=None):
    """The exact path for a tile (K at LDS address kaddr, first key in scalar j0): its raw scores into S(sbuf), the
    mask, each row's maximum, the reference's rule for moving the running maximum (outputs and sums rescaled when it
    moves), the exponentials, P and the sums (TMP[0], TMP[4]). first: the wave's first tile, where the outputs and
    sums are still zero and need no rescaling, Q is still arriving (q_waits), and tiles 1 and 2 are staged
    between its MFMAs (early_dma)."""
    mfmas = qk_mfmas(dtype, sbuf)
    dma = early_dma() if first else None
    phase(e, "X", k_reads(kaddr), mfmas, [], fwait=q_waits(mfmas, len(dma[0])) if first else None, dma=dma)
    for op in wait_mfma() + (mask_general(sbuf, j0, w) if SPARSE else mask(sbuf, j0)):
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
        if not first:
            e(f"v_mul_f32 {LSUM[rb]}, {LSUM[rb]}, {f}")
    # rescale the outputs (the MFMAs that wrote them were issued before the last barrier)
    for rb in range(2 if not first else 0):
        f = TMP[8 + rb]
        for i in range(16 * NDB):
            a, tv = f"a{16 * NDB * rb + i}", TMP[10 + (i % 4)]
            e(f"v_accvgpr_read_b32 {tv}, {a}")
            e(f"v_mul_f32 {tv}, {tv}, {f}")
            e(f"v_accvgpr_write_b32 {a}, {tv}")
    for op in exps(sbuf) + pack_and_sum(sbuf, dtype):
        e(op)


def low_part_pass(e):
    """bf16 inputs: tile 0's P V once more with the parts of the probabilities that bf16 P drops, when some row of
    the wave may see few keys. P V multiplies probabilities rounded to bf16 (8 significant bits, relative error up to
    2^-8); a row that sees many keys averages those roundings away, but a row that sees a handful does not (a few keys of comparable weight whose
    values cancel leave errors of ~2^-9 |v| on a small output). In dense attention a row sees a prefix of the keys, so
    a row that sees fewer than 64 sees only tile 0's: adding V^T(0) P_lo^T, P_lo = bf16(p - P) of tile 0's f32
    exponentials p, gives those rows probabilities to ~16 bits. Taken when the wave's first row (the fewest keys: the
    row limit grows with the row) sees fewer than 64 keys; sparse: when the stream's tile 0 is not a pass all of whose
    64 keys every row sees (the order puts such a pass first when the list has one). Runs before iteration 0, in
    S(1)'s registers (free until its phase QK), from buffer 0 (tile 0's V)."""
    skip = lbl("L_nolo")
    if SPARSE:
        t = SROT["k"]
        e(f"s_and_b32 {t}, s78, s79")
        e(f"s_cmp_eq_u32 {t}, -1")
        e(f"s_cbranch_scc0 {lbl('L_lo')}")
        e(f"s_add_u32 {t}, s76, 64")
        e(f"s_cmp_le_u32 {t}, %[lmin]")
        e(f"s_cbranch_scc1 {skip}")
        e.label("L_lo")
    else:
        e("s_cmp_ge_u32 %[lmin], 64")
        e(f"s_cbranch_scc1 {skip}")
    lo = {}
    ops_a, ops_b, ops_c = [], [], []
    k = 0
    for rb in range(2):
        for cc in range(4):
            t, r0 = cc // 2, 8 * (cc % 2)
            for i in range(4):
                hi, lr, tr = P(rb, cc, i), f"v{64 + 16 * rb + 4 * cc + i}", f"v{96 + k}"
                a, b = S(0, rb, t, r0 + 2 * i), S(0, rb, t, r0 + 2 * i + 1)
                ops_a += [f"v_lshlrev_b32 {lr}, 16, {hi}", f"v_and_b32 {tr}, 0xffff0000, {hi}"]
                ops_b += [f"v_sub_f32 {lr}, {a}, {lr}", f"v_sub_f32 {tr}, {b}, {tr}"]
                ops_c.append(f"v_cvt_pk_bf16_f32 {lr}, {lr}, {tr}")
                k += 1
    for op in ops_a + ops_b + ops_c:
        e(op)
    mfmas = []
    for f in range(4 * NDB):
        cc, db = f // NDB, f % NDB
        for rb in range(2):
            plo = f"v[{64 + 16 * rb + 4 * cc}:{64 + 16 * rb + 4 * cc + 3}]"
            mfmas.append((f, f"v_mfma_f32_32x32x16_bf16 {O(rb, db)}, {{ring}}, {plo}, {O(rb, db)}"))
    interleave(e, v_reads(), mfmas, [])
    e.label("L_nolo")


def epilogue(e, out_dtype):
    """Normalise and store this wave's rows of O, then the LSE. The rows go through LDS (free once every wave has
    passed the barrier here with its loads landed): each lane writes its 4-dim pieces of rows c32 and c32 + 32 into
    the wave's region (row-major, 16-byte chunk c of row R at c ^ (R % 8), so the writes of a row group hit distinct
    banks), then reads back whole-row chunks, so each global store writes 1 KiB of contiguous row segments (4 rows of
    bf16 / f16, 2 of f32) instead of 16 bytes of each of 32 rows. The stores are non-temporal (O is not read again
    here): measured against plain stores, 3 % off the block-sparse S16384 call and ~1 % off the S4096 prefill. Rows
    past n_q fall outside the output buffer and are dropped; LSE offsets of rows past n_q are outside its buffer."""
    e("s_waitcnt vmcnt(0) lgkmcnt(0)")
    e("s_barrier")
    if SPARSE:
        # rows past n_q are dropped (%[mlive] is 0 for them)
        e("v_cmp_ne_u32 vcc, 0, %[mlive]")
        e("s_nop 1")
        e(f"v_cndmask_b32 {MAPV}, -1, {MAPV}, vcc")
    for op in wait_mfma():
        e(op)
    sz = {"f32": 4, "bf16": 2, "f16": 2}[out_dtype]
    row = D * sz
    inv = (TMP[1], TMP[2])
    for rb in range(2):
        lt = TMP[0]
        e(f"ds_bpermute_b32 {lt}, %[swp], {LSUM[rb]}")
        e("s_waitcnt lgkmcnt(0)")
        e(f"v_add_f32 {lt}, {lt}, {LSUM[rb]}")
        e(f"v_rcp_f32 {inv[rb]}, {lt}")
        e(f"v_cmp_lt_f32 vcc, 0, {lt}")
        e("s_nop 1")
        e(f"v_cndmask_b32 {inv[rb]}, {ZERO}, {inv[rb]}, vcc")
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
    # writes: piece (rb, db, r4) is head dims 32 db + 8 r4 + 4 g .. + 3 of row 32 rb + c32; its address is
    # %[ew] ^ (16 x its chunk without the lane's part), %[ew] holding the row, the lane's part and the swizzle
    n = 0
    for rb in range(2):
        for db in range(NDB):
            for r4 in range(4):
                vals = [f"v{4 * n + i}" for i in range(4)]
                addr = f"v{128 + n}"
                for i in range(4):
                    e(f"v_accvgpr_read_b32 {vals[i]}, {O(rb, db, 4 * r4 + i)}")
                for i in range(4):
                    e(f"v_mul_f32 {vals[i]}, {vals[i]}, {inv[rb]}")
                chunk = 4 * db + r4 if sz == 2 else 8 * db + 2 * r4
                e(f"v_xor_b32 {addr}, {16 * chunk}, %[ew]")
                if sz == 4:
                    e(f"ds_write_b128 {addr}, v[{4 * n}:{4 * n + 3}] offset:{32 * row * rb}")
                else:
                    cvt = "v_cvt_pk_bf16_f32" if out_dtype == "bf16" else "v_cvt_pk_f16_f32"
                    e(f"{cvt} {vals[0]}, {vals[0]}, {vals[1]}")
                    e(f"{cvt} {vals[1]}, {vals[2]}, {vals[3]}")
                    e(f"ds_write_b64 {addr}, v[{4 * n}:{4 * n + 1}] offset:{32 * row * rb}")
                n += 1
    e("s_waitcnt lgkmcnt(0)")
    # reads: load i covers rows (rows_i) i .. of the wave's 64 (16 lanes a row for 2-byte outputs, 32 for f32); the
    # lane's chunk swizzle depends on the row through i, folded in by an xor of %[er]
    rows_i = 1024 // row
    n_ld = 64 // rows_i
    for i in range(n_ld):
        swz = ((rows_i * i) & 7) * 16
        addr = f"v{128 + i}"
        e(f"v_xor_b32 {addr}, {swz}, %[er]")
        e(f"ds_read_b128 v[{4 * i}:{4 * i + 3}], {addr} offset:{1024 * i}")
    if SPARSE:
        # output row map[q0 + row] from the lane holding it (MAPV), as a 64-bit address: row x (width x bytes) +
        # %[ocol] (o, the head's columns and the lane's chunk); dropped rows (-1) are left out of exec for their store
        for i in range(n_ld):
            a = f"v{128 + i}"
            e(f"v_add_u32 {a}, {4 * rows_i * i}, %[mp]")
            e(f"ds_bpermute_b32 {a}, {a}, {MAPV}")
        e("s_waitcnt lgkmcnt(0)")
        pairs = [(int(TMP[8 + 2 * k][1:]), int(TMP[9 + 2 * k][1:])) for k in range(4)]
        for i in range(n_ld):
            a = f"v{128 + i}"
            lo, hi = pairs[i % 4]
            e(f"v_mad_u64_u32 v[{lo}:{hi}], {SCMP[1]}, {a}, %[ows], %[ocol]")
            e(f"v_cmp_le_i32 vcc, 0, {a}")
            e("s_nop 1")
            e(f"s_and_saveexec_b64 {SCMP[0]}, vcc")
            e(f"global_store_dwordx4 v[{lo}:{hi}], v[{4 * i}:{4 * i + 3}], off nt")
            e(f"s_mov_b64 exec, {SCMP[0]}")
        return
    # global addresses alternate between two registers, each moved on by two loads' rows after its store
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

def body(in_dtype, out_dtype, sparse=False, d=128):
    """The stream for one item (a workgroup's rows) at head width d; sparse: the block-sparse one (tiles from the
    pass table, heads of 128)."""
    global SPARSE
    assert d == 128 or not sparse
    SPARSE = sparse
    set_dim(d)
    try:
        return body_of(in_dtype, out_dtype)
    finally:
        SPARSE = False
        set_dim(128)


def body_of(in_dtype, out_dtype):
    e = Emit()
    if SPARSE:
        # the pass table's first entries: the first keys of tiles 0-3, entry 1 (iteration 0 masks tile 1), entry 0
        # (tile 0's exact path, in ST); and the row map
        for i, r in enumerate(("s88", "s89", "s90", "s91")):
            e(f"s_load_dword {r}, %[ent], {16 * i}")
        e(f"s_load_dword {SEJ}, %[ent], 16")
        e(f"s_load_dwordx2 {SEW}, %[ent], 24")
        e(f"s_load_dwordx4 s[76:79], %[ent], 0")
        e(f"buffer_load_dword {MAPV}, %[mo], %[mrs], 0 offen")
    e(f"s_mov_b32 {S256}, 0x43800000")
    for r in TMP[8:12]:   # zeros for the MFMAs that clear the outputs
        e(f"v_mov_b32 {r}, 0")
    e(f"v_mov_b32 {NINF}, 0xff800000")
    e(f"v_mov_b32 {ZERO}, 0")
    for rb in range(2):
        e(f"v_mov_b32 {NEGMU[rb]}, 0")
        e(f"v_mov_b32 {LSUM[rb]}, 0")
        e(f"v_mov_b32 {MAXV[rb]}, {NINF}")
    # load sources of tile 0
    for r, pre in ((KRS, "k"), (VRS, "v")):
        e(f"s_mov_b32 {r[0]}, %[{pre}b0]")
        e(f"s_mov_b32 {r[1]}, %[{pre}b1]")
        e(f"s_mov_b32 {r[2]}, %[{pre}n]")
        e(f"s_mov_b32 {r[3]}, 0x20000")
    e(f"s_mov_b32 {SBW}, 0")
    # M0 is the compiler's: kept in SM0 while the stream uses it, restored at the end
    e(f"s_mov_b32 {SM0}, m0")
    # tile 0 into buffer 0, then Q into the accumulator registers (rows past n_q load as zeros); outputs zeroed
    # meanwhile; tiles 1 and 2 go into buffers 1 and 2 between tile 0's score MFMAs (early_dma). Loads retire in
    # order: the first barrier waits for tile 0 only, tile 0's score MFMAs each wait for the Q pair they use
    # (q_waits), and a barrier after tile 0 for tile 1.
    e(f"s_mov_b32 {SKW}, %[skw]")
    e(f"s_mov_b32 {SKWW}, %[skww]")
    e(f"s_mov_b32 {SVWW}, %[svww]")
    if SPARSE:
        e("s_waitcnt lgkmcnt(0)")
    if SPARSE:
        e(f"s_mov_b32 {SD}, s88")
    for op in dma_issue():
        e(op)
    e(f"v_add_u32 {TMP[0]}, {64 * D:#x}, %[qo]")   # row block 1: 32 rows of 2 d bytes on
    for kk in range(NKK):
        for rb in range(2):
            e(f"buffer_load_dwordx4 {Q(rb, kk)}, {'%[qo]' if rb == 0 else TMP[0]}, %[qrs], 0 offen "
              f"offset:{32 * kk}")
    # the outputs cleared by MFMAs of zero operands: a few issue slots, the matrix unit does the rest (128
    # v_accvgpr_write took ~700 cycles of the prologue)
    z = f"v[{TMP[8][1:]}:{TMP[11][1:]}]"
    for i in range(2 * NDB):
        e(f"v_mfma_f32_32x32x16_{in_dtype} a[{16 * i}:{16 * i + 15}], {z}, {z}, 0")
    body_rest(e, in_dtype, out_dtype)
    return e.out


def body_rest(e, in_dtype, out_dtype):
    e(f"s_mov_b32 {SJ}, 0")
    e(f"s_mov_b32 {SBK}, 0")
    e(f"s_mov_b32 {SBV}, 0")
    # the first barrier: every wave's loads of tile 0 have landed (Q may still be in flight)
    e(f"s_waitcnt vmcnt({2 * NKK}) lgkmcnt(0)")
    e("s_barrier")
    e("s_cmp_eq_u32 %[ntw], 0")
    e(f"s_cbranch_scc0 {lbl('L_live')}")
    # a wave with no rows: its share of tiles 1 and 2, the barrier for tile 1 as the others, then the load-only loop
    groups, tail = early_dma()
    for op in sum(groups, []) + tail + barrier():
        e(op)
    e(f"s_branch {lbl('L_tail')}")
    e.label("L_live")
    # tile 0 by the exact path
    if SPARSE:
        exact_tile(e, in_dtype, 0, "%[kr]", ST[0], first=True, w="s[78:79]")
    else:
        e(f"s_mov_b32 {SJX}, 0")
        exact_tile(e, in_dtype, 0, "%[kr]", SJX, first=True)
    e(f"v_add_f32 {LSUM[0]}, {LSUM[0]}, {TMP[0]}")
    e(f"v_add_f32 {LSUM[1]}, {LSUM[1]}, {TMP[4]}")
    if in_dtype == "bf16":
        low_part_pass(e)
    for op in barrier():   # every wave's loads of tile 1 have landed
        e(op)

    def iteration(par, variant, masked_next=False):
        """Iteration j with S_cur = S(par), S_nxt = S(1 - par). variant: 'plain' (tile j + 1 fully seen by the
        wave's rows), 'masked' (by the row limits), 'general' (sparse: the limits and the validity words), 'last'
        (no tile j + 1), 'first' (j = 0: tile 0's P and sums came from the exact path; masked_next: tile 1's mask
        kind). Reads run across the phases: V^T(j)'s first reads go out in phase
        QK's tail, and phase PV holds barrier j (after its V^T reads have landed) and then the first reads of
        K(j + 2) for the next iteration's phase QK."""
        cur, nxt = par, 1 - par
        tag = f"{variant}{par}"
        # the staging of tile j + 3: DMA loads spread between phase QK's MFMAs
        dma = dma_groups() if variant != "last" else None
        valu = []
        if variant != "first":
            valu += pack_and_sum(cur, in_dtype)
        n_v = 0
        if variant != "last":
            n_v = phase(e, "K", k_reads("%[kr]"), qk_mfmas(in_dtype, nxt), valu, pre=0 if variant == "first" else N_K_AHEAD,
                        nxt=("V", v_reads()), dma=dma)
        else:
            # the wave's last tile, but the workgroup's other waves may still read tile j + 3 (a wave of 64 rows
            # sees up to three tiles fewer than the workgroup's last): its share is staged here as in any iteration,
            # so the barriers' waits keep their meaning (barrier j + 1 waits for it)
            for op in valu + iteration_last_staging():
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
            exact_v[tag] = n_v
        if variant != "last":
            for op in rotate(SBK, "k", KREGS, K_TILE):
                e(op)
        # phase PV, with barrier j
        valu = []
        if variant != "last":
            kind = masked_next or variant
            m = mask(nxt, SJ0) if kind == "masked" else mask_general(nxt, SJ0, SEW) if kind == "general" else []
            # sparse: the next entries load once this phase has read SEW (the general mask's third instruction)
            loads = entry_loads() if SPARSE else []
            valu = ["s_nop 7", "s_nop 7"] + m[:3] + loads + m[3:] + exps(nxt)
        elif SPARSE:
            valu = entry_loads()
        n_k = phase(e, "V", v_reads(), pv_mfmas(in_dtype), valu, pre=n_v, nxt=None if variant == "last" else ("K", k_reads("%[kr]")),
                    gate_at=BAR_AT, gate=barrier())
        assert variant == "last" or n_k == N_K_AHEAD
        for op in rotate(SBV, "v", VREGS, V_TILE):
            e(op)

    exact_v = {}

    def exact_block(par, variant):
        tag = f"{variant}{par}"
        e.label(f"L_exact_{tag}")
        # K of tile j is in buffer SBV (the buffer whose V^T is read next)
        e(f"s_mul_i32 {ST[0]}, {SBV}, {K_TILE}")
        e(f"v_add_u32 {TMP[15]}, {ST[0]}, %[kr0]")
        if SPARSE:
            # tile j's entry (its first key and validity words) into ST
            e(f"s_lshl_b32 {SROT['wk']}, {SJ}, 4")
            e(f"s_load_dwordx4 s[76:79], %[ent], {SROT['wk']}")
            e("s_waitcnt lgkmcnt(0)")
            exact_tile(e, in_dtype, par, TMP[15], ST[0], w="s[78:79]")
        else:
            e(f"s_lshl_b32 {SJX}, {SJ}, 6")
            exact_tile(e, in_dtype, par, TMP[15], SJX)
        e(f"v_add_f32 {LSUM[0]}, {LSUM[0]}, {TMP[0]}")
        e(f"v_add_f32 {LSUM[1]}, {LSUM[1]}, {TMP[4]}")
        # the V^T reads phase QK sent ahead (their ring slots were reused here), again, as the last LDS instructions
        reads = v_reads()
        for f in range(exact_v[tag]):
            for text in reads[f]:
                e(ring_fmt(text, f % RING))
        e(f"s_branch {lbl('L_back_' + tag)}")

    def dispatch(par, first=False):
        """The variant of iteration SJ: this wave's last, one whose next tile needs the mask, plain (sparse: also
        one whose next tile has keys that are not valid)."""
        name = "first" if first else f"iter{par}"
        e.label(f"L_{name}")
        e(f"s_add_u32 {ST[1]}, {SJ}, 1")
        e(f"s_cmp_ge_u32 {ST[1]}, %[ntw]")
        e(f"s_cbranch_scc1 {lbl(f'L_last_{name}')}")
        if SPARSE:
            e(f"s_mov_b32 {SJ0}, {SEJ}")
            e(f"s_and_b32 {ST[2]}, {SEW_LO}, {SEW_HI}")
            e(f"s_cmp_eq_u32 {ST[2]}, -1")
            e(f"s_cbranch_scc0 {lbl(f'L_general_{name}')}")
        else:
            e(f"s_lshl_b32 {SJ0}, {ST[1]}, 6")
        e(f"s_add_u32 {ST[2]}, {SJ0}, 64")
        e(f"s_cmp_le_u32 {ST[2]}, %[lmin]")
        e(f"s_cbranch_scc0 {lbl(f'L_masked_{name}')}")
        iteration(par, "first" if first else "plain")
        e(f"s_branch {lbl(f'L_next_{name}')}")
        e.label(f"L_masked_{name}")
        if first:
            iteration(0, "first", masked_next="masked")
        else:
            iteration(par, "masked")
        if SPARSE:
            e(f"s_branch {lbl(f'L_next_{name}')}")
            e.label(f"L_general_{name}")
            if first:
                iteration(0, "first", masked_next="general")
            else:
                iteration(par, "general")
        e.label(f"L_next_{name}")
        e(f"s_add_u32 {SJ}, {SJ}, 1")

    for op in rotate(SBK, "k", KREGS, K_TILE):
        e(op)
    dispatch(0, first=True)
    dispatch(1)
    dispatch(0)
    e(f"s_branch {lbl('L_iter1')}")
    # the last iteration of the wave, by entry point
    e.label("L_last_first")
    for op in staging():
        e(op)
    phase(e, "V", v_reads(), pv_mfmas(in_dtype), [], gate_at=BAR_AT, gate=barrier())
    for op in rotate(SBV, "v", VREGS, V_TILE):
        e(op)
    e(f"s_add_u32 {SJ}, {SJ}, 1")
    e(f"s_branch {lbl('L_tail')}")
    for par in (1, 0):
        e.label(f"L_last_iter{par}")
        iteration(par, "last")
        e(f"s_add_u32 {SJ}, {SJ}, 1")
        e(f"s_branch {lbl('L_tail')}")
    for par in (0, 1):
        for variant in ("plain", "masked", "last") + (("general",) if SPARSE else ()):
            exact_block(par, variant)
    # load-only iterations for the tiles the workgroup's other waves still compute: the staging of iteration SJ,
    # then its barrier
    e.label("L_tail")
    e("s_cmp_ge_u32 %s, %%[nt]" % SJ)
    e(f"s_cbranch_scc1 {lbl('L_epi')}")
    if SPARSE:
        e(f"s_lshl_b32 {ST[0]}, {SJ}, 4")
        e(f"s_add_u32 {ST[0]}, {ST[0]}, 48")
        e(f"s_load_dword {SD}, %[ent], {ST[0]}")
        e("s_waitcnt lgkmcnt(0)")
    for op in staging() + barrier():
        e(op)
    e(f"s_add_u32 {SJ}, {SJ}, 1")
    e(f"s_branch {lbl('L_tail')}")
    e.label("L_epi")
    epilogue(e, out_dtype)
    e(f"s_mov_b32 m0, {SM0}")


def clobbers(sparse=False):
    regs = [f'"v{i}"' for i in range(CLOBBER_V_SPARSE if sparse else CLOBBER_V)]
    regs += [f'"a{i}"' for i in range(CLOBBER_A)]
    regs += [f'"s{i}"' for i in range(*(CLOBBER_S_SPARSE if sparse else CLOBBER_S))]
    return ", ".join(regs)


def check_registers(lines, sparse=False):
    """Every register the stream names must be one the clobber list reserves (the wave is only given those)."""
    import re
    for ln in lines:
        for kind, one, lo, hi in re.findall(r"\b([vas])(?:(\d+)|\[(\d+):(\d+)\])", ln.split(";")[0]):
            top = int(one) if one else int(hi)
            bot = int(one) if one else int(lo)
            limit = {"v": (0, CLOBBER_V_SPARSE if sparse else CLOBBER_V), "a": (0, CLOBBER_A),
                     "s": CLOBBER_S_SPARSE if sparse else CLOBBER_S}[kind]
            assert limit[0] <= bot and top < limit[1], f"{kind}{bot}..{top} outside the reserved registers: {ln}"
            assert one or bot % 2 == 0, f"{kind}[{bot}:{top}]: a register tuple must start on an even register: {ln}"


def main():
    out = ["// Generated by gen_attn_fwd64.py (the instruction stream of flash_fwd_r64; the design is described there).",
           "// Do not edit: change the generator and run it.", "#pragma once", ""]
    kinds = [(False, 128), (True, 128), (False, 64)]
    for sparse, d in kinds:
        for ind in ("bf16", "f16"):
            for outd in ("f32", ind):
                lines = body(ind, outd, sparse, d)
                check_registers(lines, sparse)
                kind = "SPARSE64" if sparse else "FWD64" if d == 128 else "FWD64_D64"
                name = f"MAKO_{kind}_ASM_{ind.upper()}_{outd.upper()}"
                out.append(f"#define {name} \\")
                for ln in lines:
                    out.append(f'    "{ln}\\n" \\')
                out.append('    ""')
                out.append("")
    out.append(f"#define MAKO_FWD64_CLOBBERS {clobbers()}")
    out.append(f"#define MAKO_SPARSE64_CLOBBERS {clobbers(True)}")
    out.append(f"#define MAKO_FWD64_NBUF {NBUF}")
    out.append("")
    with open(os.path.join(HERE, "attn_fwd64_asm.inc"), "w") as f:
        f.write("\n".join(out))


if __name__ == "__main__":
    main()
