"""Runs flash_sparse_r64's generated stream (gen_attn_fwd64.py, sparse=True) on the emulator (fwd64_emu.py) for a
small block-sparse case, with the pass table and the per-lane operands attn_sparse64.hip computes restated here, and
compares the outputs (through the row map) and the LSE with the oracle's."""
import time

import numpy as np

import fwd64_emu as E
import fwd64_run as R
import gen_attn_fwd64 as G
import oracle as O

NONE = 0xFFFFFFFF

VOPS = ['ocol', 'ocol_hi', 'kr', 'vr0', 'vr1', 'kd0', 'kd1', 'kd2', 'kd3', 'kd4', 'vd', 'lim0', 'lim1',
        'kr0', 'qo', 'lo0', 'lo1', 'swp', 'ew', 'er', 'mp', 'mlive', 'mo', 'g32']
SOPS = {'qrs': 's[0:3]', 'lrs': 's[4:7]', 'mrs': 's[8:11]', 'ent': 's[12:13]', 'c': 's20', 'nt': 's21', 'ntw': 's22',
        'lmin': 's23', 'has_lse': 's24', 'ows': 's25', 'kb0': 's26', 'kb1': 's27', 'kn': 's28', 'vb0': 's29',
        'vb1': 's30', 'vn': 's31', 'skw': 's32', 'skww': 's33', 'svww': 's34'}
VREG = {n: f'v{G.CLOBBER_V_SPARSE + 1 + i}' for i, n in enumerate(VOPS)}  # + 1: an even register pair for ocol


def program(ind, outd):
    lines = G.body(ind, outd, sparse=True)
    lo = int(VREG['ocol'][1:])
    assert lo % 2 == 0
    out = []
    for ln in lines:
        ln = ln.replace('%=', '0').replace('%[ocol]', f'v[{lo}:{lo + 1}]')
        for n, r in VREG.items():
            ln = ln.replace(f'%[{n}]', r)
        for n, r in SOPS.items():
            ln = ln.replace(f'%[{n}]', r)
        out.append(ln)
    return E.parse(out)


def pass_table(sel, nsel, valid, *, n_q, n_k, kv_heads, n_cubes, max_sel, dense0, dense1, causal):
    """The pass table of every (kv head, query tile) list: entry ps = {first key (-1: none), 0, W0, W1}, -1 entries
    past the list (at least 4). A pass's keys: its cube's 64 (ps < ns) or a 64-key step of the dense rows; a key may
    be seen when it is before the pass's end and valid; a causal pass wholly after the tile's rows is none; the first
    pass that neither the causal bound nor the pass's end cuts trades places with pass 0."""
    n_qt = (n_q + 63) // 64
    nd_c = (dense1 - dense0 + 63) // 64 if dense1 > dense0 else 0
    nd_l = (n_k + 63) // 64 if n_qt > n_cubes else 0
    n_ent = max(max_sel + nd_c, nd_l) + 4
    table = np.zeros((kv_heads, n_qt, n_ent, 4), np.uint32)
    table[..., 0] = NONE
    counts = np.zeros((kv_heads, n_qt), np.uint32)
    g = np.arange(2)[:, None]
    e = np.arange(32)[None, :]
    key_of = 32 * (e // 16) + 16 * ((e % 16) >> 3) + 8 * g + (e % 8)  # [g][bit]
    for kvh in range(kv_heads):
        for qt in range(n_qt):
            cube = qt < n_cubes
            ns = min(int(nsel[kvh, qt]), max_sel) if cube else 0
            lo, hi_all = (dense0, dense1) if cube else (0, n_k)
            nd = (hi_all - lo + 63) // 64 if hi_all > lo else 0
            counts[kvh, qt] = ns + nd

            def rng_of(i):
                if i < ns:
                    return int(sel[kvh, qt, i]) * 64, int(sel[kvh, qt, i]) * 64 + 64
                j = lo + (i - ns) * 64
                return j, min(j + 64, hi_all)
            # the first pass no bound cuts trades places with pass 0
            first = next((i for i in range(ns + nd) if rng_of(i)[1] == rng_of(i)[0] + 64 and
                          not (causal and rng_of(i)[0] + 64 > 64 * qt + 1)), ns + nd)
            for ps in range(ns + nd):
                src = ps if first == ns + nd else first if ps == 0 else 0 if ps == first else ps
                j0, hi = rng_of(src)
                if causal and j0 > 64 * qt + 63:
                    continue
                keys = j0 + np.arange(64)
                ok = (keys < hi) & (valid[np.minimum(keys, len(valid) - 1)] != 0) & (keys < len(valid))
                w = [int(sum(int(ok[key_of[gg, b]]) << b for b in range(32))) for gg in range(2)]
                table[kvh, qt, ps] = (j0, 0, w[0], w[1])
    return table, counts


def run(heads, kv, sel, nsel, valid, map_, *, n_q, q_pad, n_k, k_pad, n_cubes, max_sel, dense0, dense1, causal,
        ind='bf16', outd='f32', seed=0, verbose=True):
    rng = np.random.default_rng(seed)
    dt = O.BF16 if ind == 'bf16' else O.F16
    conv = O.to_bf16_bits if ind == 'bf16' else O.to_f16_bits
    qb = conv(rng.standard_normal((heads, q_pad, 128), dtype=np.float32))
    kb = conv(rng.standard_normal((kv, k_pad, 128), dtype=np.float32))
    vb = conv(rng.standard_normal((kv, k_pad, 128), dtype=np.float32))
    width = heads * 128
    so = 4 if outd == 'f32' else 2
    o_rows = q_pad
    table, counts = pass_table(sel, nsel, valid, n_q=n_q, n_k=n_k, kv_heads=kv, n_cubes=n_cubes, max_sel=max_sel,
                               dense0=dense0, dense1=dense1, causal=causal)
    n_qt, n_ent = table.shape[1], table.shape[2]
    mp32 = np.asarray(map_, np.int32)
    sizes = [qb.nbytes, kb.nbytes, vb.nbytes, o_rows * width * so + 4096, heads * q_pad * 4 + 4096,
             table.nbytes + 4096, mp32.nbytes + 4096]
    offs = np.cumsum([4096] + [((x + 4095) // 4096) * 4096 for x in sizes])
    Q0, K0, V0, O0, L0, T0, M0 = [int(x) for x in offs[:7]]
    mem = E.Mem(int(offs[-1]) + 4096)
    for base, arr in ((Q0, qb), (K0, kb), (V0, vb), (T0, table), (M0, mp32)):
        mem.b[base:base + arr.nbytes] = arr.view(np.uint8).ravel()
    sentinel = np.full(o_rows * width, 1234.5, np.float32) if so == 4 else conv(np.full(o_rows * width, 1234.5,
                                                                                        np.float32))
    mem.b[O0:O0 + sentinel.nbytes] = sentinel.view(np.uint8)
    prog, labels = program(ind, outd)
    group = heads // kv
    assert group % 4 == 0
    n_hg = heads // 4
    c = np.float32(1.0 / np.sqrt(128.0)) * np.float32(1.4426950408889634)
    lane = np.arange(64)
    g, c32 = lane >> 5, lane & 31
    lbase = 0
    vbase = lbase + G.NBUF * G.K_TILE
    t0 = time.time()
    n_instr = 0
    early = 0
    big = 0x7FFFFFFF
    for qt in range(n_qt):
        for hg in range(n_hg):
            emu = E.Emu(prog, labels, mem, G.NBUF * (G.K_TILE + G.V_TILE))
            waves = []
            kvh = hg * 4 // group
            nt = int(counts[kvh, qt])
            q0 = 64 * qt
            for w in range(4):
                W = E.Wave(w)
                h = hg * 4 + w
                rows0 = q0 + c32
                if causal:
                    lim0, lim1, lmin = rows0 + 1 - 8 * g, rows0 + 33 - 8 * g, q0 + 1
                else:
                    lim0, lim1, lmin = np.full(64, big), np.full(64, big), big
                kr = lbase + c32 * G.K_ROW + 16 * g
                vr = R.v_read_regs(vbase, 128, lane)

                def kd_of(i):
                    b = 1024 * i + 16 * lane
                    Rr, cc = b // G.K_ROW, (b % G.K_ROW) // 16
                    return np.array([R.slot_of(int(r)) for r in Rr]) * 256 + 16 * np.where(cc < 16, cc, 0)
                kds = [kd_of(w + 4 * m) for m in range(4)] + [kd_of(16)]
                orow = 128 * so
                lpr = orow // 16
                obase = lbase + w * 64 * orow
                if so == 4:
                    ew = obase + c32 * orow + 16 * ((c32 & 7) ^ g)
                else:
                    ew = obase + c32 * orow + 8 * g + 16 * (c32 & 7)
                er = obase + (lane // lpr) * orow + 16 * ((lane % lpr) ^ (lane // lpr))
                ocol = O0 + h * orow + 16 * (lane % lpr)
                vals = dict(kr=kr, vr0=vr[0], vr1=vr[1], kd0=kds[0], kd1=kds[1], kd2=kds[2],
                            kd3=kds[3], kd4=kds[4], vd=4096 * w + R.vd_lane(128, lane), lim0=lim0, lim1=lim1, kr0=kr,
                            qo=((q0 + c32) * 128 + 8 * g) * 2,
                            lo0=np.where(q0 + c32 < n_q, (h * q_pad + q0 + c32) * 4, NONE),
                            lo1=np.where(q0 + 32 + c32 < n_q, (h * q_pad + q0 + 32 + c32) * 4, NONE),
                            swp=(lane ^ 32) * 4, ew=ew, er=er, mp=4 * (lane // lpr), ocol=ocol & 0xFFFFFFFF,
                            ocol_hi=ocol >> 32, mlive=(q0 + lane < n_q).astype(np.int64), mo=(q0 + lane) * 4,
                            g32=32 * g)
                for n, arr in vals.items():
                    W.v[int(VREG[n][1:])] = np.asarray(arr, np.int64).astype(np.uint32) if np.ndim(arr) else \
                        np.full(64, int(arr) & 0xFFFFFFFF, np.uint32)

                def rs(sidx, base, nbytes):
                    W.s[sidx] = base & 0xFFFFFFFF
                    W.s[sidx + 1] = (base >> 32) & 0xFFFF
                    W.s[sidx + 2] = nbytes & 0xFFFFFFFF
                    W.s[sidx + 3] = 0x00020000
                rs(0, Q0 + h * q_pad * 256, n_q * 256)
                rs(4, L0, heads * q_pad * 4)
                rs(8, M0, n_q * 4)
                ent = T0 + ((kvh * n_qt + qt) * n_ent) * 16
                W.s[12], W.s[13] = ent & 0xFFFFFFFF, ent >> 32
                kbase = K0 + kvh * k_pad * 256
                ibase = V0 + kvh * k_pad * 256
                W.s[26], W.s[27], W.s[28] = kbase & 0xFFFFFFFF, (kbase >> 32) & 0xFFFF, 0
                W.s[29], W.s[30], W.s[31] = ibase & 0xFFFFFFFF, (ibase >> 32) & 0xFFFF, 0
                W.s[32], W.s[33], W.s[34] = lbase, lbase + 1024 * w, vbase + 4096 * w
                W.s[20] = int(np.float32(c).view(np.uint32))
                W.s[21], W.s[22], W.s[23], W.s[24], W.s[25] = nt, nt, lmin & 0xFFFFFFFF, 1, width * so
                waves.append(W)
            emu.run_wg(waves)
            n_instr += emu.count
            early += emu.early
    if verbose:
        print(f'emulated {n_instr} wave-instructions in {time.time() - t0:.1f} s')
    if so == 4:
        o = mem.b[O0:O0 + o_rows * width * 4].view(np.float32).reshape(o_rows, width).astype(np.float64)
    else:
        o = O.bits_to_f32(mem.b[O0:O0 + o_rows * width * 2].view(np.uint16), dt).reshape(o_rows, width)
        o = o.astype(np.float64)
    lse = mem.b[L0:L0 + heads * q_pad * 4].view(np.float32).reshape(heads, q_pad).astype(np.float64)
    want_o, want_l = O.attn_sparse(qb, kb, vb, sel, nsel, valid, map_, n_q=n_q, q_pad=q_pad, n_k=n_k, k_pad=k_pad,
                                   heads=heads, kv_heads=kv, n_cubes=n_cubes, max_sel=max_sel, dense0=dense0,
                                   dense1=dense1, causal=causal, sel_heads=kv, dtype=dt,
                                   o_fill=np.full((o_rows, width), 1234.5))
    written = np.zeros(o_rows, bool)
    written[mp32[:n_q][mp32[:n_q] >= 0]] = True
    sent = float(o[~written].ravel()[0]) if (~written).any() else 1234.5
    err = np.abs(o - want_o)
    bad = ~(err <= 2e-3 + 1e-2 * np.abs(want_o)) & written[:, None]
    rows = np.nonzero(mp32[:n_q] >= 0)[0]
    lerr = np.abs(lse[:, rows] - want_l[:, rows])
    lbad = ~(lerr <= 1e-3) & np.isfinite(want_l[:, rows])
    sent16 = float(O.bits_to_f32(conv(np.full(1, 1234.5, np.float32)), dt)[0])
    untouched = int((o[~written] != sent).sum()) + int(sent not in (1234.5, sent16))
    if verbose:
        print(f'sparse h{heads} kv{kv} q{n_q} k{n_k} causal{causal}: out bad {int(bad.sum())} / {bad.size} '
              f'(max err {np.nanmax(np.where(written[:, None], err, 0)):.3g}), lse bad {int(lbad.sum())}, '
              f'unmapped rows written {untouched}')
    return dict(out_bad=int(bad.sum()), lse_bad=int(lbad.sum()), untouched=untouched, early_reads=early)
