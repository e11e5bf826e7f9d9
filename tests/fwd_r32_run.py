"""Runs flash_fwd_r32's generated stream (heads of 256, 32 rows a wave) on the emulator (fwd64_emu.py) for a small
case, with the per-lane operands attn_fwd64.hip computes restated here, and compares the outputs and LSE with the
oracle's."""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "mako-common_amd", "csrc"))
import fwd64_emu as E  # noqa: E402
import fwd64_run as R64  # noqa: E402
import gen_attn_fwd_r32 as G  # noqa: E402
import oracle as O  # noqa: E402

D = 256
LAST = {}   # the last run's outputs and the oracle's, for a look at a failing case
VOPS = ['kr', 'vr0', 'vr1', 'vr2', 'vr3'] + [f'kd{m}' for m in range(G.NKP + 1)] + [
    'vd', 'vdo', 'vd2', 'vdo2', 'lim0', 'qo', 'lo0', 'swp', 'ew', 'er', 'og']
SOPS = R64.SOPS
VREG = {n: f'v{G.CLOBBER_V + i}' for i, n in enumerate(VOPS)}


def vd_lane(lane, r0):
    """The V byte (relative to its 1 KiB piece of two 512-byte rows) lane l's LDS slot holds, for a piece whose first
    row is r0 mod 4: slot byte 16 l is row r, physical unit p, half; it holds the unit G.v_unit places at p."""
    b = 16 * lane
    r, pos = b // (2 * D), b % (2 * D)
    x = (pos // 32) ^ ((r + r0) & 3)      # the physical unit's logical unit: x ^ 4 (x % 2) (G.v_unit's inverse)
    u = x ^ (4 * (x & 1))
    return r * 2 * D + 32 * u + 16 * ((pos // 16) & 1)


def program(ind, outd, lines=None):
    lines = lines if lines is not None else G.body(ind, outd)
    out = []
    for ln in lines:
        ln = ln.replace('%=', '0')
        for n, r in sorted(VREG.items(), key=lambda x: -len(x[0])):   # longer names first
            ln = ln.replace(f'%[{n}]', r)
        for n, r in SOPS.items():
            ln = ln.replace(f'%[{n}]', r)
        out.append(ln)
    return E.parse(out)


def run(heads, kv, S_q, S_k, q_pos0, block, ind='bf16', outd='f32', seed=0, verbose=True, kgrow=0.0, lines=None,
        vscale=None):
    rng = np.random.default_rng(seed)
    dt = O.BF16 if ind == 'bf16' else O.F16
    q_pad = (S_q + 63) // 64 * 64
    k_pad = (S_k + 127) // 128 * 128
    conv = O.to_bf16_bits if ind == 'bf16' else O.to_f16_bits
    qb = conv(rng.standard_normal((heads, q_pad, D), dtype=np.float32))
    kf = rng.standard_normal((kv, k_pad, D), dtype=np.float32)
    if kgrow:
        kf *= (1 + kgrow * (np.arange(k_pad) // 64))[None, :, None].astype(np.float32)
    kb = conv(kf)
    vf = rng.standard_normal((kv, k_pad, D), dtype=np.float32)
    if vscale is not None:
        vf *= vscale
    vb = conv(vf)
    width = heads * D
    row_b = 2 * D
    so = 4 if outd == 'f32' else 2
    sizes = [qb.nbytes, kb.nbytes, vb.nbytes, S_q * width * so + 4096, heads * S_q * 4 + 4096]
    offs = np.cumsum([4096] + [((x + 4095) // 4096) * 4096 for x in sizes])
    Q0, K0, V0, O0, L0 = [int(x) for x in offs[:5]]
    mem = E.Mem(int(offs[-1]) + 4096)
    mem.b[Q0:Q0 + qb.nbytes] = qb.view(np.uint8).ravel()
    mem.b[K0:K0 + kb.nbytes] = kb.view(np.uint8).ravel()
    mem.b[V0:V0 + vb.nbytes] = vb.view(np.uint8).ravel()
    if so == 4:
        fill = np.full(S_q * width, np.nan, np.float32)
        mem.b[O0:O0 + fill.nbytes] = fill.view(np.uint8)
    prog, labels = program(ind, outd, lines)
    group = heads // kv
    hq = 4 if group % 4 == 0 else 2 if group % 2 == 0 else 1
    rows_wg = 128 // hq
    n_qblk = (S_q + rows_wg - 1) // rows_wg
    n_hg = heads // hq
    c = np.float32(1.0 / np.sqrt(float(D))) * np.float32(1.4426950408889634)
    lane = np.arange(64)
    g, c32 = lane >> 5, lane & 31
    lbase = 0
    vbase = lbase + 2 * G.K_TILE
    t0 = time.time()
    n_instr = 0
    early = 0
    worst = {}
    for hg in range(n_hg):
        for qbk in range(n_qblk):
            emu = E.Emu(prog, labels, mem, G.LDS_BYTES)
            waves = []
            for w in range(4):
                W = E.Wave(w)
                h = hg * hq + w % hq
                kvh = hg * hq // group
                wg_q0 = qbk * rows_wg
                q0 = wg_q0 + (w // hq) * 32
                wg_last = q_pos0 + min(wg_q0 + rows_wg, S_q) - 1
                n_keys = S_k if wg_last >= block else min(S_k, wg_last + 1)
                live = q0 < S_q
                w_last = q_pos0 + min(q0 + 32, S_q) - 1
                w_keys = 0 if not live else (S_k if w_last >= block else min(S_k, w_last + 1))
                nt, ntw = (n_keys + 63) // 64, (w_keys + 63) // 64
                p0 = q_pos0 + q0
                lmin = R64.lim_of(p0, S_k, block)
                lim0 = np.array([R64.lim_of(p0 + cc, S_k, block) for cc in c32]) - 8 * g
                kr = lbase + c32 * G.K_ROW + 16 * g
                hh, ii = (lane >> 4) & 1, lane & 15
                vr = [vbase + (8 * g + ii // 4) * 2 * D + 8 * (ii % 4) +
                      32 * np.array([G.v_unit(2 * d + int(a), int(b) // 4) for a, b in zip(hh, ii)]) for d in range(4)]

                def kd_of(i):
                    b = 1024 * i + 16 * lane
                    Rr, cch = b // G.K_ROW, (b % G.K_ROW) // 16
                    return np.array([R64.slot_of(int(r)) for r in Rr]) * row_b + 16 * np.where(cch < D // 8, cch, 0)
                kds = [kd_of(w + 4 * m) for m in range(G.NKP)] + [kd_of(4 * G.NKP)]
                vd = (G.V_TILE // 4) * w + vd_lane(lane, 0)
                vdo = (G.V_TILE // 4) * w + vd_lane(lane, 2)
                qo = ((q0 + c32) * D + 8 * g) * 2
                orow = D * so
                lpr = orow // 16
                obase = lbase + w * 32 * orow
                if so == 4:
                    ew = obase + c32 * orow + 16 * ((c32 & 7) ^ g)
                else:
                    ew = obase + c32 * orow + 8 * g + 16 * (c32 & 7)
                er = obase + (lane // lpr) * orow + 16 * ((lane % lpr) ^ (lane // lpr))
                og = (q0 + lane // lpr) * width * so + h * orow + 16 * (lane % lpr)
                ogs = (64 // lpr) * width * so
                lo0 = np.where(q0 + c32 < S_q, (h * S_q + q0 + c32) * 4, 0xffffffff)
                swp = (lane ^ 32) * 4
                vals = dict(kr=kr, vr0=vr[0], vr1=vr[1], vr2=vr[2], vr3=vr[3], vd=vd, vdo=vdo, vd2=vd + 4096, vdo2=vdo + 4096, lim0=lim0, qo=qo, lo0=lo0, swp=swp,
                            ew=ew, er=er, og=og)
                vals.update({f'kd{m}': kds[m] for m in range(G.NKP + 1)})
                for n, arr in vals.items():
                    W.v[int(VREG[n][1:])] = np.asarray(arr, np.int64).astype(np.uint32) if np.ndim(arr) else \
                        np.full(64, int(arr) & 0xFFFFFFFF, np.uint32)

                def rs(sidx, base, nbytes):
                    W.s[sidx] = base & 0xFFFFFFFF
                    W.s[sidx + 1] = (base >> 32) & 0xFFFF
                    W.s[sidx + 2] = nbytes & 0xFFFFFFFF
                    W.s[sidx + 3] = 0x00020000
                rs(0, Q0 + h * q_pad * row_b, S_q * row_b)
                kbase = K0 + kvh * k_pad * row_b
                vrow = V0 + kvh * k_pad * row_b
                W.s[26], W.s[27], W.s[28] = kbase & 0xFFFFFFFF, (kbase >> 32) & 0xFFFF, n_keys * row_b
                W.s[29], W.s[30], W.s[31] = vrow & 0xFFFFFFFF, (vrow >> 32) & 0xFFFF, n_keys * row_b
                W.s[32], W.s[33], W.s[34] = lbase, lbase + 1024 * w, vbase + (G.V_TILE // 4) * w
                rs(12, O0, S_q * width * so)
                rs(16, L0, heads * S_q * 4)
                W.s[20] = int(np.float32(c).view(np.uint32))
                W.s[21], W.s[22], W.s[23], W.s[24], W.s[25] = nt, ntw, lmin, 1, ogs
                waves.append(W)
            emu.run_wg(waves)
            n_instr += emu.count
            early += emu.early
            for k_, v_ in emu.conflicts.items():
                worst[k_] = max(worst.get(k_, 1), v_)
    if verbose:
        print(f'emulated {n_instr} wave-instructions in {time.time() - t0:.1f} s; LDS worst multiplicity {worst}')
    if so == 4:
        o = mem.b[O0:O0 + S_q * width * 4].view(np.float32).reshape(S_q, width).astype(np.float64)
    else:
        bitsv = mem.b[O0:O0 + S_q * width * 2].view(np.uint16)
        o = O.bits_to_f32(bitsv, dt).reshape(S_q, width).astype(np.float64)
    lse = mem.b[L0:L0 + heads * S_q * 4].view(np.float32).reshape(heads, S_q).astype(np.float64)
    want_o, want_l = O.attn_dense(qb, kb, vb, n_q=S_q, q_pad=q_pad, n_k=S_k, k_pad=k_pad, heads=heads, kv_heads=kv,
                                  q_pos0=q_pos0, block=block, dim=D, dtype=dt)
    LAST.update(o=o, want=want_o, lse=lse, want_lse=want_l)
    err = np.abs(o - want_o)
    bad = ~(err <= 2e-3 + 1e-2 * np.abs(want_o))
    lerr = np.abs(lse - want_l)
    lbad = ~(lerr <= 1e-3) & np.isfinite(want_l)
    if verbose:
        print(f'h{heads} kv{kv} q{S_q} k{S_k} p{q_pos0} b{block}: out bad {bad.sum()} / {bad.size} '
              f'(max err {np.nanmax(err) if err.size else 0:.3g}), lse bad {lbad.sum()}')
    return dict(out_bad=int(bad.sum()), lse_bad=int(lbad.sum()), lds_worst=worst,
                max_err=float(np.nanmax(err)) if err.size and not np.isnan(err).all() else float('nan'),
                early_reads=early)
