"""Static scan of flash_fwd_r64's generated stream for the gfx950 software hazards it must respect (wait states
counted conservatively: an MFMA counts as one, s_nop N as N + 1; each variant scanned linearly in emission order).
The rules are the ones hipcc applies to the same instruction pairs."""
import re

RULES = {
    'vsgpr_mask': 2,   # VALU writes an SGPR pair / vcc -> VALU reads it
    'trans': 1,        # v_exp / v_log / v_rcp result -> read
    'mfma_raw': 18,    # MFMA dst -> VALU / accvgpr / store / MFMA srcA,B read
    'valu_mfma': 2,    # VALU writes -> MFMA reads
    'mfma_war_ab': 4,  # MFMA reads srcA/B -> VALU writes it
    'mfma_war_c': 11,  # MFMA reads srcC -> VALU writes it
    'dot': 3,          # v_dot2 result -> VALU read
    'valu_dot': 1,     # VALU write -> v_dot2 read
    'm0_dma': 1,       # SALU write of m0 -> LDS DMA
    'store_data': 2,   # a VMEM / DS store of more than 8 bytes -> VALU writes its data registers
}
REG = re.compile(r'-?([vas])(?:(\d+)|\[(\d+):(\d+)\])')


def regs(tok):
    out = []
    for m in REG.finditer(tok):
        k, one, lo, hi = m.groups()
        if one is not None:
            out.append(f'{k}{one}')
        else:
            out += [f'{k}{i}' for i in range(int(lo), int(hi) + 1)]
    if tok.strip() == 'vcc':
        out = ['vcc']
    return out


def check(lines, name):
    clock = 0
    last = {}     # reg -> (clock, kind)
    readers = {}  # reg -> (clock, kind) of MFMA reads
    stores = {}   # reg -> clock of a wide store reading it
    n_bad = 0
    for idx, ln in enumerate(lines):
        ln = ln.strip()
        if ln.endswith(':') or not ln:
            continue
        parts = ln.split(None, 1)
        mn = parts[0]
        args = [a.strip() for a in parts[1].split(',')] if len(parts) > 1 else []
        args = [re.sub(r'\s*offset:\d+', '', a).replace(' offen', '') for a in args]
        if mn == 's_nop':
            clock += int(args[0]) + 1
            continue
        clock += 1
        if mn.startswith('s_waitcnt') or mn.startswith('s_barrier') or mn.startswith('s_branch') or \
                mn.startswith('s_cbranch'):
            continue
        is_mfma = mn.startswith('v_mfma')
        if mn.startswith('buffer_load') and ln.endswith(' lds'):
            if 'm0' in last and clock - last['m0'][0] - 1 < RULES['m0_dma']:
                n_bad += 1
                print(f'{name}: line {idx}: {ln!r} reads m0 {clock - last["m0"][0] - 1} wait states after its write')
        if mn.startswith('s_') and args and args[0] == 'm0':
            last['m0'] = (clock, 'salu')
        is_valu = mn.startswith('v_')
        # which operands are written / read
        if mn.startswith('buffer_store') or mn.startswith('ds_write'):
            dst, srcs = [], args
        elif mn.startswith('v_cmp'):
            dst, srcs = args[:1], args[1:]
        elif mn.startswith('s_'):
            dst, srcs = args[:1], args[1:]
        else:
            dst, srcs = args[:1], args[1:]
        if mn.startswith('v_cndmask') and len(srcs) == 3:
            pass
        # reads
        for si, tok in enumerate(srcs):
            for r in regs(tok):
                if r not in last:
                    continue
                wclk, wkind = last[r]
                d = clock - wclk - 1
                need = 0
                if wkind == 'vsgpr' and is_valu:
                    need = RULES['vsgpr_mask']
                elif wkind == 'trans' and (is_valu or is_mfma):
                    need = RULES['trans']
                elif wkind == 'mfma':
                    if is_mfma and si == 2 and tok == args[0]:
                        need = 0  # accumulate chain on the same registers
                    elif is_valu or is_mfma or mn.startswith('buffer_store') or mn.startswith('ds_'):
                        need = RULES['mfma_raw']
                elif wkind == 'valu' and is_mfma:
                    need = RULES['valu_mfma']
                elif wkind == 'dot' and is_valu and not (mn.startswith('v_dot2') and si == 2):
                    need = RULES['dot']
                elif wkind == 'valu' and mn.startswith('v_dot2'):
                    need = RULES['valu_dot']
                if d < need:
                    n_bad += 1
                    if n_bad <= 12:
                        print(f'{name}: line {idx}: {ln!r} reads {r} {d} wait states after {wkind} (needs {need})')
        # WAR on the data of wide stores
        if is_valu:
            for tok in dst:
                for r in regs(tok):
                    if r in stores and clock - stores[r] - 1 < RULES['store_data']:
                        n_bad += 1
                        if n_bad <= 12:
                            print(f'{name}: line {idx}: {ln!r} writes {r} {clock - stores[r] - 1} after a wide store read it')
        if (mn.startswith('buffer_store_dwordx') or mn.startswith('ds_write_b')) and ('x4' in mn or 'x3' in mn or 'b128' in mn or 'b96' in mn):
            dtok = args[1] if mn.startswith('ds_') else args[0]
            for r in regs(dtok):
                stores[r] = clock
        # writes
        for tok in dst:
            for r in regs(tok):
                if r in readers and is_valu and not is_mfma:
                    rclk, rkind = readers[r]
                    d = clock - rclk - 1
                    need = RULES['mfma_war_c'] if rkind == 'c' else RULES['mfma_war_ab']
                    if d < need:
                        n_bad += 1
                        if n_bad <= 12:
                            print(f'{name}: line {idx}: {ln!r} writes {r} {d} after an MFMA read it as src{rkind}')
                if is_mfma:
                    last[r] = (clock, 'mfma')
                elif mn.startswith('v_cmp') and (tok.startswith('s') or tok == 'vcc'):
                    last[r] = (clock, 'vsgpr')
                elif mn in ('v_exp_f32', 'v_log_f32', 'v_rcp_f32'):
                    last[r] = (clock, 'trans')
                elif mn.startswith('v_dot2'):
                    last[r] = (clock, 'dot')
                elif is_valu:
                    last[r] = (clock, 'valu')
                else:
                    last.pop(r, None)
        if is_mfma:
            for si, tok in enumerate(srcs):
                for r in regs(tok):
                    readers[r] = (clock, 'c' if si == 2 else 'ab')
    print(f'{name}: {n_bad} hazards')
    return n_bad


