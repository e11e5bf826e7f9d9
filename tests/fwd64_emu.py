"""CPU emulator of the instruction subset gen_attn_fwd64.py emits (flash_fwd_r64's stream), so the stream's logic is
checked without a GPU: register-exact ALU, MFMA and LDS semantics in program order, one workgroup at a time with its
barriers. Vector-memory loads land only at the s_waitcnt vmcnt that retires them, and LDS reads (and lane permutes)
only at the s_waitcnt lgkmcnt that retires them, reading LDS then (their destinations hold all-ones until they land),
so a read that does not wait, a read into a register an earlier instruction still needs, a load into an LDS buffer
still being read, or an LDS read left in flight across a barrier, shows in the results. The waves of the workgroup run
one at a time from barrier to barrier, starting with a different wave each time. It
reports LDS bank-conflict multiplicities too. Wait states (hardware hazards) are checked by fwd64_hazards.py."""
import re

import numpy as np

F32 = np.float32


def f2u(x):
    return np.asarray(x, F32).view(np.uint32)


def u2f(x):
    return np.asarray(x, np.uint32).view(F32)


def f16_rne(x):
    return np.asarray(x, F32).astype(np.float16)


def f16_rtz(x):
    x = np.asarray(x, F32)
    h = x.astype(np.float16)
    hf = h.astype(F32)
    # step toward zero where rounding went away from zero
    bad = np.abs(hf) > np.abs(x)
    hb = h.view(np.uint16).copy()
    hb[bad] -= 1  # magnitude down one ulp (sign-magnitude)
    h = hb.view(np.float16)
    inf = np.isinf(h) & np.isfinite(x)
    h = np.where(inf, np.copysign(np.float16(65504), x).astype(np.float16), h)
    return h


def bf16_rne_bits(x):
    u = f2u(x).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = np.isnan(np.asarray(x, F32))
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint32)


def h2bits(h):
    return np.asarray(h, np.float16).view(np.uint16).astype(np.uint32)


def bits2h(b):
    return (np.asarray(b, np.uint32) & 0xFFFF).astype(np.uint16).view(np.float16)


EXACT_COUNT = [0, 0]  # (exact-path branches taken, checks made)
REG = re.compile(r'^(-?)([vas])(?:(\d+)|\[(\d+):(\d+)\])$')


class Op:
    __slots__ = ('mn', 'args', 'mods', 'line')


def parse(lines):
    prog, labels = [], {}
    for ln in lines:
        ln = ln.strip()
        if not ln:
            continue
        if ln.endswith(':'):
            labels[ln[:-1]] = len(prog)
            continue
        parts = ln.split(None, 1)
        op = Op()
        op.mn = parts[0]
        op.line = ln
        rest = parts[1] if len(parts) > 1 else ''
        mods = {}
        if rest.endswith(' lds'):
            mods['lds'] = True
            rest = rest[:-4]
        for cm in (' nt', ' sc0', ' sc1'):   # cache policy: no effect on the values
            if rest.endswith(cm):
                mods[cm.strip()] = True
                rest = rest[:-len(cm)]
        if 'offen' in rest:
            mods['offen'] = True
        m = re.search(r'offset:(\d+)', rest)
        if m:
            mods['offset'] = int(m.group(1))
            rest = re.sub(r'\s*offset:\d+', '', rest)
        rest = rest.replace(' offen', '')
        op.args = [a.strip() for a in rest.split(',')] if rest else []
        op.mods = mods
        prog.append(op)
    return prog, labels


class Mem:
    def __init__(self, size):
        self.b = np.zeros(size, np.uint8)


POISON = [False]   # registers start as garbage (as on the GPU) instead of zeros


class Wave:
    def __init__(self, wid):
        self.v = np.zeros((256, 64), np.uint32)
        self.a = np.zeros((256, 64), np.uint32)
        self.s = np.zeros(128, np.uint32)
        if POISON[0]:
            rng = np.random.default_rng(1000 + wid)
            self.v = rng.integers(0, 2 ** 32, (256, 64), dtype=np.uint64).astype(np.uint32)
            self.a = rng.integers(0, 2 ** 32, (256, 64), dtype=np.uint64).astype(np.uint32)
            self.s = rng.integers(0, 2 ** 32, 128, dtype=np.uint64).astype(np.uint32)
        self.vcc = np.zeros(64, bool)
        self.scc = 0
        self.pc = 0
        self.done = False
        self.wid = wid
        self.vmq = []       # outstanding vector-memory loads: callables that land their data
        self.lq = []        # outstanding LDS instructions, in issue order (LDS returns in order)
        self.sq = []        # outstanding scalar loads: they return in any order, so they land at lgkmcnt(0) only
        self.exec = np.ones(64, bool)


def parse_reg(x):
    m = REG.match(x)
    if not m:
        return None
    neg, kind, one, lo, hi = m.groups()
    if one is not None:
        return kind, int(one), 1, bool(neg)
    return kind, int(lo), int(hi) - int(lo) + 1, bool(neg)


def lit(x):
    if x == 'vcc':
        return None
    try:
        if x.startswith('0x') or x.startswith('-0x'):
            return int(x, 16) & 0xFFFFFFFF
        if '.' in x:
            return int(f2u(F32(float(x))))
        return int(x) & 0xFFFFFFFF
    except ValueError:
        return None


class Emu:
    def __init__(self, prog, labels, gmem, lds_bytes):
        self.prog, self.labels = prog, labels
        self.g = gmem
        self.lds = np.zeros(lds_bytes, np.uint8)
        self.pend = np.zeros(lds_bytes, np.int32)  # LDS DMA loads in flight over each byte (issued, not landed)
        self.early = 0   # LDS reads that sampled bytes a DMA load in flight had not yet written
        self.count = 0
        self.conflicts = {}  # instruction text -> worst multiplicity seen

    def check_landed(self, addr, size):
        idx = np.clip(np.asarray(addr, np.int64)[:, None] + np.arange(size), 0, len(self.lds) - 1)
        if self.pend[idx].any():
            self.early += 1

    # operand read: returns a (64,) uint32 array (per lane) for scalar-or-vector 32-bit operands
    def rd(self, w, x):
        neg = False
        r = parse_reg(x)
        if r is None:
            if x == 'vcc':
                raise ValueError
            v = lit(x)
            if v is None:
                raise ValueError(f'operand {x}')
            return np.full(64, v, np.uint32)
        kind, i, n, neg = r
        if kind == 'v':
            val = w.v[i].copy()
        elif kind == 'a':
            val = w.a[i].copy()
        else:
            val = np.full(64, w.s[i], np.uint32)
        if neg:
            val = f2u(-u2f(val))
        return val

    def rdf(self, w, x):
        return u2f(self.rd(w, x))

    def wr(self, w, x, val):
        kind, i, n, _ = parse_reg(x)
        if kind == 'v':
            w.v[i] = val
        elif kind == 'a':
            w.a[i] = val
        else:
            raise ValueError(x)

    def wrf(self, w, x, val):
        self.wr(w, x, f2u(np.asarray(val, F32)))

    def sread(self, w, x):
        if x == 'm0':
            return int(w.s[124])
        r = parse_reg(x)
        if r is None:
            return lit(x)
        return int(w.s[r[1]])

    def rsrc(self, w, x):
        kind, i, n, _ = parse_reg(x)
        base = int(w.s[i]) | ((int(w.s[i + 1]) & 0xFFFF) << 32)
        return base, int(w.s[i + 2])

    def mask_of(self, w, x):
        if x == 'vcc':
            return w.vcc
        kind, i, n, _ = parse_reg(x)
        lo, hi = int(w.s[i]), int(w.s[i + 1])
        bits = lo | (hi << 32)
        return np.array([(bits >> l) & 1 for l in range(64)], bool)

    def set_mask(self, w, x, m):
        if x == 'vcc':
            w.vcc = m.copy()
            return
        kind, i, n, _ = parse_reg(x)
        bits = 0
        for l in range(64):
            if m[l]:
                bits |= 1 << l
        w.s[i] = bits & 0xFFFFFFFF
        w.s[i + 1] = bits >> 32

    def step(self, w):
        op = self.prog[w.pc]
        w.pc += 1
        self.count += 1
        mn, A = op.mn, op.args
        if mn == 's_waitcnt':
            m = re.search(r'vmcnt\((\d+)\)', ' '.join(A))
            if m:
                self.retire(w, int(m.group(1)))
            m = re.search(r'lgkmcnt\((\d+)\)', ' '.join(A))
            if m:
                self.retire_lds(w, int(m.group(1)))
                if int(m.group(1)) == 0:
                    while w.sq:
                        w.sq.pop(0)()
            return
        if mn == 's_nop':
            return
        if mn == 's_barrier':
            return 'barrier'
        if mn == 's_mov_b32':
            w.s[self.sidx(A[0])] = self.sread(w, A[1])
        elif mn == 's_add_u32':
            r = self.sread(w, A[1]) + self.sread(w, A[2])
            w.s[self.sidx(A[0])] = r & 0xFFFFFFFF
            w.scc = int(r >> 32)
        elif mn == 's_addc_u32':
            r = self.sread(w, A[1]) + self.sread(w, A[2]) + w.scc
            w.s[self.sidx(A[0])] = r & 0xFFFFFFFF
            w.scc = int(r >> 32)
        elif mn == 's_sub_u32':
            a, b = self.sread(w, A[1]), self.sread(w, A[2])
            w.s[self.sidx(A[0])] = (a - b) & 0xFFFFFFFF
            w.scc = int(a < b)
        elif mn == 's_lshl_b32':
            r = (self.sread(w, A[1]) << self.sread(w, A[2])) & 0xFFFFFFFF
            w.s[parse_reg(A[0])[1]] = r
            w.scc = int(r != 0)
        elif mn == 's_and_b32':
            r = self.sread(w, A[1]) & self.sread(w, A[2])
            w.s[parse_reg(A[0])[1]] = r
            w.scc = int(r != 0)
        elif mn.startswith('s_load_dword'):
            # scalar load: base pair A[1] + offset A[2] (register or immediate); the destination holds garbage until
            # an lgkmcnt(0) wait
            kind, i, n, _ = parse_reg(A[0])
            _, b, _, _ = parse_reg(A[1])
            addr = int(w.s[b]) | ((int(w.s[b + 1]) & 0xFFFF) << 32)
            addr += self.sread(w, A[2])
            vals = self.g.b[addr:addr + 4 * n].view(np.uint32).copy()
            for q in range(n):
                w.s[i + q] = 0xDEADBEEF

            def land(w=w, i=i, vals=vals):
                for q in range(len(vals)):
                    w.s[i + q] = vals[q]
            w.sq.append(land)
        elif mn == 's_and_saveexec_b64':
            m = self.mask_of(w, A[1])
            self.set_mask(w, A[0], w.exec.copy())
            w.exec = w.exec & m
            w.scc = int(w.exec.any())
        elif mn == 's_mov_b64' and A[0] == 'exec':
            w.exec = self.mask_of(w, A[1])
        elif mn == 'v_lshrrev_b64':
            kd, di, _, _ = parse_reg(A[0])
            sh = self.rd(w, A[1]).astype(np.uint64) & 63
            _, si, _, _ = parse_reg(A[2])
            val = np.uint64(int(w.s[si]) | (int(w.s[si + 1]) << 32))
            r = np.array([int(val) >> int(x) for x in sh], np.uint64)
            w.v[di] = (r & 0xFFFFFFFF).astype(np.uint32)
            w.v[di + 1] = (r >> np.uint64(32)).astype(np.uint32)
        elif mn == 'v_bfe_u32':
            src, off, wid = self.rd(w, A[1]), self.rd(w, A[2]) & 31, self.rd(w, A[3]) & 31
            self.wr(w, A[0], ((src >> off) & ((np.uint32(1) << wid) - np.uint32(1))).astype(np.uint32))
        elif mn == 'v_mad_u64_u32':
            kd, di, _, _ = parse_reg(A[0])
            a, b = self.rd(w, A[2]).astype(np.uint64), self.rd(w, A[3]).astype(np.uint64)
            ck, ci, _, _ = parse_reg(A[4])
            c = (w.v[ci].astype(np.uint64) | (w.v[ci + 1].astype(np.uint64) << np.uint64(32))) if ck == 'v' else \
                np.full(64, int(w.s[ci]) | (int(w.s[ci + 1]) << 32), np.uint64)
            r = a * b + c
            w.v[di] = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32)
            w.v[di + 1] = (r >> np.uint64(32)).astype(np.uint32)
        elif mn == 'global_store_dwordx4':
            _, ai, _, _ = parse_reg(A[0])
            _, di, n, _ = parse_reg(A[1])
            for l in range(64):
                if not w.exec[l]:
                    continue
                addr = int(w.v[ai][l]) | (int(w.v[ai + 1][l]) << 32)
                assert 0 <= addr and addr + 16 <= len(self.g.b), f'global store at {addr:#x} out of range'
                for q in range(4):
                    self.g.b[addr + 4 * q:addr + 4 * q + 4] = np.frombuffer(np.uint32(w.v[di + q][l]).tobytes(),
                                                                            np.uint8)
        elif mn == 's_mul_i32':
            w.s[parse_reg(A[0])[1]] = (self.sread(w, A[1]) * self.sread(w, A[2])) & 0xFFFFFFFF
        elif mn.startswith('s_cmp_'):
            a, b = self.sread(w, A[0]), self.sread(w, A[1])
            w.scc = int({'eq': a == b, 'ge': a >= b, 'le': a <= b}[mn.split('_')[2]])
        elif mn == 's_cselect_b32':
            w.s[parse_reg(A[0])[1]] = self.sread(w, A[1]) if w.scc else self.sread(w, A[2])
        elif mn == 's_or_b64':
            m = self.mask_of(w, A[1]) | self.mask_of(w, A[2])
            self.set_mask(w, A[0], m)
            w.scc = int(m.any())
        elif mn == 's_branch':
            w.pc = self.labels[A[0]]
        elif mn == 's_cbranch_scc0':
            if not w.scc:
                w.pc = self.labels[A[0]]
        elif mn == 's_cbranch_scc1':
            if w.scc:
                w.pc = self.labels[A[0]]
        elif mn == 's_cbranch_vccnz':
            EXACT_COUNT[1] += 1
            if w.vcc.any():
                EXACT_COUNT[0] += 1
                w.pc = self.labels[A[0]]
        elif mn == 'v_mov_b32':
            self.wr(w, A[0], self.rd(w, A[1]))
        elif mn == 'v_add_u32':
            self.wr(w, A[0], (self.rd(w, A[1]).astype(np.uint64) + self.rd(w, A[2])).astype(np.uint32))
        elif mn == 'v_sub_u32':
            self.wr(w, A[0], (self.rd(w, A[1]).astype(np.int64) - self.rd(w, A[2]).astype(np.int64)).astype(np.uint32))
        elif mn == 'v_add_f32':
            self.wrf(w, A[0], self.rdf(w, A[1]) + self.rdf(w, A[2]))
        elif mn == 'v_sub_f32':
            self.wrf(w, A[0], self.rdf(w, A[1]) - self.rdf(w, A[2]))
        elif mn == 'v_mul_f32':
            self.wrf(w, A[0], self.rdf(w, A[1]) * self.rdf(w, A[2]))
        elif mn == 'v_fma_f32':
            self.wrf(w, A[0], (self.rdf(w, A[1]).astype(np.float64) * self.rdf(w, A[2]) + self.rdf(w, A[3])).astype(F32))
        elif mn == 'v_exp_f32':
            with np.errstate(over='ignore'):
                self.wrf(w, A[0], np.exp2(self.rdf(w, A[1])))
        elif mn == 'v_log_f32':
            with np.errstate(divide='ignore', invalid='ignore'):
                self.wrf(w, A[0], np.log2(self.rdf(w, A[1])))
        elif mn == 'v_rcp_f32':
            with np.errstate(divide='ignore'):
                self.wrf(w, A[0], F32(1) / self.rdf(w, A[1]))
        elif mn == 'v_max_f32':
            self.wrf(w, A[0], np.fmax(self.rdf(w, A[1]), self.rdf(w, A[2])))
        elif mn == 'v_max3_f32':
            self.wrf(w, A[0], np.fmax(np.fmax(self.rdf(w, A[1]), self.rdf(w, A[2])), self.rdf(w, A[3])))
        elif mn.startswith('v_cmp_'):
            _, _, cond, ty = mn.split('_')
            if ty == 'i32':
                a, b = self.rd(w, A[1]).view(np.int32), self.rd(w, A[2]).view(np.int32)
            elif ty == 'u32':
                a, b = self.rd(w, A[1]), self.rd(w, A[2])
            else:
                a, b = self.rdf(w, A[1]), self.rdf(w, A[2])
            with np.errstate(invalid='ignore'):
                m = {'lt': a < b, 'gt': a > b, 'le': a <= b, 'ne': a != b, 'eq': a == b,
                     'nle': ~(a <= b)}[cond]
            self.set_mask(w, A[0], m)
        elif mn == 'v_cndmask_b32':
            m = self.mask_of(w, A[3])
            self.wr(w, A[0], np.where(m, self.rd(w, A[2]), self.rd(w, A[1])))
        elif mn == 'v_lshlrev_b32':
            self.wr(w, A[0], (self.rd(w, A[2]).astype(np.uint64) << self.rd(w, A[1])).astype(np.uint32))
        elif mn == 'v_xor_b32':
            self.wr(w, A[0], self.rd(w, A[1]) ^ self.rd(w, A[2]))
        elif mn == 'v_and_b32':
            self.wr(w, A[0], self.rd(w, A[1]) & self.rd(w, A[2]))
        elif mn in ('v_cvt_pk_f16_f32', 'v_cvt_pkrtz_f16_f32'):
            cv = f16_rne if mn == 'v_cvt_pk_f16_f32' else f16_rtz
            lo, hi = h2bits(cv(self.rdf(w, A[1]))), h2bits(cv(self.rdf(w, A[2])))
            self.wr(w, A[0], lo | (hi << 16))
        elif mn == 'v_cvt_pk_bf16_f32':
            lo, hi = bf16_rne_bits(self.rdf(w, A[1])), bf16_rne_bits(self.rdf(w, A[2]))
            self.wr(w, A[0], lo | (hi << 16))
        elif mn == 'v_perm_b32':
            s0, s1, sel = self.rd(w, A[1]), self.rd(w, A[2]), self.rd(w, A[3])
            full = (s0.astype(np.uint64) << 32) | s1
            out = np.zeros(64, np.uint32)
            for byte in range(4):
                bs = (sel >> (8 * byte)) & 0xFF
                val = ((full >> (8 * bs.astype(np.uint64))) & 0xFF).astype(np.uint32)
                val = np.where(bs == 0x0C, 0, val)
                out |= val << (8 * byte)
            self.wr(w, A[0], out)
        elif mn == 'v_pk_add_f16':
            x, y = self.rd(w, A[1]), self.rd(w, A[2])
            lo = bits2h(x) + bits2h(y)
            hi = bits2h(x >> 16) + bits2h(y >> 16)
            self.wr(w, A[0], h2bits(lo) | (h2bits(hi) << 16))
        elif mn == 'v_dot2_f32_f16':
            a, b, c = self.rd(w, A[1]), self.rd(w, A[2]), self.rdf(w, A[3])
            r = (bits2h(a).astype(np.float64) * bits2h(b) + bits2h(a >> 16).astype(np.float64) * bits2h(b >> 16)
                 + c)
            self.wrf(w, A[0], r.astype(F32))
        elif mn == 'v_accvgpr_read_b32':
            self.wr(w, A[0], self.rd(w, A[1]))
        elif mn == 'v_accvgpr_write_b32':
            self.wr(w, A[0], self.rd(w, A[1]))
        elif mn.startswith('v_mfma_f32_32x32x16_'):
            ty = mn.split('_')[-1]
            self.mfma(w, A, ty)
        elif mn == 'ds_read_b128':
            kind, i, n, _ = parse_reg(A[0])
            addr = self.rd(w, A[1]).astype(np.int64) + op.mods.get('offset', 0)
            self.bank(op, addr, 16)
            dst = w.v if kind == 'v' else w.a
            for q in range(4):
                dst[i + q] = 0xFFFFFFFF

            def land(dst=dst, i=i, addr=addr):
                self.check_landed(addr, 16)
                for q in range(4):
                    dst[i + q] = np.array([self.lds[x + 4 * q: x + 4 * q + 4].view(np.uint32)[0]
                                           if 0 <= x + 4 * q + 4 <= len(self.lds) else 0 for x in addr], np.uint32)
            w.lq.append(land)
        elif mn == 'ds_read_b64_tr_b16':
            # transpose read (gfx950, lane layout checked on the GPU): in each group of 16 lanes, lane i receives
            # element i % 4 of the 8 bytes lanes i // 4, 4 + i // 4, 8 + i // 4 and 12 + i // 4 address, in that order
            kind, i, n, _ = parse_reg(A[0])
            addr = self.rd(w, A[1]).astype(np.int64) + op.mods.get('offset', 0)
            self.bank(op, addr, 8)
            dst = w.v if kind == 'v' else w.a
            for q in range(2):
                dst[i + q] = 0xFFFFFFFF

            def land(dst=dst, i=i, addr=addr):
                self.check_landed(addr, 8)
                chunks = np.zeros((64, 4), np.uint32)
                for l in range(64):
                    x = int(addr[l])
                    if 0 <= x and x + 8 <= len(self.lds):
                        chunks[l] = self.lds[x:x + 8].view(np.uint16)
                lane = np.arange(64)
                grp, li = lane & ~15, lane & 15
                el = np.stack([chunks[grp + 4 * y + li // 4, li % 4] for y in range(4)], axis=1)
                dst[i] = el[:, 0] | (el[:, 1] << 16)
                dst[i + 1] = el[:, 2] | (el[:, 3] << 16)
            w.lq.append(land)
        elif mn in ('ds_write_b128', 'ds_write_b64'):
            kind, i, n, _ = parse_reg(A[1])
            addr = self.rd(w, A[0]).astype(np.int64) + op.mods.get('offset', 0)
            self.bank(op, addr, 4 * n)
            src = w.v if kind == 'v' else w.a
            for l in range(64):
                for q in range(n):
                    x = addr[l] + 4 * q
                    if 0 <= x and x + 4 <= len(self.lds):
                        self.lds[x:x + 4] = np.frombuffer(np.uint32(src[i + q][l]).tobytes(), np.uint8)
            w.lq.append(lambda: None)
        elif mn == 'ds_bpermute_b32':
            addr = self.rd(w, A[1])
            src = self.rd(w, A[2])
            val = src[(addr // 4) % 64]
            self.wr(w, A[0], np.full(64, 0xFFFFFFFF, np.uint32))
            w.lq.append(lambda w=w, d=A[0], val=val: self.wr(w, d, val))
        elif mn == 'buffer_load_dwordx4' and op.mods.get('lds'):
            # LDS DMA: lane l's 16 bytes land at m0 + offset + 16 l when a vmcnt wait retires the load; until then
            # the destination holds garbage (catches reads that do not wait, and loads into buffers still read)
            base, nrec = self.rsrc(w, A[1])
            off = self.rd(w, A[0]).astype(np.int64) + op.mods.get('offset', 0)
            dst0 = int(w.s[124]) + op.mods.get('offset', 0)
            data = np.zeros((64, 16), np.uint8)
            for l in range(64):
                if off[l] < nrec:
                    data[l] = self.g.b[base + off[l]: base + off[l] + 16]
            assert 0 <= dst0 and dst0 + 1024 <= len(self.lds), f'LDS DMA to {dst0} out of range'
            self.lds[dst0:dst0 + 1024] = 0xFF
            self.pend[dst0:dst0 + 1024] += 1
            flat = data.reshape(-1).copy()

            def land(d0=dst0, flat=flat):
                self.lds[d0:d0 + 1024] = flat
                self.pend[d0:d0 + 1024] -= 1
            w.vmq.append(land)
        elif mn in ('buffer_load_dwordx4', 'buffer_load_dword'):
            kind, i, n, _ = parse_reg(A[0])
            base, nrec = self.rsrc(w, A[2])
            off = self.rd(w, A[1]).astype(np.int64) + op.mods.get('offset', 0)
            dst = w.v if kind == 'v' else w.a
            got = []
            nq = 4 if mn.endswith('x4') else 1
            for q in range(nq):
                vals = np.zeros(64, np.uint32)
                for l in range(64):
                    o = off[l] + 4 * q
                    if off[l] < nrec:  # range check on the whole access
                        vals[l] = self.g.b[base + o: base + o + 4].view(np.uint32)[0]
                got.append(vals)
                dst[i + q] = 0xFFFFFFFF

            def land(dst=dst, i=i, got=got):
                for q in range(len(got)):
                    dst[i + q] = got[q]
            w.vmq.append(land)
        elif mn.startswith('buffer_store_dword'):
            kind, i, n, _ = parse_reg(A[0])
            base, nrec = self.rsrc(w, A[2])
            off = self.rd(w, A[1]).astype(np.int64) + op.mods.get('offset', 0)
            for l in range(64):
                if off[l] < nrec:
                    for q in range(n):
                        o = base + off[l] + 4 * q
                        self.g.b[o:o + 4] = np.frombuffer(np.uint32(w.v[i + q][l]).tobytes(), np.uint8)
        else:
            raise NotImplementedError(op.line)

    def sidx(self, x):
        return 124 if x == 'm0' else parse_reg(x)[1]

    def retire(self, w, n):
        while len(w.vmq) > n:
            w.vmq.pop(0)()

    def retire_lds(self, w, n):
        while len(w.lq) > n:
            w.lq.pop(0)()

    def bank(self, op, addr, size):
        # lanes are served 128 bytes at a time: groups of 128 / size consecutive lanes must hit distinct
        # (addr / size) % (128 / size) slots; the transpose read in passes of 32 lanes over the 64 banks (256 bytes),
        # as SQ_LDS_BANK_CONFLICT measures it (about 2 cycles a read for a layout whose 32-lane pass covers 32 banks
        # twice, none for one that covers the 64 once)
        per = (256 if op.mn == 'ds_read_b64_tr_b16' else 128) // size
        worst = 1
        for g0 in range(0, 64, per):
            sl = (addr[g0:g0 + per] // size) % per
            worst = max(worst, int(np.bincount(sl.astype(np.int64)).max()))
        key = re.sub(r'\d+', '#', op.mn + ' ' + op.args[0])
        self.conflicts[op.mn] = max(self.conflicts.get(op.mn, 1), worst)

    def mfma(self, w, A, ty):
        kd, di, dn, _ = parse_reg(A[0])
        ka, ai, _, _ = parse_reg(A[1])
        kb, bi, _, _ = parse_reg(A[2])
        regs = {'v': w.v, 'a': w.a}

        def elems(kind, base):
            # lane l: 8 16-bit elements from 4 dwords
            d = regs[kind][base:base + 4]  # (4, 64)
            out = np.zeros((64, 8), np.float64)
            for q in range(4):
                lo, hi = d[q] & 0xFFFF, d[q] >> 16
                if ty == 'bf16':
                    out[:, 2 * q] = u2f(lo << 16)
                    out[:, 2 * q + 1] = u2f(hi << 16)
                else:
                    out[:, 2 * q] = bits2h(lo)
                    out[:, 2 * q + 1] = bits2h(hi)
            return out
        ea, eb = elems(ka, ai), elems(kb, bi)
        Am = np.zeros((32, 16))
        Bm = np.zeros((16, 32))
        for l in range(64):
            Am[l % 32, 8 * (l // 32): 8 * (l // 32) + 8] = ea[l]
            Bm[8 * (l // 32): 8 * (l // 32) + 8, l % 32] = eb[l]
        if A[3] == '0':
            C = np.zeros((32, 32))
        else:
            kc, ci, _, _ = parse_reg(A[3])
            C = np.zeros((32, 32))
            for l in range(64):
                for r in range(16):
                    C[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32] = u2f(regs[kc][ci + r][l])
        D = (Am @ Bm + C).astype(F32)
        dst = regs[kd]
        for r in range(16):
            vals = np.zeros(64, np.uint32)
            for l in range(64):
                vals[l] = f2u(D[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32])
            dst[di + r] = vals

    def run_wg(self, waves):
        rnd = 0
        while True:
            progressed = False
            at_barrier = []
            k = rnd % len(waves)
            rnd += 1
            for w in waves[k:] + waves[:k]:
                if w.done:
                    continue
                while True:
                    if w.pc >= len(self.prog):
                        self.retire(w, 0)
                        self.retire_lds(w, 0)
                        w.done = True
                        break
                    r = self.step(w)
                    if r == 'barrier':
                        at_barrier.append(w)
                        break
                progressed = True
            live = [w for w in waves if not w.done]
            if not live:
                return
            if len(at_barrier) != len(live):
                raise RuntimeError(f'barrier mismatch: {len(at_barrier)} at barrier, {len(live)} live')
