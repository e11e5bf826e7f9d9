"""The decode split's work partition, restated in Python from csrc/attn_decode.hip (Ranges, decode_split's piece
loop, decode_merge's lookup), checked for the properties the kernels rely on: every K/V row is in exactly one piece,
piece ids (wave + segment) are unique and inside the partial buffer, and the merge finds exactly the pieces of each
segment (empty sequences, empty waves when there are fewer rows than waves, the batch-16 shape): as many as the
waves w_lo .. w_hi over it (the segment's rows when there are fewer rows than waves). decode_coop cuts the same way
over workgroups (one range a workgroup, segments = kv heads), and its waves' tiles (column group w % ncg, every
(8 / ncg)-th 32-key tile from the piece's start) must cover every key of a piece exactly once for each column
group."""
import random


def rs(w, T, n): return w * T // n
def wave_of(x, T, n):
    w = x * n // T
    while w + 1 < n and rs(w + 1, T, n) <= x: w += 1
    while w > 0 and rs(w, T, n) > x: w -= 1
    return w
def simulate(ctx, KV, n_waves, max_ctx):
    ctx = [min(c, max_ctx) for c in ctx]
    B = len(ctx); total = sum(ctx) * KV
    written = {}; cover = [0] * total
    for wave in range(n_waves):
        r0, r1 = rs(wave, total, n_waves), rs(wave + 1, total, n_waves)
        if r0 >= r1: continue
        b = 0; seg0 = 0
        while b < B:
            ln = ctx[b] * KV
            if r0 < seg0 + ln: break
            seg0 += ln; b += 1
        c = ctx[b]; kvh = (r0 - seg0) // c; row = r0
        while row < r1:
            s_start = seg0 + kvh * c
            kb = row - s_start; ke = min(c, r1 - s_start)
            assert 0 <= kb < ke <= c
            seg = b * KV + kvh
            pid = wave + seg
            assert pid < n_waves + B * KV and pid not in written, (pid, wave, seg)
            written[pid] = (b, kvh, kb, ke)
            for r in range(s_start + kb, s_start + ke): cover[r] += 1
            row = s_start + ke
            kvh += 1
            if kvh == KV:
                kvh = 0; seg0 += c * KV; b += 1
                while b < B and ctx[b] == 0: b += 1
                if b >= B: break
                c = ctx[b]
    assert all(x == 1 for x in cover), "rows not covered exactly once"
    # pieces a segment gets: the waves over it (its rows when there are fewer rows than waves)
    per_seg = {}
    for (b, kvh, kb, ke) in written.values():
        per_seg[(b, kvh)] = per_seg.get((b, kvh), 0) + 1
    q = total // n_waves
    seq0 = 0
    for b in range(B):
        for kvh in range(KV):
            c = ctx[b]
            if c == 0: continue
            s_start = seq0 * KV + kvh * c
            lo, hi = wave_of(s_start, total, n_waves), wave_of(s_start + c - 1, total, n_waves)
            target = hi - lo + 1 if q > 0 else c
            assert per_seg[(b, kvh)] == target, (b, kvh, per_seg[(b, kvh)], target)
        seq0 += ctx[b]
    # merge lookup
    seq0 = 0
    for b in range(B):
        for kvh in range(KV):
            c = ctx[b]
            if c == 0: continue
            s_start = seq0 * KV + kvh * c
            lo, hi = wave_of(s_start, total, n_waves), wave_of(s_start + c - 1, total, n_waves)
            got = []
            for w in range(lo, hi + 1):
                if rs(w, total, n_waves) == rs(w + 1, total, n_waves): continue
                pid = w + b * KV + kvh
                assert pid in written and written[pid][:2] == (b, kvh), (b, kvh, w)
                got.append(written[pid][2:])
            assert sorted(got)[0][0] == 0 and sum(e - s for s, e in got) == c
        seq0 += ctx[b]
    return len(written)

def test_partition_properties():
    random.seed(0)
    cases = [([1, 511, 512, 1025], 8, 2048), ([0, 64, 700], 8, 2048), ([2048, 2999], 2, 2048), ([33, 31, 32, 100, 300], 4, 2048),
             ([4096], 1, 2048), ([4999, 1234, 77], 4, 2048), ([0], 8, 2048), ([0, 0, 5], 8, 2048), ([7] * 300, 8, 2048)]
    cases += [([random.randint(1024, 32768) for _ in range(16)], 8, 2048)]
    cases += [([random.randint(0, 50) for _ in range(random.randint(1, 40))], random.choice([1, 2, 4, 8]), random.choice([4, 8, 64, 2048])) for _ in range(300)]
    for ctx, KV, n in cases:
        simulate(ctx, KV, n, max(max(ctx), 1))
    # split > 0 path: n_waves = ceil(B*KV*max_ctx/split) rounded to 4, capped
    for ctx, KV, split in [([4999, 1234, 77], 4, 64), ([4999, 1234, 77], 4, 512), ([1, 100, 160], 2, 64), ([0, 64, 700], 8, 64)]:
        mc = max(ctx); want = max(1, -(-len(ctx) * KV * mc // split)); n = min(want, 2048); n = -(-n // 4) * 4
        simulate(ctx, KV, n, mc)



def coop_tiles(kb, ke, ncg, waves=8):
    """Keys each column group's waves visit in a piece [kb, ke): wave w (cg = w % ncg, kw = w // ncg) takes the
    32-key tiles at kb + 32 (kw + j (waves // ncg)) below ke (decode_coop -> wave_keys)."""
    n_kw = waves // ncg
    seen = {cg: [] for cg in range(ncg)}
    for w in range(waves):
        cg, kw = w % ncg, w // ncg
        j0 = kb + 32 * kw
        while j0 < ke:
            seen[cg] += [j for j in range(j0, j0 + 32) if j < ke]
            j0 += 32 * n_kw
    return seen


def test_coop_partition_and_tiles():
    random.seed(1)
    # the few-row route: one sequence, kv heads x n_keys rows over ceil(rows / 1024) <= 256 workgroups
    for kv, n_keys in [(8, 32768), (8, 3000), (2, 4100), (4, 5000), (4, 103), (8, 1), (2, 2047), (1, 1025)]:
        rows = kv * n_keys
        n_wg = min(max(-(-rows // 1024), 1), 256)
        simulate([n_keys], kv, n_wg, n_keys)
    # and batches of sequences (empty ones included), with fewer rows than workgroups
    for _ in range(200):
        ctx = [random.randint(0, 3000) for _ in range(random.randint(1, 6))]
        simulate(ctx, random.choice([1, 2, 4, 8]), random.choice([1, 3, 64, 256]), max(max(ctx), 1))
    for kb, ke in [(0, 1024), (0, 1000), (17, 1024), (1000, 1001), (5, 300), (0, 32), (0, 33)]:
        for ncg in (1, 2):
            seen = coop_tiles(kb, ke, ncg)
            for cg in range(ncg):
                assert sorted(seen[cg]) == list(range(kb, ke)), (kb, ke, ncg, cg)
