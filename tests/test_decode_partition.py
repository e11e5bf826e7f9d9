"""The decode split's work partition, restated in Python from csrc/attn_decode.hip (Ranges, decode_split's piece
loop, decode_merge's lookup), checked for the properties the kernels rely on: every K/V row is in exactly one piece,
piece ids (wave + segment) are unique and inside the partial buffer, and the merge finds exactly the pieces of each
segment (empty sequences, empty waves when there are fewer rows than waves, the batch-16 shape)."""
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

