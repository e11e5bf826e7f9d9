#!/usr/bin/env python3
"""Benchmark of the attention path on one MI355X, through the C ABI (mako-common_amd/lib/libmako_attn.so).

Headline (one JSON line): causal GQA prefill at the Qwen3-8B shape (batch 1, 32 query heads over 8 kv heads,
D 128, S 4096, bf16 in and out, fp32 accumulate, LSE), in TFLOP/s counting only the unmasked pairs
(4 * D * S (S + 1) / 2 * 32). Beside it: batch-16 decode against a contiguous f16 KV cache (contexts drawn
uniformly from [1024, 32768], seed 2026) in GB/s of K + V read (sum of 4096 * ctx bytes), and the bidirectional
S16384 24-head case, the S16384 causal block-sparse case, MiniMax-H3's block-sparse call (cube_select and
per-head lists) and its dense 56-head S19308 bidirectional case (the reference's one published shape) in TFLOP/s,
the head tiles of the prefill step
(fp32 rows to normed, rotated bf16 tiles) in GB/s, the split-K / gathered latent-cache helpers of a sparse latent
decode, each against its own roof, the output projection after attention (Qwen3-8B o_proj) in TFLOP/s, and the
gated delta rule of the linear-attention layers in TFLOP/s. Inputs are synthetic N(0, 1), resident in
HBM before the timed region. `value` and ms_per_step come from --steps back-to-back launches bracketed by HIP
events on the launch stream, after --warmup untimed ones; the roofline's `achieved` divides by the mean of each
launch's own event pair (the kernel's duration, which rocprofv3's kernel trace also reports). The CPU baseline is
the oracle (oracle/attn_oracle.c, double precision, pthreads) on the host's cores (at most 16 threads: one GPU's
share of the host), timed on the whole S512 case and on a bounded random sample of the rows of every other
configuration, scaled to the metric's unit by the sample's share of the algorithmic work; the same sampled rows are
the parity check of the GPU output against the oracle.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
                  [--only prefill,s512,decode,bidir,sparse,h3_sparse,h3_bidir,heads,step,gather,proj,scan,copy]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mako-common_amd"))

PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA
PEAK_GBPS = 8000.0    # MI355X HBM3E
U32_MAX = 0xFFFFFFFF
CPU_SECONDS = 8.0     # wall-clock budget of each CPU-baseline leg
WARM_SECONDS = 0.3    # least untimed GPU work before each timed region


def time_launches(torch, fn, steps, warmup):
    """Times `steps` back-to-back launches of fn after `warmup` untimed ones, by HIP events on the current stream
    (the stream the C ABI launches on). Returns (ms a step over a timed region of `steps` calls with nothing
    between them, the mean of each launch's own event pair over a second such region): the first is the step time,
    the second the kernel duration the roofline divides (an event pair around every call adds its own gaps to the
    stream, so the two regions are separate). The untimed warmup also runs for at least WARM_SECONDS, so the GPU's
    clocks have settled before the timed regions."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARM_SECONDS:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, sum(a.elapsed_time(b) for a, b in ev) / steps


def traffic(kernel):
    """HBM bytes a launch of `kernel` moves, from the committed counter summary (profiles/traffic.json: two
    rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, each scaled by what it reads for a copy of known size);
    None when the summary does not cover the kernel."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get("kernels", {}).get(kernel)
    return None if entry is None else entry["bytes_per_launch"]


def cpu_threads():
    """Threads of the CPU baseline: the cores this process may run on, at most 16 (the host's share for one GPU)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def cpu_info():
    """What the CPU baseline ran on: the thread count used, the host's logical CPUs, and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return {"cores": cpu_threads(), "nproc": os.cpu_count(), "affinity": avail, "cpu_model": model,
            "threads": "oracle pthreads over (head, row) items, min(16, CPUs available to the process)"}


ATOL, RTOL, LSE_TOL = 2e-3, 1e-2, 1e-3


def parity_of(got, want, dim, lse_got=None, lse_want=None):
    """Parity of GPU rows against the oracle's: max abs error, max relative error (over |ref| >= 1e-2), the worst
    error as a fraction of the element tolerance 2e-3 + 1e-2 |ref|, the worst row's relative L2 (the reference's
    measure, threshold 5e-3) and the LSE's max abs error."""
    import numpy as np

    got = np.asarray(got, np.float64).reshape(-1, dim)
    want = np.asarray(want, np.float64).reshape(-1, dim)
    err = np.abs(got - want)
    big = np.abs(want) >= 1e-2
    nrm = np.maximum((want ** 2).sum(1), 1e-30)
    out = {"rows": int(got.shape[0]), "max_abs_err": float(err.max()),
           "max_rel_err": float((err[big] / np.abs(want[big])).max()) if big.any() else 0.0,
           "worst_over_tol": float((err / (ATOL + RTOL * np.abs(want))).max()),
           "worst_row_rel_l2": float(np.sqrt(((got - want) ** 2).sum(1) / nrm).max())}
    ok = bool(np.all(err <= ATOL + RTOL * np.abs(want))) and out["worst_row_rel_l2"] < 5e-3
    if lse_got is not None:
        lg, lw = np.asarray(lse_got, np.float64).ravel(), np.asarray(lse_want, np.float64).ravel()
        fin = np.isfinite(lw)
        out["lse_max_abs_err"] = float(np.abs(lg[fin] - lw[fin]).max()) if fin.any() else 0.0
        ok = ok and out["lse_max_abs_err"] <= LSE_TOL and bool(np.array_equal(np.isfinite(lg), fin))
    out["tolerance"] = "|err| <= 2e-3 + 1e-2 |ref| element-wise, worst row rel L2 < 5e-3, lse within 1e-3"
    out["within_tolerance"] = ok
    return out


def bits(torch, t):
    return t.cpu().view(torch.int16).numpy().view("uint16")


def cpu_sample(run, n0, budget):
    """Runs run(n) with n doubling from n0 until one run takes at least budget / 4 seconds; returns (n, seconds)
    of the last run."""
    n = n0
    while True:
        t0 = time.perf_counter()
        run(n)
        dt = time.perf_counter() - t0
        if dt >= budget / 4 or n >= 1 << 16:
            return n, dt
        n = int(n * min(8.0, max(2.0, budget / 2 / max(dt, 1e-3))))


def dense_cpu_leg(torch, M, O, q, k, v, o, lse, args, dtype, seed, n0, label, full=False):
    """The CPU baseline and parity of a dense leg: the oracle on every (head, row) pair (full) or on a random sample
    of them, timed; the sampled rows of the GPU output (o [n_q][heads * D], lse [heads][n_q]) against the oracle's.
    Returns (cpu_baseline, parity)."""
    import numpy as np

    H, D, S, nk = args["heads"], args["dim"], args["n_q"], args["n_k"]
    qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
    rng = np.random.default_rng(seed)
    gpu_o, gpu_l = o.float().cpu().numpy(), lse.cpu().numpy()
    state = {}

    def keys_of(r):  # keys row r sees (prefix-causal rule with q_pos0)
        pos = args["q_pos0"] + int(r)
        return nk if pos >= args["block"] else min(nk, pos + 1)

    def run(n):
        if full:
            hr = np.stack(np.meshgrid(np.arange(H), np.arange(S), indexing="ij"), -1).reshape(-1, 2).astype(np.uint32)
        else:
            hr = np.stack([rng.integers(0, H, n), rng.integers(0, S, n)], 1).astype(np.uint32)
        want, wl = O.attn_dense_rows(qb, kb, vb, hr, dtype=dtype, nthreads=cpu_threads(), **args)
        state["hr"], state["want"], state["wl"] = hr, want, wl

    if full:
        t0 = time.perf_counter()
        run(0)
        n, dt = H * S, time.perf_counter() - t0
    else:
        n, dt = cpu_sample(run, n0, CPU_SECONDS)
    hr, want, wl = state["hr"], state["want"], state["wl"]
    sample_flop = float(sum(4.0 * D * keys_of(r) for _, r in hr))
    got = np.stack([gpu_o[r, h * D:(h + 1) * D] for h, r in hr])
    got_l = np.array([gpu_l[h, r] for h, r in hr])
    base = {"value": sample_flop / dt / 1e12, "unit": "TFLOP/s", "kind": "port", "extrapolated": not full,
            "sample": (f"every (head, row) pair of {label}" if full else
                       f"{n} random (head, row) pairs of {label}") +
                      f", double precision, {dt:.2f} s wall; TFLOP/s of the unmasked pairs computed"}
    base.update(cpu_info())
    return base, parity_of(got, want, D, got_l, wl), (hr, want, wl)


def bench_prefill(torch, M, steps, warmup, with_cpu):
    import numpy as np

    S, H, KV, D = 4096, 32, 8, 128
    gen = torch.Generator(device="cuda").manual_seed(4096)
    q = torch.randn((H, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn((KV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((KV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    o = torch.empty((S, H * D), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((H, S), dtype=torch.float32, device="cuda")
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=H, kv_heads=KV, q_pos0=0, block=U32_MAX, dim=D)
    ms, kms = time_launches(torch, lambda: M.attn_fwd(q, k, v, o, lse=lse, **args), steps, warmup)
    flop = 4.0 * D * (S * (S + 1) / 2) * H
    tflops, ktflops = flop / (ms * 1e-3) / 1e12, flop / (kms * 1e-3) / 1e12
    out = {"ms": ms, "kernel_ms": kms, "tflops": tflops, "flop": flop,
           "roofline": {"bound": "mfma", "achieved": ktflops, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": ktflops / PEAK_TFLOPS, "traffic": traffic("flash_fwd_causal_s4096"),
                        "kernel": "flash_fwd_r64<bf16,bf16> (one launch a call)", "kernel_ms": kms}}
    if with_cpu:
        import oracle as O

        base, par, (hr, want, _) = dense_cpu_leg(torch, M, O, q, k, v, o, lse, args, O.BF16, 7, 64,
                                                 "the S4096 causal prefill")
        # The same rows with an f32 output: the kernel's own error, apart from the rounding of the bf16 output
        # (half an ulp of bf16 is 7.8e-3 at |o| in [2, 4)).
        o32 = torch.empty((S, H * D), dtype=torch.float32, device="cuda")
        M.attn_fwd(q, k, v, o32, **args)
        g32 = o32.cpu().numpy()
        par["f32_output"] = {k_: v_ for k_, v_ in parity_of(np.stack([g32[r, h * D:(h + 1) * D] for h, r in hr]),
                                                            want, D).items() if k_ != "tolerance"}
        out["cpu_baseline"], out["parity"] = base, par
    return out


def bench_s512(torch, M, steps, warmup, with_cpu):
    """The reference-CPU-runnable case: causal GQA, 16 query heads over 8 kv heads, D 128, S 512, f16 in, f32 out
    (the reference's output), LSE; the CPU baseline runs it whole and every output row is checked."""
    S, H, KV, D = 512, 16, 8, 128
    gen = torch.Generator(device="cuda").manual_seed(512)
    q = torch.randn((H, S, D), generator=gen, device="cuda").half()
    k = torch.randn((KV, S, D), generator=gen, device="cuda").half()
    v = torch.randn((KV, S, D), generator=gen, device="cuda").half()
    o = torch.empty((S, H * D), dtype=torch.float32, device="cuda")
    lse = torch.empty((H, S), dtype=torch.float32, device="cuda")
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=H, kv_heads=KV, q_pos0=0, block=U32_MAX, dim=D)
    ms, kms = time_launches(torch, lambda: M.attn_fwd(q, k, v, o, lse=lse, **args), steps, warmup)
    flop = 4.0 * D * (S * (S + 1) / 2) * H
    kt = flop / (kms * 1e-3) / 1e12
    out = {"value": round(flop / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
           "dtype": "f16",
           "roofline": {"bound": "mfma", "achieved": kt, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": kt / PEAK_TFLOPS, "traffic": traffic("flash_fwd_causal_s512"),
                        "kernel": "flash_fwd_r64<f16,f32> (one launch a call)", "kernel_ms": kms,
                        "note": "1.08 GFLOP: 16 workgroups on 256 CUs, launch- and latency-bound"},
           "config": {"workload": "causal GQA prefill, batch 1, 16 query heads / 8 kv heads, D 128, S 512, f16 in, "
                                  "f32 out, LSE (the reference-CPU-runnable case)"}}
    if with_cpu:
        import oracle as O

        out["cpu_baseline"], out["parity"], _ = dense_cpu_leg(torch, M, O, q, k, v, o, lse, args, O.F16, 0, 0,
                                                              "the S512 causal prefill", full=True)
    return out


def bench_decode(torch, M, steps, warmup, with_cpu):
    import numpy as np

    B, H, KV, D, cap = 16, 32, 8, 128, 32768
    ctx = np.random.default_rng(2026).integers(1024, 32769, B).astype(np.uint32)
    gen = torch.Generator(device="cuda").manual_seed(2026)
    q = torch.randn((B, H, D), generator=gen, device="cuda").half()
    k = torch.randn((B, KV, cap, D), generator=gen, device="cuda").half()
    v = torch.randn((B, KV, cap, D), generator=gen, device="cuda").half()
    ctx_d = torch.from_numpy(ctx.astype(np.int32)).to("cuda")
    o = torch.empty((B, H * D), dtype=torch.float16, device="cuda")
    lse = torch.empty((B, H), dtype=torch.float32, device="cuda")
    a = M.decode_args(batch=B, heads=H, kv_heads=KV, dim=D, cap=cap, max_ctx=cap)
    ws = torch.empty(M.decode_workspace(a), dtype=torch.uint8, device="cuda")
    ms, kms = time_launches(torch, lambda: M.attn_decode(a, q, k, v, ctx_d, o, ws, lse=lse), steps, warmup)
    nbytes = float(4096 * ctx.astype(np.int64).sum())  # K + V: kv_heads * D * 2 bytes * 2 tensors per token
    gbps, kgbps = nbytes / (ms * 1e-3) / 1e9, nbytes / (kms * 1e-3) / 1e9
    out = {"ms": ms, "kernel_ms": kms, "gbps": gbps, "bytes": nbytes, "sum_ctx": int(ctx.sum()),
           "roofline": {"bound": "hbm", "achieved": kgbps, "peak": PEAK_GBPS, "unit": "GB/s",
                        "frac": kgbps / PEAK_GBPS, "traffic": traffic("decode_batch16"),
                        "kernel": "decode_split<f16> + decode_merge<f16> (one step, both kernels)",
                        "kernel_ms": kms}}
    if with_cpu:
        import oracle as O

        qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
        rng = np.random.default_rng(11)
        gpu_o, gpu_l = o.float().cpu().numpy(), lse.cpu().numpy()
        state = {}

        def run(n):
            sh = np.stack([rng.integers(0, B, n), rng.integers(0, H, n)], 1).astype(np.uint32)
            want, wl = O.attn_decode_rows(qb, kb, vb, ctx, sh, batch=B, heads=H, kv_heads=KV, dim=D, cap=cap,
                                          dtype=O.F16, nthreads=cpu_threads())
            state["sh"], state["want"], state["wl"] = sh, want, wl

        n, dt = cpu_sample(run, 16, CPU_SECONDS)
        sh, want, wl = state["sh"], state["want"], state["wl"]
        # a (sequence, head) pair's share of the K + V bytes: its kv head's rows serve H / KV query heads
        sample_bytes = float(sum(4096 * int(ctx[b]) / H for b, _ in sh))
        got = np.stack([gpu_o[b, h * D:(h + 1) * D] for b, h in sh])
        out["cpu_baseline"] = {"value": sample_bytes / dt / 1e9, "unit": "GB/s", "kind": "port", "extrapolated": True,
                               "sample": f"{n} random (sequence, head) pairs of the batch-16 decode, double "
                                         f"precision, {dt:.2f} s wall; each pair credited its share of K + V bytes"}
        out["cpu_baseline"].update(cpu_info())
        out["parity"] = parity_of(got, want, D, np.array([gpu_l[b, h] for b, h in sh]), wl)
    return out


def bench_few_rows(torch, M, steps, warmup, with_cpu, nqs=(1, 4, 16)):
    """attention() with a few query rows (the reference's decode is attention(n_q = 1, q_pos0 = ctx - 1)): n_q 1, 4
    and 16 at ctx 32768, 32 query heads over 8 kv heads, bf16, through mako_attn_fwd (its split-K route). HBM-bound:
    each call reads K + V once, 8 x 32768 x 256 bytes each."""
    import numpy as np

    H, KV, D, n = 32, 8, 128, 32768
    gen = torch.Generator(device="cuda").manual_seed(32768)
    k = torch.randn((KV, n, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((KV, n, D), generator=gen, device="cuda").to(torch.bfloat16)
    nbytes = 2.0 * KV * n * D * 2
    out = {}
    for nq in (1, 4, 16):
        q = torch.randn((H, nq, D), generator=gen, device="cuda").to(torch.bfloat16)
        if nq not in nqs:
            continue
        o = torch.empty((nq, H * D), dtype=torch.bfloat16, device="cuda")
        lse = torch.empty((H, nq), dtype=torch.float32, device="cuda")
        args = dict(n_q=nq, q_pad=nq, n_k=n, k_pad=n, heads=H, kv_heads=KV, q_pos0=n - nq, block=U32_MAX, dim=D)
        ms, kms = time_launches(torch, lambda: M.attn_fwd(q, k, v, o, lse=lse, **args), steps, warmup)
        kg = nbytes / (kms * 1e-3) / 1e9
        leg = {"ms": round(ms, 5), "kernel_ms": round(kms, 5), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
               "roofline": {"bound": "hbm", "achieved": kg, "peak": PEAK_GBPS, "unit": "GB/s",
                            "frac": kg / PEAK_GBPS, "traffic": traffic(f"few_rows_nq{nq}"),
                            "kernel": "decode_coop<bf16> (%d column group%s) + decode_merge<bf16> (one call, both "
                                      "kernels)" % ((1, "") if nq * H // KV <= 32 else (2, "s")), "kernel_ms": kms}}
        if with_cpu:
            import oracle as O

            qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
            rng = np.random.default_rng(nq)
            gpu_o, gpu_l = o.float().cpu().numpy(), lse.cpu().numpy()
            state = {}

            def run(m):
                hr = np.stack([rng.integers(0, H, m), rng.integers(0, nq, m)], 1).astype(np.uint32)
                want, wl = O.attn_dense_rows(qb, kb, vb, hr, dtype=O.BF16, nthreads=cpu_threads(), **args)
                state["hr"], state["want"], state["wl"] = hr, want, wl

            m, dt = cpu_sample(run, 8, CPU_SECONDS / 3)
            hr = state["hr"]
            got = np.stack([gpu_o[r, h * D:(h + 1) * D] for h, r in hr])
            leg["cpu_baseline"] = {"value": m * nbytes / (H * nq) / dt / 1e9, "unit": "GB/s", "kind": "port",
                                   "extrapolated": True,
                                   "sample": f"{m} random (head, row) pairs, double precision, {dt:.2f} s wall; each "
                                             f"pair credited its share of the K + V bytes"}
            leg["cpu_baseline"].update(cpu_info())
            leg["parity"] = parity_of(got, state["want"], D, np.array([gpu_l[h, r] for h, r in hr]), state["wl"])
        out[f"n_q={nq}"] = leg
    return out


def bench_bidir(torch, M, steps, warmup, with_cpu):
    S, H, D = 16384, 24, 128
    gen = torch.Generator(device="cuda").manual_seed(16384)
    q, k, v = (torch.randn((H, S, D), generator=gen, device="cuda").to(torch.bfloat16) for _ in range(3))
    o = torch.empty((S, H * D), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((H, S), dtype=torch.float32, device="cuda")
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=H, kv_heads=H, q_pos0=0, block=0, dim=D)
    ms, kms = time_launches(torch, lambda: M.attn_fwd(q, k, v, o, lse=lse, **args), steps, warmup)
    flop = 4.0 * D * S * S * H
    kt = flop / (kms * 1e-3) / 1e12
    out = {"value": round(flop / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
           "kernel_ms": round(kms, 4), "frac": round(kt / PEAK_TFLOPS, 4), "dtype": "bf16",
           "roofline": {"bound": "mfma", "achieved": kt, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": kt / PEAK_TFLOPS, "traffic": traffic("flash_fwd_bidir_s16384"),
                        "kernel": "flash_fwd_r64<bf16,bf16> (one launch a call)", "kernel_ms": kms},
           "config": {"workload": "bidirectional MHA, 24 heads, D 128, S 16384, bf16 in/out, LSE"}}
    if with_cpu:
        import oracle as O

        out["cpu_baseline"], out["parity"], _ = dense_cpu_leg(torch, M, O, q, k, v, o, lse, args, O.BF16, 5, 16,
                                                              "the S16384 bidirectional case")
    return out


def bench_other_dims(torch, M, steps, warmup, with_cpu, names=None):
    """The attention path's other head widths, each against the MFMA roof: heads of 256 causal (the Qwen3.5 gated
    attention layers, qwen_text.cpp:418, at a Qwen3-Next-style shape: 16 query heads over 2 kv heads, S 4096) on
    flash_fwd_wide, and heads of 64 bidirectional (the H3 VAE decoder's ViT attention, h3_vae.cpp:219: MHA, 16
    heads, 4096 tokens) on flash_fwd. bf16 in and out, LSE."""
    legs = {
        "d256_causal": dict(H=16, KV=2, D=256, S=4096, block=U32_MAX, seed=256,
                            kernel="flash_fwd_r32<bf16,bf16> (one launch a call)",
                            workload="causal GQA, 16 query heads / 2 kv heads, D 256, S 4096, bf16 in/out, LSE "
                                     "(Qwen3.5 gated attention)"),
        "d64_bidir": dict(H=16, KV=16, D=64, S=4096, block=0, seed=64,
                          kernel="flash_fwd_r64<bf16,bf16,64> (one launch a call)",
                          workload="bidirectional MHA, 16 heads, D 64, S 4096, bf16 in/out, LSE (H3 VAE ViT)"),
    }
    out = {}
    for name, c in legs.items():
        if names is not None and name not in names:
            continue
        H, KV, D, S = c["H"], c["KV"], c["D"], c["S"]
        gen = torch.Generator(device="cuda").manual_seed(c["seed"])
        q = torch.randn((H, S, D), generator=gen, device="cuda").to(torch.bfloat16)
        k = torch.randn((KV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
        v = torch.randn((KV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
        o = torch.empty((S, H * D), dtype=torch.bfloat16, device="cuda")
        lse = torch.empty((H, S), dtype=torch.float32, device="cuda")
        args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=H, kv_heads=KV, q_pos0=0, block=c["block"], dim=D)
        ms, kms = time_launches(torch, lambda: M.attn_fwd(q, k, v, o, lse=lse, **args), steps, warmup)
        pairs = S * (S + 1) / 2 if c["block"] == U32_MAX else S * S
        flop = 4.0 * D * pairs * H
        kt = flop / (kms * 1e-3) / 1e12
        leg = {"value": round(flop / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
               "kernel_ms": round(kms, 4), "frac": round(kt / PEAK_TFLOPS, 4), "dtype": "bf16",
               "roofline": {"bound": "mfma", "achieved": kt, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": kt / PEAK_TFLOPS, "traffic": traffic(name), "kernel": c["kernel"],
                            "kernel_ms": kms},
               "config": {"workload": c["workload"], "flop": flop}}
        if with_cpu:
            import oracle as O

            leg["cpu_baseline"], leg["parity"], _ = dense_cpu_leg(torch, M, O, q, k, v, o, lse, args, O.BF16,
                                                                  c["seed"], 16, f"the {name} case")
        out[name] = leg
    return out


def bench_sparse(torch, M, steps, warmup, with_cpu):
    """Block-sparse causal attention, S16384, 32 query heads over 8 kv heads, 64x64 blocks: each block attends
    itself (causal), the 8 before it and 8 random earlier ones (seed 16384, one list per kv head). MFMA-bound: the
    gathered K / V (each block once per query block and kv head, 1.105 GB) is mostly served by the L2s (the byte
    counters measure about half a gigabyte of HBM traffic), so the roofline divides the unmasked-pair FLOPs."""
    import numpy as np

    S, H, KV, D = 16384, 32, 8, 128
    nb = S // 64
    sel, nsel = M.window_random_blocks(nb, KV, seed=16384)
    gen = torch.Generator(device="cuda").manual_seed(16384)
    q = torch.randn((H, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn((KV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((KV, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    o = torch.empty((S, H * D), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((H, S), dtype=torch.float32, device="cuda")
    sel_d = torch.from_numpy(sel.view(np.int16)).to("cuda")
    nsel_d = torch.from_numpy(nsel.view(np.int16)).to("cuda")
    valid = torch.ones(S, dtype=torch.uint8, device="cuda")
    map_ = torch.arange(S, dtype=torch.int32, device="cuda")
    args = dict(n_q=S, q_pad=S, n_k=S, k_pad=S, heads=H, kv_heads=KV, n_cubes=nb, max_sel=sel.shape[2], dense0=S,
                dense1=S, causal=1, sel_heads=KV)
    ms, kms = time_launches(torch, lambda: M.attn_sparse(q, k, v, o, sel_d, nsel_d, valid, map_, lse=lse, **args),
                            steps, warmup)
    blocks = int(nsel[0].astype(np.int64).sum())          # blocks a head attends (the same count for every list)
    pairs = (blocks - nb) * 64 * 64 + nb * (64 * 65 // 2)  # full blocks, plus the causal diagonal ones
    flop = 4.0 * D * pairs * H
    gathered = float(blocks) * KV * 64 * D * 2 * 2        # K + V of each block once per (query block, kv head)
    kt = flop / (kms * 1e-3) / 1e12
    hbm = traffic("flash_sparse_s16384")
    out = {"value": round(flop / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
           "kernel_ms": round(kms, 4), "dtype": "bf16", "blocks": blocks,
           "gathered_gbps": round(gathered / (kms * 1e-3) / 1e9, 1),
           "roofline": {"bound": "mfma", "achieved": kt, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": kt / PEAK_TFLOPS, "traffic": hbm,
                        "kernel": "sparse_prep (pass table) + flash_sparse_r64<bf16,bf16> (one call, both kernels)",
                        "kernel_ms": kms,
                        "hbm_frac": None if hbm is None else hbm / (kms * 1e-3) / 1e9 / PEAK_GBPS,
                        "note": "gathered K + V (1.105 GB) is L2 traffic; HBM moves the counted bytes"},
           "config": {"workload": "causal block-sparse, 32 query heads / 8 kv heads, D 128, S 16384, 64x64 blocks: "
                                  "diagonal + 8 preceding + 8 random earlier (seed 16384, per kv head), bf16",
                      "blocks_per_head": blocks}}
    if with_cpu:
        import oracle as O

        qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
        rng = np.random.default_rng(3)
        gpu_o, gpu_l = o.float().cpu().numpy(), lse.cpu().numpy()
        valid_h = np.ones(S, np.uint8)
        state = {}

        def run(n):
            hr = np.stack([rng.integers(0, H, n), rng.integers(0, S, n)], 1).astype(np.uint32)
            want, wl = O.attn_sparse_rows(qb, kb, vb, sel, nsel, valid_h, hr, dtype=O.BF16, nthreads=cpu_threads(),
                                          **args)
            state["hr"], state["want"], state["wl"] = hr, want, wl

        n, dt = cpu_sample(run, 64, CPU_SECONDS)
        hr, want, wl = state["hr"], state["want"], state["wl"]
        # keys a row sees: 64 per full block of its list, plus the causal part of its diagonal block
        sample_flop = float(sum(4.0 * D * ((int(nsel[h // (H // KV), r // 64]) - 1) * 64 + r % 64 + 1)
                                for h, r in hr))
        got = np.stack([gpu_o[r, h * D:(h + 1) * D] for h, r in hr])
        out["cpu_baseline"] = {"value": sample_flop / dt / 1e12, "unit": "TFLOP/s", "kind": "port",
                               "extrapolated": True,
                               "sample": f"{n} random (head, row) pairs of the S16384 block-sparse case, double "
                                         f"precision, {dt:.2f} s wall; TFLOP/s of the unmasked pairs computed"}
        out["cpu_baseline"].update(cpu_info())
        out["parity"] = parity_of(got, want, D, np.array([gpu_l[h, r] for h, r in hr]), wl)
    return out


def h3_cubes(frames, ph, pw, dense):
    """The row layout of MiniMax-H3's sparse attention (h3.cpp:510-547): the video rows of `frames` latent frames
    of ph x pw patches in 4 x 4 x 4 cubes of (frame, patch row, patch column), the grid padded to multiples of 4 with
    rows that are no token (valid 0, map -1), then the `dense` text, conditioning and audio rows. The model's rows
    are the dense ones first, then the video frame by frame. Returns n_cubes, the attention rows, the cube-grid
    stride of one latent frame step (yc * xc), map [rows] i32, valid [rows] u8 and the cubes' row counts."""
    import numpy as np

    fc, yc, xc = (-(-frames // 4), -(-ph // 4), -(-pw // 4))
    n = fc * yc * xc
    vrows = n * 64
    rows = vrows + dense
    map_ = np.full(rows, -1, np.int32)
    valid = np.zeros(rows, np.uint8)
    f, y, x = np.meshgrid(np.arange(frames), np.arange(ph), np.arange(pw), indexing="ij")
    cube = ((f // 4) * yc + y // 4) * xc + x // 4
    r = cube * 64 + ((f % 4) * 4 + y % 4) * 4 + x % 4
    map_[r.ravel()] = (dense + (f * ph + y) * pw + x).ravel()
    valid[r.ravel()] = 1
    map_[vrows:] = np.arange(dense)
    valid[vrows:] = 1
    cnt = np.bincount(cube.ravel(), minlength=n).astype(np.uint32)
    return n, rows, yc * xc, map_, valid, cnt


def bench_h3_sparse(torch, M, steps, warmup, with_cpu):
    """MiniMax-H3's block-sparse attention as its engine calls it (h3.cpp:342-366, 510-547; runtime.hpp:96-106):
    56 heads of 128 (MHA), f16 tiles, f32 output through the row map; cube_select with per-head lists (top 1/8 of the
    cubes, the local option 3: a cube and its neighbours one latent-frame step before and after lead each list),
    then attention over the selected cubes plus the dense rows; tiles past the cubes see every key. The layout: a
    960x544 video at 9 latent frames of 34 x 60 patches (18360 video rows in 405 cubes, 25920 rows padded) and 948
    dense rows: the 19308 rows of the reference's own attention benchmark. Roofline: MFMA, over the unmasked pairs
    (valid rows against the valid keys of their passes); the pairs of the visited tiles are reported beside them."""
    import numpy as np

    H, D, dense, ratio, local = 56, 128, 948, 0.125, 3
    n, rows, stride, map_h, valid_h, cnt_h = h3_cubes(9, 34, 60, dense)
    S = int(map_h.max()) + 1
    q_pad, k_pad = -(-rows // 64) * 64, -(-rows // 128) * 128
    topk = max(1, int(np.ceil(ratio * n)))
    gen = torch.Generator(device="cuda").manual_seed(19308)
    live = torch.zeros(max(q_pad, k_pad), dtype=torch.float16, device="cuda")
    live[:rows] = torch.from_numpy(valid_h).to("cuda").half()
    q, k, v = ((torch.randn((H, p, D), generator=gen, device="cuda").half() * live[:p, None]).contiguous()
               for p in (q_pad, k_pad, k_pad))
    o = torch.zeros((S, H * D), dtype=torch.float32, device="cuda")
    lse = torch.empty((H, q_pad), dtype=torch.float32, device="cuda")
    sel = torch.zeros((H, n, topk), dtype=torch.int16, device="cuda")
    nsel = torch.zeros((H, n), dtype=torch.int16, device="cuda")
    ws = torch.empty(M.cube_select_workspace(H, n), dtype=torch.uint8, device="cuda")
    cnt = torch.from_numpy(cnt_h.view(np.int32)).to("cuda")
    valid = torch.zeros(k_pad, dtype=torch.uint8, device="cuda")
    valid[:rows] = torch.from_numpy(valid_h).to("cuda")
    map_ = torch.full((q_pad,), -1, dtype=torch.int32, device="cuda")
    map_[:rows] = torch.from_numpy(map_h).to("cuda")
    sargs = dict(heads=H, q_pad=q_pad, k_pad=k_pad, n_cubes=n, topk=topk, local=local, stride=stride)
    args = dict(n_q=rows, q_pad=q_pad, n_k=rows, k_pad=k_pad, heads=H, kv_heads=H, n_cubes=n, max_sel=topk,
                dense0=n * 64, dense1=rows, causal=0, sel_heads=H)

    def select():
        M.cube_select(q, k, cnt, sel, nsel, ws, **sargs)

    def attend(lse_out=None):
        M.attn_sparse(q, k, v, o, sel, nsel, valid, map_, lse=lse_out, **args)

    def call():
        select()
        attend()

    select()
    torch.cuda.synchronize()
    ns = nsel.cpu().numpy().view(np.uint16).astype(np.int64)
    sl = sel.cpu().numpy().view(np.uint16).astype(np.int64)
    # algorithmic work: the unmasked (query row, key) pairs, valid rows against the valid keys of their lists and
    # the dense rows (the tiles past the cubes: every valid key); the pairs of the visited tiles as information
    cnt64 = cnt_h.astype(np.int64)
    kvalid = np.where(np.arange(topk)[None, None, :] < ns[:, :, None], cnt64[sl], 0).sum(-1) + dense
    pairs = float((cnt64[None, :] * kvalid).sum() + H * (rows - n * 64) * int(valid_h.sum()))
    # the tiles the kernel computes: 32-key halves of the listed cubes that hold a valid key, the dense rows
    halves = valid_h[:n * 64].reshape(n, 2, 32).any(-1).sum(-1).astype(np.int64)
    n_halves = np.where(np.arange(topk)[None, None, :] < ns[:, :, None], halves[sl], 0).sum(-1)
    visited = float(64 * (32 * n_halves + dense).sum() + H * (rows - n * 64) * rows)
    flop = 4.0 * D * pairs
    ms_sel, kms_sel = time_launches(torch, select, steps, warmup)
    ms_att, kms_att = time_launches(torch, attend, steps, warmup)
    ms, _ = time_launches(torch, call, steps, warmup)
    kt = flop / (kms_att * 1e-3) / 1e12
    vt = 4.0 * D * visited / (kms_att * 1e-3) / 1e12
    out = {"value": round(flop / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
           "attention": {"ms_per_step": round(ms_att, 4), "kernel_ms": round(kms_att, 4),
                         "tflops": round(kt, 2), "frac": round(kt / PEAK_TFLOPS, 4),
                         "visited_tflops": round(vt, 2), "visited_frac": round(vt / PEAK_TFLOPS, 4)},
           "cube_select": {"ms_per_step": round(ms_sel, 4), "kernel_ms": round(kms_sel, 4)},
           "dtype": "f16",
           "roofline": {"bound": "mfma", "achieved": kt, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": kt / PEAK_TFLOPS, "traffic": traffic("flash_sparse_h3"),
                        "kernel": "the attention of the call (per-head lists)", "kernel_ms": kms_att},
           "config": {"workload": "MiniMax-H3 block-sparse attention at 960x544: 56 heads of 128 (MHA), 405 cubes "
                                  f"of 64 rows, per-head lists of the top {topk} (1/8, local 3, stride {stride}), "
                                  f"{dense} dense rows, {rows} attention rows mapped to {S} model rows, f16 in, f32 "
                                  "out; value: cube_select + attention a step",
                      "pairs": pairs, "flop": flop, "visited_pairs": visited,
                      "flop_note": "unmasked pairs only (valid rows x valid keys); the kernel also computes the "
                                   "masked rows and keys inside the 32-key tiles it visits (visited_pairs: the "
                                   "cube padding of the layout)"}}
    if with_cpu:
        import oracle as O

        attend(lse)
        torch.cuda.synchronize()
        qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
        sel_h, nsel_h = sel.cpu().numpy().view(np.uint16), nsel.cpu().numpy().view(np.uint16)
        t0 = time.perf_counter()
        want_sel, want_nsel = O.cube_select(qb, kb, cnt_h, dim=D, dtype=O.F16, **sargs)
        t_sel = time.perf_counter() - t0
        gpu_o, gpu_l = o.cpu().numpy(), lse.cpu().numpy()
        rng = np.random.default_rng(56)
        live_rows = np.flatnonzero(map_h >= 0)
        state = {}

        def run(m):
            hr = np.stack([rng.integers(0, H, m), live_rows[rng.integers(0, len(live_rows), m)]], 1)
            hr = hr.astype(np.uint32)
            want, wl = O.attn_sparse_rows(qb, kb, vb, sel_h, nsel_h, np.pad(valid_h, (0, k_pad - rows)), hr,
                                          dtype=O.F16, nthreads=cpu_threads(), **args)
            state["hr"], state["want"], state["wl"] = hr, want, wl

        m, dt = cpu_sample(run, 64, CPU_SECONDS)
        hr, want, wl = state["hr"], state["want"], state["wl"]
        keys = [(int(ns[h, r // 64]) * 64 + dense) if r < n * 64 else rows for h, r in hr]
        got = np.stack([gpu_o[map_h[r], h * D:(h + 1) * D] for h, r in hr])
        out["cpu_baseline"] = {"value": 4.0 * D * sum(keys) / dt / 1e12, "unit": "TFLOP/s", "kind": "port",
                               "extrapolated": True,
                               "sample": f"{m} random (head, live row) pairs of the attention, double precision, "
                                         f"{dt:.2f} s wall, over the GPU's lists; cube_select of all 56 heads "
                                         f"{t_sel:.2f} s, one thread"}
        out["cpu_baseline"].update(cpu_info())
        out["parity"] = parity_of(got, want, D, np.array([gpu_l[h, r] for h, r in hr]), wl)
        out["parity"]["cube_select_exact"] = bool(np.array_equal(sel_h, want_sel) and
                                                  np.array_equal(nsel_h, want_nsel))
    return out


def bench_h3_bidir(torch, M, steps, warmup, with_cpu):
    """The one shape the reference publishes a time for: its attention benchmark's default, MiniMax-H3's dense
    sequence at 960x544 (bench/attn_bench.cpp:1-2, 36-39): 56 heads of 128, 19308 query rows over 19308 keys,
    bidirectional, f16 in and f32 out, no LSE. The reference's figure, 302 ms for flash_attn_coop_128_32
    (ops.metal:227-228), is from an Apple GPU, not from this hardware; vs_baseline is that time over this one."""
    S, H, D = 19308, 56, 128
    q_pad, k_pad = -(-S // 64) * 64, -(-S // 128) * 128
    gen = torch.Generator(device="cuda").manual_seed(302)
    q = torch.randn((H, q_pad, D), generator=gen, device="cuda").half()
    k = torch.randn((H, k_pad, D), generator=gen, device="cuda").half()
    v = torch.randn((H, k_pad, D), generator=gen, device="cuda").half()
    o = torch.empty((S, H * D), dtype=torch.float32, device="cuda")
    args = dict(n_q=S, q_pad=q_pad, n_k=S, k_pad=k_pad, heads=H, kv_heads=H, q_pos0=0, block=0, dim=D)
    ms, kms = time_launches(torch, lambda: M.attn_fwd(q, k, v, o, **args), steps, warmup)
    flop = 4.0 * D * S * S * H
    kt = flop / (kms * 1e-3) / 1e12
    ref_ms = 302.0
    out = {"value": round(flop / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
           "kernel_ms": round(kms, 4), "frac": round(kt / PEAK_TFLOPS, 4), "dtype": "f16",
           "vs_baseline": round(ref_ms / ms, 2),
           "baseline": {"ms": ref_ms, "tflops": round(flop / (ref_ms * 1e-3) / 1e12, 2),
                        "hardware": "Apple GPU (unnamed), the reference's published figure, not MI355X",
                        "source": "src/kernels/ops.metal:227-228; bench/attn_bench.cpp:1-2"},
           "roofline": {"bound": "mfma", "achieved": kt, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": kt / PEAK_TFLOPS, "traffic": traffic("flash_fwd_h3_s19308"),
                        "kernel": "flash_fwd_r64<f16,f32> (one launch a call)", "kernel_ms": kms},
           "config": {"workload": "MiniMax-H3 dense attention at 960x544: 56 heads of 128 (MHA), 19308 x 19308, "
                                  "bidirectional, f16 in, f32 out, no LSE", "flop": flop}}
    if with_cpu:
        import oracle as O

        lse = torch.empty((H, S), dtype=torch.float32, device="cuda")  # [heads][n_q]
        M.attn_fwd(q, k, v, o, lse=lse, **args)
        torch.cuda.synchronize()
        out["cpu_baseline"], out["parity"], _ = dense_cpu_leg(torch, M, O, q, k, v, o, lse, args, O.F16, 19, 16,
                                                              "the 56-head S19308 bidirectional case")
    return out


def bench_heads(torch, M, steps, warmup):
    """The head tiles of a Qwen3-8B prefill step (src/models/qwen_text.cpp:415-417): 4096 tokens, q 32 heads and
    k 8 heads of 128 RMS-normed and rotated over the whole head, v 8 heads sliced, from fp32 rows into bf16 tiles;
    one step is the three calls. Bytes: the fp32 rows read, the angle table read once, the tiles written."""
    T, D = 4096, 128
    gen = torch.Generator(device="cuda").manual_seed(4096)
    xq = torch.randn((T, 32 * D), generator=gen, device="cuda")
    xk = torch.randn((T, 8 * D), generator=gen, device="cuda")
    xv = torch.randn((T, 8 * D), generator=gen, device="cuda")
    ang = torch.rand((T, D // 2), generator=gen, device="cuda") * 6.283
    cs = torch.stack([ang.cos(), ang.sin()], -1).contiguous()
    wq, wk = (torch.rand(D, generator=gen, device="cuda") + 0.5 for _ in range(2))
    yq = torch.empty((32, T, D), dtype=torch.bfloat16, device="cuda")
    yk, yv = (torch.empty((8, T, D), dtype=torch.bfloat16, device="cuda") for _ in range(2))
    base = dict(rows=T, col0=0, stride=D, dim=D, n_pad=T)

    def step():
        M.heads(xq, yq, ld=32 * D, heads=32, rope=1, rot=D, eps=1e-6, cs=cs, w=wq, **base)
        M.heads(xk, yk, ld=8 * D, heads=8, rope=1, rot=D, eps=1e-6, cs=cs, w=wk, **base)
        M.heads(xv, yv, ld=8 * D, heads=8, **base)
    ms, kms = time_launches(torch, step, steps, warmup)
    nbytes = 48.0 * T * D * (4 + 2) + T * D // 2 * 8
    gbps = nbytes / (kms * 1e-3) / 1e9
    return {"ms": ms, "kernel_ms": kms, "gbps": gbps, "bytes": nbytes, "frac": gbps / PEAK_GBPS}


def bench_step(torch, M, steps, warmup):
    """The attention of a Qwen3-8B prefill step from the projections' fp32 rows (src/models/qwen_text.cpp:308-311,
    the q / k norms folded into the producers): 4096 tokens, q 32 heads and k 8 heads of 128 RMS-normed and rotated,
    v 8 heads, causal GQA attention into bf16 rows with the LSE. Timed two ways on the same inputs: one call of
    mako_attn_fwd_rows (qkv_prep, flash_fwd_r64), and the separate calls (mako_heads three times, then
    mako_attn_fwd: heads_vec x 3, flash_fwd_r64); both give the same bits (checked here, untimed)."""
    T, D, H, KV = 4096, 128, 32, 8
    gen = torch.Generator(device="cuda").manual_seed(4096)
    xq = torch.randn((T, H * D), generator=gen, device="cuda")
    xk = torch.randn((T, KV * D), generator=gen, device="cuda")
    xv = torch.randn((T, KV * D), generator=gen, device="cuda")
    ang = torch.rand((T, D // 2), generator=gen, device="cuda") * 6.283
    cs = torch.stack([ang.cos(), ang.sin()], -1).contiguous()
    wq, wk = (torch.rand(D, generator=gen, device="cuda") + 0.5 for _ in range(2))
    yq = torch.empty((H, T, D), dtype=torch.bfloat16, device="cuda")
    yk, yv = (torch.empty((KV, T, D), dtype=torch.bfloat16, device="cuda") for _ in range(2))
    o = torch.empty((T, H * D), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((H, T), dtype=torch.float32, device="cuda")
    hq = dict(rows=T, ld=H * D, col0=0, stride=D, dim=D, heads=H, rope=1, rot=D, eps=1e-6)
    hk = dict(hq, ld=KV * D, heads=KV)
    hv = dict(rows=T, ld=KV * D, col0=0, stride=D, dim=D, heads=KV)
    attn = dict(n_q=T, n_k=T, heads=H, kv_heads=KV, q_pos0=0, block=U32_MAX)

    def fused():
        M.attn_fwd_rows(xq, xk, xv, o, hq, hk, hv, in_dtype=M.BF16, cs=cs, wq=wq, wk=wk, lse=lse, **attn)

    def separate():
        M.heads(xq, yq, n_pad=T, cs=cs, w=wq, **hq)
        M.heads(xk, yk, n_pad=T, cs=cs, w=wk, **hk)
        M.heads(xv, yv, n_pad=T, **hv)
        M.attn_fwd(yq, yk, yv, o, lse=lse, q_pad=T, k_pad=T, dim=D, **attn)

    fused()
    torch.cuda.synchronize()
    got = (o.view(torch.int16).clone(), lse.clone())
    separate()
    torch.cuda.synchronize()
    same = bool(torch.equal(got[0], o.view(torch.int16)) and torch.equal(got[1].view(torch.int32),
                                                                         lse.view(torch.int32)))
    ms_f, kms_f = time_launches(torch, fused, steps, warmup)
    ms_s, kms_s = time_launches(torch, separate, steps, warmup)
    flop = 4.0 * D * (T * (T + 1) / 2) * H
    prep_bytes = 48.0 * T * D * 4 + T * D // 2 * 8 + (H + 2 * KV) * T * D * 2.0
    return {"value": round(kms_f * 1e3, 1), "unit": "us a step", "higher_is_better": False,
            "ms_per_step": round(ms_f, 4), "kernel_ms": round(kms_f, 4),
            "separate_calls": {"ms_per_step": round(ms_s, 4), "kernel_ms": round(kms_s, 4)},
            "speedup_vs_separate": round(kms_s / kms_f, 3), "same_bits_as_separate": same,
            "attention_tflops_over_step": round(flop / (kms_f * 1e-3) / 1e12, 1),
            "qkv_prep_bytes": prep_bytes,
            "config": {"workload": "Qwen3-8B prefill attention step from fp32 projection rows: 4096 tokens, q 32 and "
                                   "k 8 heads of 128 RMS-normed and rotated (rope over the whole head), v 8 heads, "
                                   "causal GQA, bf16 tiles and output, LSE"}}


def bench_gather(torch, M, steps, warmup):
    """The split-K and gathered latent-cache helpers (src/kernels/gemm.metal:683-870) at a sparse latent decode
    shape: a 65536-row cache of 512-wide f16 latent rows; 64 consecutive query tokens of 64 heads, each over its own
    list of 2048 rows (attn_gather_scores, then attn_gather_pv in one split); attn_pv of 64 heads over 32768 keys in
    splits of 512; the float indexer (idx_dots) of 32 heads of 128 over 16384 pooled keys. Each kernel is timed on
    its own; bytes are what it must move (rows gathered, probabilities and scores once, outputs once); the roofline
    of each is the larger of its HBM and MFMA times (f16 MFMA 2.5 PFLOP/s, f32 MFMA 157.3 TFLOP/s)."""
    import numpy as np

    R, T, H, D, S = 65536, 64, 64, 512, 2048
    gen = torch.Generator(device="cuda").manual_seed(512)
    kv = (torch.randn((R, D), generator=gen, device="cuda") * 0.1).half()
    q = (torch.randn((T, H, D), generator=gen, device="cuda") * 0.1).half()
    rng = np.random.default_rng(512)
    lst = torch.from_numpy(np.stack([rng.choice(R, S, replace=False) for _ in range(T)]).astype(np.int32)).cuda()
    cnt = torch.full((T,), S, dtype=torch.int32, device="cuda")
    scores = torch.empty((T, H, S), dtype=torch.float32, device="cuda")
    p = torch.softmax(torch.randn((T, H, S), generator=gen, device="cuda"), -1)
    part = torch.empty((1, T, H, D), dtype=torch.float32, device="cuda")
    NK, KPS = 32768, 512
    pk = torch.softmax(torch.randn((H, NK), generator=gen, device="cuda"), -1)
    kpart = torch.empty((NK // KPS, H, D), dtype=torch.float32, device="cuda")
    IH, ID, PL = 32, 128, 16384
    iq = torch.randn((T, IH, ID), generator=gen, device="cuda")
    pooled = torch.randn((PL, ID), generator=gen, device="cuda")
    dots = torch.empty((T, IH, PL), dtype=torch.float32, device="cuda")
    g = dict(heads=H, dim=D, stride=S, tokens=T)
    legs = {
        "attn_gather_scores": (lambda: M.attn_gather_scores(q, kv, lst, cnt, scores, **g),
                               T * S * D * 2 + T * H * D * 2 + T * S * 4 + T * H * S * 4, 2.0 * T * H * S * D, 2500),
        "attn_gather_pv": (lambda: M.attn_gather_pv(p, kv, lst, cnt, part, splits=1, **g),
                           T * S * D * 2 + T * H * S * 4 + T * S * 4 + T * H * D * 4, 2.0 * T * H * S * D, 2500),
        "attn_pv": (lambda: M.attn_pv(pk, kv, kpart, heads=H, dim=D, n_kv=NK, keys_per_split=KPS),
                    NK * D * 2 + H * NK * 4 + NK // KPS * H * D * 4, 2.0 * H * NK * D, 2500),
        "idx_dots": (lambda: M.idx_dots(iq, pooled, dots, tokens=T, heads=IH, dim=ID, pools=PL, stride=PL),
                     T * IH * ID * 4 + PL * ID * 4 + T * IH * PL * 4, 2.0 * T * IH * PL * ID, 157.3),
    }
    out = {}
    for name, (fn, nbytes, flop, peak_tf) in legs.items():
        ms, kms = time_launches(torch, fn, steps, warmup)
        t_hbm, t_mfma = nbytes / (PEAK_GBPS * 1e9), flop / (peak_tf * 1e12)
        out[name] = {"ms": round(ms, 4), "kernel_ms": round(kms, 4), "bytes": nbytes, "flop": flop,
                     "gbps": round(nbytes / (kms * 1e-3) / 1e9, 1), "tflops": round(flop / (kms * 1e-3) / 1e12, 2),
                     "bound": "mfma" if t_mfma > t_hbm else "hbm",
                     "frac": round(max(t_hbm, t_mfma) / (kms * 1e-3), 4)}
    return out


def bench_proj(torch, M, steps, warmup):
    """The output projection after attention at Qwen3-8B's prefill shape (src/models/qwen_text.cpp:312): 4096
    tokens x 4096 -> 4096, bf16 weights, f32 output. Three forms: bf16 activations as the attention writes them (the
    headline of this leg), f32 activations rounded in the GEMM's loads, and f32 with the bf16 split (twice the
    MFMA work). TFLOP/s count 2 t k n (4 t k n with the split)."""
    t = k = n = 4096
    gen = torch.Generator(device="cuda").manual_seed(312)
    w = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    xf = torch.randn((t, k), generator=gen, device="cuda")
    xb = xf.to(torch.bfloat16)
    y = torch.empty((t, n), dtype=torch.float32, device="cuda")
    out = {}
    for name, x, split in (("bf16_x", xb, 0), ("f32_x", xf, 0), ("f32_x_split", xf, 1)):
        ms, kms = time_launches(torch, lambda: M.proj_bf16(w, x, y, t=t, k=k, n=n, split=split), steps, warmup)
        flop = 2.0 * t * k * n * (2 if split else 1)
        out[name] = {"ms": round(ms, 4), "kernel_ms": round(kms, 4), "flop": flop,
                     "tflops": round(flop / (kms * 1e-3) / 1e12, 1),
                     "frac": round(flop / (kms * 1e-3) / 1e12 / PEAK_TFLOPS, 4)}
    # For scale only: the vendor library on the same shape (torch.matmul on bf16, f32 accumulate, bf16 output)
    yb = torch.empty((t, n), dtype=torch.bfloat16, device="cuda")
    wt = w.t()
    ms, kms = time_launches(torch, lambda: torch.matmul(xb, wt, out=yb), steps, warmup)
    out["vendor_library_bf16_out"] = {"kernel_ms": round(kms, 4), "tflops": round(2.0 * t * k * n / (kms * 1e-3) / 1e12, 1)}
    return out


def bench_scan(torch, M, steps, warmup):
    """The gated delta rule (kda_scan) at the shape of Qwen3.5's linear-attention layers: 32 heads of 128 over 4096
    tokens, f32, q and k unit-norm per head, g a log-decay in [-0.5, 0], beta in (0, 1), the state zeroed before
    each call. VALU work: 896 flops a (token, head, state row) (the decay, and three 128-term fused multiply-add
    sums); the roofline is the vector f32 peak (157.3 TFLOP/s counts packed FP32, which these kernels do not use:
    78.6 without it)."""
    T, H, D = 4096, 32, 128
    gen = torch.Generator(device="cuda").manual_seed(459)
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)
    q = unit(torch.randn((T, H, D), generator=gen, device="cuda")).reshape(T, H * D).contiguous()
    k = unit(torch.randn((T, H, D), generator=gen, device="cuda")).reshape(T, H * D).contiguous()
    v = torch.randn((T, H * D), generator=gen, device="cuda")
    g = -0.5 * torch.rand((T, H * D), generator=gen, device="cuda")
    beta = torch.rand((T, H), generator=gen, device="cuda") * 0.9 + 0.05
    state = torch.zeros((H, D, D), device="cuda")
    o = torch.empty((T, H * D), device="cuda")
    ms, kms = time_launches(torch, lambda: M.kda_scan(q, k, v, g, beta, state, o, tokens=T, heads=H), steps, warmup)
    flop = 896.0 * T * H * D
    nbytes = 4.0 * T * H * D * 5 + 4.0 * T * H + 2 * 4.0 * H * D * D
    return {"ms": round(ms, 4), "kernel_ms": round(kms, 4), "flop": flop, "bytes": nbytes,
            "tflops": round(flop / (kms * 1e-3) / 1e12, 2), "gbps": round(nbytes / (kms * 1e-3) / 1e9, 1),
            "frac_of_157": round(flop / (kms * 1e-3) / 1e12 / 157.3, 4),
            "frac_of_78_6_unpacked": round(flop / (kms * 1e-3) / 1e12 / 78.6, 4)}


def bench_copy(torch, steps, warmup):
    """A plain device copy of known size: the reference point that scales the HBM byte counters."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    ms, kms = time_launches(torch, lambda: dst.copy_(src), steps, warmup)
    return {"bytes_read": n, "bytes_written": n, "ms": ms, "kernel_ms": kms, "gbps": 2 * n / (kms * 1e-3) / 1e9}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline and parity legs")
    ap.add_argument("--only", default=None,
                    help="comma-separated legs to run alone (no CPU legs unless --cpu): prefill, s512, decode, "
                         "few_rows, bidir, dims, sparse, h3_sparse, h3_bidir, heads, step, gather, proj, scan, copy; "
                         "few_rows:N runs the n_q = N "
                         "case alone, dims:NAME one head width (d256_causal, d64_bidir)")
    ap.add_argument("--cpu", action="store_true", help="with --only: run the legs' CPU-baseline and parity parts")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the attention path is built and "
              f"measured on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    import mako_attn as M

    M.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    if args.only:
        c = args.cpu
        sub = {}
        for leg in args.only.split(","):
            name, _, case = leg.partition(":")
            if case:
                sub.setdefault(name, []).append(int(case) if name == "few_rows" else case)
        fn = {"prefill": lambda: bench_prefill(torch, M, args.steps, args.warmup, c),
              "s512": lambda: bench_s512(torch, M, args.steps, args.warmup, c),
              "decode": lambda: bench_decode(torch, M, args.steps, args.warmup, c),
              "few_rows": lambda: bench_few_rows(torch, M, args.steps, args.warmup, c,
                                                 tuple(sub.get("few_rows", (1, 4, 16)))),
              "bidir": lambda: bench_bidir(torch, M, args.steps, args.warmup, c),
              "dims": lambda: bench_other_dims(torch, M, args.steps, args.warmup, c, sub.get("dims")),
              "sparse": lambda: bench_sparse(torch, M, args.steps, args.warmup, c),
              "h3_sparse": lambda: bench_h3_sparse(torch, M, args.steps, args.warmup, c),
              "h3_bidir": lambda: bench_h3_bidir(torch, M, args.steps, args.warmup, c),
              "heads": lambda: bench_heads(torch, M, args.steps, args.warmup),
              "step": lambda: bench_step(torch, M, args.steps, args.warmup),
              "gather": lambda: bench_gather(torch, M, args.steps, args.warmup),
              "proj": lambda: bench_proj(torch, M, args.steps, args.warmup),
              "scan": lambda: bench_scan(torch, M, args.steps, args.warmup),
              "copy": lambda: bench_copy(torch, args.steps, args.warmup)}
        for leg in dict.fromkeys(x.partition(":")[0] for x in args.only.split(",")):
            if leg not in fn:
                ap.error(f"--only: unknown leg {leg!r}")
            print(json.dumps({leg: fn[leg]()}), flush=True)
        return
    with_cpu = not args.no_cpu
    pre = bench_prefill(torch, M, args.steps, args.warmup, with_cpu)
    s512 = bench_s512(torch, M, args.steps, args.warmup, with_cpu)
    dec = bench_decode(torch, M, args.steps, args.warmup, with_cpu)
    few = bench_few_rows(torch, M, args.steps, args.warmup, with_cpu)
    bid = bench_bidir(torch, M, max(1, args.steps // 4), max(1, args.warmup), with_cpu)
    dims = bench_other_dims(torch, M, max(1, args.steps // 2), args.warmup, with_cpu)
    spa = bench_sparse(torch, M, args.steps, args.warmup, with_cpu)
    h3s = bench_h3_sparse(torch, M, max(1, args.steps // 4), max(1, args.warmup), with_cpu)
    h3d = bench_h3_bidir(torch, M, max(1, args.steps // 8), max(1, args.warmup), with_cpu)
    hds = bench_heads(torch, M, args.steps, args.warmup)
    stp = bench_step(torch, M, args.steps, args.warmup)
    gat = bench_gather(torch, M, args.steps, args.warmup)
    prj = bench_proj(torch, M, max(1, args.steps // 2), args.warmup)
    scn = bench_scan(torch, M, max(1, args.steps // 4), max(1, args.warmup))
    line = {
        "metric": "attn prefill TFLOP/s (Qwen3-8B shape, seq 4096) + decode KV HBM GB/s, 1 GPU",
        "value": round(pre["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1), seeded, resident in HBM",
        "config": {"workload": "causal GQA prefill, batch 1, 32 query heads / 8 kv heads, D 128, S 4096, bf16 "
                               "in/out, fp32 accumulate, LSE", "global_batch": 1, "seq_len": 4096,
                   "parallelism": "single GPU"},
        "roofline": pre["roofline"],
        "prefill_s512": s512,
        "decode": {"value": round(dec["gbps"], 1), "unit": "GB/s", "ms_per_step": round(dec["ms"], 4),
                   "dtype": "f16", "config": {"workload": "decode, batch 16, 32 query heads / 8 kv heads, D 128, "
                                                          "contexts U[1024, 32768] seed 2026, f16 cache",
                                              "sum_ctx": dec["sum_ctx"]},
                   "roofline": dec["roofline"]},
        "few_rows": {"value": few["n_q=1"]["gbps"], "unit": "GB/s", "dtype": "bf16",
                     "roofline": few["n_q=1"]["roofline"],
                     "per_n_q": few,
                     "config": {"workload": "attention() with n_q 1, 4, 16 rows at q_pos0 = ctx - n_q, ctx 32768, "
                                            "32 query heads / 8 kv heads, D 128, bf16 in/out, LSE (split-K route)",
                                "bytes": 2 * 8 * 32768 * 256}},
        "bidirectional": bid,
        "other_head_widths": dims,
        "block_sparse": spa,
        "h3_block_sparse": h3s,
        "h3_bidirectional": h3d,
        "head_tiles": {"value": round(hds["gbps"], 1), "unit": "GB/s", "ms_per_step": round(hds["ms"], 4),
                       "kernel_ms": round(hds["kernel_ms"], 4), "bound": "hbm", "frac": round(hds["frac"], 4),
                       "config": {"workload": "Qwen3-8B prefill head tiles: 4096 tokens, q 32 and k 8 heads of 128 "
                                              "RMS-normed and rotated, v 8 heads sliced, fp32 rows to bf16 tiles",
                                  "bytes": hds["bytes"]}},
        "prefill_step_from_rows": stp,
        "latent_decode": {name: {"kernel_ms": v["kernel_ms"], "gbps": v["gbps"], "tflops": v["tflops"],
                                 "bound": v["bound"], "frac": v["frac"]} for name, v in gat.items()},
    }
    line["output_projection"] = {
        "value": prj["bf16_x"]["tflops"], "unit": "TFLOP/s", "kernel_ms": prj["bf16_x"]["kernel_ms"],
        "bound": "mfma", "frac": prj["bf16_x"]["frac"],
        "f32_rows": {k: prj["f32_x"][k] for k in ("kernel_ms", "tflops", "frac")},
        "f32_rows_bf16_split": {k: prj["f32_x_split"][k] for k in ("kernel_ms", "tflops", "frac")},
        "vendor_library_bf16_out_tflops": prj["vendor_library_bf16_out"]["tflops"],
        "config": {"workload": "Qwen3-8B o_proj after a 4096-token prefill: 4096 x 4096 bf16 weights over the "
                               "attention's bf16 rows [4096][32 * 128], f32 output"}}
    line["linear_attention"] = {
        "value": scn["tflops"], "unit": "TFLOP/s", "kernel_ms": scn["kernel_ms"], "bound": "valu",
        "frac": scn["frac_of_157"], "frac_without_packed_fp32": scn["frac_of_78_6_unpacked"],
        "config": {"workload": "gated delta rule (kda_scan), 32 heads of 128 over 4096 tokens, f32, state zeroed"}}
    line["latent_decode"]["config"] = {"workload": "sparse latent decode helpers: 65536-row cache of 512-wide f16 "
                                                   "latent rows, 64 tokens x 64 heads over lists of 2048 (scores, "
                                                   "then P V in one split), attn_pv of 64 heads over 32768 keys in "
                                                   "splits of 512, f32 indexer 64 x 32 heads of 128 over 16384 "
                                                   "pooled keys"}
    if with_cpu:
        line["cpu_baseline"] = pre["cpu_baseline"]
        line["parity"] = pre["parity"]
        line["decode"]["cpu_baseline"] = dec["cpu_baseline"]
        line["decode"]["parity"] = dec["parity"]
    line["configs"] = configs_summary(line, pre, dec, few)
    print(json.dumps(line), flush=True)


def configs_summary(line, pre, dec, few):
    """The five configurations, the other head widths and the few-row route in a few numbers each, last in the JSON
    line (so a record that keeps only the line's tail still holds them): value, unit, kernel ms, fraction of the
    roofline, and the parity of the sampled rows (within tolerance, max abs error)."""
    def par(p):
        return {} if not p else {"within_tolerance": p["within_tolerance"], "max_abs_err": round(p["max_abs_err"], 6)}

    def entry(value, unit, kernel_ms, frac, parity):
        return dict({"value": round(value, 2), "unit": unit, "kernel_ms": round(kernel_ms, 4),
                     "frac": round(frac, 4)}, **par(parity))
    s512, bid, spa = line["prefill_s512"], line["bidirectional"], line["block_sparse"]
    h3s, h3d = line["h3_block_sparse"], line["h3_bidirectional"]
    f1 = few["n_q=1"]
    return {
        "C1_causal_s512_f16": entry(s512["value"], "TFLOP/s", s512["roofline"]["kernel_ms"], s512["roofline"]["frac"],
                                    s512.get("parity")),
        "C2_causal_s4096_bf16": entry(pre["tflops"], "TFLOP/s", pre["kernel_ms"], pre["roofline"]["frac"],
                                      pre.get("parity")),
        "C3_decode_b16": entry(dec["gbps"], "GB/s", dec["kernel_ms"], dec["roofline"]["frac"], dec.get("parity")),
        "C4_block_sparse_s16384": entry(spa["value"], "TFLOP/s", spa["kernel_ms"], spa["roofline"]["frac"],
                                        spa.get("parity")),
        "C5_bidirectional_s16384": entry(bid["value"], "TFLOP/s", bid["kernel_ms"], bid["frac"], bid.get("parity")),
        **{f"heads_{name}": entry(h["value"], "TFLOP/s", h["kernel_ms"], h["frac"], h.get("parity"))
           for name, h in line["other_head_widths"].items() if isinstance(h, dict) and "kernel_ms" in h},
        "few_rows_n_q1": entry(f1["gbps"], "GB/s", f1["kernel_ms"], f1["roofline"]["frac"], f1.get("parity")),
        "h3_sparse_per_head_lists": entry(h3s["attention"]["tflops"], "TFLOP/s", h3s["attention"]["kernel_ms"],
                                          h3s["roofline"]["frac"], h3s.get("parity")),
        "h3_bidirectional_s19308_f16_f32": dict(entry(h3d["value"], "TFLOP/s", h3d["kernel_ms"], h3d["frac"],
                                                      h3d.get("parity")),
                                                vs_baseline=h3d["vs_baseline"],
                                                baseline="302 ms on an Apple GPU (reference's published figure)"),
    }


if __name__ == "__main__":
    main()
