"""Benchmark of the KV-cache attention path on one MI355X.

Headline (BASELINE.json metric "decode attn HBM GB/s (% of peak) @ctx 8K"):
Llama-2-7B-shaped full-stack decode (config C2 shapes) at context 8K -- 32
layers x 32 q heads x 32 KV heads x head_dim 128, f16 KV cache already
holding 8192 rows.  One step = one decoded token: for each of the 32 layers,
one launch appends the token's K/V row (f32 -> f16) and runs decode
attention over all rows so far; the cache grows by one row per step.

  value    = algorithmic bytes of all attention launches in the timed steps
             / wall time of those steps (appends and launch gaps included);
  roofline = the decode kernel: algorithmic bytes per launch / its average
             launch duration from HIP events on the kernel's stream (a re-run
             of the same launches bracketed by two events).
Algorithmic bytes per (layer, step) = 2*L*n_kv*d*sizeof(kv) + n_heads*d*(4+4).

Secondary (metric "prefill attn TFLOP/s (% MFMA peak)"): Llama-3-8B causal
prefill (config C4) at 8192 tokens, bf16, FLOPs = 4*n_heads*d*L(L+1)/2.

cpu_baseline: the CPU oracle (a C restatement of vantablack's cpuAttention,
oracle/attn_oracle.c) on a bounded sample of the same decode workload, on
the host's cores, once faithfully single-threaded (as vantablack runs
attention) and once split over heads on a pool.zig-style pool.

roofline.traffic: HBM-side bytes per launch of the same kernel shape, read
from profiles/traffic.json.  That file comes from two rocprofv3 counter runs
over `bench.py --pmc-workload` (FETCH_SIZE, then WRITE_SIZE), each scaled by
what the counter reads for vtb_copy_f32 over a buffer of known size, and is
written by `bench.py --pmc-summary FETCH_DIR WRITE_DIR`.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--ctx 8192]
       python bench.py --pmc-workload              (the counter-run workload)
       python bench.py --pmc-summary FETCH_DIR WRITE_DIR
       python bench.py --trace-summary TRACE_DIR   (kernel-trace table by bench
                                                    section; trace taken with
                                                    VTB_BENCH_ROCTX=1 and
                                                    --marker-trace)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode attn HBM GB/s (% of peak) @ctx 8K; prefill attn TFLOP/s (% MFMA peak)"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
PMC_COPY_FLOATS = 64 << 20  # calibration copy: 256 MiB read + 256 MiB written
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class _Phases:
    """ROCTx ranges around the bench sections when VTB_BENCH_ROCTX=1, so a
    `rocprofv3 --kernel-trace --marker-trace` run of this script can be cut
    by section (`--trace-summary`).  A no-op otherwise."""

    def __init__(self):
        self.lib = None
        if os.environ.get("VTB_BENCH_ROCTX") == "1":
            import ctypes
            try:
                self.lib = ctypes.CDLL("librocprofiler-sdk-roctx.so.1")
                self.lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            except OSError:
                self.lib = None

    def __call__(self, name):
        phases = self

        class _Range:
            def __enter__(self):
                if phases.lib is not None:
                    phases.lib.roctxRangePushA(name.encode())

            def __exit__(self, *exc):
                if phases.lib is not None:
                    phases.lib.roctxRangePop()
        return _Range()


phase = _Phases()


def decode_bytes(L, n_heads, n_kv, d, kv_bytes):
    return 2 * L * n_kv * d * kv_bytes + n_heads * d * 8


def bench_decode(ctx, torch, args):
    import numpy as np
    import vantablack_amd as vb

    n_layers, n_heads, n_kv, d = 32, 32, 32, 128
    L0 = args.ctx
    total_steps = args.warmup + args.steps
    max_seq = L0 + total_steps
    dev = torch.device("cuda:0")
    stream = torch.cuda.ExternalStream(ctx.stream)
    # Layer-major cache [n_layers][max_seq][n_kv][d], f16, rows [0, L0) filled.
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    log(f"bench: allocating f16 KV cache {2 * n_layers * max_seq * n_kv * d * 2 / 2**30:.2f} GiB")
    kc = torch.empty((n_layers, max_seq, n_kv, d), dtype=torch.float16, device=dev)
    vc = torch.empty_like(kc)
    kc.normal_(generator=g)
    vc.normal_(generator=g)
    q = (torch.randn((n_layers, n_heads * d), generator=g, device=dev) / np.sqrt(d)).contiguous()
    kcur = torch.randn((n_layers, total_steps, n_kv * d), generator=g, device=dev)
    vcur = torch.randn((n_layers, total_steps, n_kv * d), generator=g, device=dev)
    out = torch.empty((n_layers, n_heads * d), device=dev)
    torch.cuda.synchronize()

    kb, vbuf = ctx.wrap_tensor(kc), ctx.wrap_tensor(vc)
    row_bytes = n_kv * d * 2
    layer_bytes = max_seq * row_bytes
    inv = 1.0 / np.sqrt(d)

    # Each layer reads its own q row and writes its own output row.
    qbs = [ctx.wrap_tensor(q[l]) for l in range(n_layers)]
    obs = [ctx.wrap_tensor(out[l]) for l in range(n_layers)]

    # The token's K/V rows per (layer, step), as the f32 k_cur/v_cur views the
    # fused launch appends.
    kcs = [[ctx.wrap_tensor(kcur[l, s]) for s in range(total_steps)] for l in range(n_layers)]
    vcs = [[ctx.wrap_tensor(vcur[l, s]) for s in range(total_steps)] for l in range(n_layers)]

    def step_layers(seg, s):
        # One launch per layer: KV-slot append fused with decode attention
        # (forward.zig:466-483 as one call), cache growing by one row per step.
        pos = L0 + s
        for l in range(n_layers):
            seg.attn_decode_append(obs[l], qbs[l], kb, l * layer_bytes, vbuf, l * layer_bytes, kcs[l][s], vcs[l][s],
                                   n_heads, n_kv, d, pos + 1, inv, vb.F16)

    with ctx.segment() as seg:
        for s in range(args.warmup):
            step_layers(seg, s)
    ctx.wait_idle()
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    with ctx.segment() as seg:
        for s in range(args.warmup, total_steps):
            step_layers(seg, s)
    ctx.wait_idle()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    alg = sum(n_layers * decode_bytes(L0 + s + 1, n_heads, n_kv, d, 2) for s in range(args.warmup, total_steps))
    value_gbs = alg / wall / 1e9

    # Kernel timing: the same decode launches (same lengths, slot rewritten
    # with the same rows) bracketed by two HIP events on the context stream,
    # divided by the launch count -- the launches run back to back, so this
    # is the kernel's average duration including the inter-kernel gap.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    with ctx.segment() as seg:
        for s in range(args.warmup, total_steps):
            step_layers(seg, s)
    e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    avg_launch = e0.elapsed_time(e1) * 1e-3 / (args.steps * n_layers)
    L_mid = L0 + args.warmup + (args.steps + 1) // 2
    per_launch = sum(decode_bytes(L0 + args.warmup + s + 1, n_heads, n_kv, d, 2)
                     for s in range(args.steps)) / args.steps
    achieved = per_launch / avg_launch / 1e9
    log(f"decode: wall {wall * 1e3:.2f} ms for {args.steps} steps, {value_gbs:.1f} GB/s whole-step; "
        f"kernel avg {avg_launch * 1e6:.2f} us/launch -> {achieved:.1f} GB/s")
    for b in qbs + obs + [kb, vbuf] + [x for row in kcs + vcs for x in row]:
        b.release()
    del kc, vc
    torch.cuda.empty_cache()
    return {
        "value": value_gbs, "ms_per_step": wall * 1e3 / args.steps, "avg_launch_s": avg_launch,
        "bytes_per_launch": per_launch, "achieved_gbs": achieved, "L_mid": L_mid,
    }


def bench_decode_cfg(ctx, torch, name, n_layers, n_heads, n_kv, d, kv, L, steps=8, warmup=2, seed=7, rope=False):
    """Decode of one BASELINE config shape: every step runs the fused
    append + attention launch for each of n_layers layers, the token at
    attended length L (the cache holds the L attended rows; a sliding
    window is the caller's offset shift of forward.zig:470-483, so only
    the window's rows need to exist).  Returns per-launch time from HIP
    events on the context stream and the algorithmic GB/s.  rope=True fuses
    the RoPE of q and k_cur at position L (interleaved form, base 10000) into
    every launch (attn_decode_rope_append)."""
    import numpy as np
    import vantablack_amd as vb
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[kv]
    vdt = {"f32": vb.F32, "f16": vb.F16, "bf16": vb.BF16}[kv]
    eb = {"f32": 4, "f16": 2, "bf16": 2}[kv]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rows = L + 1
    kc = torch.randn((n_layers, rows, n_kv, d), generator=g, device=dev).to(tdt)
    vc = torch.randn((n_layers, rows, n_kv, d), generator=g, device=dev).to(tdt)
    q = (torch.randn((n_layers, n_heads * d), generator=g, device=dev) / np.sqrt(d)).contiguous()
    kcur = torch.randn((n_layers, n_kv * d), generator=g, device=dev)
    vcur = torch.randn((n_layers, n_kv * d), generator=g, device=dev)
    out = torch.empty((n_layers, n_heads * d), device=dev)
    torch.cuda.synchronize()
    kb, vbuf = ctx.wrap_tensor(kc), ctx.wrap_tensor(vc)
    qbs = [ctx.wrap_tensor(q[l]) for l in range(n_layers)]
    obs = [ctx.wrap_tensor(out[l]) for l in range(n_layers)]
    kcs = [ctx.wrap_tensor(kcur[l]) for l in range(n_layers)]
    vcs = [ctx.wrap_tensor(vcur[l]) for l in range(n_layers)]
    layer_bytes = rows * n_kv * d * eb
    inv = 1.0 / np.sqrt(d)
    stream = torch.cuda.ExternalStream(ctx.stream)

    def one_step(seg):
        for l in range(n_layers):
            if rope:
                seg.attn_decode_rope_append(obs[l], qbs[l], kb, l * layer_bytes, vbuf, l * layer_bytes, kcs[l],
                                            vcs[l], n_heads, n_kv, d, L, inv, vdt, L, 10000.0, False)
            else:
                seg.attn_decode_append(obs[l], qbs[l], kb, l * layer_bytes, vbuf, l * layer_bytes, kcs[l], vcs[l],
                                       n_heads, n_kv, d, L, inv, vdt)

    with ctx.segment() as seg:
        for _ in range(warmup):
            one_step(seg)
    ctx.wait_idle()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    with ctx.segment() as seg:
        for _ in range(steps):
            one_step(seg)
    e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / (steps * n_layers)
    per = decode_bytes(L, n_heads, n_kv, d, eb)
    for b in qbs + obs + kcs + vcs + [kb, vbuf]:
        b.release()
    del kc, vc
    torch.cuda.empty_cache()
    log(f"decode {name}: h{n_heads}/{n_kv} d{d} {kv} L={L}: {t * 1e6:.2f} us/launch -> {per / t / 1e9:.1f} GB/s")
    return {"us_per_launch": round(t * 1e6, 3), "gbs": round(per / t / 1e9, 1),
            "pct_of_hbm_peak": round(100.0 * per / t / 1e9 / HBM_PEAK_GBS, 2), "bytes_per_launch": per,
            "shape": f"{n_layers} layers, {n_heads}q/{n_kv}kv heads, d{d}, {kv} KV, attended L={L}"}


def bench_decode_c2_run(ctx, torch, n_layers=32, L0=4096, steps=256):
    """BASELINE config 2 as written: Llama-2-7B shapes (32 layers, 32/32
    heads, d128, f16 KV) with the cache holding 4096 rows, then 256 decode
    steps, each appending the token's K/V row and attending every row so far
    in every layer (L = 4097 .. 4352).  One untimed pass of the 256 steps,
    then a timed pass of the same launches (each step rewrites its row with
    the same values).  Returns the run's time from HIP events on the context
    stream and its algorithmic GB/s."""
    import vantablack_amd as vb
    n_heads, n_kv, d = 32, 32, 128
    max_seq = L0 + steps
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(4352)
    kc = torch.empty((n_layers, max_seq, n_kv, d), dtype=torch.float16, device=dev)
    vc = torch.empty_like(kc)
    kc.normal_(generator=g)
    vc.normal_(generator=g)
    q = (torch.randn((n_layers, n_heads * d), generator=g, device=dev) / np.sqrt(d)).contiguous()
    kcur = torch.randn((n_layers, steps, n_kv * d), generator=g, device=dev)
    vcur = torch.randn((n_layers, steps, n_kv * d), generator=g, device=dev)
    out = torch.empty((n_layers, n_heads * d), device=dev)
    torch.cuda.synchronize()
    kb, vbuf = ctx.wrap_tensor(kc), ctx.wrap_tensor(vc)
    qbs = [ctx.wrap_tensor(q[l]) for l in range(n_layers)]
    obs = [ctx.wrap_tensor(out[l]) for l in range(n_layers)]
    kcs = [[ctx.wrap_tensor(kcur[l, s]) for s in range(steps)] for l in range(n_layers)]
    vcs = [[ctx.wrap_tensor(vcur[l, s]) for s in range(steps)] for l in range(n_layers)]
    layer_bytes = max_seq * n_kv * d * 2
    inv = 1.0 / np.sqrt(d)
    stream = torch.cuda.ExternalStream(ctx.stream)

    def run(seg):
        for s in range(steps):
            for l in range(n_layers):
                seg.attn_decode_append(obs[l], qbs[l], kb, l * layer_bytes, vbuf, l * layer_bytes, kcs[l][s],
                                       vcs[l][s], n_heads, n_kv, d, L0 + s + 1, inv, vb.F16)

    with ctx.segment() as seg:
        run(seg)
    ctx.wait_idle()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    with ctx.segment() as seg:
        run(seg)
    e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t = e0.elapsed_time(e1) * 1e-3
    alg = sum(n_layers * decode_bytes(L0 + s + 1, n_heads, n_kv, d, 2) for s in range(steps))
    for b in qbs + obs + [kb, vbuf] + [x for r in kcs + vcs for x in r]:
        b.release()
    del kc, vc, kcur, vcur
    torch.cuda.empty_cache()
    log(f"decode C2 run: {steps} steps x {n_layers} layers, L {L0 + 1}->{L0 + steps}: {t * 1e3:.2f} ms "
        f"({t / steps * 1e3:.4f} ms/step, wall {wall * 1e3:.1f} ms) -> {alg / t / 1e9:.1f} GB/s")
    return {"ms_total": round(t * 1e3, 3), "ms_per_step": round(t / steps * 1e3, 4),
            "us_per_launch": round(t / (steps * n_layers) * 1e6, 3), "wall_ms": round(wall * 1e3, 2),
            "gbs": round(alg / t / 1e9, 1), "pct_of_hbm_peak": round(100.0 * alg / t / 1e9 / HBM_PEAK_GBS, 2),
            "bytes_total": alg,
            "shape": f"{n_layers} layers, {n_heads}q/{n_kv}kv heads, d{d}, f16 KV, {steps} steps, "
                     f"L {L0 + 1}->{L0 + steps} (BASELINE config 2 as written)"}


def decode_kernel_name(n_heads, n_kv, d, kv):
    """The decode kernel one launch runs, by the launcher's rule
    (launch_decode / decode_heads_per_wg in vantablack_amd/csrc/vtb_hip.cpp):
    the MFMA form for f16/bf16 caches with GQA groups of 4 or more, the
    head-group form (two KV heads per workgroup) for uniform groups of 1-2
    when a row of two heads fits one load instruction, else the one-head
    scalar form; the group width rounds up to 1, 2, 4, 8 or 16."""
    g = -(-n_heads // n_kv)
    G = next(x for x in (1, 2, 4, 8, 16) if x >= g)
    eb = {"f32": 4, "f16": 2, "bf16": 2}[kv]
    hg = 2 if 64 // (d * eb // 16) >= 2 else 1
    head_group = not (eb == 2 and G >= 4) and G <= 2 and n_heads == n_kv * G and hg > 1 and n_kv % hg == 0
    return f"vtb_decode{'h' if head_group else ''}_{kv}_d{d}_g{G}"


def prefill_flops(L, n_heads, d):
    return 4 * n_heads * d * L * (L + 1) // 2


def prefill_kernel_name(torch, n_heads, n_q, d):
    """The attention kernel one attn_prefill call runs (launch_prefill_mfma in
    vantablack_amd/csrc/vtb_hip.cpp): one per head_dim, and the key-split
    form for d <= 128 when 128-query workgroups would fill at most half the
    CUs."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if d <= 128 and 2 * n_heads * ((n_q + 127) // 128) <= cus:
        return f"vtb_prefill_ks_d{d}"
    return f"vtb_prefill_d{d}"


def bench_prefill(ctx, torch, n_heads, n_kv, d, L, reps=20, warm_s=0.05):
    """Causal prefill of L tokens (pos0 = 0), bf16 Q/K/V resident in HBM.
    Returns the average launch time from HIP events on the context stream.

    The timed launches follow `warm_s` seconds of back-to-back launches of the
    same call: under this load the clock governor first lowers the clock (a
    long prompt's launches run up to 30% slower for the first ~10 ms) and then
    settles, so a short warmup times the transient rather than the sustained
    rate a serving loop sees.  The mean over `reps` launches is reported."""
    import numpy as np
    import vantablack_amd as vb
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(4321)
    q = torch.randn((L, n_heads * d), generator=g, device=dev)  # f32, as prefill.zig's s.q
    k = torch.randn((L, n_kv * d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((L, n_kv * d), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty((L, n_heads * d), device=dev)
    torch.cuda.synchronize()
    qb, kb, vbuf, ob = ctx.wrap_tensor(q), ctx.wrap_tensor(k), ctx.wrap_tensor(v), ctx.wrap_tensor(out)
    stream = torch.cuda.ExternalStream(ctx.stream)
    inv = 1.0 / np.sqrt(d)
    # Warm-up in growing chunks, each timed with events, until warm_s of
    # calls have run (at most 4000 calls).
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    warmup, spent, chunk = 0, 0.0, 1
    while spent < warm_s and warmup < 4000:
        with ctx.segment() as seg:
            e0.record(stream)
            for _ in range(chunk):
                seg.attn_prefill(ob, qb, kb, vbuf, 0, L, 0, vb.NO_WINDOW, n_heads, n_kv, d, inv, vb.BF16)
            e1.record(stream)
        ctx.wait_idle()
        torch.cuda.synchronize()
        spent += e0.elapsed_time(e1) * 1e-3
        warmup += chunk
        chunk = min(2 * chunk, 256)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    with ctx.segment() as seg:
        for e0, e1 in ev:
            e0.record(stream)
            seg.attn_prefill(ob, qb, kb, vbuf, 0, L, 0, vb.NO_WINDOW, n_heads, n_kv, d, inv, vb.BF16)
            e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    t = sum(e0.elapsed_time(e1) for e0, e1 in ev) / reps * 1e-3
    fl = prefill_flops(L, n_heads, d)
    for b in (qb, kb, vbuf, ob):
        b.release()
    log(f"prefill h{n_heads}/{n_kv} d{d} L{L}: {t * 1e6:.1f} us/launch -> {fl / t / 1e12:.1f} TFLOP/s "
        f"({warmup} warm launches, mean of {reps})")
    return {"avg_launch_s": t, "flops": fl, "tflops": fl / t / 1e12, "warm_launches": warmup, "reps": reps,
            "kernel": prefill_kernel_name(torch, n_heads, L, d)}


QUANT_BLOCK = {"q8_0": (34, 32), "q4_k": (144, 256), "q5_k": (176, 256), "q6_k": (210, 256)}
# Llama-2-7B projections per layer: q, k, v, o (4096 x 4096), gate, up
# (11008 x 4096), down (4096 x 11008) -- segMatmulQuant's shapes
# (forward.zig:400-417) on either side of the attention.
LLAMA2_7B_PROJ = [("qkvo", 4096, 4096, 4), ("gate_up", 11008, 4096, 2), ("down", 4096, 11008, 1)]


def bench_gemv(ctx, torch, kind, m, k, reps=20, pool_bytes=512 << 20):
    """One quantised GEMV (m x k, `kind` blocks) per launch, cycling over
    enough distinct weight copies (>= pool_bytes) that every launch streams
    its weights from HBM rather than the 256 MB MALL.  Random weight bytes
    (the arithmetic does not depend on them).  Returns us/launch and the
    algorithmic GB/s (weights + activations + outputs)."""
    import vantablack_amd as vb
    bb, be = QUANT_BLOCK[kind]
    row_bytes = k // be * bb
    wbytes = m * row_bytes
    copies = max(2, -(-pool_bytes // wbytes))
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    w = torch.randint(0, 256, (copies, wbytes), generator=g, dtype=torch.uint8, device=dev)
    x = torch.randn(k, generator=g, device=dev)
    out = torch.empty(m, device=dev)
    torch.cuda.synchronize()
    wb, xb, ob = ctx.wrap_tensor(w), ctx.wrap_tensor(x), ctx.wrap_tensor(out)
    stream = torch.cuda.ExternalStream(ctx.stream)
    with ctx.segment() as seg:
        for i in range(copies):
            seg.matmul_quant(kind, ob, wb, i * wbytes, xb, m, k)
    ctx.wait_idle()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    with ctx.segment() as seg:
        for i in range(reps):
            seg.matmul_quant(kind, ob, wb, (i % copies) * wbytes, xb, m, k)
    e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    for b in (wb, xb, ob):
        b.release()
    del w
    torch.cuda.empty_cache()
    nbytes = wbytes + 4 * k + 4 * m
    log(f"gemv {kind} {m}x{k}: {t * 1e6:.2f} us/launch -> {nbytes / t / 1e9:.1f} GB/s")
    return {"us_per_launch": round(t * 1e6, 3), "gbs": round(nbytes / t / 1e9, 1),
            "pct_of_hbm_peak": round(100.0 * nbytes / t / 1e9 / HBM_PEAK_GBS, 2), "bytes_per_launch": nbytes}


def bench_gemv_layer(ctx, torch, kind):
    """The seven Llama-2-7B projections of one layer in `kind`: per-shape
    figures and the layer total (time-weighted GB/s)."""
    res, tot_t, tot_b = {}, 0.0, 0
    for name, m, k, count in LLAMA2_7B_PROJ:
        r = bench_gemv(ctx, torch, kind, m, k)
        res[name] = r
        tot_t += count * r["us_per_launch"]
        tot_b += count * r["bytes_per_launch"]
    res["layer"] = {"us": round(tot_t, 2), "gbs": round(tot_b / (tot_t * 1e-6) / 1e9, 1),
                    "pct_of_hbm_peak": round(100.0 * tot_b / (tot_t * 1e-6) / 1e9 / HBM_PEAK_GBS, 2)}
    return res


# Llama-3-8B (C4's model) layer projections: (name, m, k, count per layer).
LLAMA3_8B_PROJ = (("q_o", 4096, 4096, 2), ("k_v", 1024, 4096, 2), ("gate_up", 14336, 4096, 2),
                  ("down", 4096, 14336, 1))


def bench_qgemm_layer(ctx, torch, kind, n_tokens, reps=3):
    """matmulBatched's seven projections of one Llama-3-8B layer for a prompt
    of n_tokens (the C4 prefill's other half), `kind` weights.  Reference
    flops are 2*m*k*B per projection; the MFMA work is twice that (the
    activations enter as two f16 pieces), reported against the dense
    f16/bf16 peak."""
    import vantablack_amd as vb
    bb, be = QUANT_BLOCK[kind]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    res, tot_t, tot_f = {}, 0.0, 0.0
    for name, m, k, count in LLAMA3_8B_PROJ:
        wbytes = m * (k // be * bb)
        w = torch.randint(0, 256, (wbytes,), generator=g, dtype=torch.uint8, device=dev)
        x = torch.randn(n_tokens, k, generator=g, device=dev)
        out = torch.empty(n_tokens, m, device=dev)
        torch.cuda.synchronize()
        wb, xb, ob = ctx.wrap_tensor(w), ctx.wrap_tensor(x), ctx.wrap_tensor(out)
        with ctx.segment() as seg:
            seg.matmul_batched(kind, ob, wb, 0, xb, m, k, n_tokens)
        ctx.wait_idle()
        stream = torch.cuda.ExternalStream(ctx.stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with ctx.segment() as seg:
            for _ in range(reps):
                seg.matmul_batched(kind, ob, wb, 0, xb, m, k, n_tokens)
        e1.record(stream)
        ctx.wait_idle()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        for b in (wb, xb, ob):
            b.release()
        del w, x, out
        torch.cuda.empty_cache()
        fl = 2.0 * m * k * n_tokens
        log(f"qgemm {kind} {m}x{k} B={n_tokens}: {t * 1e6:.1f} us -> {fl / t / 1e12:.1f} TFLOP/s "
            f"(MFMA {2 * fl / t / 1e12:.1f})")
        res[name] = {"us": round(t * 1e6, 1), "tflops": round(fl / t / 1e12, 1),
                     "mfma_tflops": round(2 * fl / t / 1e12, 1),
                     "pct_of_bf16_peak": round(100.0 * 2 * fl / t / 1e12 / BF16_PEAK_TFLOPS, 2)}
        tot_t += count * t
        tot_f += count * fl
    res["layer"] = {"us": round(tot_t * 1e6, 1), "tflops": round(tot_f / tot_t / 1e12, 1),
                    "mfma_tflops": round(2 * tot_f / tot_t / 1e12, 1),
                    "pct_of_bf16_peak": round(100.0 * 2 * tot_f / tot_t / 1e12 / BF16_PEAK_TFLOPS, 2)}
    return res


def bench_full_decode(ctx, torch, ctx_rows=8192, steps=6, warmup=2):
    """Whole-token decode of a Llama-2-7B-shaped model on the GPU, as
    vantablack's gpuLayerStep x 32 + gpuFinalStep encode it
    (forward.zig:419-520), through vantablack_amd.layer.gpu_token_step: per
    layer (residual add +) rmsnorm, the Q/K/V GEMVs (one grouped launch), RoPE +
    K/V append + attention (one launch), O GEMV, residual add + rmsnorm (one
    launch), gate/up GEMVs + SwiGLU (one gated launch), down GEMV; then the last
    residual add + output norm and the 32000-row logits GEMV.  Q4_K projections (random blocks with small
    f16 scales), f32 norm weights, f16 KV cache holding ctx_rows rows.
    Returns ms per token from HIP events on the context stream."""
    import numpy as np
    from vantablack_amd import layer as ly
    dim, nh, nkv, hd, ffn, n_layers, vocab = 4096, 32, 32, 128, 11008, 32, 32000
    c = ly.LayerConfig(dim=dim, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn_dim=ffn,
                       max_seq=ctx_rows + warmup + steps, kv_dtype=1)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    qb, qe = QUANT_BLOCK["q4_k"]
    scale = torch.tensor([0.01], dtype=torch.float16, device=dev).view(torch.uint8)

    def q4k(m, k):
        w = torch.randint(0, 256, (m * k // qe, qb), generator=g, dtype=torch.uint8, device=dev)
        w[:, 0:2] = scale
        w[:, 2:4] = scale
        return w.reshape(-1)

    shapes = [("q", dim, dim), ("k", nkv * hd, dim), ("v", nkv * hd, dim), ("o", dim, dim),
              ("gate", ffn, dim), ("up", ffn, dim), ("down", dim, ffn)]
    tensors, offs, pos = [], [], 0

    def put(t):
        nonlocal pos
        off = pos
        tensors.append(t)
        pos += t.numel()
        return off

    norm = torch.ones(dim, dtype=torch.float32, device=dev).view(torch.uint8)
    for _ in range(n_layers):
        an = put(norm)
        o = {n: put(q4k(m, k)) for n, m, k in shapes}
        fn = put(norm)
        offs.append(ly.LayerOffsets(an, o["q"], o["k"], o["v"], o["o"], fn, o["gate"], o["up"], o["down"],
                                    *(["q4_k"] * 7)))
    out_norm_off = put(norm)
    out_off = put(q4k(vocab, dim))
    blob = torch.cat(tensors)
    del tensors
    weight_bytes = blob.numel()
    kc = torch.empty((n_layers, c.max_seq, nkv, hd), dtype=torch.float16, device=dev)
    vc = torch.empty_like(kc)
    kc.normal_(generator=g)
    vc.normal_(generator=g)
    torch.cuda.synchronize()
    wb, kb, vb_ = ctx.wrap_tensor(blob), ctx.wrap_tensor(kc), ctx.wrap_tensor(vc)
    s = ly.LayerScratch(ctx, c, vocab)
    ctx.upload(s.x, np.zeros(dim, np.float32) + np.float32(0.1))

    def token(seg, p):
        ly.gpu_token_step(seg, s, wb, offs, kb, vb_, c, p, out_norm_off, out_off, "q4_k", vocab)

    with ctx.segment() as seg:
        for t in range(warmup):
            token(seg, ctx_rows + t)
    ctx.wait_idle()
    stream = torch.cuda.ExternalStream(ctx.stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    with ctx.segment() as seg:
        for t in range(steps):
            token(seg, ctx_rows + warmup + t)
    e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    t_tok = e0.elapsed_time(e1) * 1e-3 / steps
    L_mid = ctx_rows + warmup + steps // 2
    kv_bytes = n_layers * decode_bytes(L_mid, nh, nkv, hd, 2)
    s.release()
    for b in (wb, kb, vb_):
        b.release()
    del blob, kc, vc
    torch.cuda.empty_cache()
    log(f"full decode: {t_tok * 1e3:.3f} ms/token ({1 / t_tok:.1f} tok/s), "
        f"{(weight_bytes + kv_bytes) / t_tok / 1e9:.0f} GB/s over weights + KV")
    return {"ms_per_token": round(t_tok * 1e3, 3), "tok_per_s": round(1 / t_tok, 1),
            "launches_per_token": n_layers * 7 + 2, "weight_bytes": weight_bytes,
            "kv_bytes_per_token": kv_bytes,
            "hbm_gbs": round((weight_bytes + kv_bytes) / t_tok / 1e9, 1),
            "pct_of_hbm_peak": round(100.0 * (weight_bytes + kv_bytes) / t_tok / 1e9 / HBM_PEAK_GBS, 1)}


def bench_full_prefill(ctx, torch, B=8192, reps=2):
    """A whole-prompt prefill of B tokens through a Llama-3-8B-shaped model
    on the GPU (prefillLayer x 32, prefill.zig:151-231, through
    vantablack_amd.layer.gpu_prefill_layer): per layer per-token rmsnorm,
    Q/K/V projections on MFMA, batched RoPE, the K/V rows into a bf16 cache,
    MFMA causal attention, O projection + residual, rmsnorm, gate/up, SwiGLU,
    down + residual; then, as prefillCpu ends (prefill.zig:143-146), the final
    rmsnorm and the LM head (128256 x 4096, Q6_K) on the last token's row.
    Q4_K projections (random blocks, small f16 scales), a distinct weight set
    per layer (3.9 GB).  Returns ms per prompt from HIP events on the context
    stream."""
    import vantablack_amd as vb
    from vantablack_amd import layer as ly
    dim, nh, nkv, hd, ffn, n_layers = 4096, 32, 8, 128, 14336, 32
    c = ly.LayerConfig(dim=dim, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn_dim=ffn, max_seq=B,
                       rope_base=500000.0, kv_dtype=2)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(78)
    qb, qe = QUANT_BLOCK["q4_k"]
    scale = torch.tensor([0.002], dtype=torch.float16, device=dev).view(torch.uint8)
    tensors, offs, pos = [], [], 0

    def put(t):
        nonlocal pos
        off = pos
        tensors.append(t)
        pos += t.numel()
        return off

    def q4k(m, k):
        w = torch.randint(0, 256, (m * k // qe, qb), generator=g, dtype=torch.uint8, device=dev)
        w[:, 0:2] = scale
        w[:, 2:4] = scale
        return w.reshape(-1)

    norm = torch.ones(dim, dtype=torch.float32, device=dev).view(torch.uint8)
    shapes = [("q", dim, dim), ("k", nkv * hd, dim), ("v", nkv * hd, dim), ("o", dim, dim),
              ("gate", ffn, dim), ("up", ffn, dim), ("down", dim, ffn)]
    for _ in range(n_layers):
        an = put(norm)
        o = {n: put(q4k(m, k)) for n, m, k in shapes}
        fn = put(norm)
        offs.append(ly.LayerOffsets(an, o["q"], o["k"], o["v"], o["o"], fn, o["gate"], o["up"], o["down"],
                                    *(["q4_k"] * 7)))
    vocab = 128256
    out_norm = put(norm)
    qb6, qe6 = QUANT_BLOCK["q6_k"]
    w6 = torch.randint(0, 256, (vocab * dim // qe6, qb6), generator=g, dtype=torch.uint8, device=dev)
    w6[:, qb6 - 2:] = scale  # Q6_K's f16 d sits at the end of the block
    out_w = put(w6.reshape(-1))
    blob = torch.cat(tensors)
    del tensors, w6
    kc = torch.zeros((n_layers, B, nkv, hd), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    x0 = (torch.randn((B, dim), generator=g, device=dev) * 0.1).contiguous()
    torch.cuda.synchronize()
    wb, kb, vb_ = ctx.wrap_tensor(blob), ctx.wrap_tensor(kc), ctx.wrap_tensor(vc)
    xin = ctx.wrap_tensor(x0)
    s = ly.PrefillScratch(ctx, c, B)
    last = ctx.wrap(s.x.ptr + (B - 1) * dim * 4, dim * 4, keepalive=s.x)
    logits = ctx.alloc(vocab * 4)

    def prompt(seg):
        seg.copy(s.x, 0, xin, 0, B * dim)
        for l in range(n_layers):
            ly.gpu_prefill_layer(seg, s, wb, offs[l], kb, vb_, c, l, 0)
        # Final RMSNorm + LM head on the last position only (prefill.zig:143-146).
        seg.rmsnorm(last, last, wb, out_norm, dim, c.rms_eps)
        seg.matmul_quant("q6_k", logits, wb, out_w, last, vocab, dim)

    with ctx.segment() as seg:
        prompt(seg)
    ctx.wait_idle()
    stream = torch.cuda.ExternalStream(ctx.stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    with ctx.segment() as seg:
        for _ in range(reps):
            prompt(seg)
    e1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    proj_flops = 2.0 * B * n_layers * sum(m * k for _, m, k in shapes) + 2.0 * vocab * dim
    attn_flops = n_layers * prefill_flops(B, nh, hd)
    # The last layer's attention on the model's own q / K / V (s.q and the
    # cache rows stay as the prompt left them): its time per call, and the
    # share of (head, query block) work items that take two f16 pieces.
    row_bytes = nkv * hd * 2
    inv = 1.0 / math.sqrt(hd)
    lo = (n_layers - 1) * B * row_bytes
    ea = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(3)]
    with ctx.segment() as seg:
        for a0, a1 in ea:
            a0.record(stream)
            seg.attn_prefill(s.attn_out, s.q, kb, vb_, lo, B, 0, vb.NO_WINDOW, nh, nkv, hd, inv, vb.BF16)
            a1.record(stream)
    ctx.wait_idle()
    torch.cuda.synchronize()
    t_attn = sum(a0.elapsed_time(a1) for a0, a1 in ea) / len(ea) * 1e-3
    qm = torch.from_numpy(ctx.download(s.q, np.float32, B * nh * hd)).to(dev).view(B, nh, hd)
    paths = prefill_paths(torch, qm, kc[n_layers - 1].float(), vc[n_layers - 1].float(), inv)
    del qm
    s.release()
    for b in (wb, kb, vb_, xin, last, logits):
        b.release()
    del blob, kc, vc, x0
    torch.cuda.empty_cache()
    log(f"full prefill: {t * 1e3:.1f} ms per {B}-token prompt ({B / t:.0f} tok/s), "
        f"{(proj_flops + attn_flops) / t / 1e12:.0f} TFLOP/s (reference flops)")
    log(f"full prefill: last layer's attention {t_attn * 1e6:.1f} us per call; work items with two-piece "
        f"q {paths['xq_frac']:.3f}, P {paths['xp_frac']:.3f} (score bound median {paths['bound_median']:.1f}, "
        f"max {paths['bound_max']:.1f}; value crest max {paths['crest_max']:.2f})")
    return {"ms_per_prompt": round(t * 1e3, 2), "tok_per_s": round(B / t, 1),
            "ms_per_layer": round(t * 1e3 / n_layers, 3),
            "tflops_reference": round((proj_flops + attn_flops) / t / 1e12, 1),
            "attn_last_layer_us": round(t_attn * 1e6, 2),
            "attn_last_layer_tflops": round(prefill_flops(B, nh, hd) / t_attn / 1e12, 1),
            "attn_precision_paths": paths}


def prefill_paths(torch, q, k, v, inv_sqrt_hd, bm=128, tile=64):
    """The prefill kernel's precision choice (prefill_entry) for every
    (head, causal query block) of a pos0 = 0 prompt, from q [B][n_heads][D]
    and the cache rows k, v [B][n_kv][D] (f32): two-piece q where
    max |q| * max |k_t| * scale_log2 over the block's key tiles exceeds 32,
    two-piece P where the values' crest factor over those tiles exceeds 8."""
    B, nh, D = q.shape
    nkv = k.shape[1]
    nblk, nt = -(-B // bm), -(-B // tile)
    pad = nt * tile - B
    qn = q.norm(dim=2)                                                     # [B][nh]
    qn = torch.nn.functional.pad(qn, (0, 0, 0, nblk * bm - B)).view(nblk, bm, nh).amax(1)
    kn2 = torch.nn.functional.pad((k * k).sum(2), (0, 0, 0, pad)).view(nt, tile, nkv).amax(1)
    va = torch.nn.functional.pad(v.abs().amax(2), (0, 0, 0, pad)).view(nt, tile, nkv).amax(1)
    vs = torch.nn.functional.pad((v.double() ** 2).sum(2), (0, 0, 0, pad)).view(nt, tile, nkv).sum(1)
    kend = torch.clamp(torch.arange(1, nblk + 1, device=q.device) * bm, max=B)
    last = (kend + tile - 1) // tile - 1                                   # last tile of each block
    kmax = torch.cummax(kn2, 0).values[last]                               # [nblk][nkv]
    vmax = torch.cummax(va, 0).values[last]
    vss = torch.cumsum(vs, 0)[last]
    kvh = torch.arange(nh, device=q.device) * nkv // nh
    bound = qn * kmax[:, kvh].sqrt() * (inv_sqrt_hd * 1.4426950408889634)
    crest2 = (vmax.double() ** 2) * (kend[:, None].double() * D) / vss
    xq = bound > 32.0
    xp = (crest2 > 64.0)[:, kvh]
    return {"items": nblk * nh, "xq_frac": round(xq.float().mean().item(), 4),
            "xp_frac": round(xp.float().mean().item(), 4),
            "bound_median": round(bound.median().item(), 2), "bound_max": round(bound.max().item(), 2),
            "crest_max": round(crest2.max().sqrt().item(), 2)}


def _timed(fn, budget_s):
    """Seconds per call of fn, repeated until budget_s is spent (at least once)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            return el / n, n


def _cpu_workers():
    # Workers: the CPUs this process may run on, capped at the GPU box's CPU
    # share (16); pool.zig's own default is (ncpu + 1) / 2 workers
    # (pool.zig:53), timed as well.
    affinity = len(os.sched_getaffinity(0))
    workers = min(affinity, int(os.environ.get("VTB_CPU_WORKERS", "16")))
    return affinity, (("faithful_1t", 1), ("pool", workers), ("pool_default", (workers + 1) // 2))


def _oracle_cache(orc, rng, n_kv, d, rows, kv):
    """One-layer oracle cache of `rows` rows holding exactly-upcast values of
    the KV dtype (f32 storage, as vantablack's cache holds them)."""
    cache = orc.OracleKvCache(1, n_kv, d, rows)
    for arr in (cache.k, cache.v):
        x = rng.standard_normal(arr.size, dtype=np.float32)
        arr[:] = x if kv == "f32" else orc.to_dtype(x, kv)[1]
    return cache


def cpu_baseline(seconds_budget=6.0):
    """Time the CPU oracle on a bounded sample of the headline decode
    workload: one C2 layer at L=8192 (f32 values of the f16 cache, as
    vantablack's f32 cache would hold them), each line repeated for about
    seconds_budget / 3."""
    from oracle import oracle as orc
    n_heads, n_kv, d, L = 32, 32, 128, 8192
    rng = np.random.default_rng(0)
    cache = orc.OracleKvCache(1, n_kv, d, L)
    cache.k[:] = rng.standard_normal(cache.k.size, dtype=np.float32).astype(np.float16).astype(np.float32)
    cache.v[:] = rng.standard_normal(cache.v.size, dtype=np.float32).astype(np.float16).astype(np.float32)
    cache.pos = L - 1
    c = orc.config(n_heads, n_kv, d, L)
    q = (rng.standard_normal(n_heads * d, dtype=np.float32) / np.float32(np.sqrt(d)))
    # The oracle reads f32 K/V (vantablack's cache dtype), so its rate is
    # counted in f32 bytes; the f16-equivalent rate is reported beside it.
    per = decode_bytes(L, n_heads, n_kv, d, 4)
    per16 = decode_bytes(L, n_heads, n_kv, d, 2)
    res = {}
    affinity, lines = _cpu_workers()
    for label, nw in lines:
        pool = orc.Pool(nw)
        try:
            t, n = _timed(lambda: pool.attention(q, cache, c, 0, L - 1), seconds_budget / 3)
        finally:
            pool.close()
        res[label] = {"gbs": per / t / 1e9, "gbs_f16_equiv": per16 / t / 1e9,
                      "ms_per_layer": t * 1e3, "layers": n, "workers": nw}
        log(f"cpu {label}: {res[label]['ms_per_layer']:.2f} ms per layer-step ({n} runs)")
    res["affinity_cpus"] = affinity
    res["cpu_model"] = cpu_model()
    return res


# The BASELINE configs as the CPU oracle runs them (forward.zig:187-228 per
# decode layer, prefill.zig:237-287 per prompt row).  Decode: (name, n_heads,
# n_kv, d, KV dtype, layers per step, [(cur_pos, window)] sampled layer
# calls, steps, note).  Prefill: (name, n_heads, n_kv, d, KV dtype, prompt
# tokens, every k-th row sampled).
CPU_DECODE_CFGS = (
    ("C1", 32, 4, 64, "f32", 1, [(511, 0)], 1, "one layer at L=512, the whole config"),
    ("C2_256", 32, 32, 128, "f16", 32, [(4096, 0), (4351, 0)], 256,
     "one layer at the first (L=4097) and last (L=4352) step; a step is 32 layers, the run 256 steps, "
     "extrapolated linearly in L from the two"),
    ("C3", 32, 8, 128, "bf16", 32, [(16383, 4096)], 1,
     "one layer at pos 16383 with window 4096 (L=4096); a step is 32 layers"),
    ("C5_decode", 8, 1, 256, "bf16", 26, [(32767, 0)], 1, "one layer at L=32768; a step is 26 layers"),
)
CPU_PREFILL_CFGS = (
    ("C4_L512", 32, 8, 128, "bf16", 512, 1),
    ("C4_L2048", 32, 8, 128, "bf16", 2048, 8),
    ("C4_L8192", 32, 8, 128, "bf16", 8192, 64),
    ("C5_prefill", 8, 1, 256, "bf16", 4096, 32),
)


def cpu_baseline_configs(seconds_per_line=1.5):
    """The CPU oracle on every BASELINE config, three lines each: faithful
    (one thread, as vantablack runs attention), and split over heads on a
    pool.zig-style pool at the box's CPU share and at pool.zig's default
    worker count.  Each line times a bounded sample of the config (named in
    its `sample`) for about seconds_per_line and extrapolates to the whole
    config's work: decode steps from per-layer calls, a prefill from every
    k-th prompt row (row b attends b + 1 keys, so the sample's share of the
    L(L+1)/2 causal pairs scales it up exactly)."""
    from oracle import oracle as orc
    rng = np.random.default_rng(11)
    _, lines = _cpu_workers()
    out = {}
    for name, nh, nkv, d, kv, layers, calls, steps, note in CPU_DECODE_CFGS:
        rows = max(p for p, _ in calls) + 1
        cache = _oracle_cache(orc, rng, nkv, d, rows, kv)
        q = rng.standard_normal(nh * d, dtype=np.float32) / np.float32(np.sqrt(d))
        scores = np.zeros(nh * rows, np.float32)
        o = np.zeros(nh * d, np.float32)
        cfgs = [(pos, orc.config(nh, nkv, d, rows, w if w else orc.NO_WINDOW)) for pos, w in calls]
        attended = [pos + 1 - orc.window_start(pos, w if w else orc.NO_WINDOW) for pos, w in calls]
        step_bytes = layers * sum(decode_bytes(a, nh, nkv, d, 4) for a in attended) / len(attended)
        e = {"workload": f"{nh}q/{nkv}kv heads, d{d}, {kv} values as f32, {layers} layers per step, "
                         f"{steps} step(s)", "sample": note}
        for label, nw in lines:
            pool = orc.Pool(nw)
            try:
                t, n = _timed(lambda: [pool.attention(q, cache, cf, 0, pos, scores=scores, out=o)
                                       for pos, cf in cfgs], seconds_per_line)
            finally:
                pool.close()
            t_layer = t / len(cfgs)
            e[label] = {"cores": nw, "ms_per_layer": round(t_layer * 1e3, 4),
                        "ms_per_step": round(t_layer * layers * 1e3, 3),
                        "ms_total": round(t_layer * layers * steps * 1e3, 3),
                        "gbs_f32": round(step_bytes / (t_layer * layers) / 1e9, 3), "runs": n}
            log(f"cpu {name} {label}: {t_layer * 1e3:.3f} ms per layer ({n} runs)")
        out[name] = e
        del cache
    for name, nh, nkv, d, kv, B, k in CPU_PREFILL_CFGS:
        cache = _oracle_cache(orc, rng, nkv, d, B, kv)
        c = orc.config(nh, nkv, d, B)
        sample = list(range(k - 1, B, k))
        qs = rng.standard_normal((len(sample), nh * d), dtype=np.float32)
        scores = np.zeros(nh * B, np.float32)
        o = np.zeros(nh * d, np.float32)
        work_all = B * (B + 1) // 2
        work_sample = sum(b + 1 for b in sample)
        flops = prefill_flops(B, nh, d)
        e = {"workload": f"{nh}q/{nkv}kv heads, d{d}, {kv} values as f32, {B}-token causal prompt (pos0 0)",
             "sample": (f"every {k}-th prompt row ({len(sample)} rows, {work_sample} of {work_all} causal "
                        f"pairs), scaled by {work_all / work_sample:.3f}" if k > 1 else "every prompt row")}
        for label, nw in lines:
            pool = orc.Pool(nw)
            try:
                t, n = _timed(lambda: [pool.attention(qs[i], cache, c, 0, b, scores=scores, out=o)
                                       for i, b in enumerate(sample)], seconds_per_line)
            finally:
                pool.close()
            t_all = t * work_all / work_sample
            e[label] = {"cores": nw, "ms_per_call": round(t_all * 1e3, 2),
                        "tflops": round(flops / t_all / 1e12, 5), "runs": n}
            log(f"cpu {name} {label}: {t_all * 1e3:.1f} ms per call (extrapolated; {n} sample runs)")
        out[name] = e
        del cache
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# Kernel shapes of the counter-run workload: (label, n_heads, n_kv, d, kv dtype,
# attended rows, layers).  C3's window of 4096 is the attended range.
PMC_DECODE = [("C2", 32, 32, 128, "f16", 8193, 4), ("C3", 32, 8, 128, "bf16", 4096, 4),
              ("C5", 8, 1, 256, "bf16", 32768, 4)]
PMC_PREFILL = [("C4", 32, 8, 128, 8192), ("C5", 8, 1, 256, 4096)]


def pmc_workload():
    """The launches of every measured kernel shape, for rocprofv3 --pmc runs:
    the calibration copy (vtb_copy_f32); the fused append + decode launch of
    C2 (vtb_decodeh_f16_d128_g1), C3 (vtb_decode_bf16_d128_g4) and C5
    (vtb_decode_bf16_d256_g8, with its merge launch vtb_decode_merge), each
    over PMC_DECODE's layer count of distinct cache layers; and the C4 (8192 tokens) and C5 (4096 tokens) causal
    prefill calls: the pre-pass (vtb_kvt_*: tile statistics and the f16
    operands) and the attention kernels (vtb_prefill_d128,
    vtb_prefill_d256)."""
    import numpy as np
    import torch
    import vantablack_amd as vb
    ctx = vb.Context()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(99)
    src = torch.randn(PMC_COPY_FLOATS, generator=g, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    with ctx.segment() as seg:
        seg.copy(ctx.wrap_tensor(dst), 0, ctx.wrap_tensor(src), 0, PMC_COPY_FLOATS)
    ctx.wait_idle()
    log("pmc: copy done")
    del src, dst
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}
    for label, n_heads, n_kv, d, kv, L, n_layers in PMC_DECODE:
        kc = torch.randn((n_layers, L, n_kv, d), generator=g, device=dev).to(tdt[kv])
        vc = torch.randn((n_layers, L, n_kv, d), generator=g, device=dev).to(tdt[kv])
        q = torch.randn((n_layers, n_heads * d), generator=g, device=dev) / np.sqrt(d)
        kcur, vcur = torch.randn(n_kv * d, device=dev), torch.randn(n_kv * d, device=dev)
        out = torch.empty(n_heads * d, device=dev)
        torch.cuda.synchronize()
        kb, vbuf = ctx.wrap_tensor(kc), ctx.wrap_tensor(vc)
        lb = L * n_kv * d * 2
        with ctx.segment() as seg:
            for l in range(n_layers):
                seg.attn_decode_append(ctx.wrap_tensor(out), ctx.wrap_tensor(q[l]), kb, l * lb, vbuf, l * lb,
                                       ctx.wrap_tensor(kcur), ctx.wrap_tensor(vcur), n_heads, n_kv, d, L,
                                       1.0 / np.sqrt(d), vb.hip.DTYPES[kv])
        ctx.wait_idle()
        log(f"pmc: decode {label} done")
        del kc, vc
    for label, n_heads, n_kv, d, L in PMC_PREFILL:
        qp = torch.randn((L, n_heads * d), generator=g, device=dev)
        kp = torch.randn((L, n_kv * d), generator=g, device=dev).to(torch.bfloat16)
        vp = torch.randn((L, n_kv * d), generator=g, device=dev).to(torch.bfloat16)
        op = torch.empty((L, n_heads * d), device=dev)
        torch.cuda.synchronize()
        with ctx.segment() as seg:
            seg.attn_prefill(ctx.wrap_tensor(op), ctx.wrap_tensor(qp), ctx.wrap_tensor(kp), ctx.wrap_tensor(vp), 0,
                             L, 0, vb.NO_WINDOW, n_heads, n_kv, d, 1.0 / np.sqrt(d), vb.BF16)
        ctx.wait_idle()
        log(f"pmc: prefill {label} done")
        del qp, kp, vp, op
    ctx.close()


def pmc_read(dirs):
    """Per-dispatch average of every counter of the vtb_* kernels in the
    rocprofv3 --pmc csv outputs under dirs: {kernel: {counter: value}}."""
    import csv
    import glob
    vals = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Kernel_Name"].startswith("vtb_"):
                    name = r["Kernel_Name"].split("(")[0]
                    vals.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in vals.items()}


def trace_summary(dirs):
    """Markdown table of the vtb_* dispatches in rocprofv3 kernel-trace csv
    outputs under dirs, one row per (bench section, kernel, grid, block) in
    dispatch order.  Sections come from the ROCTx ranges bench.py opens when
    VTB_BENCH_ROCTX=1 (`--marker-trace` output); a dispatch belongs to the
    range its start lies in."""
    import csv
    import glob

    def files(pat):
        return [f for d in dirs for f in glob.glob(os.path.join(d, "**", pat), recursive=True)]

    def col(r, *names):
        for n in names:
            if n in r and r[n] != "":
                return r[n]
        return None

    ranges = []
    for f in files("*marker_api_trace.csv"):
        for r in csv.DictReader(open(f)):
            name = col(r, "Function", "Message", "Name")
            t0, t1 = col(r, "Start_Timestamp"), col(r, "End_Timestamp")
            if name and t0 and t1 and int(t1) > int(t0):
                ranges.append((int(t0), int(t1), name))
    ranges.sort()
    rows = {}
    for f in files("*kernel_trace.csv"):
        for r in csv.DictReader(open(f)):
            kname = r["Kernel_Name"].split("(")[0]
            if not kname.startswith("vtb_"):
                continue
            t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            sec = ""
            for a, b, n in ranges:  # innermost (latest-starting) range holding t0
                if a <= t0 < b:
                    sec = n
            grid = "x".join(col(r, f"Grid_Size_{c}") or "1" for c in "XYZ")
            block = col(r, "Workgroup_Size_X", "Workgroup_Size") or "?"
            key = (sec, kname, grid, block)
            e = rows.setdefault(key, {"first": t0, "us": [], "vgpr": col(r, "Arch_VGPR_Count", "VGPR_Count"),
                                      "agpr": col(r, "Accum_VGPR_Count"), "lds": col(r, "LDS_Block_Size", "Lds_Size"),
                                      "scratch": col(r, "Scratch_Size", "Private_Segment_Size")})
            e["first"] = min(e["first"], t0)
            e["us"].append((t1 - t0) / 1e3)
    print("| section | kernel | launches | avg us | min us | max us | grid (threads) | block | arch VGPR | AGPR | "
          "LDS B | scratch B |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|")
    for (sec, kname, grid, block), e in sorted(rows.items(), key=lambda kv: kv[1]["first"]):
        us = e["us"]
        print(f"| {sec or '-'} | {kname} | {len(us)} | {sum(us) / len(us):.2f} | {min(us):.2f} | {max(us):.2f} | "
              f"{grid} | {block} | {e['vgpr']} | {e['agpr']} | {e['lds']} | {e['scratch']} |")


def pmc_summary(fetch_dir, write_dir):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the vtb_* kernels from
    two rocprofv3 --pmc csv outputs, scaled by the copy calibration, written
    to profiles/traffic.json and printed as a markdown table."""
    fetch = {k: v["FETCH_SIZE"] for k, v in pmc_read([fetch_dir]).items() if "FETCH_SIZE" in v}
    write = {k: v["WRITE_SIZE"] for k, v in pmc_read([write_dir]).items() if "WRITE_SIZE" in v}
    copy_kib = PMC_COPY_FLOATS * 4 / 1024
    f_fetch = copy_kib / fetch["vtb_copy_f32"]
    f_write = copy_kib / write["vtb_copy_f32"]
    kernels = {}
    for name in sorted(set(fetch) & set(write)):
        kernels[name] = {"fetch_kib": round(fetch[name], 1), "write_kib": round(write[name], 1),
                         "traffic_bytes": int(round((fetch[name] * f_fetch + write[name] * f_write) * 1024))}
    out = {"calibration": {"kernel": "vtb_copy_f32", "bytes_each_way": PMC_COPY_FLOATS * 4,
                           "fetch_factor": round(f_fetch, 4), "write_factor": round(f_write, 4)},
           "workload": "bench.py --pmc-workload: decode " +
                       ", ".join(f"{c[0]} ({c[1]}q/{c[2]}kv d{c[3]} {c[4]} L={c[5]})" for c in PMC_DECODE) +
                       " with the KV append fused; prefill " +
                       ", ".join(f"{c[0]} ({c[1]}q/{c[2]}kv d{c[3]} bf16, {c[4]} tokens)" for c in PMC_PREFILL),
           "kernels": kernels}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(f"calibration (vtb_copy_f32, {PMC_COPY_FLOATS * 4 >> 20} MiB each way): "
          f"FETCH x{f_fetch:.4f}, WRITE x{f_write:.4f}\n")
    print("| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | calibrated traffic MB |")
    print("|---|---|---|---|")
    for k, v in kernels.items():
        print(f"| {k} | {v['fetch_kib']:.1f} | {v['write_kib']:.1f} | {v['traffic_bytes'] / 1e6:.2f} |")


COUNTERS_FILE = os.path.join(ROOT, "profiles", "counters.json")


def pmc_sq_summary(dirs):
    """Shader (SQ) and GRBM counters of the vtb_* kernels from rocprofv3
    --pmc csv runs over `bench.py --pmc-workload`, with each dispatch's
    duration from the same runs, written to profiles/counters.json and
    printed as a markdown table.

    Normalisation (gfx950, from the runs' agent_info: 8 XCDs, 256 CUs, 4 SIMDs
    per CU, 2.4 GHz peak engine clock):
      GRBM_GUI_ACTIVE is summed over the XCDs, so the dispatch's cycles on
        one XCD are GRBM_GUI_ACTIVE / 8 (that window also holds about 20k
        cycles of dispatch set-up: clock_ghz is only meaningful for long
        kernels);
      SQ_VALU_MFMA_BUSY_CYCLES is summed over every SIMD (a 32x32x16 f16 MFMA
        counts 32), so mfma_busy = busy / (1024 SIMDs x cycles), with cycles
        from GRBM (at the clock the kernel ran at) or from duration x 2.4 GHz
        (against the peak clock, i.e. the dense-peak fraction);
      SQ_INSTS_VALU_MFMA_MOPS_* count units of 512 flops;
      SQ_ACTIVE_INST_VALU counts quad-cycles (4 clocks) per wave, summed, so
        valu_busy = 4 x that / (1024 SIMDs x duration x 2.4 GHz)."""
    import csv
    import glob
    agent = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*agent_info.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Agent_Type"] == "GPU":
                    agent = {"xcc": int(r["Num_Xcc"]), "cus": int(r["Cu_Count"]),
                             "simds": int(r["Cu_Count"]) * int(r["Simd_Per_Cu"]),
                             "clk_mhz": int(r["Max_Engine_Clk_Fcompute"])}
    vals, durs = {}, {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            seen = set()
            for r in csv.DictReader(open(f)):
                if not r["Kernel_Name"].startswith("vtb_"):
                    continue
                name = r["Kernel_Name"].split("(")[0]
                vals.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
                key = (f, r["Dispatch_Id"])
                if key not in seen:
                    seen.add(key)
                    durs.setdefault(name, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9)
    clk = agent["clk_mhz"] * 1e6
    kernels = {}
    for name in sorted(vals):
        c = {k: sum(v) / len(v) for k, v in vals[name].items()}
        dur = sum(durs[name]) / len(durs[name])
        e = {"dispatches": len(durs[name]), "dur_us": round(dur * 1e6, 2),
             "counters": {k: int(round(v)) for k, v in sorted(c.items())}}
        grbm_cyc = c.get("GRBM_GUI_ACTIVE", 0) / agent["xcc"]
        if grbm_cyc:
            e["clock_ghz"] = round(grbm_cyc / dur / 1e9, 3)
        mops = c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0) + c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0)
        if mops:
            e["mfma_flops"] = int(mops * 512)
            busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0)
            if grbm_cyc:
                e["mfma_busy_at_clock"] = round(busy / (agent["simds"] * grbm_cyc), 4)
            e["mfma_busy_at_peak_clock"] = round(busy / (agent["simds"] * dur * clk), 4)
        if c.get("SQ_ACTIVE_INST_VALU"):
            e["valu_busy_at_peak_clock"] = round(4 * c["SQ_ACTIVE_INST_VALU"] / (agent["simds"] * dur * clk), 4)
        if c.get("SQ_WAVES"):
            e["valu_insts_per_wave"] = round(c.get("SQ_INSTS_VALU", 0) / c["SQ_WAVES"], 1)
            e["waves"] = int(c["SQ_WAVES"])
        kernels[name] = e
    out = {"agent": agent, "dirs": [os.path.basename(d.rstrip("/")) for d in dirs],
           "workload": "bench.py --pmc-workload (see profiles/traffic.json for the shapes)",
           "kernels": kernels}
    with open(COUNTERS_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print("| kernel | dispatches | dur us | clock GHz (GRBM) | MFMA flops | MFMA busy @clock | MFMA busy @2.4GHz "
          "| VALU busy @2.4GHz | VALU insts/wave | waves |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for k, e in kernels.items():
        print(f"| {k} | {e['dispatches']} | {e['dur_us']} | {e.get('clock_ghz', '')} | {e.get('mfma_flops', '')} | "
              f"{e.get('mfma_busy_at_clock', '')} | {e.get('mfma_busy_at_peak_clock', '')} | "
              f"{e.get('valu_busy_at_peak_clock', '')} | {e.get('valu_insts_per_wave', '')} | {e.get('waves', '')} |")
    # Per wave: quad-cycle counters divided by SQ_WAVES; instruction counts
    # per wave; LDS bank conflicts as a total.
    print()
    print("| kernel | waves | wave life | waiting (SQ_WAIT_ANY) | issuing (SQ_ACTIVE_INST_ANY) | of which VALU | "
          "VMEM reads | LDS insts | MFMA insts | LDS bank conflicts (total) |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for k, e in kernels.items():
        c = e["counters"]
        w = c.get("SQ_WAVES")
        if not w or "SQ_WAVE_CYCLES" not in c:
            continue
        life = c["SQ_WAVE_CYCLES"] / w

        def pw(n):
            return c.get(n, 0) / w
        print(f"| {k} | {int(w)} | {life:.0f} | {pw('SQ_WAIT_ANY'):.0f} ({100 * pw('SQ_WAIT_ANY') / life:.0f}%) | "
              f"{pw('SQ_ACTIVE_INST_ANY'):.0f} ({100 * pw('SQ_ACTIVE_INST_ANY') / life:.0f}%) | "
              f"{pw('SQ_ACTIVE_INST_VALU'):.0f} | {pw('SQ_INSTS_VMEM_RD'):.0f} | {pw('SQ_INSTS_LDS'):.0f} | "
              f"{pw('SQ_INSTS_MFMA'):.0f} | {int(c.get('SQ_LDS_BANK_CONFLICT', 0))} |")


def load_counters():
    try:
        with open(COUNTERS_FILE) as f:
            return json.load(f)["kernels"]
    except (OSError, ValueError, KeyError):
        return {}


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["kernels"]
    except (OSError, ValueError, KeyError):
        return {}


def mfma_busy_field(e):
    """The prefill kernel's MFMA-busy figures from profiles/counters.json."""
    if not e or "mfma_busy_at_clock" not in e:
        return None
    return {"at_clock": e["mfma_busy_at_clock"], "at_2p4ghz": e["mfma_busy_at_peak_clock"],
            "clock_ghz": e.get("clock_ghz"), "dur_us": e["dur_us"],
            "source": "profiles/counters.json: SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x cycles); cycles = "
                      "GRBM_GUI_ACTIVE / 8 XCDs (at_clock) or duration x 2.4 GHz (at_2p4ghz); C4 8192 tokens"}


def decode_counter_field(kname, tr, e, merge_tr=None):
    """HBM traffic and VALU figures of one decode kernel from profiles/;
    merge_tr: the traffic of its merge launch (vtb_decode_merge), when the
    config takes one, added to the decode launch's."""
    if not tr and not e:
        return None
    out = {"kernel": kname}
    if tr:
        out["traffic_bytes"] = tr["traffic_bytes"] + (merge_tr["traffic_bytes"] if merge_tr else 0)
        if merge_tr:
            out["traffic_bytes_merge_launch"] = merge_tr["traffic_bytes"]
    if e:
        out.update({"valu_busy_at_2p4ghz": e.get("valu_busy_at_peak_clock"),
                    "valu_insts_per_wave": e.get("valu_insts_per_wave"), "waves": e.get("waves"),
                    "profiled_dur_us": e["dur_us"]})
    out["source"] = "profiles/traffic.json (FETCH_SIZE, WRITE_SIZE) and profiles/counters.json (SQ counters)"
    return out


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-workload":
        return pmc_workload()
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-summary":
        return pmc_summary(sys.argv[2], sys.argv[3])
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-sq-summary":
        return pmc_sq_summary(sys.argv[2:])
    if len(sys.argv) > 1 and sys.argv[1] == "--trace-summary":
        return trace_summary(sys.argv[2:])
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-dump":
        return print(json.dumps(pmc_read(sys.argv[2:]), indent=1))
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-more", action="store_true", help="skip the C1/C3/C5 decode lines")
    ap.add_argument("--no-gemv", action="store_true", help="skip the quantised GEMV / batched matmul lines")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; how the path would shard across GPUs "
                                   "is a design only (head-parallel decode/prefill, no exchange inside "
                                   "attention). Run with --gpus 1."}))
        sys.exit(2)

    import torch
    import vantablack_amd as vb
    ctx = vb.Context()

    def run(name, fn, *a, **kw):
        with phase(name):
            return fn(*a, **kw)

    dec = run("C2 decode @8K", bench_decode, ctx, torch, args)
    # The other decode configs (3, 5), reported
    # beside the headline.  C3: window 4096 at position 16383 -> 4096 rows.
    dec_more = {} if args.no_more else {
        "C1": run("C1 decode", bench_decode_cfg, ctx, torch, "C1", 1, 32, 4, 64, "f32", 512, steps=64),
        "C3": run("C3 decode", bench_decode_cfg, ctx, torch, "C3", 32, 32, 8, 128, "bf16", 4096),
        "C5": run("C5 decode", bench_decode_cfg, ctx, torch, "C5", 26, 8, 1, 256, "bf16", 32768),
        # C2's shape at 8K with the layer's RoPE of q and k_cur fused into
        # the same launch (the next-row prologue), to price the rotation.
        "C2_rope_fused": run("C2 + RoPE decode", bench_decode_cfg, ctx, torch, "C2+RoPE", 32, 32, 32, 128, "f16",
                             8192, rope=True),
        # C2 as BASELINE.json writes it: 256 steps, L 4097 -> 4352.
        "C2_256": run("C2 256 steps", bench_decode_c2_run, ctx, torch),
    }
    pre = {} if args.no_prefill else {
        "C4_L512": run("C4 prefill 512", bench_prefill, ctx, torch, 32, 8, 128, 512),
        "C4_L2048": run("C4 prefill 2048", bench_prefill, ctx, torch, 32, 8, 128, 2048),
        "C4_L8192": run("C4 prefill 8192", bench_prefill, ctx, torch, 32, 8, 128, 8192),
        "C5_L4096": run("C5 prefill 4096", bench_prefill, ctx, torch, 8, 1, 256, 4096),
    }
    # The next row beside attention: segMatmulQuant's GEMVs at Llama-2-7B
    # shapes, HBM-bound (weights streamed once per launch).
    gemv = None if args.no_gemv else {kind: run(f"GEMV {kind}", bench_gemv_layer, ctx, torch, kind)
                                       for kind in ("q4_k", "q5_k", "q6_k", "q8_0")}
    # matmulBatched (the prefill projections) at the C4 prompt length.
    qgemm = None if args.no_gemv else run("batched projections", bench_qgemm_layer, ctx, torch, "q4_k", 8192)
    # The whole token: every layer on the GPU (gpuLayerStep x 32 + gpuFinalStep).
    full = None if args.no_gemv else run("full decode", bench_full_decode, ctx, torch, ctx_rows=args.ctx)
    fullp = None if (args.no_gemv or args.no_prefill) else run("full prefill", bench_full_prefill, ctx, torch)
    cpu = None if args.no_cpu else cpu_baseline()
    cpu_cfg = None if args.no_cpu else cpu_baseline_configs()
    ctx.close()
    traffic = load_traffic()
    counters = load_counters()
    dec_kernel = decode_kernel_name(32, 32, 128, "f16")
    dec_tr = traffic.get(dec_kernel, {}).get("traffic_bytes")
    pre_kernel = pre["C4_L8192"]["kernel"] if pre else None
    pre_tr = traffic.get(pre_kernel, {}).get("traffic_bytes") if pre_kernel else None

    line = {
        "metric": METRIC,
        "value": round(dec["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (torch.randn on device; random f16 KV cache)",
        "config": {
            "workload": f"C2 Llama-2-7B full-stack decode attention @ctx {args.ctx // 1024}K: 32 layers x "
                        f"32q/32kv heads x d128, f16 KV, L {args.ctx + args.warmup + 1}->"
                        f"{args.ctx + args.warmup + args.steps}, 1 token/step (KV append + attention per layer)",
            "n_layers": 32, "n_heads": 32, "n_kv_heads": 32, "head_dim": 128, "kv_dtype": "f16",
            "ctx": args.ctx,
        },
        "pct_of_hbm_peak": round(100.0 * dec["value"] / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(dec["achieved_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dec["achieved_gbs"] / HBM_PEAK_GBS, 4), "traffic": dec_tr,
            "traffic_source": "profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated; L=8193)"
            if dec_tr else None,
            "kernel": f"{dec_kernel} (KV append fused)",
            "avg_launch_us": round(dec["avg_launch_s"] * 1e6, 3),
            "bytes_per_launch": int(dec["bytes_per_launch"]),
        },
    }
    if dec_more:
        # C5 (one query, 256 splits) merges in a second launch (vtb_decode_merge), the
        # only config of the counter workload that takes one.
        for cfg, kname, merge in (("C3", decode_kernel_name(32, 8, 128, "bf16"), None),
                                  ("C5", decode_kernel_name(8, 1, 256, "bf16"), "vtb_decode_merge")):
            if cfg in dec_more:
                dec_more[cfg]["counters"] = decode_counter_field(kname, traffic.get(kname), counters.get(kname),
                                                                 traffic.get(merge) if merge else None)
        line["decode_other_configs"] = dec_more
    if gemv:
        line["quant_gemv"] = {
            "workload": "Llama-2-7B layer projections q,k,v,o 4096x4096, gate,up 11008x4096, down 4096x11008; "
                        "f32 activations; weights cycled over >= 512 MB so each launch reads HBM",
            **gemv,
        }
    if fullp:
        line["full_prefill"] = dict(
            workload="Llama-3-8B shapes (32 layers, 32q/8kv heads x d128, ffn 14336), 8192-token prompt, Q4_K "
                     "projections on MFMA, bf16 KV, MFMA causal attention, then the final rmsnorm and the "
                     "128256-row Q6_K LM head on the last token (prefill.zig:143-146); every op on the GPU",
            **fullp)
    if full:
        line["full_decode"] = dict(
            workload="Llama-2-7B shapes, 32 layers + output norm and 32000-row logits, Q4_K projections, "
                     f"f16 KV at ctx {args.ctx}, one token per step; every op on the GPU",
            **full)
    if qgemm:
        line["prefill_projections"] = {
            "workload": "Llama-3-8B layer projections (q,o 4096x4096; k,v 1024x4096; gate,up 14336x4096; "
                        "down 4096x14336), Q4_K weights, f32 activations, 8192 tokens (C4 prompt length)",
            "flops": "reference flops 2*m*k*B; MFMA work 2x (activations as two f16 pieces, 22 bits)",
            "q4_k": qgemm,
        }
    if pre:
        p8 = pre["C4_L8192"]
        line["prefill"] = {
            "metric": "prefill attn TFLOP/s (% MFMA peak)",
            "workload": "C4 Llama-3-8B causal prefill: 32q/8kv heads x d128, bf16, 8192 tokens, pos0 0",
            "value": round(p8["tflops"], 2), "unit": "TFLOP/s",
            "pct_of_bf16_peak": round(100.0 * p8["tflops"] / BF16_PEAK_TFLOPS, 2),
            "roofline": {"bound": "mfma", "achieved": round(p8["tflops"], 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(p8["tflops"] / BF16_PEAK_TFLOPS, 4), "traffic": pre_tr,
                         "kernel": pre_kernel, "avg_launch_us": round(p8["avg_launch_s"] * 1e6, 2),
                         "timed_span": "one attn_prefill call: the pre-pass (vtb_kvt_bf16_d128: tile "
                                       "statistics, f16 K and V^T) and the attention kernel",
                         "flops_per_launch": p8["flops"],
                         "mfma_busy": mfma_busy_field(counters.get(pre_kernel))},
            "all": {k: {"tflops": round(v["tflops"], 2), "us": round(v["avg_launch_s"] * 1e6, 2)}
                    for k, v in pre.items()},
        }
    if cpu:
        line["cpu_baseline"] = {
            "value": round(cpu["pool"]["gbs"], 3), "unit": "GB/s", "cores": cpu["pool"]["workers"],
            "kind": "port",
            "sample": "one C2 layer at L=8192 (32 heads, d128, f32 K/V values, as vantablack's f32 cache "
                      "holds them), repeated ~6 s per line (three lines); GB/s counts the f32 bytes the "
                      "oracle reads; pool = heads split over pool.zig-style workers (vantablack itself runs "
                      "attention single-threaded)",
            "cpu_model": cpu["cpu_model"], "affinity_cpus": cpu["affinity_cpus"],
            "f16_equivalent_gbs": round(cpu["pool"]["gbs_f16_equiv"], 3),
            "faithful_1t": {"value": round(cpu["faithful_1t"]["gbs"], 3), "cores": 1,
                            "ms_per_layer": round(cpu["faithful_1t"]["ms_per_layer"], 3)},
            "pool_ms_per_layer": round(cpu["pool"]["ms_per_layer"], 3),
            "pool_default": {"value": round(cpu["pool_default"]["gbs"], 3), "cores": cpu["pool_default"]["workers"],
                             "ms_per_layer": round(cpu["pool_default"]["ms_per_layer"], 3),
                             "note": "pool.zig's default worker count, (workers + 1) / 2"},
        }
    if cpu_cfg:
        # The same GPU run's figure beside each CPU config line.
        gpu = {}
        if dec_more:
            layers = {"C1": 1, "C3": 32, "C5_decode": 26}
            for name, key in (("C1", "C1"), ("C3", "C3"), ("C5_decode", "C5")):
                if key in dec_more:
                    gpu[name] = {"ms_per_step": round(dec_more[key]["us_per_launch"] * layers[name] / 1e3, 4)}
            if "C2_256" in dec_more:
                gpu["C2_256"] = {"ms_total": dec_more["C2_256"]["ms_total"],
                                 "ms_per_step": dec_more["C2_256"]["ms_per_step"]}
        if pre:
            for name, key in (("C4_L512", "C4_L512"), ("C4_L2048", "C4_L2048"), ("C4_L8192", "C4_L8192"),
                              ("C5_prefill", "C5_L4096")):
                gpu[name] = {"ms_per_call": round(pre[key]["avg_launch_s"] * 1e3, 4)}
        for name, e in cpu_cfg.items():
            if name in gpu:
                e["gpu"] = gpu[name]
                k = "ms_per_call" if "ms_per_call" in gpu[name] else "ms_per_step"
                e["gpu"]["speedup_vs_pool"] = round(e["pool"][k] / gpu[name][k], 1)
        line.setdefault("cpu_baseline", {})["configs"] = cpu_cfg
        line["cpu_baseline"]["configs_note"] = (
            "every BASELINE config on the CPU oracle (C restatement of cpuAttention / attentionCausal, "
            "f32 values of the KV dtype): faithful_1t = one thread, as vantablack runs attention; pool / "
            "pool_default = heads split over a pool.zig-style pool at the box's CPU share and at pool.zig's "
            "default worker count; each line a bounded sample (see `sample`) extrapolated to the config")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
