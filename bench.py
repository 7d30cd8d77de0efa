#!/usr/bin/env python3
"""Benchmark of the RoPE-aware attention prologue on one MI355X (gfx950).

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

Headline workload (``value``): the ``optimized_attention`` query path of the
reference (src/e1_rope_publication_v1.py:661-726) at Qwen3-8B per-layer shape,
B=1, S=4096, causal, theta=1e6 -- one step = both launches of
``launch_attention(mode='query')`` (K RMSNorm+RoPE once, then causal GQA flash
attention with Q's RMSNorm+RoPE in the prologue), the reference's timing unit
(rope:665-666).  ``value`` is causal TFLOP/s (4*B*Hq*D*S(S+1)/2 per step) over
the K timed steps, inputs resident in HBM; the K steps are recorded once into
a HIP graph and replayed (the reference times graph replays too,
fusion_harness.py:32-79), and the eager per-step figures ride along.

The same line carries, as nested objects:
  * ``roofline``      -- the attention kernel alone, timed with HIP events on the
                         stream it is launched on, against dense-BF16 MFMA peak;
  * ``norm_rope``     -- the isolated Q/K RMSNorm+RoPE bandwidth sweep (six
                         shapes), rotating buffer sets so the 256 MB Infinity
                         Cache cannot serve replays, against HBM peak;
  * ``prefill_shapes``-- S=2048, S=8192 and the ragged B=4,S=1000 prefill;
  * ``factored``      -- the no-RoPE factored launch (Hq16/Hkv8/D256, B=2, S=2048);
  * ``cpu_baseline``  -- the eager FP32 CPU path (the oracle), timed on the host
                         cores on a bounded sample of the headline workload, and
                         the parity of the GPU output on that sample.

Inputs are synthetic (seeded CPU generator, BF16, copied to the GPU).  Only
one GPU is supported.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
METRIC = "µs + HBM GB/s fused QK-norm+RoPE; TFLOP/s fused-prologue GQA prefill"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense BF16 MFMA, published
SWEEP = [(1, 512), (1, 2048), (1, 8192), (4, 2048), (8, 1024), (16, 512)]
QWEN3_8B = (32, 8, 128)
GEMMA3_12B = (16, 8, 256)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed steps of the headline workload")
    ap.add_argument("--warmup", type=int, default=300, help="untimed steps first")
    ap.add_argument("--settle-ms", type=float, default=400.0,
                    help="after the warmup steps, further untimed steps until this much wall time of "
                         "continuous load has passed: the GPU clock needs a few hundred ms of load to settle, "
                         "whatever --warmup is")
    ap.add_argument("--seq", type=int, default=4096, help="headline sequence length")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--norm-style", default="fp32", choices=["fp32", "hf", "legacy"])
    ap.add_argument("--quick", action="store_true", help="headline workload only (no sweep, extra shapes, CPU)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget per workload")
    ap.add_argument("--sweep-only", action="store_true",
                    help="only the norm+RoPE six-shape sweep (for a kernel-trace profile of rows_kernel); prints "
                         "a JSON line with the sweep")
    ap.add_argument("--pmc", action="store_true",
                    help="short run for rocprofv3 counter passes: a few launches of each kernel plus a "
                         "copy of known size for calibration; prints a JSON line of what ran")
    return ap.parse_args()


def _events():
    import torch
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


SETTLE_MS = 300.0  # untimed replays before every graph-timed measurement (GPU clock)


def time_graph(fn, n, replays=10):
    """Average device time (ms) per call of ``fn(i)``, i = 0..n-1, as one HIP
    graph block replayed ``replays`` times (median), with the package's paced
    timing protocol (kernelfuser_amd.timing), after SETTLE_MS of untimed
    replays of the same block so every measurement starts at the settled
    clock, whatever ran before it."""
    from kernelfuser_amd import timing
    return timing.block_time_us(fn, n, replays=replays, settle_ms=SETTLE_MS) * 1e-3


def load_traffic():
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return {}
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return {}


NOMINAL_GHZ = 2.4  # MI355X peak engine clock, at which MFMA_BF16_PEAK_TFS is quoted


def clock_of(kf, fn, launches=200):
    """Shader clock during `fn`'s attention launches: `launches` back-to-back
    calls with per-workgroup clock stamps on (kfmi_clock_stamps), summarised
    over the last launch's workgroups; results are unchanged by the stamps.
    None (and a note on stderr) if the stamps cannot be read: the clock is
    reported beside the measured figures, never in place of them."""
    try:
        with kf._lib.tuning(clock_stamps=1):
            for _ in range(launches):
                fn()
        return kf._lib.clock_summary(kf._lib.clock_stamps())
    except (RuntimeError, ValueError) as e:
        print(f"bench: clock stamps unavailable: {e}", file=sys.stderr, flush=True)
        return None


def at_clock(tflops, clock):
    """Fraction of the MFMA peak scaled to the measured clock (None without one)."""
    return None if clock is None else tflops / (MFMA_BF16_PEAK_TFS * clock["ghz_median"] / NOMINAL_GHZ)


def headline(args, torch, kf):
    """Timed steps of launch_attention(mode='query') plus the attention kernel alone."""
    b, s = args.batch, args.seq
    hq, hkv, d = QWEN3_8B
    xs_cpu = kf.make_inputs(b, s, QWEN3_8B, 1909)
    xs = xs_cpu.to("cuda:0")
    out = torch.empty_like(xs.q)
    kn = torch.empty_like(xs.k)
    step = lambda: kf.launch_attention(xs.reference7, out, causal=True, mode="query", bm=128, bn=64, kn=kn,
                                       norm_style=args.norm_style)
    t_settle = time.perf_counter()
    for _ in range(args.warmup):
        step()
    settle_steps = 0
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(20):
            step()
        settle_steps += 20
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    # Eager steps: one host call per step.
    ev0, ev1 = _events()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    eager_wall_ms = (time.perf_counter() - t0) * 1e3
    eager_dev_ms = ev0.elapsed_time(ev1)
    # The timed steps: the same K steps recorded once into a HIP graph and
    # replayed, as the reference times its arms (fusion_harness.py:32-79);
    # the replay is bracketed by synchronisations, so the host clock sees
    # exactly the K steps' device work.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        step()
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(args.steps):
                step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:  # the clock settles under the replayed load
        graph.replay()
        torch.cuda.synchronize()
    ev0, ev1 = _events()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    dev_ms = ev0.elapsed_time(ev1)
    del graph
    flops = kf.attention_flops(b, hq, s, d, True)
    ms_step = wall_ms / args.steps
    res = {"flops_per_step": flops, "ms_per_step": ms_step, "device_ms_per_step": dev_ms / args.steps,
           "tflops": flops / (ms_step * 1e-3) / 1e12, "settle_steps": settle_steps,
           "eager_ms_per_step": eager_wall_ms / args.steps, "eager_device_ms_per_step": eager_dev_ms / args.steps}
    # The two kernels separately (events on the launch stream).
    attn_ms = time_graph(lambda i: kf.attention_prefill(xs.q, kn, xs.v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin,
                                                           causal=True, fuse_q=True, norm_style=args.norm_style),
                         20)
    # The preparation launch of the step: K norm+RoPE rows.
    prep_ms = time_graph(lambda i: kf.prepare_attention(xs.reference7, None, kn, only_k=True, rope=True,
                                                        norm_style=args.norm_style), 100)
    res["attention_kernel_us"] = attn_ms * 1e3
    res["clock"] = clock_of(kf, lambda: kf.attention_prefill(xs.q, kn, xs.v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin,
                                                              causal=True, fuse_q=True, norm_style=args.norm_style))
    res["prep_kernel_us"] = prep_ms * 1e3
    res["attention_kernel_tflops"] = flops / (attn_ms * 1e-3) / 1e12
    prep_bytes = kf.k_prep_bytes(b, hkv, s, d)
    res["prep_bytes"] = prep_bytes
    res["prep_gbs"] = prep_bytes / (prep_ms * 1e-3) / 1e9
    return res, xs_cpu, out


def norm_rope_sweep(args, torch, kf):
    """Isolated Q+K norm+RoPE, one launch per call, buffer sets rotated (> 512 MB total)."""
    hq, hkv, d = QWEN3_8B
    rows = []
    for b, s in SWEEP:
        nbytes = kf.norm_rope_bytes(b, hq, hkv, s, d)
        nsets = max(2, min(64, -(-768 * 2 ** 20 // nbytes)))
        base = kf.make_inputs(b, s, QWEN3_8B, 1909, with_v=False).to("cuda:0")
        sets = []
        for i in range(nsets):
            q = base.q if i == 0 else base.q.roll(i, dims=2).contiguous()
            k = base.k if i == 0 else base.k.roll(i, dims=2).contiguous()
            sets.append((q, k, torch.empty_like(q), torch.empty_like(k)))
        fn = lambda i: kf.norm_rope(sets[i % nsets][0], sets[i % nsets][1], base.gq, base.gk, base.cos, base.sin,
                                    norm_style=args.norm_style, qn=sets[i % nsets][2], kn=sets[i % nsets][3])
        ms = time_graph(fn, max(4 * nsets, 40))
        rows.append({"B": b, "S": s, "bytes": nbytes, "us": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9,
                     "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "buffer_sets": nsets})
        del sets, base
        torch.cuda.empty_cache()
    big = [r for r in rows if r["bytes"] > 100e6]
    best = max(big, key=lambda r: r["gbs"])
    return {"kernel": "rows_kernel (Q+K rows, one launch)", "norm_style": args.norm_style, "shapes": rows,
            "roofline": {"bound": "hbm", "achieved": best["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": best["gbs"] / HBM_PEAK_GBS, "shape": [best["B"], best["S"]],
                         "traffic": load_traffic().get("norm_rope_b%d_s%d" % (best["B"], best["S"]))},
            "min_frac_large_shapes": min(r["frac_hbm"] for r in big)}


def prefill_shapes(args, torch, kf):
    hq, hkv, d = QWEN3_8B
    rows = []
    for b, s in [(1, 2048), (1, 8192), (4, 1000)]:
        xs = kf.make_inputs(b, s, QWEN3_8B, 2909).to("cuda:0")
        out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
        step = lambda: kf.launch_attention(xs.reference7, out, causal=True, mode="query", bm=128, bn=64, kn=kn,
                                           norm_style=args.norm_style)
        ms = time_graph(lambda i: step(), 20)
        f = kf.attention_flops(b, hq, s, d, True)
        clk = clock_of(kf, step)
        tf = f / (ms * 1e-3) / 1e12
        rows.append({"B": b, "S": s, "kernel": kf._lib.attention_kernel(b, hq, hkv, s, d, True, kf._lib.MODE_QUERY),
                     "us": ms * 1e3, "tflops": tf, "frac_mfma": tf / MFMA_BF16_PEAK_TFS,
                     "clock_ghz": None if clk is None else clk["ghz_median"], "frac_mfma_at_clock": at_clock(tf, clk)})
        del xs, out, kn
    return rows


def factored(args, torch, kf):
    b, s = 2, 2048
    hq, hkv, d = GEMMA3_12B
    xs = kf.make_inputs(b, s, GEMMA3_12B, 1909, rope=False).to("cuda:0")
    out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
    inv = torch.empty(xs.q.shape[:-1], device="cuda:0", dtype=torch.float32)
    step = lambda: kf.launch_factored_attention((xs.q, xs.k, xs.v, xs.gq, xs.gk), out, inv, kn, causal=True, bm=128,
                                                bn=64)
    ms = time_graph(lambda i: step(), 20)
    f = kf.attention_flops(b, hq, s, d, True)
    clk = clock_of(kf, step)
    tf = f / (ms * 1e-3) / 1e12
    return {"B": b, "S": s, "Hq": hq, "Hkv": hkv, "D": d, "causal": True, "us": ms * 1e3,
            "tflops": tf, "frac_mfma": tf / MFMA_BF16_PEAK_TFS,
            "clock_ghz": None if clk is None else clk["ghz_median"], "frac_mfma_at_clock": at_clock(tf, clk)}


def cpu_baseline(args, torch, xs_cpu, out_gpu):
    """The eager FP32 CPU path (oracle restatement of rope:295-302) on a bounded
    sample of the headline workload: KV group 0 (Q heads 0-3, KV head 0) of
    B=1, S=seq.  Also checks the GPU output on that sample (attention gate)."""
    import oracle
    host_cpus = os.cpu_count() or 1
    threads = max(1, min(16, host_cpus))  # the box's CPU share is 16 threads
    torch.set_num_threads(threads)
    hq, hkv, d = QWEN3_8B
    g = hq // hkv
    q, k, v = xs_cpu.q[:, :g].contiguous(), xs_cpu.k[:, :1].contiguous(), xs_cpu.v[:, :1].contiguous()
    times, ref = [], None
    t_end = time.perf_counter() + args.cpu_seconds
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        ref = oracle.oracle_fp32(q, k, v, xs_cpu.gq, xs_cpu.gk, xs_cpu.cos, xs_cpu.sin, True)
        times.append(time.perf_counter() - t0)
    f = 4 * q.shape[0] * g * d * (q.shape[2] * (q.shape[2] + 1) // 2)
    med = statistics.median(times[1:] if len(times) > 2 else times)
    gate = oracle.attention_gate(out_gpu[:, :g].float().cpu(), ref)
    res = {"value": f / med / 1e12, "unit": "TFLOP/s", "cores": threads, "host_cpus": host_cpus, "kind": "port",
           "sample_share_of_workload": g / hq,
           "sample": (f"oracle_fp32 (eager FP32 torch: RMSNorm, RoPE, SDPA) on KV group 0 of the headline "
                      f"workload (1/{hkv} of its FLOPs): B=1, Hq={g}, Hkv=1, S={q.shape[2]}, D=128, causal; "
                      f"{len(times)} calls in {sum(times):.1f} s, median {med * 1e3:.1f} ms; rate = that "
                      f"sample's FLOPs / its median time, on {threads} threads"),
           "parity": {k2: gate[k2] for k2 in ("max_abs", "mean_abs", "relative_l2", "pass")}}
    # norm+RoPE CPU leg on the largest sweep shape, in GB/s.
    nr = None
    xs = None
    try:
        from kernelfuser_amd.inputs import make_inputs
        xs = make_inputs(1, 8192, QWEN3_8B, 1909, with_v=False)
        nt = []
        t_end = time.perf_counter() + args.cpu_seconds / 2
        while time.perf_counter() < t_end or len(nt) < 2:
            t0 = time.perf_counter()
            oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin).to(torch.bfloat16)
            oracle.norm_rope_fp32(xs.k, xs.gk, xs.cos, xs.sin).to(torch.bfloat16)
            nt.append(time.perf_counter() - t0)
        m = statistics.median(nt[1:] if len(nt) > 2 else nt)
        by = 4 * 8192 * 40 * 128 + 2 * 8192 * 128 + 4 * 128
        nr = {"value": by / m / 1e9, "unit": "GB/s", "cores": threads, "host_cpus": host_cpus, "kind": "port",
              "sample": f"norm_rope_fp32 of Q and K at B=1, S=8192 (Qwen3-8B heads), {len(nt)} calls, "
                        f"median {m * 1e3:.1f} ms"}
    finally:
        del xs
    res["norm_rope"] = nr
    return res


def pmc_run(torch, kf):
    """A few launches of each kernel at the headline shapes plus one copy of
    known size, for rocprofv3 --pmc passes (FETCH_SIZE / WRITE_SIZE)."""
    xs = kf.make_inputs(1, 4096, QWEN3_8B, 1909).to("cuda:0")
    out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
    for _ in range(3):
        kf.launch_attention(xs.reference7, out, causal=True, mode="query", bm=128, bn=64, kn=kn, norm_style="fp32")
    # the general kernel's configurations: B=1 S=2048, B=4 S=1000, factored D=256
    for b, s in ((1, 2048), (4, 1000)):
        gx = kf.make_inputs(b, s, QWEN3_8B, 2909).to("cuda:0")
        go, gk = torch.empty_like(gx.q), torch.empty_like(gx.k)
        for _ in range(3):
            kf.launch_attention(gx.reference7, go, causal=True, mode="query", bm=128, bn=64, kn=gk, norm_style="fp32")
        del gx, go, gk
    fx = kf.make_inputs(2, 2048, GEMMA3_12B, 1909, rope=False).to("cuda:0")
    fo, fk = torch.empty_like(fx.q), torch.empty_like(fx.k)
    finv = torch.empty(fx.q.shape[:-1], device="cuda:0", dtype=torch.float32)
    for _ in range(3):
        kf.launch_factored_attention((fx.q, fx.k, fx.v, fx.gq, fx.gk), fo, finv, fk, causal=True, bm=128, bn=64)
    del fx, fo, fk, finv
    # norm+RoPE: the six sweep shapes, in the sweep's order (B=1 S=512 and
    # S=8192 run two heads per workgroup, B=1 S=2048 and the three 170 MB
    # shapes four)
    for b, s in SWEEP:
        nr = kf.make_inputs(b, s, QWEN3_8B, 1909, with_v=False).to("cuda:0")
        qn, kn2 = torch.empty_like(nr.q), torch.empty_like(nr.k)
        for _ in range(3):
            kf.norm_rope(nr.q, nr.k, nr.gq, nr.gk, nr.cos, nr.sin, norm_style="fp32", qn=qn, kn=kn2)
        del nr, qn, kn2
    src = torch.ones(256 * 2 ** 20 // 4, device="cuda:0", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_run": True, "copy_bytes_each_way": src.numel() * 4,
                      "attention": "B=1 S=4096 causal", "general": ["B=1 S=2048", "B=4 S=1000", "factored D=256 B=2 S=2048"], "norm_rope": [f"B={b} S={s}" for b, s in SWEEP]}), flush=True)


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (multi-GPU sharding is "
                                   "a design note, not built)", "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible; bench.py needs an MI355X"}), flush=True)
        sys.exit(1)
    sys.path.insert(0, str(ROOT))
    import kernelfuser_amd as kf
    from kernelfuser_amd import _lib
    _lib.load()
    if args.pmc:
        pmc_run(torch, kf)
        return
    if args.sweep_only:
        print(json.dumps({"norm_rope": norm_rope_sweep(args, torch, kf)}), flush=True)
        return
    head, xs_cpu, out = headline(args, torch, kf)
    traffic = load_traffic().get("attention_b%d_s%d" % (args.batch, args.seq))
    line = {
        "metric": METRIC,
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded CPU torch.Generator, N(0,1) Q/K/V, gamma=1+0.1N, theta=1e6)",
        "config": {"workload": "optimized_attention mode=query (K norm+RoPE launch + fused-prologue causal "
                               "GQA prefill), Qwen3-8B per-layer heads",
                   "B": args.batch, "S": args.seq, "Hq": 32, "Hkv": 8, "D": 128, "causal": True,
                   "norm_style": args.norm_style, "flops_per_step": head["flops_per_step"],
                   "flops_convention": "4*B*Hq*D*S(S+1)/2"},
        "roofline": {"bound": "mfma", "kernel": "attn_pp_kernel (fused Q norm+RoPE prologue, ping-pong waves)",
                     "achieved": head["attention_kernel_tflops"], "peak": MFMA_BF16_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": head["attention_kernel_tflops"] / MFMA_BF16_PEAK_TFS,
                     "kernel_us": head["attention_kernel_us"], "traffic": traffic,
                     "frac_step_device": head["flops_per_step"] / (head["device_ms_per_step"] * 1e-3) / 1e12
                     / MFMA_BF16_PEAK_TFS,
                     "frac_step_wall": head["tflops"] / MFMA_BF16_PEAK_TFS,
                     "frac_note": "frac: attention kernel alone (graph-replay events); frac_step_*: the whole "
                                  "step (K-prep launch + attention, K steps replayed as one HIP graph) by "
                                  "device events / by the host clock",
                     "clock": None if head["clock"] is None else dict(
                         head["clock"], nominal_ghz=NOMINAL_GHZ,
                         peak_at_clock=MFMA_BF16_PEAK_TFS * head["clock"]["ghz_median"] / NOMINAL_GHZ,
                         frac_at_clock=at_clock(head["attention_kernel_tflops"], head["clock"]),
                         note="shader clock of the attention kernel's workgroups (per-workgroup "
                              "s_memtime / s_memrealtime stamps, 200 back-to-back launches, last "
                              "launch); peak_at_clock scales the 2.5 PFLOP/s peak to that clock")},
        "kernels": {"attention_us": head["attention_kernel_us"],
                    "prep_us": head["prep_kernel_us"], "prep_bytes": head["prep_bytes"],
                    "prep_gbs": head["prep_gbs"], "prep": "K RMSNorm+RoPE rows (one launch)",
                    "device_ms_per_step": head["device_ms_per_step"], "settle_steps": head["settle_steps"],
                    "step_timing": "K steps recorded once into a HIP graph and replayed (host clock around "
                                   "the replay, synchronised on both sides)",
                    "eager_ms_per_step": head["eager_ms_per_step"],
                    "eager_device_ms_per_step": head["eager_device_ms_per_step"]},
    }
    if not args.quick:
        line["norm_rope"] = norm_rope_sweep(args, torch, kf)
        line["prefill_shapes"] = prefill_shapes(args, torch, kf)
        line["factored"] = factored(args, torch, kf)
    if not args.quick and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args, torch, xs_cpu, out)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
