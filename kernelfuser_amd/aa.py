"""A/A noise-floor runner for the fused attention prologue on gfx950.

Counterpart of the reference's A/A control (src/e7_rope_aa.py:116-191, with
``stats`` of src/e1_qk_publication_v3.py:206-220).  Both arms run the SAME
path -- ``optimized_attention`` of this package -- on bitwise-identical
inputs, so any timing difference between them is measurement noise.  The
protocol follows the reference:

* every round captures a fresh HIP graph per arm (after warmups) and checks
  that A1, A2 and an eager call give finite, bitwise-equal outputs before
  timing and again after it;
* each sample replays both graphs once, in a random order drawn per pair;
* per round: the A1/A2 ratio of medians and the paired-delta mean with its
  95% interval; over rounds: the pooled ratio and the interval of the
  per-round deltas;
* an independent retest repeats everything with fresh captures and another
  order seed.

Not carried over: Chrome-trace capture and the GPU-exclusivity monitor (the
reference polls NVML; here one process owns the GPU for the run).

``python -m kernelfuser_amd.aa --out results.json`` runs the reference's six
Qwen3-8B short-prefill shapes (B in 1, 8, 32; S in 128, 256; causal).
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import random
import statistics
import time
from pathlib import Path

import torch

from .inputs import QWEN3_8B, make_inputs

WARMUPS = 20
RETEST_SEED_OFFSET = 1000003


def stats(xs) -> dict:
    """Summary of event samples in ms (the fields of qk:206-220)."""
    if not xs:
        raise ValueError("timing sample collection is empty")
    vals = [float(x) for x in xs]
    if not all(math.isfinite(x) and x >= 0.0 for x in vals):
        raise ValueError(f"timing samples must be finite and non-negative: {vals!r}")
    mean = statistics.fmean(vals)
    sem = statistics.stdev(vals) / math.sqrt(len(vals)) if len(vals) > 1 else 0.0
    return {"n": len(vals), "mean_ms": mean, "sem_ms": sem, "two_sem_ms": 2.0 * sem,
            "p50_ms": statistics.median(vals), "p95_ms": sorted(vals)[math.ceil(.95 * len(vals)) - 1],
            "samples_ms": vals}


def exact_check(left: torch.Tensor, right: torch.Tensor) -> dict:
    """Finite and bitwise-equal outputs (e7:44-54)."""
    if left.is_cuda or right.is_cuda:
        torch.cuda.synchronize()
    finite = bool(torch.isfinite(left).all().item() and torch.isfinite(right).all().item())
    equal = bool(torch.equal(left, right))
    return {"finite": finite, "exact_output_equal": equal,
            "max_abs": float((left.float() - right.float()).abs().max().item()) if finite else None,
            "pass": finite and equal}


def capture(fn, warmups: int = WARMUPS):
    """One independent graph of ``fn`` (captured after warmups on a side stream),
    replayed once so its output can be inspected."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmups):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        output = fn()
    graph.replay()
    torch.cuda.synchronize()
    return graph, output


def event_sample(graph) -> float:
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    end.record()
    end.synchronize()
    value = float(start.elapsed_time(end))
    if not math.isfinite(value) or value <= 0:
        raise RuntimeError(f"invalid event sample: {value}")
    return value


def measure_pair(fn_a, fn_b, reference: torch.Tensor, rounds: int, samples: int, seed: int,
                 warmups: int = WARMUPS) -> dict:
    """Fresh A1/A2 captures every round, randomized order for every pair (e7:116-191)."""
    if rounds < 1 or samples < 2:
        raise ValueError("A/A timing needs at least one round and two samples per round")
    rng = random.Random(seed)
    records = []
    for index in range(rounds):
        ga, oa = capture(fn_a, warmups)
        gb, ob = capture(fn_b, warmups)
        checks = {"A1_vs_A2": exact_check(oa, ob), "A1_vs_eager": exact_check(oa, reference),
                  "A2_vs_eager": exact_check(ob, reference)}
        if not all(c["pass"] for c in checks.values()):
            raise RuntimeError(f"A/A output check failed before timing: {checks}")
        for _ in range(warmups):
            ga.replay()
            gb.replay()
        torch.cuda.synchronize()
        a_times, b_times, orders = [], [], []
        for _ in range(samples):
            if rng.random() < 0.5:
                orders.append("A1_first")
                a_times.append(event_sample(ga))
                b_times.append(event_sample(gb))
            else:
                orders.append("A2_first")
                b_times.append(event_sample(gb))
                a_times.append(event_sample(ga))
        final = exact_check(oa, ob)
        if not final["pass"]:
            raise RuntimeError(f"A/A output changed during replay: {final}")
        deltas = [a - b for a, b in zip(a_times, b_times)]
        records.append({
            "round": index, "A1": stats(a_times), "A2": stats(b_times), "arm_order": orders,
            "ratio": statistics.median(a_times) / statistics.median(b_times),
            "paired_delta_mean_ms": statistics.fmean(deltas),
            "paired_delta_ci95_ms": 1.96 * statistics.stdev(deltas) / math.sqrt(samples),
            "correctness_before": checks, "correctness_after": final,
        })
        del ga, gb, oa, ob
        gc.collect()
        torch.cuda.empty_cache()
    a_all = [v for r in records for v in r["A1"]["samples_ms"]]
    b_all = [v for r in records for v in r["A2"]["samples_ms"]]
    ratios = [r["ratio"] for r in records]
    means = [r["paired_delta_mean_ms"] for r in records]
    return {
        "mode": "hip_graph_replay_paired_interleaved", "paired": True,
        "arm_order": "randomized_per_pair_sample", "fresh_graph_captures_per_arm": rounds,
        "warmups_per_capture": warmups, "samples_per_round": samples, "seed": seed,
        "rounds": records, "A1": stats(a_all), "A2": stats(b_all),
        "ratio": statistics.fmean(a_all) / statistics.fmean(b_all),
        "ratio_median_round": statistics.median(ratios),
        "ratio_range_round": [min(ratios), max(ratios)],
        "delta_mean_across_rounds_ms": statistics.fmean(means),
        "delta_ci95_across_rounds_ms": 1.96 * statistics.stdev(means) / math.sqrt(rounds) if rounds > 1 else None,
    }


def run_row(b: int, s: int, rounds: int, samples: int, mode: str = "query", norm_style: str = "hf",
            device: str = "cuda:0") -> dict:
    """One shape: identical inputs for both arms, eager reference, initial run
    and an independently recaptured retest."""
    from .ops import optimized_attention
    seed = 1701 + b + s + 1  # e7:252
    xs = make_inputs(b, s, QWEN3_8B, seed).to(device)
    inputs_a = xs.astuple()
    inputs_b = tuple(t.detach().clone() for t in inputs_a)
    fn = lambda t: (lambda: optimized_attention(*t, causal=True, mode=mode, norm_style=norm_style))
    with torch.inference_mode():
        reference = fn(inputs_a)()
        eager_b = fn(inputs_b)()
        row = {"model": "Qwen3-8B", "B": b, "S": s, "causal": True, "mode": mode, "norm_style": norm_style,
               "geometry": {"Hq": QWEN3_8B[0], "Hkv": QWEN3_8B[1], "D": QWEN3_8B[2]}, "input_seed": seed,
               "correctness": exact_check(reference, eager_b)}
        if not row["correctness"]["pass"]:
            raise RuntimeError("eager arms differ or contain non-finite values")
        row["initial"] = measure_pair(fn(inputs_a), fn(inputs_b), reference, rounds, samples, 98431 + b + s)
        row["retest"] = measure_pair(fn(inputs_a), fn(inputs_b), reference, rounds, samples,
                                     98431 + b + s + RETEST_SEED_OFFSET)
    row["status"] = "tested_pass"
    return row


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", required=True)
    ap.add_argument("--batches", default="1,8,32")
    ap.add_argument("--sizes", default="128,256")
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--samples", type=int, default=100)
    ap.add_argument("--mode", default="query", choices=["query", "unfused"])
    ap.add_argument("--norm-style", default="hf", choices=["hf", "legacy", "fp32"])
    args = ap.parse_args(argv)
    batches = [int(x) for x in args.batches.split(",")]
    sizes = [int(x) for x in args.sizes.split(",")]
    if args.rounds < 1 or args.samples < 2 or not all(x > 0 for x in batches + sizes):
        ap.error("positive shapes, at least one round and at least two samples are required")
    reasons = []
    if sorted((b, s) for b in batches for s in sizes) != sorted((b, s) for b in (1, 8, 32) for s in (128, 256)):
        reasons.append("the full noise-floor protocol uses B=1,8,32 and S=128,256")
    if args.rounds < 5 or args.samples < 100:
        reasons.append("the full noise-floor protocol uses at least 5 rounds and 100 samples per round")
    rec = {"schema": "kernelfuser-amd-aa-v1", "scope": "optimized_attention A/A at Qwen3-8B short-prefill shapes",
           "created_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
           "gpu": torch.cuda.get_device_name(0), "torch": torch.__version__,
           "protocol": {"rounds": args.rounds, "samples": args.samples, "warmup": WARMUPS,
                        "randomized_arm_order": "per_pair_sample", "graph": "hip",
                        "correctness": "finite and bitwise-equal A1/A2/eager outputs before and after timing"},
           "protocol_gate_reasons": reasons, "rows": []}
    out = Path(args.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    for b in batches:
        for s in sizes:
            row = run_row(b, s, args.rounds, args.samples, args.mode, args.norm_style)
            rec["rows"].append(row)
            out.write_text(json.dumps(rec, indent=1) + "\n")
            print(f"Qwen3-8B B={b} S={s} {row['status']} initial={row['initial']['ratio']:.4f} "
                  f"retest={row['retest']['ratio']:.4f}", flush=True)
            gc.collect()
            torch.cuda.empty_cache()
    return rec


if __name__ == "__main__":
    main()
