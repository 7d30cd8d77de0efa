"""A/A noise floor of the fused attention prologue on one MI355X.

Counterpart of the reference's A/A control (src/e7_rope_aa.py:116-191): two
arms that run the same path -- ``optimized_attention`` of this package -- on
separate but bitwise-identical inputs, timed with the package's interleaved
graph-block protocol (``timing.interleaved``).  Whatever separates the two
arms is the noise of that protocol, which bounds the differences the
refinement runner can claim.

Per shape:
  * the eager outputs of both arms must be finite and bitwise equal;
  * a *pass* is one ``timing.interleaved`` run over both arms (fresh blocks
    every round; the last output of every block is checked bitwise against the
    eager output after the round's samples, so a replay that drifted fails the
    run);
  * the statistic is the per-sample paired ratio A1/A2 (both blocks from the
    same sample): its median with a bootstrap 95% interval, plus the ratio of
    the two arms' medians;
  * a second, independent pass (the retest) uses other input copies, fresh
    captures and another order seed.

``python -m kernelfuser_amd.aa --out results.json`` runs the reference's six
Qwen3-8B short-prefill shapes (B in 1, 8, 32; S in 128, 256; causal).
"""
from __future__ import annotations

import argparse
import gc
import json
import time
from pathlib import Path

import torch

from . import _lib, exclusive, timing
from .inputs import QWEN3_8B, make_inputs

DEFAULT_ROUNDS, DEFAULT_SAMPLES, DEFAULT_LAUNCHES = 5, 40, 20


def _bits(t: torch.Tensor) -> torch.Tensor:
    """The tensor's bit patterns as integers (so -0.0 and 0.0 differ)."""
    ints = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}
    return t.contiguous().view(ints[t.element_size()]) if t.is_floating_point() else t


def bitwise(left: torch.Tensor, right: torch.Tensor) -> dict:
    """Finite and bitwise-equal tensors (the A/A correctness condition)."""
    if left.is_cuda or right.is_cuda:
        torch.cuda.synchronize()
    finite = bool(torch.isfinite(left).all().item() and torch.isfinite(right).all().item())
    same = bool(left.shape == right.shape and left.dtype == right.dtype
                and torch.equal(_bits(left), _bits(right)))
    diff = float((left.float() - right.float()).abs().max().item()) if finite and left.shape == right.shape else None
    return {"finite": finite, "bitwise_equal": same, "max_abs": diff, "pass": finite and same}


def aa_pass(fn_a, fn_b, eager: torch.Tensor, *, rounds: int, samples: int, launches: int, seed: int) -> dict:
    """One A/A pass: both arms interleaved, replay outputs checked bitwise
    against ``eager`` after every round."""
    checks = []

    def check(name, out):
        r = bitwise(out, eager)
        checks.append({"arm": name, **r})
        if not r["pass"]:
            raise RuntimeError(f"A/A replay output of {name} differs from the eager output: {r}")

    res = timing.interleaved({"A1": fn_a, "A2": fn_b}, rounds=rounds, samples=samples, launches=launches,
                             seed=seed, baseline="A2", check=check)
    a, b = res["arms"]["A1"], res["arms"]["A2"]
    pr = res["paired_ratio"]["A1"]
    return {"A1": {k: a[k] for k in ("n", "median_us", "p10_us", "p90_us", "mean_us")},
            "A2": {k: b[k] for k in ("n", "median_us", "p10_us", "p90_us", "mean_us")},
            "ratio_of_medians": a["median_us"] / b["median_us"],
            "paired_ratio_median": pr["median"], "paired_ratio_ci95": pr["ci95"],
            "replay_checks": checks, "protocol": {k: v for k, v in res["protocol"].items() if k != "orders"},
            "orders": res["protocol"]["orders"]}


def run_row(b: int, s: int, rounds: int = DEFAULT_ROUNDS, samples: int = DEFAULT_SAMPLES,
            launches: int = DEFAULT_LAUNCHES, mode: str = "query", norm_style: str = "hf",
            device: str = "cuda:0") -> dict:
    """One shape: eager A1/A2 check, then the initial and the retest pass."""
    from .ops import optimized_attention
    seed = 7001 + 31 * b + s
    host = make_inputs(b, s, QWEN3_8B, seed)
    row = {"model": "Qwen3-8B", "B": b, "S": s, "causal": True, "mode": mode, "norm_style": norm_style,
           "geometry": {"Hq": QWEN3_8B[0], "Hkv": QWEN3_8B[1], "D": QWEN3_8B[2]}, "input_seed": seed,
           "launches_per_block": launches}
    with torch.inference_mode():
        for label, order_seed in (("initial", seed), ("retest", seed + 104729)):
            xa, xb = host.to(device).astuple(), host.to(device).astuple()  # separate copies per pass
            arm = lambda xs: (lambda: optimized_attention(*xs, causal=True, mode=mode, norm_style=norm_style))
            with _lib.record_launches() as ka:
                ea = arm(xa)()
            with _lib.record_launches() as kb:
                eb = arm(xb)()
            eager = bitwise(ea, eb)
            if not eager["pass"]:
                raise RuntimeError(f"eager A1/A2 outputs differ or are not finite: {eager}")
            # each arm's kernels of this library (the reference keeps a kernel
            # trace per arm, e7_rope_aa.py:89-113); an arm without any measured
            # something else
            eager["kernels"] = {"A1": ka.launches, "A2": kb.launches}
            if not ka.launches or not kb.launches:
                row["status"] = "invalid_no_kernel"
                row[label] = {"eager_check": eager}
                return row
            rec = aa_pass(arm(xa), arm(xb), ea, rounds=rounds, samples=samples, launches=launches,
                          seed=order_seed)
            rec["eager_check"] = eager
            row[label] = rec
            del xa, xb, ea, eb
            gc.collect()
            torch.cuda.empty_cache()
    row["status"] = "tested_pass"
    return row


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", required=True)
    ap.add_argument("--batches", default="1,8,32")
    ap.add_argument("--sizes", default="128,256")
    ap.add_argument("--rounds", type=int, default=DEFAULT_ROUNDS)
    ap.add_argument("--samples", type=int, default=DEFAULT_SAMPLES)
    ap.add_argument("--launches", type=int, default=DEFAULT_LAUNCHES)
    ap.add_argument("--mode", default="query", choices=["query", "unfused"])
    ap.add_argument("--norm-style", default="hf", choices=["hf", "legacy", "fp32"])
    args = ap.parse_args(argv)
    batches = [int(x) for x in args.batches.split(",")]
    sizes = [int(x) for x in args.sizes.split(",")]
    if args.rounds < 1 or args.samples < 2 or args.launches < 1 or not all(x > 0 for x in batches + sizes):
        ap.error("positive shapes, at least one round, two samples and one launch per block are required")
    rec = {"schema": "kernelfuser-amd-aa-v2",
           "scope": "optimized_attention A/A at Qwen3-8B short-prefill shapes",
           "created_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
           "gpu": torch.cuda.get_device_name(0), "torch": torch.__version__,
           "protocol": {"rounds": args.rounds, "samples": args.samples, "launches_per_block": args.launches,
                        "timing": "kernelfuser_amd.timing.interleaved (paced, cyclic Latin-square order)",
                        "correctness": "finite and bitwise-equal eager A1/A2 outputs; every block's last "
                                       "replay output bitwise equal to the eager output"},
           "rows": []}
    out = Path(args.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    torch.zeros(1, device="cuda:0")  # hold a context, so the GPU's process list must name this process
    mon = exclusive.ExclusiveMonitor(0).start()
    try:
        _run_rows(batches, sizes, args, rec, mon, out)
    finally:
        rec["gpu_exclusivity"] = exclusive.summarize(mon.finish())
        out.write_text(json.dumps(rec, indent=1) + "\n")
    return rec


def _run_rows(batches, sizes, args, rec, mon, out):
    for b in batches:
        for s in sizes:
            before = exclusive.gpu_snapshot(0)
            t0 = time.time()
            row = run_row(b, s, args.rounds, args.samples, args.launches, args.mode, args.norm_style)
            exclusive.guarded(row, [before, *mon.between(t0, time.time()), exclusive.gpu_snapshot(0)])
            rec["rows"].append(row)
            out.write_text(json.dumps(rec, indent=1) + "\n")
            i, r = row["initial"], row["retest"]
            print(f"Qwen3-8B B={b} S={s} {row['status']} A1 {i['A1']['median_us']:.2f} us "
                  f"paired A1/A2 {i['paired_ratio_median']:.4f} [{i['paired_ratio_ci95'][0]:.4f}, "
                  f"{i['paired_ratio_ci95'][1]:.4f}] retest {r['paired_ratio_median']:.4f}", flush=True)
            gc.collect()
            torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
