"""Device timing of attention-prologue calls on one MI355X: HIP-graph blocks,
measured back to back in a balanced, interleaved order.

This is the timing protocol of every runner in the package (bench, A/A,
refinement, Qwen3 prefill).  The reference times its arms with randomised
graph blocks and fresh captures per round (src/fusion_harness.py:32-79); the
design here differs in how a sample is taken:

* A **block** is one HIP graph holding ``launches`` consecutive calls of an
  arm, captured on a private stream after eager warm-up calls on that stream
  (lazy allocations and library set-up happen outside the capture).  The
  arm's output of the last captured call is kept, so replays can be checked.
* A **sample** enqueues every arm's block back to back, with an event before
  the first block and after each one, and synchronises once.  A pacing kernel
  (``torch.cuda._sleep``) goes first, sized from the host's own enqueue time
  of the previous sample, so the host has queued the whole sample before the
  GPU reaches it: the interval between two events is then the block's device
  time only, never host latency.  Samples whose enqueue outran the pacing are
  flagged (``paced``) and reported.
* The arm order of sample j in a round is the round's random permutation
  rotated by j (a cyclic Latin square): over len(arms) consecutive samples
  every arm takes every position once, so what one arm leaves behind (clock
  state, caches) falls on every other arm equally.
* Every round captures fresh blocks, then (``settle_ms`` > 0) replays them
  until that much wall time of continuous load has passed before its first
  sample: the MI355X clock needs a few hundred ms of load to reach its
  steady state, and capture leaves the GPU idle.  The summary per arm is the median,
  10th/90th percentiles and mean of per-launch microseconds; for a named
  baseline arm, each other arm also gets the per-sample paired ratio
  (arm/baseline, both from the same sample) with its median and a seeded
  bootstrap 95% interval of that median.
"""
from __future__ import annotations

import math
import random
import statistics
import time
from typing import Callable, Dict, Optional

import torch

_SLEEP_CYCLES_PER_US: Optional[float] = None


def sleep_cycles_per_us() -> float:
    """Cycles of ``torch.cuda._sleep`` per microsecond on this device,
    measured once per process (a 2-ms spin, timed with events)."""
    global _SLEEP_CYCLES_PER_US
    if _SLEEP_CYCLES_PER_US is None:
        cycles = 4_000_000
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(cycles // 8)  # first call loads the kernel
        a.record()
        torch.cuda._sleep(cycles)
        b.record()
        b.synchronize()
        us = a.elapsed_time(b) * 1e3
        _SLEEP_CYCLES_PER_US = cycles / max(us, 1.0)
    return _SLEEP_CYCLES_PER_US


def pace(us: float) -> None:
    """Occupy the current stream for about ``us`` microseconds."""
    if us > 0:
        torch.cuda._sleep(int(us * sleep_cycles_per_us()))


class GraphBlock:
    """``launches`` consecutive calls ``fn(i)`` (i = 0 .. launches-1; ``fn()``
    when it takes no argument) captured into one HIP graph.  ``output`` is
    what the last captured call returned."""

    def __init__(self, fn: Callable, launches: int, warmups: int = 3):
        if launches < 1:
            raise ValueError("a graph block needs at least one launch")
        self.launches = launches
        call = _indexed(fn)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(warmups):
                call(i % launches)
            side.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            out = None
            with torch.cuda.graph(self.graph, stream=side):
                for i in range(launches):
                    out = call(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.output = out

    def replay(self) -> None:
        self.graph.replay()


def _indexed(fn: Callable) -> Callable[[int], object]:
    try:
        import inspect
        n = len([p for p in inspect.signature(fn).parameters.values()
                 if p.default is inspect.Parameter.empty and p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)])
    except (TypeError, ValueError):
        n = 0
    return fn if n >= 1 else (lambda i: fn())


def summary(us) -> dict:
    """Median, 10th/90th percentiles (inclusive method), mean and count of a
    list of microsecond samples; rejects empty, negative or non-finite input."""
    vals = [float(x) for x in us]
    if not vals:
        raise ValueError("no timing samples")
    if not all(math.isfinite(x) and x >= 0.0 for x in vals):
        raise ValueError(f"timing samples must be finite and non-negative: {vals!r}")
    if len(vals) == 1:
        p10 = p90 = vals[0]
    else:
        q = statistics.quantiles(vals, n=10, method="inclusive")
        p10, p90 = q[0], q[-1]
    return {"n": len(vals), "median_us": statistics.median(vals), "p10_us": p10, "p90_us": p90,
            "mean_us": statistics.fmean(vals), "samples_us": vals}


def bootstrap_median_ci(values, seed: int, resamples: int = 2000, level: float = 0.95):
    """Percentile-bootstrap interval of the median of ``values`` (seeded)."""
    vals = [float(x) for x in values]
    if not vals:
        raise ValueError("no values")
    rng = random.Random(seed)
    n = len(vals)
    meds = sorted(statistics.median(rng.choices(vals, k=n)) for _ in range(resamples))
    lo = meds[int(math.floor((1 - level) / 2 * (resamples - 1)))]
    hi = meds[int(math.ceil((1 + level) / 2 * (resamples - 1)))]
    return [lo, hi]


def latin_orders(names, samples: int, rng: random.Random):
    """Orders of one round: a random permutation rotated by the sample index."""
    base = list(names)
    rng.shuffle(base)
    k = len(base)
    return [base[j % k:] + base[:j % k] for j in range(samples)]


def interleaved(arms: Dict[str, Callable], *, rounds: int = 3, samples: int = 5, launches: int = 20,
                seed: int = 1701, baseline: Optional[str] = None, warmups: int = 3,
                check: Optional[Callable[[str, object], None]] = None, settle_ms: float = 0.0) -> dict:
    """Time every arm as described in the module docstring.  ``check(name,
    output)`` is called with each block's last output after every round's
    samples (e.g. to compare replays with an eager result); it raises to
    reject the run."""
    if not arms:
        raise ValueError("no arms to time")
    if rounds < 1 or samples < 1:
        raise ValueError("need at least one round and one sample")
    if baseline is not None and baseline not in arms:
        raise KeyError(baseline)
    rng = random.Random(seed)
    names = list(arms)
    per_arm = {n: [] for n in names}
    ratios = {n: [] for n in names if n != baseline} if baseline else {}
    orders, paced = [], []
    enqueue_us = 200.0
    for _ in range(rounds):
        capture_order = names[:]
        rng.shuffle(capture_order)
        blocks = {n: GraphBlock(arms[n], launches, warmups) for n in capture_order}
        t_settle = time.perf_counter()
        while True:  # one untimed replay each, repeated while the clock settles
            for blk in blocks.values():
                blk.replay()
            torch.cuda.synchronize()
            if (time.perf_counter() - t_settle) * 1e3 >= settle_ms:
                break
        for order in latin_orders(names, samples, rng):
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(len(order) + 1)]
            pre = torch.cuda.Event(enable_timing=True)
            pre.record()
            pace(1.5 * enqueue_us + 50.0)
            t0 = time.perf_counter()
            evs[0].record()
            for j, n in enumerate(order):
                blocks[n].replay()
                evs[j + 1].record()
            enqueue_us = (time.perf_counter() - t0) * 1e6
            evs[-1].synchronize()
            paced.append(pre.elapsed_time(evs[0]) * 1e3 >= enqueue_us)
            got = {n: evs[j].elapsed_time(evs[j + 1]) * 1e3 / launches for j, n in enumerate(order)}
            for n, v in got.items():
                per_arm[n].append(v)
            if baseline:
                for n in ratios:
                    ratios[n].append(got[n] / got[baseline])
            orders.append(order)
        if check is not None:
            for n, blk in blocks.items():
                check(n, blk.output)
        del blocks
    res = {"arms": {n: summary(v) for n, v in per_arm.items()},
           "protocol": {"rounds": rounds, "samples_per_round": samples, "launches_per_block": launches,
                        "seed": seed, "order": "cyclic Latin square of a random permutation per round",
                        "settle_ms_per_round": settle_ms,
                        "fresh_blocks_each_round": True, "orders": orders,
                        "paced_samples": sum(paced), "total_samples": len(paced)}}
    if baseline:
        res["baseline"] = baseline
        res["paired_ratio"] = {n: {"median": statistics.median(r), "ci95": bootstrap_median_ci(r, seed + i)}
                               for i, (n, r) in enumerate(ratios.items())}
    return res


def block_time_us(fn: Callable, launches: int, replays: int = 10, warmups: int = 3, settle_ms: float = 0.0) -> float:
    """Median per-launch device time (us) of ``launches`` calls of ``fn``
    replayed ``replays`` times as one block (one arm, one round), after
    ``settle_ms`` of untimed replays."""
    res = interleaved({"arm": fn}, rounds=1, samples=replays, launches=launches, warmups=warmups,
                      settle_ms=settle_ms)
    return res["arms"]["arm"]["median_us"]
