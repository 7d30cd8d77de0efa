"""Timing harness: randomized paired HIP-graph timing of several arms.

Counterpart of the reference's shared harness (src/fusion_harness.py:32-79):
each round captures a fresh graph of ``replays`` launches per arm on a side
stream (after warmups), replays every graph a few times, then takes
``samples`` event-timed replays per arm in a freshly shuffled arm order;
results are per-launch microseconds (median, p10, p90, samples).  On ROCm
``torch.cuda.CUDAGraph`` records a hipGraph.
"""
from __future__ import annotations

import random
import statistics

import torch


def capture(fn, replays: int = 50, warmups: int = 10):
    """Graph of ``replays`` consecutive calls of ``fn`` captured on a side stream."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmups):
            fn()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(replays):
                fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    return graph


def paired(functions: dict, rounds: int = 5, samples: int = 10, replays: int = 50, seed: int = 1701) -> dict:
    """Randomized graph blocks, fresh captures each round, per-launch latency (us)."""
    if rounds < 1 or samples < 1 or replays < 1:
        raise ValueError("paired timing needs rounds, samples and replays >= 1")
    rng = random.Random(seed)
    values = {name: [] for name in functions}
    orders = []
    for _ in range(rounds):
        graphs = {name: capture(fn, replays) for name, fn in functions.items()}
        for graph in graphs.values():
            for _ in range(3):
                graph.replay()
        torch.cuda.synchronize()
        for _ in range(samples):
            order = list(functions)
            rng.shuffle(order)
            orders.append(order)
            for name in order:
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record()
                graphs[name].replay()
                end.record()
                end.synchronize()
                values[name].append(start.elapsed_time(end) * 1000.0 / replays)
        del graphs
    return {
        "arms": {name: {"median_us": statistics.median(t),
                        "p10_us": sorted(t)[max(0, int(len(t) * .1))],
                        "p90_us": sorted(t)[min(len(t) - 1, int(len(t) * .9))],
                        "samples_us": t} for name, t in values.items()},
        "protocol": {"rounds": rounds, "samples_per_round": samples, "graph_launches_per_sample": replays,
                     "arm_order": orders, "seed": seed, "fresh_graphs_each_round": True},
    }


def metric(candidate: torch.Tensor, reference: torch.Tensor, atol: float = .025, rtol: float = .025) -> dict:
    """Closeness of two tensors (src/fusion_harness.py:105-109)."""
    a = candidate.detach().float()
    b = reference.detach().float().to(a.device)
    delta = a - b
    return {"pass": bool(torch.allclose(a, b, atol=atol, rtol=rtol)),
            "max_abs": delta.abs().max().item(),
            "relative_l2": (delta.norm() / b.norm().clamp_min(1e-12)).item()}
