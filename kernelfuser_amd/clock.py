"""Shader clock of the attention kernels against their input data.

The MFMA rate that bounds the attention kernels is the clock times the
matrix cores' work per cycle, and the GPU's power management sets the clock
from the power drawn, which depends on the operands the MFMAs toggle.  This
runner times the attention kernel of the fused path (K prepared once, Q's
norm and RoPE in the prologue) on the same shapes with three kinds of data,
and reads the shader clock of each launch from the kernels' per-workgroup
clock stamps (``kfmi_clock_stamps``):

  * ``random``: the synthetic inputs of bench.py (N(0,1) Q/K/V);
  * ``v_zero``: V all zero (GEMM2's V operand constant; scores unchanged);
  * ``k_zero``: the prepared K all zero (every score 0: GEMM1's K operand and
    GEMM2's probabilities constant).

The instruction stream is the same in all three, so the kernel's cycle
count (time x clock) stays put while the clock, and with it the time,
follows the data.  While the launches run back to back for a few seconds,
``amd-smi metric --power --clock`` is sampled from a child process (socket
power and the per-XCD gfx clocks; left out when amd-smi cannot be read), which
shows the board at its power limit.

``python -m kernelfuser_amd.clock --out clock.json`` runs Qwen3-8B heads,
causal, at B=1 S=4096 and S=8192 (ping-pong kernel) and B=1 S=2048 (general
kernel).  No counterpart in the reference.
"""
from __future__ import annotations

import argparse
import json
import statistics
import threading
import time

SHAPES = [(1, 4096), (1, 8192), (1, 2048)]
CASES = ("random", "v_zero", "k_zero")


def _smi_power_sample(index: int) -> tuple[float | None, list[float]]:
    """(socket power W, gfx clocks MHz per XCD) from one ``amd-smi metric``."""
    from . import exclusive as ex

    rc, out, _ = ex._run_smi(["metric", "-g", str(index), "--power", "--clock", "--json"], timeout=10)
    if rc != 0:
        return None, []
    try:
        doc = ex._json_payload(out)
    except ValueError:
        return None, []
    gpu = (doc.get("gpu_data") or [doc])[0] if isinstance(doc, dict) else doc[0]
    power = ex._as_int((gpu.get("power") or {}).get("socket_power"))
    clocks = [ex._as_int(v.get("clk")) for k, v in (gpu.get("clock") or {}).items()
              if k.startswith("gfx_") and isinstance(v, dict)]
    return (float(power) if power is not None else None), [float(c) for c in clocks if c is not None]


def power_while(fn, seconds: float = 3.0) -> dict | None:
    """Median socket power and gfx clock (amd-smi, sampled from a child process
    every ~50 ms) while ``fn`` runs back to back for ``seconds``; None when
    amd-smi cannot be read."""
    import torch

    from . import exclusive as ex

    try:
        rc, listing, _ = ex._run_smi(["list", "--json"])
        index = ex.smi_index(ex.device_bdf(torch.cuda.current_device()), listing) if rc == 0 else None
    except (ValueError, RuntimeError):
        index = None
    if index is None or _smi_power_sample(index)[0] is None:
        return None
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            samples.append(_smi_power_sample(index))
            time.sleep(0.05)

    th = threading.Thread(target=sampler)
    th.start()
    t0 = time.time()
    try:
        while time.time() - t0 < seconds:
            for _ in range(50):
                fn()
            torch.cuda.synchronize()
    finally:
        stop.set()
        th.join()
    watts = [w for w, _ in samples if w is not None]
    clks = [statistics.median(c) for _, c in samples if c]
    if not watts:
        return None
    return {"socket_w_median": statistics.median(watts), "socket_w_max": max(watts), "samples": len(watts),
            "gfx_mhz_median": statistics.median(clks) if clks else None}


def measure(b: int, s: int, case: str, *, launches: int = 20, replays: int = 10, settle_ms: float = 300.0,
            norm_style: str = "fp32", power: bool = True) -> dict:
    import torch

    from . import QWEN3_8B, _lib, attention_flops, attention_prefill, make_inputs, prepare_attention
    from .timing import block_time_us

    xs = make_inputs(b, s, QWEN3_8B, 1909).to("cuda:0")
    v = torch.zeros_like(xs.v) if case == "v_zero" else xs.v
    kn = torch.empty_like(xs.k)
    prepare_attention(xs.reference7, None, kn, only_k=True, norm_style=norm_style)
    if case == "k_zero":
        kn.zero_()
    out = torch.empty_like(xs.q)

    def fn():
        return attention_prefill(xs.q, kn, v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin, causal=True,
                                 norm_style=norm_style)

    fn()
    kernel = [r["kernel"] for r in _lib.last_launches() if r["kernel"].startswith("attn_")][0]
    us = block_time_us(fn, launches, replays=replays, settle_ms=settle_ms)
    with _lib.tuning(clock_stamps=1):
        for _ in range(200):
            fn()
    clk = _lib.clock_summary(_lib.clock_stamps())
    pw = power_while(fn) if power else None
    f = attention_flops(b, QWEN3_8B[0], s, QWEN3_8B[2], True)
    ghz = clk["ghz_median"]
    return {"B": b, "S": s, "case": case, "kernel": kernel, "us": us, "tflops": f / (us * 1e-6) / 1e12,
            "clock": clk, "power": pw, "kcycles": us * ghz, "frac_mfma": f / (us * 1e-6) / 1e12 / 2500.0,
            "frac_mfma_at_clock": f / (us * 1e-6) / 1e12 / (2500.0 * ghz / 2.4)}


def table(rows: list[dict]) -> str:
    out = ["| B | S | kernel | data | kernel us | shader clock GHz (median, min-max) | kcycles (us x GHz) | "
           "TFLOP/s | of 2.5 PFLOP/s | of the peak at that clock | socket power W (amd-smi median) |",
           "|" + "---|" * 11]
    for r in rows:
        c, pw = r["clock"], r.get("power")
        w = "n/a" if not pw else f"{pw['socket_w_median']:.0f}"
        out.append(f"| {r['B']} | {r['S']} | `{r['kernel'].split('(')[0]}` | {r['case']} | {r['us']:.1f} | "
                   f"{c['ghz_median']:.3f} ({c['ghz_min']:.3f}-{c['ghz_max']:.3f}) | {r['kcycles']:.0f} | "
                   f"{r['tflops']:.0f} | {r['frac_mfma']:.3f} | {r['frac_mfma_at_clock']:.3f} | {w} |")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", default=None)
    ap.add_argument("--shapes", default=",".join(f"{b}x{s}" for b, s in SHAPES), help="BxS,BxS,...")
    ap.add_argument("--cases", default=",".join(CASES))
    ap.add_argument("--no-power", action="store_true", help="skip the amd-smi power sampling")
    args = ap.parse_args(argv)
    rows = []
    for spec in args.shapes.split(","):
        b, s = (int(x) for x in spec.split("x"))
        for case in args.cases.split(","):
            r = measure(b, s, case, power=not args.no_power)
            print(json.dumps(r), flush=True)
            rows.append(r)
    print(table(rows), flush=True)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(rows, f, indent=1)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
