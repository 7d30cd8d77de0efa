"""Tuning runner: the dispatch alternatives of this library, each gated and
timed beside the shape-based choice on one MI355X.

Counterpart of the reference's ``tune_refinement``
(src/e1_rope_publication_v1.py:765-814).  The reference sweeps eleven Triton
tile specifications (mode, BM, BN, warps, stages, gather) over twelve shapes
(rope:776), gates every arm against its FP32 oracle, keeps each arm's
compiler evidence and times the passing arms with its paired protocol
(3 rounds x 5 samples x 20 replays, seed 32109).  This library has no free
tile arguments -- each kernel is one fixed gfx950 design -- so what is swept
is the choice the library makes by shape, forced per arm through the
calling thread's overrides (``kfmi_set_tuning``):

* attention kernel at D = 128 (``query/general``, ``query/pingpong-h1``,
  ``query/pingpong-h2``, ``query/wide``); by shape: ping-pong when the GQA
  ratio is even, there are at least 16 query blocks of 128 rows, and either
  its items fill whole rounds of CUs (non-causal: a multiple of the CU
  count; causal: the persistent pairing applies) or, causal, there are at
  least 24 blocks; else general;
* query heads per ping-pong wave group (``-h1``: two heads x 128 rows per
  item, ``-h2``: four heads x 64 rows); by shape: 2 when the ratio is a
  multiple of 4;
* the V^T operand of the ping-pong kernel (``query/pingpong-h2-vt``: the
  preparation launch also writes V transposed); the caller's choice;
* the persistent long/short pairing of causal ping-pong items
  (``query/pingpong-h2-once``: one item per workgroup); by shape: when the
  pairs fill every CU equally;
* splitting the longest query blocks' key ranges in two at D = 256, causal
  (``query/nosplit``); by shape: ``plan_split``, when the unsplit grid has
  fewer workgroups than CUs (the factored entry point takes no workspace
  and never splits);
* heads per workgroup of the Q+K preparation kernel, timed on the
  preparation alone (``prepare/rows2``, ``prepare/rows4``: the isolated
  norm+RoPE workload) and inside mode ``unfused`` (``unfused/rows2``,
  ``unfused/rows4``); by shape, with R = B(Hq+Hkv)S rows: 4 for the FP32
  style when R >= 2^18 and S <= 4096, for the HF and legacy styles when
  2^15 <= R < 2^17.

Per row: every arm is gated against ``refine.reference_fp32`` with the
reference gate and records the kernels it launched (instance, grid, block,
registers, LDS, scratch and the launch-time ``plan``); an arm whose records
do not show the kernel and plan it forced is ``dispatch_mismatch`` and is not
timed.  The passing arms are timed together with ``timing.interleaved``
(3 rounds x 5 samples x 20 launches, seed 32109, the shape-based ``query``
arm as the paired baseline).  Each decision then names the fastest option,
the option the shape-based dispatch took (the one whose kernels and plan
equal the by-shape arm's) and the per-sample paired ratio by-shape / fastest
with its bootstrap 95% interval; the by-shape choice is ``kept`` when it is
the fastest or when that interval reaches 1.0 or its median is within 1%.

``python -m kernelfuser_amd.refine --grid tune --out tune.json`` runs the
reference's twelve shapes plus this build's configurations (B=4 S=1000 first;
in the refinement inputs' rounding style and again in the FP32 style that
bench.py times) and shapes beside the ping-pong and split thresholds; the
norm+RoPE sweep's six shapes then run the preparation arms only.
"""
from __future__ import annotations

import gc
import statistics
import time

import torch

from . import _lib, exclusive, timing
from .ops import MODELS, launch_attention, launch_factored_attention, prepare_attention
from .refine import SEEDS, _norm, _rope, gate, reference_fp32, refinement_inputs

# rope:776, in the reference's order
REFERENCE_SHAPES = [
    ("Qwen3-8B", 1, 128, False, True), ("Qwen3-8B", 32, 128, True, True), ("Qwen3-8B", 8, 256, False, True),
    ("Qwen3-8B", 1, 512, False, True), ("Qwen3-8B", 8, 512, False, True), ("Qwen3-8B", 32, 512, True, True),
    ("Qwen3-8B", 1, 1024, False, False), ("Qwen3-8B", 1, 1024, True, False), ("Gemma-3-4B", 1, 1024, False, False),
    ("Gemma-3-4B", 1, 1024, True, False), ("Qwen3-32B", 1, 2048, False, False), ("Gemma-3-12B", 1, 2048, True, False)]
# the measured configurations
CONFIG_SHAPES = [
    ("Qwen3-8B", 4, 1000, True, True), ("Qwen3-8B", 1, 2048, True, True), ("Qwen3-8B", 1, 4096, True, True),
    ("Qwen3-8B", 1, 8192, True, True), ("Gemma-3-12B", 2, 2048, True, False)]
# beside the thresholds: the ping-pong one (causal and not) and the split
# plans of D = 256 with one and with two rounds of workgroups
THRESHOLD_SHAPES = [
    ("Qwen3-8B", 1, 3072, True, True), ("Qwen3-8B", 1, 2048, False, True), ("Qwen3-8B", 1, 3072, False, True),
    ("Qwen3-32B", 1, 2048, True, False), ("Gemma-3-4B", 1, 2048, True, False), ("Gemma-3-12B", 1, 1024, True, False),
    ("Gemma-3-12B", 1, 1536, True, False)]
# the isolated norm+RoPE sweep (Qwen3-8B heads, FP32 style as the bench's
# sweep; the causal flag is unused): preparation arms only
PREPARE_SHAPES = [("Qwen3-8B", b, s, False, True, "prepare") for b, s in
                  ((1, 512), (1, 2048), (1, 8192), (4, 2048), (8, 1024), (16, 512))]
# the configurations again in the FP32 rounding style that bench.py times,
# and causal grids of 8-15 query blocks that the persistent pairing fills
CONFIG_FP32_SHAPES = [r + ("fp32",) for r in CONFIG_SHAPES] + [("Qwen3-8B", 1, 3072, True, True, "fp32")]
PAIRING_SHAPES = [("Qwen3-8B", b, s, True, True, st) for b, s in ((8, 1024), (4, 1536), (16, 1024))
                  for st in ("fp32", "hf")]
SHAPES = CONFIG_SHAPES + CONFIG_FP32_SHAPES + THRESHOLD_SHAPES + PAIRING_SHAPES + REFERENCE_SHAPES + PREPARE_SHAPES
TUNE_SEED = 32109  # rope:808

# decision -> option arms (each option arm forces one alternative)
DECISIONS = {
    "attention_kernel": ("query/general", "query/pingpong-h1", "query/pingpong-h2", "query/wide"),
    "pp_heads": ("query/pingpong-h1", "query/pingpong-h2"),
    "v_transposed": ("query/pingpong-h2", "query/pingpong-h2-vt"),
    "persistent": ("query/pingpong-h2", "query/pingpong-h2-once"),
    "split": ("query", "query/nosplit"),
    "rows_heads": ("prepare/rows2", "prepare/rows4"),
    "rows_heads_unfused": ("unfused/rows2", "unfused/rows4"),
}


def _plan(rec) -> dict:
    return dict(kv.split("=", 1) for kv in rec.get("plan", "").split() if "=" in kv)


def _base(rec) -> str:
    return rec["kernel"].split("<")[0]


def _attention_record(launches):
    recs = [r for r in launches if r["kernel"].startswith("attn_")]
    return recs[-1] if recs else None


def _rows_record(launches):
    recs = [r for r in launches if r["kernel"].startswith("rows_kernel")]
    return recs[-1] if recs else None


def _spec(mode, tuning=None, vt=False, attention=None, rows=None, timed=True):
    expect = {}
    if attention:
        expect["attention"] = attention
    if rows:
        expect["rows"] = rows
    return {"mode": mode, "tuning": tuning or {}, "vt": vt, "expect": expect, "timed": timed}


def arm_specs(model: str, s: int, causal: bool, rotary: bool, prepare_only: bool = False) -> dict:
    """name -> arm: mode, overrides, whether V^T is passed, the kernel (base
    name or None) and plan entries its launch records must show per role
    ("attention", "rows"), and whether it is timed (``query/pingpong``, the
    ping-pong kernel with its own choices left to the shape, is only run for
    its launch records: the by-shape side of the ping-pong decisions)."""
    hq, hkv, d = MODELS[model]
    g = hq // hkv
    prep = {"prepare": _spec("prepare")}
    if d == 128:
        prep["prepare/rows2"] = _spec("prepare", {"rows_heads": 2}, rows=("rows_kernel", {"hpw": "2"}))
        prep["prepare/rows4"] = _spec("prepare", {"rows_heads": 4}, rows=("rows_kernel", {"hpw": "4"}))
    if prepare_only:
        return prep
    specs = {"query": _spec("query"), "full": _spec("full"), "unfused": _spec("unfused"), **prep}
    if not rotary:
        specs["factored"] = _spec("factored")
    if d == 128:
        specs["query/general"] = _spec("query", {"attn_kernel": "general"}, attention=("attn_fwd_kernel", {}))
        if g % 2 == 0:
            specs["query/pingpong"] = _spec("query", {"attn_kernel": "pingpong"},
                                            attention=("attn_pp_kernel", {}), timed=False)
            specs["query/pingpong-h1"] = _spec("query", {"attn_kernel": "pingpong", "pp_heads": 1},
                                               attention=("attn_pp_kernel", {"hpg": "1"}))
        if g % 4 == 0:
            pp2 = {"attn_kernel": "pingpong", "pp_heads": 2}
            specs["query/pingpong-h2"] = _spec("query", pp2, attention=("attn_pp_kernel", {"hpg": "2"}))
            if s % 8 == 0:  # V^T rows must be 16-byte aligned
                specs["query/pingpong-h2-vt"] = _spec("query", pp2, vt=True, attention=("attn_pp_kernel", {"hpg": "2"}))
                specs["query/pingpong-h2-vt"]["expect"]["attention_vt"] = True
            if causal:
                specs["query/pingpong-h2-once"] = _spec("query", {**pp2, "persistent": 1},
                                                        attention=("attn_pp_kernel", {"hpg": "2", "persistent": "0"}))
            specs["query/wide"] = _spec("query", {"attn_kernel": "wide"}, attention=("attn_ww_kernel", {}))
        specs["unfused/rows2"] = _spec("unfused", {"rows_heads": 2}, rows=("rows_kernel", {"hpw": "2"}))
        specs["unfused/rows4"] = _spec("unfused", {"rows_heads": 4}, rows=("rows_kernel", {"hpw": "4"}))
    elif causal:
        specs["query/nosplit"] = _spec("query", {"split": 1}, attention=("attn_fwd_kernel", {"split": "0"}))
    return specs


def build_tuning_arms(xs, specs: dict, causal: bool, rotary: bool, style: str | None = None) -> dict:
    """name -> callable returning the arm's output; every call runs under the
    arm's overrides (also while a timing block captures it).  ``style``
    defaults to refine.build_arms' choice (hf with RoPE, legacy without;
    rope:849, :856)."""
    q, k, v, gq, gk, cos, sin = xs
    style = style or ("hf" if rotary else "legacy")
    arms = {}
    for name, sp in specs.items():
        mode, tun, use_vt = sp["mode"], sp["tuning"], sp["vt"]
        out = torch.empty_like(q)
        if mode == "prepare":  # Q and K rows into one buffer (the output compared)
            qk = torch.empty(q.numel() + k.numel(), dtype=q.dtype, device=q.device)
            qn, kn = qk[:q.numel()].view_as(q), qk[q.numel():].view_as(k)

            def call(qk=qk, qn=qn, kn=kn, tun=tun):
                with _lib.tuning(**tun):
                    prepare_attention(xs, qn, kn, rope=rotary, norm_style=style)
                return qk
        elif mode == "factored":
            kn = torch.empty_like(k)
            inv = torch.empty(q.shape[:-1], device=q.device, dtype=torch.float32)

            def call(out=out, kn=kn, inv=inv, tun=tun):
                with _lib.tuning(**tun):
                    launch_factored_attention((q, k, v, gq, gk), out, inv, kn, causal=causal)
                return out
        else:
            qn = torch.empty_like(q) if mode == "unfused" else None
            kn = torch.empty_like(k) if mode != "full" else None
            vt = torch.empty_like(v) if use_vt else None

            def call(out=out, qn=qn, kn=kn, vt=vt, mode=mode, tun=tun):
                with _lib.tuning(**tun):
                    launch_attention(xs, out, causal=causal, mode=mode, rope=rotary, qn=qn, kn=kn, vt=vt,
                                     norm_style=style)
                return out
        arms[name] = call
    return arms


def dispatch_matches(launches, expect: dict) -> bool:
    """Whether the launch records show the kernel and plan an arm forced."""
    for role, want in expect.items():
        if role == "attention_vt":  # the kernel instance that reads V^T
            rec = _attention_record(launches)
            if rec is None or not rec["kernel"].endswith(", true>"):
                return False
            continue
        kernel, plan = want
        rec = _attention_record(launches) if role == "attention" else _rows_record(launches)
        if rec is None or (kernel and _base(rec) != kernel):
            return False
        got = _plan(rec)
        if any(got.get(k_) != v_ for k_, v_ in plan.items()):
            return False
    return True


def signature(launches) -> tuple:
    """Kernels and plans of one arm's launches: equal signatures ran the same
    dispatch."""
    return tuple((r["kernel"], r["grid"], r.get("plan", "")) for r in launches)


def _paired(samples_a, samples_b, seed: int) -> dict:
    r = [a / b for a, b in zip(samples_a, samples_b)]
    return {"median": statistics.median(r), "ci95": timing.bootstrap_median_ci(r, seed)}


def decide(row: dict, timed: dict, seed: int) -> dict:
    """Per decision: options timed, the fastest, the by-shape option and the
    paired ratio by-shape / fastest."""
    arms, checks = timed["arms"], row["correctness"]
    sig = {n: signature(c["kernels"]) for n, c in checks.items() if c.get("pass")}
    out = {}
    for i, (dec, options) in enumerate(DECISIONS.items()):
        opts = [o for o in options if o in arms]
        if len(opts) < 2:
            continue
        by = {"rows_heads": "prepare", "rows_heads_unfused": "unfused", "pp_heads": "query/pingpong",
              "persistent": "query/pingpong"}.get(dec, "query")
        if len({sig.get(o) for o in opts}) == 1:
            continue  # the alternatives ran the same launches (no split or pairing at this shape)
        if dec == "v_transposed":
            by_shape = "query/pingpong-h2"  # the caller's choice; ops.launch_attention's default is no V^T
        else:
            same = [o for o in opts if sig.get(o) == sig.get(by)]
            by_shape = same[0] if same else None
        med = {o: arms[o]["median_us"] for o in opts}
        best = min(opts, key=med.get)
        rec = {"options_median_us": med, "fastest": best, "by_shape": by_shape}
        if by_shape is None:
            rec["verdict"] = "by_shape_not_among_options"
        elif by_shape == best:
            rec["verdict"] = "kept"
            rec["by_shape_over_fastest"] = {"median": 1.0, "ci95": [1.0, 1.0]}
        else:
            pr = _paired(arms[by_shape]["samples_us"], arms[best]["samples_us"], seed + i)
            rec["by_shape_over_fastest"] = pr
            rec["verdict"] = "kept" if pr["ci95"][0] <= 1.0 or pr["median"] <= 1.01 else "by_shape_slower"
        out[dec] = rec
    return out


def prepared_fp32(xs, rotary: bool) -> torch.Tensor:
    """FP32 RMSNorm*gamma (+ RoPE) of the Q rows, then the K rows, flattened
    (the layout of a preparation arm's output)."""
    q, k, _, gq, gk, cos, sin = xs
    qn, kn = _norm(q, gq), _norm(k, gk)
    if rotary:
        qn, kn = _rope(qn, cos, sin), _rope(kn, cos, sin)
    return torch.cat([qn.flatten(), kn.flatten()])


def tune_row(model: str, b: int, s: int, causal: bool, rotary: bool, prepare_only: bool = False, *, rounds=3,
             samples=5, launches=20, settle_ms: float = 150.0, style: str | None = None, device="cuda:0") -> dict:
    """One shape: gate and evidence for every arm, interleaved timing,
    decisions.  ``prepare_only``: the preparation arms alone, in the FP32
    style of the isolated norm+RoPE workload.  ``style``: the rounding style
    of every arm (default: refine.build_arms' choice)."""
    xs = refinement_inputs(model, b, s, SEEDS[0], rotary, device)
    ref = None if prepare_only else reference_fp32(xs, causal, rotary)
    ref_prep = prepared_fp32(xs, rotary)
    specs = arm_specs(model, s, causal, rotary, prepare_only)
    style = "fp32" if prepare_only else style
    arms = build_tuning_arms(xs, specs, causal, rotary, style)
    checks = {}
    for name, call in list(arms.items()):
        try:
            with _lib.record_launches() as rec:
                out = call()
            torch.cuda.synchronize()
            want = ref_prep if specs[name]["mode"] == "prepare" else ref
            checks[name] = {**gate(out, want), "kernels": rec.launches}
            if not rec.launches:
                checks[name]["pass"] = False
                checks[name]["error"] = "no kernel of this library launched"
            elif not dispatch_matches(rec.launches, specs[name]["expect"]):
                checks[name]["pass"] = False
                checks[name]["error"] = "dispatch_mismatch"
        except Exception as exc:  # an override this shape cannot run
            checks[name] = {"pass": False, "error": repr(exc)}
        if not checks[name]["pass"]:
            del arms[name]
    del ref, ref_prep
    row = {"model": model, "shape": [b, s, causal], "rotary": rotary, "geometry": list(MODELS[model]),
           "prepare_only": prepare_only, "style": style or ("hf" if rotary else "legacy"), "correctness": checks}
    if any(not c["pass"] for c in checks.values()):
        row["status"] = "failed_gate"  # every alternative offered here must run and pass
        return row
    arms = {n: a for n, a in arms.items() if specs[n]["timed"]}
    eager = {n: arms[n]().clone() for n in arms}

    def replay_check(name, out):
        if not torch.equal(out, eager[name]):
            raise RuntimeError(f"{model} {b}x{s}: graph replay of {name} differs from its eager output")

    timed = timing.interleaved(arms, rounds=rounds, samples=samples, launches=launches, seed=TUNE_SEED,
                               baseline="prepare" if prepare_only else "query", check=replay_check,
                               settle_ms=settle_ms)
    row["timing"] = {**timed, "protocol": {k: v for k, v in timed["protocol"].items() if k != "orders"}}
    row["decisions"] = decide(row, timed, TUNE_SEED)
    row["status"] = "passed"
    return row


def run(rows, *, launches: int = 20, rounds: int = 3, samples: int = 5, save=None) -> dict:
    """The tuning grid (``refine --grid tune``): one record with a row per
    shape, GPU exclusivity observed throughout."""
    rec = {"schema": "kernelfuser-amd-tune-v1",
           "created_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
           "environment": {"gpu": torch.cuda.get_device_name(0), "torch": torch.__version__,
                           "hip": torch.version.hip},
           "protocol": {"rounds": rounds, "samples": samples, "launches_per_block": launches, "seed": TUNE_SEED,
                        "baseline": "query (shape-based dispatch)",
                        "gate": "finite, allclose(atol=rtol=0.025), relative L2 <= 0.025 vs FP32; "
                                "launch records must show the forced kernel and plan"},
           "rows": []}
    torch.zeros(1, device="cuda:0")  # hold a context, so the GPU's process list must name this process
    rec["gpu_before"] = exclusive.gpu_snapshot(0)
    mon = exclusive.ExclusiveMonitor(0).start()
    try:
        with torch.inference_mode():
            for model, b, s, causal, rotary, *kind in rows:
                t0 = time.time()
                row = tune_row(model, b, s, causal, rotary, kind == ["prepare"], rounds=rounds, samples=samples,
                               launches=launches, style=kind[0] if kind and kind[0] in ("fp32", "hf", "legacy") else None)
                exclusive.guarded(row, mon.between(t0, time.time()))
                rec["rows"].append(row)
                if save:
                    save(rec)
                print(f"{len(rec['rows'])} {model} B={b} S={s} causal={causal} rope={rotary} {row['status']} "
                      + " ".join(f"{d}:{v['verdict']}({v['by_shape']}->{v['fastest']})"
                                 for d, v in row.get("decisions", {}).items()), flush=True)
                gc.collect()
                torch.cuda.empty_cache()
    finally:
        obs = mon.finish()
        rec["gpu_after"] = exclusive.gpu_snapshot(0)
        rec["gpu_exclusivity"] = exclusive.summarize([rec["gpu_before"], *obs, rec["gpu_after"]])
    bad = [r for r in rec["rows"] if r["status"] != "passed"]
    rec["status"] = "passed" if not bad else "failed"
    rec["decisions_needing_change"] = [
        {"row": [r["model"], *r["shape"], r["rotary"]], "decision": d, **v}
        for r in rec["rows"] for d, v in r.get("decisions", {}).items() if v["verdict"] != "kept"]
    if save:
        save(rec)
    return rec
