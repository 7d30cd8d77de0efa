"""Host logic of the tuning runner (kernelfuser_amd.tune): arm lists per
geometry, the launch-record checks and the decision rule, on synthetic
records (no GPU)."""
import pytest

from kernelfuser_amd import tune


def _rec(kernel, plan, grid=256):
    return {"kernel": kernel, "grid": grid, "block": 512, "registers": 128, "lds_bytes": 0, "scratch_bytes": 0,
            "plan": plan}


def test_arms_follow_geometry():
    q8 = tune.arm_specs("Qwen3-8B", 1000, True, True)  # G = 4, D = 128
    assert {"query/general", "query/pingpong-h1", "query/pingpong-h2", "query/pingpong-h2-vt",
            "query/pingpong-h2-once", "query/wide", "unfused/rows2", "unfused/rows4"} <= set(q8)
    assert not q8["query/pingpong"]["timed"]
    assert "query/pingpong-h2-vt" not in tune.arm_specs("Qwen3-8B", 1001, True, True)  # V^T needs S % 8 == 0
    assert "query/pingpong-h2-once" not in tune.arm_specs("Qwen3-8B", 1000, False, True)
    g4 = tune.arm_specs("Gemma-3-4B", 1024, True, False)  # D = 256
    assert set(g4) == {"query", "full", "unfused", "factored", "query/nosplit", "prepare"}
    assert set(tune.arm_specs("Gemma-3-4B", 1024, False, False)) == {"query", "full", "unfused", "factored", "prepare"}
    assert set(tune.arm_specs("Qwen3-8B", 512, False, True, True)) == {"prepare", "prepare/rows2", "prepare/rows4"}
    assert tune.SHAPES[0] == ("Qwen3-8B", 4, 1000, True, True)
    assert len(tune.REFERENCE_SHAPES) == 12  # rope:776
    assert all(r[-1] == "prepare" for r in tune.PREPARE_SHAPES) and len(tune.PREPARE_SHAPES) == 6
    assert all(r[-1] == "fp32" for r in tune.CONFIG_FP32_SHAPES) and len(tune.CONFIG_FP32_SHAPES) == 6


def test_dispatch_matches():
    rows = _rec("rows_kernel<128, 1, true, true, false, 2>", "hpw=2")
    pp2 = [rows, _rec("attn_pp_kernel<true, 2, 1, false>", "hpg=2 persistent=1 xcd=1")]
    assert tune.dispatch_matches(pp2, {"attention": ("attn_pp_kernel", {"hpg": "2"})})
    assert not tune.dispatch_matches(pp2, {"attention": ("attn_pp_kernel", {"hpg": "1"})})
    assert not tune.dispatch_matches(pp2, {"attention": ("attn_fwd_kernel", {})})
    assert not tune.dispatch_matches(pp2, {"attention_vt": True})
    vt = [rows, _rec("attn_pp_kernel<true, 2, 1, true>", "hpg=2 persistent=1 xcd=1")]
    assert tune.dispatch_matches(vt, {"attention_vt": True})
    assert tune.dispatch_matches(pp2, {"rows": ("rows_kernel", {"hpw": "2"})})
    assert not tune.dispatch_matches(pp2, {"rows": ("rows_kernel", {"hpw": "4"})})
    assert not tune.dispatch_matches([], {"attention": (None, {})})


def _row(sigs):
    return {"correctness": {n: {"pass": True, "kernels": [_rec(k, p)]} for n, (k, p) in sigs.items()}}


def _arms(times):
    return {"arms": {n: {"median_us": sorted(v)[len(v) // 2], "samples_us": v} for n, v in times.items()}}


def test_decide_rule():
    gen, pp1, pp2 = ("attn_fwd_kernel<>", "split=0"), ("attn_pp_kernel<>", "hpg=1"), ("attn_pp_kernel<>", "hpg=2")
    row = _row({"query": gen, "query/general": gen, "query/pingpong": pp2, "query/pingpong-h1": pp1,
                "query/pingpong-h2": pp2})
    # general is the by-shape choice and 20% slower than ping-pong h2 in every sample
    timed = _arms({"query": [12.0] * 5, "query/general": [12.0, 12.1, 11.9, 12.0, 12.2],
                   "query/pingpong-h1": [11.0] * 5, "query/pingpong-h2": [10.0, 10.1, 9.9, 10.0, 10.0]})
    dec = tune.decide(row, timed, 1)
    k = dec["attention_kernel"]
    assert k["by_shape"] == "query/general" and k["fastest"] == "query/pingpong-h2"
    assert k["verdict"] == "by_shape_slower" and k["by_shape_over_fastest"]["median"] == pytest.approx(1.2)
    assert dec["pp_heads"]["by_shape"] == "query/pingpong-h2" and dec["pp_heads"]["verdict"] == "kept"
    # within 1%: kept
    timed = _arms({"query": [10.05] * 5, "query/general": [10.05] * 5, "query/pingpong-h1": [11.0] * 5,
                   "query/pingpong-h2": [10.0] * 5})
    assert tune.decide(row, timed, 1)["attention_kernel"]["verdict"] == "kept"
    # options that ran the same launches are not a decision
    same = _row({"query": gen, "query/nosplit": gen})
    assert "split" not in tune.decide(same, _arms({"query": [1.0] * 3, "query/nosplit": [1.1] * 3}), 1)
