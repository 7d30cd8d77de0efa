"""Tuning runner on the GPU (one short row per kind): every forced
alternative runs, passes the FP32 gate and shows the kernel and plan it
forced in its launch records; the decisions name a fastest option and the
by-shape one (src/e1_rope_publication_v1.py:765-814)."""
import pytest

from helpers import announce

pytestmark = pytest.mark.gpu


def _check_row(row):
    assert row["status"] == "passed", {n: c.get("error", c.get("relative_l2")) for n, c in row["correctness"].items()}
    assert all(c["pass"] and c["kernels"] for c in row["correctness"].values())
    for dec, d in row["decisions"].items():
        assert d["fastest"] in d["options_median_us"], dec
        assert d["verdict"] in ("kept", "by_shape_slower"), (dec, d)
        assert d["by_shape_over_fastest"]["median"] >= 1.0 or d["by_shape"] != d["fastest"]


def test_tune_row_b4_s1000(gpu):
    """The ping-pong threshold's first shape: general (by shape), ping-pong
    with two and four heads per item, V^T, one item per workgroup, wide;
    rows kernel with 2 and 4 heads per workgroup."""
    from kernelfuser_amd import tune
    announce("tune row Qwen3-8B B=4 S=1000 causal rope")
    row = tune.tune_row("Qwen3-8B", 4, 1000, True, True, rounds=1, samples=2, launches=3, settle_ms=0.0)
    _check_row(row)
    ker = {n: [r["kernel"].split("<")[0] for r in c["kernels"]] for n, c in row["correctness"].items()}
    assert ker["query/general"][-1] == "attn_fwd_kernel" and ker["query/wide"][-1] == "attn_ww_kernel"
    assert ker["query/pingpong-h1"][-1] == ker["query/pingpong-h2"][-1] == "attn_pp_kernel"
    assert {"attention_kernel", "pp_heads", "v_transposed", "rows_heads", "rows_heads_unfused"} <= set(row["decisions"])
    assert row["decisions"]["pp_heads"]["by_shape"] == "query/pingpong-h2"  # GQA ratio 4


def test_tune_row_split_d256(gpu):
    """D = 256, causal: the split key ranges of the longest query blocks
    against one workgroup per block, in modes query and factored."""
    from kernelfuser_amd import tune
    announce("tune row Gemma-3-4B B=1 S=1024 causal no-rope")
    row = tune.tune_row("Gemma-3-4B", 1, 1024, True, False, rounds=1, samples=2, launches=3, settle_ms=0.0)
    _check_row(row)
    plans = {n: [r["plan"] for r in c["kernels"] if r["kernel"].startswith("attn_")][-1]
             for n, c in row["correctness"].items() if n != "prepare"}
    assert plans["query/nosplit"].startswith("split=0") and not plans["query"].startswith("split=0")
    assert row["decisions"]["split"]["by_shape"] == "query"


def test_tune_row_prepare_only(gpu):
    """The isolated norm+RoPE workload: two and four heads per workgroup of
    the preparation kernel, gated against FP32 RMSNorm + RoPE."""
    from kernelfuser_amd import tune
    announce("tune prepare row Qwen3-8B B=16 S=512")
    row = tune.tune_row("Qwen3-8B", 16, 512, False, True, True, rounds=1, samples=2, launches=3, settle_ms=0.0)
    _check_row(row)
    assert set(row["correctness"]) == {"prepare", "prepare/rows2", "prepare/rows4"}
    assert row["decisions"]["rows_heads"]["by_shape"] == "prepare/rows4"  # 2^18 rows or more, S <= 4096
