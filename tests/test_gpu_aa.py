"""A/A runner and the timing protocol on the GPU: both arms of
optimized_attention are bitwise equal to each other and to the eager call,
before timing and on every block's replay."""
import math

import pytest

from helpers import announce

pytestmark = pytest.mark.gpu


def test_aa_row_short(gpu):
    from kernelfuser_amd import aa
    announce("A/A B=1 S=128, 1 round x 4 samples x 5 launches")
    row = aa.run_row(1, 128, rounds=1, samples=4, launches=5)
    assert row["status"] == "tested_pass"
    for key in ("initial", "retest"):
        rec = row[key]
        assert rec["eager_check"]["pass"]
        kern = rec["eager_check"]["kernels"]
        assert [r["kernel"].split("<")[0] for r in kern["A1"]] == ["rows_kernel", "attn_fwd_kernel"]
        assert [r["kernel"] for r in kern["A1"]] == [r["kernel"] for r in kern["A2"]]
        assert len(rec["replay_checks"]) == 2 and all(c["pass"] for c in rec["replay_checks"])
        assert rec["A1"]["n"] == 4 and rec["A2"]["n"] == 4
        assert math.isfinite(rec["paired_ratio_median"]) and 0.5 < rec["paired_ratio_median"] < 2.0
        lo, hi = rec["paired_ratio_ci95"]
        assert lo <= rec["paired_ratio_median"] <= hi
        assert len(rec["orders"]) == 4


def test_interleaved_blocks_time_the_device(gpu):
    """A block of 20 launches is timed per launch, and a pacing kernel keeps
    host enqueue latency out of the intervals: a spin of known length reads
    back at that length."""
    import torch
    from kernelfuser_amd import timing
    announce("timing: paced spin arms")
    cyc = timing.sleep_cycles_per_us()
    assert cyc > 0
    arms = {"spin50": lambda: torch.cuda._sleep(int(50 * cyc)), "spin100": lambda: torch.cuda._sleep(int(100 * cyc))}
    res = timing.interleaved(arms, rounds=2, samples=4, launches=5, seed=3, baseline="spin50")
    m50, m100 = res["arms"]["spin50"]["median_us"], res["arms"]["spin100"]["median_us"]
    assert 40 < m50 < 70 and 85 < m100 < 130, (m50, m100)
    assert 1.6 < res["paired_ratio"]["spin100"]["median"] < 2.4
    assert res["protocol"]["paced_samples"] >= res["protocol"]["total_samples"] - 1
