"""A/A runner on the GPU: both arms of optimized_attention are bitwise equal to
each other and to an eager call, before and after graph-replay timing."""
import math

import pytest

from helpers import announce

pytestmark = pytest.mark.gpu


def test_aa_row_short(gpu):
    from kernelfuser_amd import aa
    announce("A/A B=1 S=128, 1 round x 4 samples")
    row = aa.run_row(1, 128, rounds=1, samples=4)
    assert row["status"] == "tested_pass" and row["correctness"]["pass"]
    for key in ("initial", "retest"):
        rec = row[key]
        assert rec["fresh_graph_captures_per_arm"] == 1 and len(rec["rounds"]) == 1
        r0 = rec["rounds"][0]
        assert all(c["pass"] for c in r0["correctness_before"].values()) and r0["correctness_after"]["pass"]
        assert math.isfinite(rec["ratio"]) and 0.5 < rec["ratio"] < 2.0
        assert len(r0["arm_order"]) == 4
