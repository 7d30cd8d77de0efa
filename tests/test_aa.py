"""Host logic of the timing protocol and of the A/A noise-floor runner
(src/fusion_harness.py:32-79 and src/e7_rope_aa.py:116-191 in the reference),
on CPU: sample summaries, the bootstrap interval, the balanced arm order and
the bitwise output check."""
import math
import random
import statistics

import pytest
import torch

from kernelfuser_amd import aa, timing


def test_summary_known_values():
    s = timing.summary([4.0, 1.0, 3.0, 2.0])
    assert s["n"] == 4 and s["median_us"] == 2.5 and s["mean_us"] == 2.5
    # inclusive deciles of 1..4: positions 1 + 0.1*3 and 1 + 0.9*3
    assert math.isclose(s["p10_us"], 1.3) and math.isclose(s["p90_us"], 3.7)
    one = timing.summary([7.0])
    assert one["p10_us"] == one["p90_us"] == one["median_us"] == 7.0
    big = timing.summary(list(range(0, 101)))
    assert big["p10_us"] == 10.0 and big["p90_us"] == 90.0 and big["median_us"] == 50.0


@pytest.mark.parametrize("bad", [[], [1.0, float("nan")], [1.0, -0.5], [float("inf")]])
def test_summary_rejects_invalid_samples(bad):
    with pytest.raises(ValueError):
        timing.summary(bad)


def test_bootstrap_interval_brackets_median_and_is_seeded():
    rng = random.Random(3)
    vals = [1.0 + 0.01 * rng.gauss(0, 1) for _ in range(200)]
    lo, hi = timing.bootstrap_median_ci(vals, seed=11)
    assert lo <= statistics.median(vals) <= hi
    assert hi - lo < 0.01  # the median of 200 values with sd 0.01 is known to ~1e-3
    assert timing.bootstrap_median_ci(vals, seed=11) == [lo, hi]
    assert timing.bootstrap_median_ci([2.0] * 5, seed=1) == [2.0, 2.0]
    with pytest.raises(ValueError):
        timing.bootstrap_median_ci([], seed=1)


def test_latin_orders_balance_positions():
    names = ["a", "b", "c", "d"]
    orders = timing.latin_orders(names, 8, random.Random(5))
    assert all(sorted(o) == names for o in orders)
    for pos in range(4):
        counts = {n: sum(o[pos] == n for o in orders) for n in names}
        assert set(counts.values()) == {2}, counts  # 8 samples: every arm twice in every position
    # rotations of one permutation
    assert orders[1] == orders[0][1:] + orders[0][:1]


def test_bitwise_check():
    a = torch.randn(3, 5, dtype=torch.bfloat16)
    assert aa.bitwise(a, a.clone())["pass"]
    b = a.clone()
    b[1, 2] = b[1, 2] * 2 + 1
    r = aa.bitwise(a, b)
    assert not r["pass"] and r["finite"] and not r["bitwise_equal"] and r["max_abs"] > 0
    z, nz = torch.zeros(4), -torch.zeros(4)
    assert torch.equal(z, nz) and not aa.bitwise(z, nz)["pass"]  # -0.0 is a different bit pattern
    b[0, 0] = float("nan")
    r = aa.bitwise(a, b)
    assert not r["pass"] and not r["finite"] and r["max_abs"] is None


def test_cli_rejects_bad_protocol(tmp_path):
    with pytest.raises(SystemExit):
        aa.main(["--out", str(tmp_path / "x.json"), "--samples", "1"])
