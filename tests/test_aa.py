"""Host logic of the A/A noise-floor runner (src/e7_rope_aa.py:116-191 in the
reference): the sample statistics and the bitwise output check, on CPU."""
import math

import pytest
import torch

from kernelfuser_amd import aa


def test_stats_known_values():
    s = aa.stats([1.0, 2.0, 3.0, 4.0])
    assert s["n"] == 4 and s["mean_ms"] == 2.5 and s["p50_ms"] == 2.5
    assert math.isclose(s["sem_ms"], math.sqrt(5 / 3) / 2)  # stdev (n-1) / sqrt(n)
    assert math.isclose(s["two_sem_ms"], 2 * s["sem_ms"])
    assert s["p95_ms"] == 4.0  # ceil(.95 * 4) - 1 = index 3
    assert aa.stats([5.0])["sem_ms"] == 0.0
    p = aa.stats(list(range(1, 101)))
    assert p["p95_ms"] == 95.0


@pytest.mark.parametrize("bad", [[], [1.0, float("nan")], [1.0, -0.5], [float("inf")]])
def test_stats_rejects_invalid_samples(bad):
    with pytest.raises(ValueError):
        aa.stats(bad)


def test_exact_check():
    a = torch.randn(3, 5)
    assert aa.exact_check(a, a.clone())["pass"]
    b = a.clone()
    b[1, 2] += 1e-6
    r = aa.exact_check(a, b)
    assert not r["pass"] and r["finite"] and not r["exact_output_equal"] and r["max_abs"] > 0
    b[0, 0] = float("nan")
    r = aa.exact_check(a, b)
    assert not r["pass"] and not r["finite"] and r["max_abs"] is None


def test_cli_rejects_bad_protocol(tmp_path):
    with pytest.raises(SystemExit):
        aa.main(["--out", str(tmp_path / "x.json"), "--samples", "1"])
