"""Both sides of every correctness gate (oracle/gates.py).

The GPU parity tests are only as strong as the gates they call, so each gate
is fed cases that must fail, built so that exactly one criterion is violated
(a threshold typo such as 2e-1 for 2e-2 makes the matching case pass and the
test fail), and cases just inside each threshold that must pass.

Gates: the reference metric (src/e1_rope_publication_v1.py:287-293: finite,
allclose atol=rtol=.025, relative-L2 <= .025); attention max-abs <= 2e-2;
norm+RoPE max-abs <= 1.6e-2 and mean-abs <= 2e-3.
"""
import pytest
import torch

import oracle


def _ref(n=4096, seed=0):
    return torch.randn(n, generator=torch.Generator().manual_seed(seed)).clamp(-3, 3)


def _with_spike(ref, delta, at=17):
    x = ref.clone()
    x[at] += delta
    return x


def test_metric_passes_identical_and_near_thresholds():
    r = _ref()
    assert oracle.metric(r.clone(), r)["pass"]
    # one element off by 0.024 (< atol): allclose holds, relative-L2 tiny
    assert oracle.metric(_with_spike(r, 0.024), r)["pass"]
    # uniform 2.4% relative error: allclose (|b| <= 3) and relative-L2 0.024
    m = oracle.metric(r * 1.024, r)
    assert m["pass"] and abs(m["relative_l2"] - 0.024) < 1e-4, m


@pytest.mark.parametrize("gate", [oracle.metric, oracle.attention_gate, oracle.norm_rope_gate])
def test_every_gate_fails_on_nan_and_inf(gate):
    r = _ref()
    for bad in (float("nan"), float("inf"), -float("inf")):
        x = r.clone()
        x[5] = bad
        m = gate(x, r)
        assert not m["finite"] and not m["pass"], (bad, m)


@pytest.mark.parametrize("gate", [oracle.metric, oracle.attention_gate, oracle.norm_rope_gate])
def test_every_gate_fails_on_relative_l2(gate):
    """3% uniform relative error: allclose holds for |b| <= 5 (0.03|b| <=
    0.025 + 0.025|b|); on a reference scaled to |b| <= 0.15 the largest error
    is 0.0045 and the mean 0.0012, inside every max-abs and mean-abs gate, so
    only the relative-L2 criterion (0.03 > 0.025) fails."""
    r = _ref() * 0.05
    x = r * 1.03
    m = gate(x, r)
    assert torch.allclose(x, r, atol=.025, rtol=.025)
    assert m["max_abs"] < 1.6e-2 and m["mean_abs"] < 2e-3
    assert abs(m["relative_l2"] - 0.03) < 1e-4
    assert not m["pass"], m


@pytest.mark.parametrize("gate", [oracle.metric, oracle.attention_gate, oracle.norm_rope_gate])
def test_every_gate_fails_on_allclose_miss(gate):
    """One element of a near-zero reference off by 0.1: allclose fails
    (0.1 > 0.025 + 0.025|b|) while relative-L2 stays far below 0.025."""
    r = _ref()
    r[17] = 0.0
    x = _with_spike(r, 0.1)
    m = gate(x, r)
    assert m["relative_l2"] < 0.01
    assert not torch.allclose(x, r, atol=.025, rtol=.025)
    assert not m["pass"], m


def test_attention_gate_max_abs_threshold():
    r = _ref()
    near = oracle.attention_gate(_with_spike(r, 0.019), r)
    assert near["pass"], near
    # 0.021: inside allclose (atol .025) and relative-L2, outside max-abs 2e-2
    over = oracle.attention_gate(_with_spike(r, 0.021), r)
    assert oracle.metric(_with_spike(r, 0.021), r)["pass"]
    assert abs(over["max_abs"] - 0.021) < 1e-6 and not over["pass"], over


def test_norm_rope_gate_max_abs_threshold():
    r = _ref()
    assert oracle.norm_rope_gate(_with_spike(r, 0.015), r)["pass"]
    over = oracle.norm_rope_gate(_with_spike(r, 0.017), r)
    assert oracle.attention_gate(_with_spike(r, 0.017), r)["pass"]
    assert not over["pass"], over


def test_norm_rope_gate_mean_abs_threshold():
    """A uniform offset: 0.0019 passes, 0.0021 fails on mean-abs alone (max-abs,
    allclose and relative-L2 ~0.002 all hold)."""
    r = _ref()
    assert oracle.norm_rope_gate(r + 0.0019, r)["pass"]
    m = oracle.norm_rope_gate(r + 0.0021, r)
    assert oracle.attention_gate(r + 0.0021, r)["pass"]
    assert abs(m["mean_abs"] - 0.0021) < 1e-5 and not m["pass"], m
