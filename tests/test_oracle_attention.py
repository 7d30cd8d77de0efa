"""Pins of the oracle's attention (CPU only).

The oracle's attention restates src/e1_rope_publication_v1.py:170 (GQA
expansion by repeat_interleave) and :295-302 (FP32 SDPA, default scale
D^-1/2).  The checks below use float64 brute force, known answers that the
mathematics fixes (single-key rows, constant V, zero queries, two-key closed
form), the GQA head map, and agreement of the full-matrix and row-sample
forms; each family is also run against a planted mistake to show it would
catch one.
"""
import math

import numpy as np
import pytest
import torch

import oracle


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _qkv(b, hq, hkv, s, d, seed):
    return _rand((b, hq, s, d), seed), _rand((b, hkv, s, d), seed + 1), _rand((b, hkv, s, d), seed + 2)


# --------------------------------------------------------------------------
# float64 brute force
# --------------------------------------------------------------------------

@pytest.mark.parametrize("b,hq,hkv,s,d,causal", [(2, 4, 2, 9, 16, True), (1, 4, 1, 17, 32, False),
                                                  (1, 2, 2, 33, 16, True), (1, 8, 2, 5, 8, False)])
def test_attention_matches_float64_bruteforce(b, hq, hkv, s, d, causal):
    q, k, v = _qkv(b, hq, hkv, s, d, 11 + s)
    got = oracle.attention_fp32(q, k, v, causal).double().numpy()
    want = oracle.attention_bruteforce(q, k, v, causal)
    assert np.abs(got - want).max() < 2e-6


def test_bruteforce_catches_planted_mistakes():
    q, k, v = _qkv(1, 4, 2, 12, 16, 5)
    want = oracle.attention_bruteforce(q, k, v, True)
    # off-by-one causal mask (a row cannot see itself)
    qf, kf, vf = (t.double().numpy() for t in (q, k, v))
    bad = np.zeros_like(want)
    for h in range(4):
        for i in range(12):
            n = max(i, 1)
            sc = (kf[0, h // 2, :n] @ qf[0, h, i]) / math.sqrt(16)
            w = np.exp(sc - sc.max())
            bad[0, h, i] = (w / w.sum()) @ vf[0, h // 2, :n]
    assert np.abs(bad - want).max() > 1e-2
    # scale 1/D instead of 1/sqrt(D)
    wrong_scale = oracle.attention_fp32(q, k, v, True, scale=1.0 / 16).double().numpy()
    assert np.abs(wrong_scale - want).max() > 1e-2
    # non-causal where causal is asked
    assert np.abs(oracle.attention_fp32(q, k, v, False).double().numpy() - want).max() > 1e-2


# --------------------------------------------------------------------------
# known answers
# --------------------------------------------------------------------------

def test_causal_row0_is_v0():
    q, k, v = _qkv(2, 4, 2, 40, 128, 21)
    out = oracle.attention_fp32(q, k, v, True)
    for h in range(4):
        assert torch.equal(out[:, h, 0], v[:, h // 2, 0].float())


def test_constant_v_gives_constant_output():
    q, k, _ = _qkv(1, 4, 2, 64, 128, 31)
    v = torch.empty(1, 2, 64, 128, dtype=torch.bfloat16)
    v[:, 0] = 1.5
    v[:, 1] = -0.25
    for causal in (True, False):
        out = oracle.attention_fp32(q, k, v, causal)
        assert torch.allclose(out[:, :2], torch.full_like(out[:, :2], 1.5), atol=1e-6, rtol=0)
        assert torch.allclose(out[:, 2:], torch.full_like(out[:, 2:], -0.25), atol=1e-6, rtol=0)


def test_zero_query_gives_prefix_mean():
    _, k, v = _qkv(1, 2, 1, 50, 128, 41)
    q = torch.zeros(1, 2, 50, 128, dtype=torch.bfloat16)
    out = oracle.attention_fp32(q, k, v, True)
    prefix_mean = torch.cumsum(v.double(), dim=2) / torch.arange(1, 51, dtype=torch.float64)[None, None, :, None]
    for h in range(2):
        assert torch.allclose(out[:, h].double(), prefix_mean[:, 0], atol=1e-6, rtol=0)
    full = oracle.attention_fp32(q, k, v, False)
    assert torch.allclose(full[:, 0].double(), v.double().mean(2, keepdim=True).expand(1, 1, 50, 128)[:, 0],
                          atol=1e-6, rtol=0)


def test_two_key_closed_form_fixes_the_scale():
    """Row with keys k0 = t*e0 and k1 = 0, values e0 and e1: the output is
    (sigmoid(t*q0/sqrt(D)), 1 - sigmoid(...), 0, ...) -- pins the default
    D^-1/2 scale of rope:302 (scale=None)."""
    d = 128
    q = torch.zeros(1, 1, 2, d, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 2, d, dtype=torch.bfloat16)
    v = torch.zeros(1, 1, 2, d, dtype=torch.bfloat16)
    q[0, 0, :, 0] = 2.0
    k[0, 0, 0, 0] = 3.0
    v[0, 0, 0, 0] = 1.0
    v[0, 0, 1, 1] = 1.0
    out = oracle.attention_fp32(q, k, v, False)[0, 0, 0]
    p = 1.0 / (1.0 + math.exp(-6.0 / math.sqrt(d)))
    assert abs(float(out[0]) - p) < 1e-6 and abs(float(out[1]) - (1 - p)) < 1e-6
    assert float(out[2:].abs().max()) == 0.0
    wrong = oracle.attention_fp32(q, k, v, False, scale=1.0)[0, 0, 0]
    assert abs(float(wrong[0]) - p) > 1e-2


# --------------------------------------------------------------------------
# GQA head map (rope:170, kernel rope:616)
# --------------------------------------------------------------------------

def _gqa_constant_case(hq, hkv):
    s, d = 24, 128
    q, k, _ = _qkv(1, hq, hkv, s, d, 51)
    v = torch.empty(1, hkv, s, d, dtype=torch.bfloat16)
    for j in range(hkv):
        v[:, j] = float(j + 1)
    return q, k, v


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 8), (8, 1)])
def test_gqa_map_is_h_div_group(hq, hkv):
    q, k, v = _gqa_constant_case(hq, hkv)
    out = oracle.attention_fp32(q, k, v, True)
    g = hq // hkv
    for h in range(hq):
        assert torch.allclose(out[:, h], torch.full_like(out[:, h], float(h // g + 1)), atol=1e-5)
    rows = oracle.attention_rows_fp32(q, k, v, [0, 7, 23], True)
    for h in range(hq):
        assert torch.allclose(rows[:, h], torch.full_like(rows[:, h], float(h // g + 1)), atol=1e-5)


def test_gqa_planted_mistake_tiled_expansion():
    """``repeat`` (head h -> h % Hkv) instead of ``repeat_interleave`` fails the map."""
    q, k, v = _gqa_constant_case(32, 8)
    tiled = torch.nn.functional.scaled_dot_product_attention(
        q.float(), k.float().repeat(1, 4, 1, 1), v.float().repeat(1, 4, 1, 1), is_causal=True)
    assert not torch.allclose(tiled, oracle.attention_fp32(q, k, v, True), atol=1e-3)


# --------------------------------------------------------------------------
# equivalent forms: head chunks, row samples, tails, online softmax
# --------------------------------------------------------------------------

@pytest.mark.parametrize("s", [33, 129, 200])
def test_rows_and_chunks_agree_with_full(s):
    xs_q, k, v = _qkv(1, 8, 2, s, 128, 61 + s)
    full = oracle.attention_fp32(xs_q, k, v, True)
    chunked = oracle.attention_fp32(xs_q, k, v, True, head_chunk=3)
    assert torch.allclose(full, chunked, atol=1e-6, rtol=0)
    rows = torch.tensor([0, 1, s // 2, s - 2, s - 1])
    assert torch.allclose(oracle.attention_rows_fp32(xs_q, k, v, rows, True), full[:, :, rows], atol=1e-6, rtol=0)


@pytest.mark.parametrize("s", [33, 129])
def test_oracle_rows_agree_with_full_oracle(s):
    from kernelfuser_amd.inputs import make_inputs
    xs = make_inputs(1, s, (8, 2, 128), 71)
    full = oracle.oracle_fp32(*xs.astuple(), True)
    rows = torch.tensor([0, 5, s - 1])
    got = oracle.oracle_rows_fp32(*xs.astuple(), rows, True)
    assert torch.allclose(got, full[:, :, rows], atol=1e-6, rtol=0)


def _online_softmax_attention(q, k, v, causal, block):
    """Tile-by-tile online softmax in float64 (the flash recurrence of the
    kernels, rope:629-647): running max m, denominator l, accumulator acc."""
    qd, kd, vd = q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)
    s, d = qd.shape
    out = np.zeros_like(qd)
    for i in range(s):
        n = i + 1 if causal else s
        m, l, acc = -np.inf, 0.0, np.zeros(d)
        for j0 in range(0, n, block):
            sc = kd[j0:min(n, j0 + block)] @ qd[i] / math.sqrt(d)
            m_new = max(m, sc.max())
            alpha = math.exp(m - m_new) if m > -np.inf else 0.0
            p = np.exp(sc - m_new)
            l = l * alpha + p.sum()
            acc = acc * alpha + p @ vd[j0:j0 + len(sc)]
            m = m_new
        out[i] = acc / l
    return out


@pytest.mark.parametrize("block", [4, 16, 64])
def test_online_softmax_equals_one_pass(block):
    q, k, v = _qkv(1, 1, 1, 70, 32, 81)
    got = _online_softmax_attention(q[0, 0].float().numpy(), k[0, 0].float().numpy(), v[0, 0].float().numpy(),
                                    True, block)
    want = oracle.attention_bruteforce(q, k, v, True)[0, 0]
    assert np.abs(got - want).max() < 1e-12
