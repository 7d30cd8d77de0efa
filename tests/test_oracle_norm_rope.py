"""Pins of the oracle's RMSNorm, RoPE and rotary tables (CPU only).

The oracle restates src/e1_rope_publication_v1.py:137-183 and :295-301 of the
reference.  These checks do not retype its formulas: they use closed forms,
invariants of the rotation, float64 brute force, and a scalar restatement of
the BF16 rounding chain with bit-level round-to-nearest-even.  Each family
also runs against a deliberately wrong variant ("planted mistake") to show
that the check would catch it.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from helpers import rne_bf16
from kernelfuser_amd.inputs import make_inputs, rope_tables as product_tables

pytestmark = []


# --------------------------------------------------------------------------
# rotary tables (rope:179-183)
# --------------------------------------------------------------------------

def _table_closed_form_error(cos, sin, theta):
    """Max |table - closed form| in units of (BF16 ulp + FP32 angle error)."""
    S, D = cos.shape
    pos = np.arange(S, dtype=np.float64)[:, None]
    i = np.arange(D // 2, dtype=np.float64)[None, :]
    ang = pos * theta ** (-2.0 * i / D)
    want_c = np.concatenate([np.cos(ang)] * 2, axis=1)
    want_s = np.concatenate([np.sin(ang)] * 2, axis=1)
    # FP32 angle: relative error ~2^-23 of |ang| propagates to cos/sin.
    tol = 2.0 ** -8 + np.concatenate([ang] * 2, axis=1) * 2.0 ** -22 + 1e-7
    ec = np.abs(cos.float().numpy() - want_c) / tol
    es = np.abs(sin.float().numpy() - want_s) / tol
    return max(ec.max(), es.max())


@pytest.mark.parametrize("S,D,theta", [(64, 128, 1e6), (300, 256, 1e4), (2048, 128, 1e6)])
def test_tables_closed_form(S, D, theta):
    cos, sin = oracle.rope_tables(S, D, theta)
    assert cos.dtype == torch.bfloat16 and cos.shape == (S, D)
    assert _table_closed_form_error(cos, sin, theta) <= 1.0
    assert torch.equal(cos[:, : D // 2], cos[:, D // 2:]) and torch.equal(sin[:, : D // 2], sin[:, D // 2:])
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)


def test_tables_planted_mistakes():
    S, D, theta = 256, 128, 1e6
    pos = torch.arange(S, dtype=torch.float32)
    # frequency exponent over D/2 instead of D
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / (D // 2)))
    ang = pos[:, None] * inv[None, :]
    bad = torch.cat([torch.cos(ang)] * 2, 1).bfloat16(), torch.cat([torch.sin(ang)] * 2, 1).bfloat16()
    assert _table_closed_form_error(*bad, theta) > 1.0
    # interleaved instead of duplicated halves
    cos, sin = oracle.rope_tables(S, D, theta)
    inter = cos[:, : D // 2].repeat_interleave(2, 1), sin[:, : D // 2].repeat_interleave(2, 1)
    assert _table_closed_form_error(*inter, theta) > 1.0


def test_product_tables_identical_to_oracle_tables():
    """Kernel and oracle must consume bit-identical tables."""
    for S, D in ((128, 128), (1000, 128), (33, 256)):
        a = product_tables(S, D, 1e6)
        b = oracle.rope_tables(S, D, 1e6)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# --------------------------------------------------------------------------
# RMSNorm (rope:298, qk:600)
# --------------------------------------------------------------------------

def test_norm_constant_row_closed_form():
    D = 128
    g = (1 + 0.1 * torch.randn(D, generator=torch.Generator().manual_seed(1))).bfloat16()
    for a in (0.25, 1.0, -3.0, 7.5):
        x = torch.full((1, 1, 1, D), a).bfloat16()
        y = oracle.norm_fp32(x, g)
        want = g.double() * a / math.sqrt(a * a + oracle.EPS)
        assert torch.allclose(y[0, 0, 0].double(), want, rtol=3e-7, atol=0)


def _norm_bruteforce(x, g, eps):
    xd = x.double().numpy()
    gd = g.double().numpy()
    out = np.empty_like(xd)
    for idx in np.ndindex(*xd.shape[:-1]):
        row = xd[idx]
        ms = sum(v * v for v in row) / len(row)
        out[idx] = row / math.sqrt(ms + eps) * gd
    return out


def test_norm_bruteforce_and_scale_invariance():
    xs = make_inputs(2, 5, (4, 2, 128), 11)
    y = oracle.norm_fp32(xs.q, xs.gq)
    ref = _norm_bruteforce(xs.q, xs.gq, oracle.EPS)
    assert np.max(np.abs(y.numpy() - ref) / (np.abs(ref) + 1e-3)) < 1e-5
    # RMSNorm is scale invariant (up to eps): norm(4x) == norm(x)
    y4 = oracle.norm_fp32((xs.q.float() * 4), xs.gq)
    assert torch.allclose(y4, y, rtol=1e-5, atol=1e-5)
    # planted mistake: mean over D replaced by sum over D fails the brute force
    bad = xs.q.float() * torch.rsqrt(xs.q.float().square().sum(-1, keepdim=True) + oracle.EPS) * xs.gq.float()
    assert np.max(np.abs(bad.numpy() - ref)) > 0.1


def test_rms_inverse_matches_norm():
    xs = make_inputs(1, 7, (2, 1, 256), 3)
    inv = oracle.rms_inverse(xs.q)
    ref = _norm_bruteforce(xs.q, torch.ones(256), oracle.EPS) / np.where(xs.q.double().numpy() == 0, 1,
                                                                          xs.q.double().numpy())
    assert np.allclose(inv.numpy()[..., 0], ref[..., 0], rtol=1e-5)


# --------------------------------------------------------------------------
# rotate-half RoPE (rope:141-168, fp32=True)
# --------------------------------------------------------------------------

def _rope_by_rotation(x, cos, sin):
    """Brute force: rotate every pair (x_i, x_{i+D/2}) by the 2x2 matrix
    [[c, -s], [s, c]] with (c, s) of frequency i, in float64."""
    xd = x.double().numpy()
    c = cos.double().numpy()
    s = sin.double().numpy()
    D = xd.shape[-1]
    h = D // 2
    out = np.empty_like(xd)
    for idx in np.ndindex(*xd.shape[:-2]):
        for p in range(xd.shape[-2]):
            for i in range(h):
                a, b = xd[idx][p, i], xd[idx][p, i + h]
                ci, si = c[p, i], s[p, i]
                out[idx][p, i] = ci * a - si * b
                out[idx][p, i + h] = si * a + ci * b
    return out


def test_rope_matches_pairwise_rotation():
    xs = make_inputs(1, 6, (2, 1, 128), 21)
    y = oracle.rope_fp32(xs.q.float(), xs.cos, xs.sin)
    ref = _rope_by_rotation(xs.q.float(), xs.cos, xs.sin)
    assert np.max(np.abs(y.numpy() - ref)) < 1e-5
    # planted mistake: the sign of the rotated term flipped in the first half
    h = 64
    bad = y.clone()
    a, b = xs.q.float()[..., :h], xs.q.float()[..., h:]
    bad[..., :h] = a * xs.cos.float()[:, :h] + b * xs.sin.float()[:, :h]
    assert np.max(np.abs(bad.numpy() - ref)) > 0.05


def test_rope_complex_multiplication_form():
    """(a + i b) * e^{i ang} = (a c - b s) + i (a s + b c) per frequency."""
    xs = make_inputs(1, 40, (3, 1, 128), 22)
    y = oracle.rope_fp32(xs.q.float(), xs.cos, xs.sin).double().numpy()
    x = xs.q.double().numpy()
    z = (x[..., :64] + 1j * x[..., 64:]) * (xs.cos.double().numpy()[:, :64] + 1j * xs.sin.double().numpy()[:, :64])
    assert np.max(np.abs(y[..., :64] - z.real)) < 1e-5 and np.max(np.abs(y[..., 64:] - z.imag)) < 1e-5


def test_rope_invariants():
    S, D = 64, 128
    xs = make_inputs(1, S, (2, 1, D), 23)
    cos32, sin32 = oracle.rope_tables(S, D, 1e4, dtype=torch.float32)
    x = xs.q.float()
    y = oracle.rope_fp32(x, cos32, sin32)
    # position 0 is the identity
    assert torch.equal(oracle.rope_fp32(x, xs.cos, xs.sin)[:, :, 0], x[:, :, 0])
    # each pair keeps its 2-norm
    pre = x[..., :64].square() + x[..., 64:].square()
    post = y[..., :64].square() + y[..., 64:].square()
    assert torch.allclose(pre, post, rtol=1e-5, atol=1e-5)
    # R(-a) R(a) = I
    back = oracle.rope_fp32(y, cos32, -sin32)
    assert torch.allclose(back, x, atol=1e-5)
    # <R(m) q, R(n) k> depends only on m - n
    q = x[0, 0, 5]
    k = x[0, 1, 9]
    def dot(m, n):
        qm = oracle.rope_fp32(q.view(1, 1, 1, D), cos32[m:m + 1], sin32[m:m + 1]).flatten()
        kn = oracle.rope_fp32(k.view(1, 1, 1, D), cos32[n:n + 1], sin32[n:n + 1]).flatten()
        return float((qm.double() * kn.double()).sum())
    assert abs(dot(10, 3) - dot(40, 33)) < 1e-3 * (1 + abs(dot(10, 3)))
    assert abs(dot(10, 3) - dot(3, 10)) > 1e-3  # not symmetric in general


def test_norm_rope_fp32_composition():
    xs = make_inputs(1, 17, (4, 1, 128), 24)
    y = oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin)
    ref = _rope_by_rotation(torch.from_numpy(_norm_bruteforce(xs.q, xs.gq, oracle.EPS)), xs.cos, xs.sin)
    assert np.max(np.abs(y.numpy() - ref)) < 2e-5


# --------------------------------------------------------------------------
# BF16 boundary chains (rope:137-168 fp32=False; kernel rope:559-581)
# --------------------------------------------------------------------------

def _hf_chain_scalar(x, g, cos, sin, eps, legacy=False):
    """Element-by-element restatement with explicit RNE rounding in numpy."""
    xf = x.float().numpy()
    gf = g.float().numpy()
    c = cos.float().numpy()
    s = sin.float().numpy()
    D = xf.shape[-1]
    h = D // 2
    out = np.empty_like(xf)
    for idx in np.ndindex(*xf.shape[:-2]):
        for p in range(xf.shape[-2]):
            row = xf[idx][p]
            ms = np.float32(np.sum(row.astype(np.float32) * row.astype(np.float32), dtype=np.float32)) / np.float32(D)
            inv = np.float32(1.0) / np.sqrt(np.float32(ms + np.float32(eps)), dtype=np.float32)
            if legacy:
                n = rne_bf16((row * inv).astype(np.float32) * gf)
            else:
                n = rne_bf16(rne_bf16(row * inv) * gf)
            a, b = n[:h], n[h:]
            p0 = rne_bf16(a * c[p, :h]); p1 = rne_bf16(b * s[p, :h])
            p2 = rne_bf16(b * c[p, :h]); p3 = rne_bf16(a * s[p, :h])
            out[idx][p, :h] = rne_bf16(p0 - p1)
            out[idx][p, h:] = rne_bf16(p2 + p3)
    return out


@pytest.mark.parametrize("legacy", [False, True])
def test_bf16_chain_scalar_restatement(legacy):
    xs = make_inputs(1, 9, (3, 1, 128), 31)
    norm = oracle.norm_legacy_bf16 if legacy else oracle.norm_hf_bf16
    got = oracle.rope_hf_bf16(norm(xs.q, xs.gq), xs.cos, xs.sin).float().numpy()
    ref = _hf_chain_scalar(xs.q, xs.gq, xs.cos, xs.sin, oracle.EPS, legacy)
    # The only freedom is the FP32 sum order of the mean square, which can move
    # inv by an ulp and flip a rounding: allow one BF16 ulp on rare elements.
    diff = np.abs(got - ref)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    assert np.all(diff <= 2 * ulp)
    assert np.mean(diff > 0) < 0.01


def test_bf16_chain_differs_from_single_rounding():
    """The HF chain is a different contract from FP32-then-round-once: it must
    not collapse to it (it rounds 4-5 times per element)."""
    xs = make_inputs(1, 64, (4, 1, 128), 32)
    hf = oracle.rope_hf_bf16(oracle.norm_hf_bf16(xs.q, xs.gq), xs.cos, xs.sin).float()
    one = oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin).bfloat16().float()
    assert float((hf != one).float().mean()) > 0.05


def test_gate_headroom_single_rounding():
    """Config 1 (B=1, S=128, Qwen3-8B, theta=1e6): one rounding of the FP32
    result passes the norm+RoPE gate; the HF chain does not (its max-abs is
    about 0.04).  This is why the gated runs use norm_style='fp32'."""
    xs = make_inputs(1, 128, (32, 8, 128), 1701, with_v=False)
    ref = oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin)
    one = ref.bfloat16()
    assert oracle.norm_rope_gate(one, ref)["pass"]
    hf = oracle.rope_hf_bf16(oracle.norm_hf_bf16(xs.q, xs.gq), xs.cos, xs.sin)
    m = oracle.norm_rope_gate(hf, ref)
    assert not m["pass"] and m["max_abs"] > 0.016
