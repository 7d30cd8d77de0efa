"""Pins of the oracle's factored no-RoPE attention (CPU only).

The factored path (src/e1_qk_publication_v3.py:592-652) scores raw Q against
KN = k * inv_k * gk * gq and multiplies each score row by Q's inverse RMS;
results/RESULTS.md:104-112 of the reference states the identity
  (q * inv_q * gq) . (k * inv_k * gk) = inv_q * (q . (k * inv_k * gk * gq)),
so the factored oracle must equal the unfused no-RoPE oracle
(src/e1_rope_publication_v1.py:736-742) up to FP32 rounding.  A planted
mistake (gamma folded the wrong way, or the wrong inverse RMS) must not.
"""
import math

import pytest
import torch

import oracle
from kernelfuser_amd.inputs import GEMMA3_12B, make_inputs


@pytest.mark.parametrize("geom,s,causal", [(GEMMA3_12B, 48, True), ((4, 2, 128), 33, False), ((8, 8, 256), 17, True)])
def test_factoring_identity(geom, s, causal):
    xs = make_inputs(1, s, geom, 91, rope=False)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, causal)
    inv_q, kn = oracle.factored_prepare_fp32(xs.q, xs.k, xs.gq, xs.gk)
    got = oracle.factored_attention_fp32(xs.q, kn, xs.v, inv_q, causal)
    assert (got - ref).abs().max() < 1e-5


def test_factoring_planted_mistakes():
    xs = make_inputs(1, 40, GEMMA3_12B, 92, rope=False, gamma_std=0.3)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True)
    inv_q, kn = oracle.factored_prepare_fp32(xs.q, xs.k, xs.gq, xs.gk)
    # gq left out of KN
    kn_no_gq = xs.k.float() * oracle.rms_inverse(xs.k) * xs.gk.float()
    assert (oracle.factored_attention_fp32(xs.q, kn_no_gq, xs.v, inv_q, True) - ref).abs().max() > 1e-3
    # K's inverse RMS used for the Q rows
    inv_k = oracle.rms_inverse(xs.k)[..., 0].repeat_interleave(2, dim=1)
    assert (oracle.factored_attention_fp32(xs.q, kn, xs.v, inv_k, True) - ref).abs().max() > 1e-3


def test_inverse_rms_closed_form():
    d = 256
    for a in (0.5, -2.0, 9.0):
        x = torch.full((1, 1, 1, d), a, dtype=torch.bfloat16)
        inv = oracle.rms_inverse(x)[0, 0, 0, 0].item()
        assert abs(inv - 1.0 / math.sqrt(a * a + oracle.EPS)) < 1e-6 / abs(a)


def test_bf16_kn_rounding_stays_within_gate():
    """The kernel rounds KN once to BF16 (qk:608); the factored result on
    that rounded KN stays within the attention gate of the unfused oracle
    (config-5 geometry, shortened)."""
    xs = make_inputs(1, 128, GEMMA3_12B, 93, rope=False)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True)
    inv_q, kn = oracle.factored_prepare_fp32(xs.q, xs.k, xs.gq, xs.gk)
    got = oracle.factored_attention_fp32(xs.q, kn.to(torch.bfloat16), xs.v, inv_q, True)
    assert oracle.attention_gate(got, ref)["pass"]
