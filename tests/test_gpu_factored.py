"""GPU parity of the factored no-RoPE path (src/e1_qk_publication_v3.py:592-652)
against the unfused FP32 oracle (src/e1_rope_publication_v1.py:736-742).

Config 5: Gemma-3-12B layout (Hq=16, Hkv=8, D=256), B=2, S=2048, causal; plus
the reference's tail checks (Gemma-3-4B, S in {33,129}, qk:723-734).
"""
import pytest
import torch

import oracle
from helpers import announce, bf16_ulp
from kernelfuser_amd import (GEMMA3_12B, factored_attention, factored_qk_attention, launch_factored_attention,
                             make_inputs, prepare_factored)

pytestmark = pytest.mark.gpu


def test_config5_b2_s2048_causal(gpu):
    xs = make_inputs(2, 2048, GEMMA3_12B, 1909, rope=False)
    announce("factored B=2 S=2048 D=256 causal")
    g = xs.to(gpu)
    out, inv, kn = factored_qk_attention(g.q, g.k, g.v, g.gq, g.gk, causal=True)
    torch.cuda.synchronize()
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True, head_chunk=4)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m
    assert m["relative_l2"] < 0.01
    inv_ref, kn_ref = oracle.factored_prepare_fp32(xs.q, xs.k, xs.gq, xs.gk)
    assert torch.allclose(inv.cpu(), inv_ref, rtol=2e-6, atol=0)
    diff = (kn.cpu().float() - kn_ref).abs()
    assert bool((diff <= bf16_ulp(kn_ref) * 0.5001 + 1e-6 * kn_ref.abs()).all())


@pytest.mark.parametrize("s", [33, 129])
@pytest.mark.parametrize("causal", [False, True])
def test_tails_gemma3_4b(gpu, s, causal):
    xs = make_inputs(1, s, (8, 4, 256), 13109, rope=False)
    g = xs.to(gpu)
    out = torch.empty_like(g.q)
    kn = torch.empty_like(g.k)
    inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
    announce(f"factored tails S={s} causal={causal}")
    launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=causal, bn=64)
    torch.cuda.synchronize()
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, causal)
    m = oracle.metric(out.cpu(), ref)
    assert m["pass"], m


def test_separate_prepare_then_attention(gpu):
    """prepare (INV for Q rows + KN) then attention reading INV equals the fused launch."""
    xs = make_inputs(1, 257, GEMMA3_12B, 2909, rope=False)
    g = xs.to(gpu)
    inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
    kn = torch.empty_like(g.k)
    out = torch.empty_like(g.q)
    announce("factored prepare + attention(read inv)")
    prepare_factored((g.q, g.k, g.v, g.gq, g.gk), inv, kn)
    factored_attention(g.q, kn, g.v, inv, out, causal=True)
    torch.cuda.synchronize()
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True)
    assert oracle.attention_gate(out.cpu(), ref)["pass"]
    inv_ref, _ = oracle.factored_prepare_fp32(xs.q, xs.k, xs.gq, xs.gk)
    assert torch.allclose(inv.cpu(), inv_ref, rtol=2e-6, atol=0)


def test_factored_d128_qwen(gpu):
    xs = make_inputs(1, 512, (32, 8, 128), 3909, rope=False)
    g = xs.to(gpu)
    announce("factored D=128 S=512 causal")
    out, inv, kn = factored_qk_attention(g.q, g.k, g.v, g.gq, g.gk, causal=True)
    torch.cuda.synchronize()
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True)
    assert oracle.attention_gate(out.cpu(), ref)["pass"]
