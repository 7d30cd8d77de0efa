"""Whole-output parity at long sequence lengths for the prologue forms that
the shorter tests cover only at small S, against the CPU FP32 oracle
(src/e1_rope_publication_v1.py:295-302, no-RoPE / factored :736-742 and
src/e1_qk_publication_v3.py:612-638):

  * mode 'full' at S=4096: one launch; Q and every one of the 64 K tiles
    normalised (and rotated) inside the general kernel (rope:619-635);
  * mode 'unfused' at S=8192: Q and K prepared by one launch, then the
    ping-pong kernel without a prologue;
  * the factored no-RoPE launch at S=4096 with D=128 (ping-pong kernel, Q's
    inverse RMS computed in its prologue) and D=256 (general kernel);
  * query mode with Gemma-3-12B heads (D=256) at S=4096 and Qwen3-32B heads
    at S=2048.
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import GEMMA3_12B, QWEN3_8B, launch_attention, launch_factored_attention, make_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode,s,style", [("full", 4096, "fp32"), ("full", 4096, "hf"), ("unfused", 8192, "fp32")])
def test_long_modes_whole_output(gpu, mode, s, style):
    xs = make_inputs(1, s, QWEN3_8B, 8080)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    qn = torch.empty_like(g.q) if mode == "unfused" else None
    kn = torch.empty_like(g.k) if mode == "unfused" else None
    announce(f"long mode {mode} {style} B=1 S={s} causal (whole output)")
    recs = list(launch_attention(g.reference7, out, causal=True, mode=mode, qn=qn, kn=kn, norm_style=style))
    torch.cuda.synchronize()
    assert any(r["kernel"].startswith("attn_") for r in recs), recs
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    gate = oracle.attention_gate if style == "fp32" else oracle.metric
    m = gate(out.cpu(), ref)
    assert m["pass"], m


@pytest.mark.parametrize("geom", [QWEN3_8B, GEMMA3_12B])
def test_long_factored_whole_output(gpu, geom):
    s = 4096
    xs = make_inputs(1, s, geom, 8181, rope=False)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
    kn = torch.empty_like(g.k)
    announce(f"long factored D={geom[2]} B=1 S={s} causal (whole output)")
    launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=True)
    torch.cuda.synchronize()
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True, head_chunk=8)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m
    inv_ref = oracle.rms_inverse(xs.q.float())[..., 0]
    assert torch.allclose(inv.cpu(), inv_ref, rtol=1e-6, atol=0)


@pytest.mark.parametrize("geom,s,causal,style", [(GEMMA3_12B, 4096, True, "fp32"), (GEMMA3_12B, 4096, False, "legacy"),
                                                 ((64, 8, 128), 2048, True, "fp32")])
def test_long_query_geometries_whole_output(gpu, geom, s, causal, style):
    """Query mode at long S off the Qwen3-8B geometry: Gemma-3-12B heads (D=256,
    general kernel, RoPE in the prologue), causal and not, and Qwen3-32B heads
    (GQA ratio 8: two four-head items per KV head; the persistent pairing fills
    every CU at S=2048)."""
    xs = make_inputs(1, s, geom, 8282)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    kn = torch.empty_like(g.k)
    announce(f"long query {geom} {style} B=1 S={s} causal={causal} (whole output)")
    launch_attention(g.reference7, out, causal=causal, mode="query", kn=kn, norm_style=style)
    torch.cuda.synchronize()
    ref = oracle.oracle_fp32(*xs.astuple(), causal, head_chunk=8)
    gate = oracle.attention_gate if style == "fp32" else oracle.metric
    m = gate(out.cpu(), ref)
    assert m["pass"], m
