"""The older API of the reference (rope:25-36, :185-212): ``fused`` with
explicit eps/scale on every geometry of the reference's MODELS table, the
broadcast table shapes, ``separate`` and ``anchor``; gated against the FP32
oracle with the model's scale (query_pre_attn_scalar for Gemma-3)."""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import MODELS, anchor, fused, launch_attention, make_inputs, model_scale, separate

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", sorted(MODELS))
def test_fused_models_gate(gpu, name):
    geom = MODELS[name]
    d = geom[2]
    xs = make_inputs(1, 65, geom, 3101)
    g = xs.to(gpu)
    announce(f"fused {name} {geom} S=65 causal")
    sc = model_scale(name, d)
    out = fused(g.q, g.k, g.v, g.gq, g.gk, g.cos, g.sin, True, scale=sc)
    torch.cuda.synchronize()
    ref = oracle.oracle_fp32(*xs.astuple(), True, scale=sc)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m


def test_fused_table_shapes_and_eps(gpu):
    xs = make_inputs(2, 40, MODELS["Qwen3-8B"], 3102, qkv_std=0.02).to(gpu)
    announce("fused table shapes / eps")
    base = fused(xs.q, xs.k, xs.v, xs.gq, xs.gk, xs.cos, xs.sin, False)
    c3, s3 = xs.cos[None].expand(2, -1, -1), xs.sin[None].expand(2, -1, -1)
    c4, s4 = xs.cos[None, None].expand(2, 1, -1, -1), xs.sin[None, None].expand(2, 1, -1, -1)
    assert torch.equal(fused(xs.q, xs.k, xs.v, xs.gq, xs.gk, c3, s3, False), base)
    assert torch.equal(fused(xs.q, xs.k, xs.v, xs.gq, xs.gk, c4, s4, False), base)
    big_eps = fused(xs.q, xs.k, xs.v, xs.gq, xs.gk, xs.cos, xs.sin, False, eps=1e-3)
    torch.cuda.synchronize()
    cpu = [t.cpu() for t in xs.astuple()]
    ref = oracle.oracle_fp32(*cpu, False, eps=1e-3)
    assert oracle.attention_gate(big_eps.cpu(), ref)["pass"]
    # with |x| ~ 0.02 the two eps give visibly different normalisations
    assert float((big_eps.float() - base.float()).abs().max()) > 1e-2


def test_separate_equals_unfused_launch(gpu):
    xs = make_inputs(1, 129, MODELS["Qwen3-8B"], 3103).to(gpu)
    announce("separate vs launch_attention unfused")
    a = separate(xs.q, xs.k, xs.v, xs.gq, xs.gk, xs.cos, xs.sin, True)
    out, qn, kn = torch.empty_like(xs.q), torch.empty_like(xs.q), torch.empty_like(xs.k)
    launch_attention(xs.reference7, out, causal=True, mode="unfused", qn=qn, kn=kn, norm_style="hf")
    torch.cuda.synchronize()
    assert torch.equal(a, out)
    ref = oracle.oracle_fp32(*[t.cpu() for t in xs.astuple()], True)
    assert oracle.attention_gate(a.cpu(), ref)["pass"]


def test_anchor_on_prepared_inputs(gpu):
    xs = make_inputs(1, 100, MODELS["Gemma-3-4B"], 3104)
    qn = oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin).to(torch.bfloat16)
    kn = oracle.norm_rope_fp32(xs.k, xs.gk, xs.cos, xs.sin).to(torch.bfloat16)
    announce("anchor D=256 S=100")
    sc = model_scale("Gemma-3-4B", 256)
    out = anchor(qn.to(gpu), kn.to(gpu), xs.v.to(gpu), None, None, True, scale=sc)
    torch.cuda.synchronize()
    ref = oracle.attention_fp32(qn, kn, xs.v, True, scale=sc)
    assert oracle.attention_gate(out.cpu(), ref)["pass"]
