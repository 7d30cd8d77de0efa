"""Whole-output parity of every path that reaches the ping-pong kernel's
one-unit-per-CU persistent form, against the CPU FP32 oracle
(src/e1_rope_publication_v1.py:295-302; no-RoPE / factored: :736-742 and
src/e1_qk_publication_v3.py:612-638).

B=4, S=1000 with Qwen3-8B heads is a causal grid of 8 query blocks of 128
rows whose persistent (long, short) pairs give each of the 256 CUs exactly
one unit; the shape-based dispatch sends it to the ping-pong kernel with
persistent=1.  S=1000 also leaves the last 64-row block ragged.  The launch
records must name the ping-pong kernel and that plan (on a device with 256
CUs; elsewhere the grid does not pair and the test is skipped).
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import QWEN3_8B, _lib, launch_attention, launch_factored_attention, make_inputs

pytestmark = pytest.mark.gpu

B, S = 4, 1000


def _check_plan(recs):
    attn = [r for r in recs if r["kernel"].startswith("attn_")]
    assert len(attn) == 1, recs
    if attn[0]["grid"] != 256 and not attn[0]["kernel"].startswith("attn_pp_kernel"):
        pytest.skip(f"device does not pair this grid: {attn[0]}")
    assert attn[0]["kernel"].startswith("attn_pp_kernel"), attn
    assert "persistent=1" in attn[0]["plan"], attn


@pytest.mark.parametrize("mode,style", [("query", "fp32"), ("query", "hf"), ("query", "legacy"),
                                        ("unfused", "fp32"), ("unfused", "hf")])
def test_paired_grid_modes_whole_output(gpu, mode, style):
    xs = make_inputs(B, S, QWEN3_8B, 6464)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    kn = torch.empty_like(g.k)
    qn = torch.empty_like(g.q) if mode == "unfused" else None
    announce(f"paired grid {mode} {style} B={B} S={S} causal (whole output)")
    recs = list(launch_attention(g.reference7, out, causal=True, mode=mode, qn=qn, kn=kn, norm_style=style))
    torch.cuda.synchronize()
    _check_plan(recs)
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    gate = oracle.attention_gate if style == "fp32" else oracle.metric
    m = gate(out.cpu(), ref)
    assert m["pass"], m


def test_paired_grid_factored_whole_output(gpu):
    """The factored no-RoPE launch at D=128 on the same grid: Q's inverse RMS
    computed in the prologue and applied per score."""
    xs = make_inputs(B, S, QWEN3_8B, 6565, rope=False)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
    kn = torch.empty_like(g.k)
    announce(f"paired grid factored D=128 B={B} S={S} causal (whole output)")
    recs = list(launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=True))
    torch.cuda.synchronize()
    _check_plan(recs)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True, head_chunk=8)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m
    inv_ref = oracle.rms_inverse(xs.q.float())[..., 0]
    assert torch.allclose(inv.cpu(), inv_ref, rtol=1e-6, atol=0)


def test_paired_grid_general_kernel_agrees(gpu):
    """The same call forced onto the general kernel passes the same gate; the
    two kernels' outputs differ by at most a few BF16 ulp (their FP32 styles
    round Q at different points)."""
    xs = make_inputs(B, S, QWEN3_8B, 6666)
    g = xs.to(gpu)
    outs = []
    for kernel in ("auto", "general"):
        out = torch.full_like(g.q, float("nan"))
        kn = torch.empty_like(g.k)
        with _lib.tuning(attn_kernel=kernel):
            launch_attention(g.reference7, out, causal=True, mode="query", kn=kn, norm_style="fp32")
        outs.append(out)
    torch.cuda.synchronize()
    announce(f"paired grid ping-pong vs general B={B} S={S}")
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    for out in outs:
        m = oracle.attention_gate(out.cpu(), ref)
        assert m["pass"], m
    d = (outs[0].float() - outs[1].float()).abs()
    assert float(d.max()) <= 2e-2
