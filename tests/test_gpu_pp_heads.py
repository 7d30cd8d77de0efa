"""Whole-output parity of the ping-pong kernel's two-heads-per-item form
(two Q heads x 128 rows per work item, `hpg=1`) against the CPU FP32 oracle
(src/e1_rope_publication_v1.py:295-302; no-RoPE / factored: :736-742 and
src/e1_qk_publication_v3.py:612-638).

The shape-based dispatch picks this form for GQA ratios that are even but
not a multiple of 4; the tests force it through the library's tuning
overrides (kfmi_set_tuning) on Qwen3 geometries as well, and check from the
launch records that it ran.  Cases: a partial last query block and key tile
(S=3000), non-causal with B=2, GQA ratios 8 and 2, the persistent pairing on
and off, and the factored no-RoPE prologue.
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import QWEN3_8B, _lib, launch_attention, launch_factored_attention, make_inputs

pytestmark = pytest.mark.gpu


def _ran_h1(recs, persistent=None):
    attn = [r for r in recs if r["kernel"].startswith("attn_")]
    assert len(attn) == 1 and attn[0]["kernel"].startswith("attn_pp_kernel"), recs
    assert "hpg=1" in attn[0]["plan"], attn
    if persistent is not None:
        assert f"persistent={persistent}" in attn[0]["plan"], attn


@pytest.mark.parametrize("geom,b,s,causal,style", [
    (QWEN3_8B, 1, 3000, True, "fp32"),
    (QWEN3_8B, 2, 1000, False, "hf"),
    ((64, 8, 128), 1, 1100, True, "legacy"),
    ((16, 8, 128), 1, 777, True, "fp32"),
])
def test_pp_two_heads_query_whole_output(gpu, geom, b, s, causal, style):
    xs = make_inputs(b, s, geom, 9090 + s)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    kn = torch.empty_like(g.k)
    announce(f"pp two heads/item {geom} {style} B={b} S={s} causal={causal} (whole output)")
    with _lib.tuning(attn_kernel="pingpong", pp_heads=1):
        recs = list(launch_attention(g.reference7, out, causal=causal, mode="query", kn=kn, norm_style=style))
    torch.cuda.synchronize()
    _ran_h1(recs)
    ref = oracle.oracle_fp32(*xs.astuple(), causal, head_chunk=8)
    gate = oracle.attention_gate if style == "fp32" else oracle.metric
    m = gate(out.cpu(), ref)
    assert m["pass"], m


def test_pp_two_heads_pairing_on_and_off(gpu):
    """B=2 S=2048 causal with Qwen3-8B heads: 16 blocks of 128 rows x 32 head
    pairs = 256 (long, short) units, one per CU; run with the persistent
    pairing and with one item per workgroup.  Both pass the gate; an item's
    arithmetic does not depend on where it runs, so they agree bit for bit."""
    xs = make_inputs(2, 2048, QWEN3_8B, 9191)
    g = xs.to(gpu)
    outs = []
    for persistent in (0, 1):
        out = torch.full_like(g.q, float("nan"))
        kn = torch.empty_like(g.k)
        announce(f"pp two heads/item B=2 S=2048 causal persistent-off={persistent}")
        with _lib.tuning(attn_kernel="pingpong", pp_heads=1, persistent=persistent):
            recs = list(launch_attention(g.reference7, out, causal=True, mode="query", kn=kn, norm_style="fp32"))
        torch.cuda.synchronize()
        attn = [r for r in recs if r["kernel"].startswith("attn_")]
        if persistent == 0 and "persistent=1" not in attn[0]["plan"]:
            pytest.skip(f"device does not pair this grid: {attn[0]}")
        _ran_h1(recs, persistent=1 - persistent)
        outs.append(out)
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.attention_gate(outs[0].cpu(), ref)
    assert m["pass"], m
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("s,causal", [(1500, True), (640, False)])
def test_pp_two_heads_factored_whole_output(gpu, s, causal):
    """The factored no-RoPE launch (Q's inverse RMS computed in the prologue,
    applied per score) on the two-heads-per-item form."""
    xs = make_inputs(1, s, QWEN3_8B, 9292 + s, rope=False)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
    kn = torch.empty_like(g.k)
    announce(f"pp two heads/item factored B=1 S={s} causal={causal} (whole output)")
    with _lib.tuning(attn_kernel="pingpong", pp_heads=1):
        recs = list(launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=causal))
    torch.cuda.synchronize()
    _ran_h1(recs)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, causal, head_chunk=8)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m
    inv_ref = oracle.rms_inverse(xs.q.float())[..., 0]
    assert torch.allclose(inv.cpu(), inv_ref, rtol=1e-6, atol=0)
