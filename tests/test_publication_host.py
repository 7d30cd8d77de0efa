"""Host logic of the publication runner (kernelfuser_amd.publication): the
PyTorch arm's rounding chain and GQA expansion against the FP32 reference
on the CPU, and the per-row gate (src/e1_rope_publication_v1.py:397-405)."""
import torch

from kernelfuser_amd import publication
from kernelfuser_amd.refine import gate, reference_fp32, refinement_inputs


def test_vendor_arm_matches_fp32_on_cpu():
    """HF chain + SDPA on K/V repeated to Hq heads, with the model's scale
    (Gemma-3-27B: D=128 but query_pre_attn_scalar 256), against the FP32
    reference; a wrong scale or head map fails the gate."""
    for name, causal in (("Qwen3-8B", True), ("Gemma-3-27B", False)):
        xs = refinement_inputs(name, 1, 48, 1701, True, device="cpu")
        scale = publication.model_scale(name, xs[0].shape[-1])
        ref = reference_fp32(xs, causal, True, scale)
        assert gate(publication.vendor_fn(*xs, causal, scale), ref)["pass"]
        wrong = reference_fp32(xs, causal, True, scale * 1.5)
        assert not gate(publication.vendor_fn(*xs, causal, scale), wrong)["pass"]
    q = torch.arange(4.0).view(1, 2, 1, 2)
    assert torch.equal(publication.expand(q, 4)[0, :, 0, 0], torch.tensor([0.0, 0.0, 2.0, 2.0]))


def test_rope_torch_rounding_points():
    """rotate-half with a BF16 rounding after every product and sum."""
    x = torch.tensor([[1.0 + 2 ** -7, 3.0, 0.5, -1.0]], dtype=torch.bfloat16)
    cos = torch.tensor([[0.7, 0.3, 0.7, 0.3]], dtype=torch.bfloat16)
    sin = torch.tensor([[0.2, 0.9, 0.2, 0.9]], dtype=torch.bfloat16)
    y = publication.rope_torch(x, cos, sin)
    bf = lambda t: t.to(torch.bfloat16)
    a, b, c, s = x[0, :2], x[0, 2:], cos[0, :2], sin[0, :2]
    want = torch.cat([bf(bf(a * c) - bf(b * s)), bf(bf(b * c) + bf(a * s))])
    assert torch.equal(y[0], want)


def _row(**kw):
    row = {"errors": [], "correctness": {"pass": True}, "torchinductor_status": "compiled",
           "torchinductor_correctness": {"pass": True}, "gpu_exclusivity": {"exclusive": None},
           "traces": ["a", "b", "c", "d"],
           "timing": {p: {"initial": {}, "retest": {}} for p in ("separate_vs_fused", "vendor_vs_fused")}}
    row.update(kw)
    return row


def test_publication_gate():
    assert publication.publication_gate(_row(), True) == {"pass": True, "reasons": []}
    assert not publication.publication_gate(_row(errors=[{"stage": "x"}]), True)["pass"]
    assert not publication.publication_gate(_row(correctness={"pass": False}), True)["pass"]
    assert not publication.publication_gate(_row(gpu_exclusivity={"exclusive": False}), True)["pass"]
    assert not publication.publication_gate(_row(traces=["a"]), True)["pass"]
    assert not publication.publication_gate(_row(timing={"vendor_vs_fused": {"initial": {}}}), True)["pass"]
    # a compile arm that PyTorch cannot build here fails the gate with its reason
    g = publication.publication_gate(_row(torchinductor_status="unavailable: X", torchinductor_correctness={},
                                          traces=["a", "b", "c"]), True)
    assert not g["pass"] and "unavailable: X" in g["reasons"][0]
    # left out on request: three traces suffice
    assert publication.publication_gate(_row(torchinductor_status="not requested", traces=["a", "b", "c"]),
                                        False)["pass"]
