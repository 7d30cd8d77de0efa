"""GPU kernels on the committed golden inputs (``tests/golden/``) against the
stored oracle outputs, through the C ABI, with the build's gates."""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from helpers import announce, bf16_ulp

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name, dev):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    t = {k[3:]: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).contiguous().to(dev)
         for k, v in g.items() if k.startswith("in_")}
    ref = {k: (torch.from_numpy(v.view(np.int16)).view(torch.bfloat16) if k.endswith("_bits") else torch.from_numpy(v))
           for k, v in g.items() if not k.startswith("in_")}
    return t, ref


def test_golden_norm_rope(gpu):
    import kernelfuser_amd as kf
    t, ref = load("norm_rope_s16", gpu)
    announce("golden norm_rope_s16")
    qn, kn = kf.norm_rope(t["q"], t["k"], t["gq"], t["gk"], t["cos"], t["sin"], norm_style="fp32")
    qh, kh = kf.norm_rope(t["q"], t["k"], t["gq"], t["gk"], t["cos"], t["sin"], norm_style="hf")
    torch.cuda.synchronize()
    assert oracle.norm_rope_gate(qn.cpu(), ref["qn_fp32"])["pass"]
    assert oracle.norm_rope_gate(kn.cpu(), ref["kn_fp32"])["pass"]
    # HF chain: the stored BF16 chain, up to a rare one-ulp flip of one rounding
    # (a last-bit difference of the FP32 inverse RMS moves a normalised value or
    # RoPE product by one ulp of the larger operand of the rotation)
    for got, key, x, g in ((qh, "qn_hf_bits", t["q"], t["gq"]), (kh, "kn_hf_bits", t["k"], t["gk"])):
        want = ref[key].float()
        y = oracle.norm_hf_bf16(x.cpu(), g.cpu()).float()
        half = y.shape[-1] // 2
        scale = torch.maximum(y.abs(), torch.cat([y[..., half:], y[..., :half]], -1).abs())
        diff = (got.cpu().float() - want).abs()
        assert bool((diff <= bf16_ulp(scale) + bf16_ulp(want)).all())
        assert float((diff > 0).float().mean()) < 2e-3


@pytest.mark.parametrize("style", ["fp32", "hf"])
def test_golden_attention(gpu, style):
    import kernelfuser_amd as kf
    t, ref = load("attention_s33", gpu)
    announce(f"golden attention_s33 {style}")
    out = kf.optimized_attention(t["q"], t["k"], t["v"], t["gq"], t["gk"], t["cos"], t["sin"], causal=True,
                                 norm_style=style)
    torch.cuda.synchronize()
    assert oracle.attention_gate(out.cpu(), ref["out_fp32"])["pass"]


def test_golden_attention_norope(gpu):
    import kernelfuser_amd as kf
    t, ref = load("attention_norope_s17", gpu)
    announce("golden attention_norope_s17")
    out = kf.optimized_attention(t["q"], t["k"], t["v"], t["gq"], t["gk"], causal=False, norm_style="legacy")
    torch.cuda.synchronize()
    assert oracle.attention_gate(out.cpu(), ref["out_fp32"])["pass"]


def test_golden_factored(gpu):
    import kernelfuser_amd as kf
    t, ref = load("factored_s17", gpu)
    announce("golden factored_s17")
    out, inv, kn = kf.factored_qk_attention(t["q"], t["k"], t["v"], t["gq"], t["gk"], causal=True)
    torch.cuda.synchronize()
    assert torch.allclose(inv.cpu(), ref["inv_q_fp32"], rtol=2e-6, atol=0)
    # KN is BF16(k*inv_k*gk*gq): within half a BF16 ulp (plus FP32 noise) of the FP32 value
    kref = ref["kn_fp32"]
    assert bool(((kn.cpu().float() - kref).abs() <= kref.abs() * 2.0 ** -8 * 1.01 + 1e-6).all())
    assert oracle.attention_gate(out.cpu(), ref["out_fp32"])["pass"]
