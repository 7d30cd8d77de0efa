"""The general attention kernel's lean softmax and its exact redo.

After the first KV tile of a work item the kernel takes p = exp2(logit -
m_run) with no per-tile max; a lane whose tile sum reaches 2^64 makes the
whole workgroup redo the item with the exact online softmax.  These inputs
put one key's logit so far above the first tile's row max (up to 163 in log2
units, where exp2 overflows) that only the redo gives finite, correct rows;
the FP32 oracle (softmax attention on the same prepared Q/K) is the check.
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import anchor

pytestmark = pytest.mark.gpu


def _spiked(b, hq, hkv, s, d, key, seed):
    g = torch.Generator().manual_seed(seed)
    q = 0.1 * torch.randn(b, hq, s, d, generator=g)
    k = 0.1 * torch.randn(b, hkv, s, d, generator=g)
    v = torch.randn(b, hkv, s, d, generator=g)
    q[..., 0] = 8.0          # every query leans along e0
    k[:, :, key, 0] = 160.0  # one key far along e0: logit 1280/sqrt(D)
    return tuple(t.to(torch.bfloat16) for t in (q, k, v))


@pytest.mark.parametrize("d,hq,hkv,s,causal", [(128, 8, 2, 700, True), (128, 8, 2, 700, False),
                                               (256, 4, 2, 640, True), (256, 4, 2, 640, False)])
def test_lean_overflow_takes_exact_redo(gpu, d, hq, hkv, s, causal):
    q, k, v = _spiked(1, hq, hkv, s, d, 300, 4242)
    announce(f"lean redo D={d} Hq={hq} Hkv={hkv} S={s} causal={causal}")
    out = anchor(q.to(gpu), k.to(gpu), v.to(gpu), None, None, causal)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isfinite(out.float()).all()
    ref = oracle.attention_fp32(q, k, v, causal)
    m = oracle.attention_gate(out, ref)
    assert m["pass"], m
    # rows that see the spiked key are its value row
    first = 300 if causal else 0
    kv_of = torch.arange(hq) // (hq // hkv)
    want = v[0, kv_of, 300].float()[:, None, :].expand(hq, s - first, d)
    assert (out[0, :, first:].float() - want).abs().max() <= 2e-2


def test_lean_matches_exact_on_ordinary_inputs(gpu):
    """Without a spike no redo happens and the result is the same softmax."""
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, h, 900, 128, generator=g).to(torch.bfloat16) for h in (8, 2, 2))
    announce("lean ordinary D=128 S=900 causal")
    out = anchor(q.to(gpu), k.to(gpu), v.to(gpu), None, None, True)
    torch.cuda.synchronize()
    m = oracle.attention_gate(out.cpu(), oracle.attention_fp32(q, k, v, True))
    assert m["pass"], m
