"""The largest shapes the boundary accepts: Q with just under 2^31 elements.

B=15, Qwen3-8B heads (Hq=32, Hkv=8, D=128), S=32768: Q and O hold
2,013,265,920 elements (4.0 GB each), so element offsets reach 2^31 and byte
offsets 2^32 - 2^26.  The preparation kernel computes 32-bit byte offsets,
which the boundary's limit (fewer than 2^31 elements per tensor) keeps below
2^32; the attention kernels address Q and O through 64-bit offsets and K/V
and the tables through per-head buffer descriptors.  Checked on the last
batch (the highest offsets) against the FP32 oracle on a row sample of every
head: the fused attention prologue (ping-pong kernel, persistent, 120 units
per CU on 256 CUs) and the isolated Q+K norm+RoPE launch.  Inputs are drawn
on the device (seeded) to keep the host out of a 10 GB generation; the
oracle sees the same bits through copies of the last batch.  The same
element count at D=256 (Gemma-3-12B heads, Hq=16, Hkv=8) runs the general
kernel, in the fused RoPE form and in the factored no-RoPE launch.
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import GEMMA3_12B, QWEN3_8B, launch_attention, launch_factored_attention, norm_rope
from kernelfuser_amd.inputs import rope_tables

pytestmark = pytest.mark.gpu

B, S = 15, 32768
HQ, HKV, D = QWEN3_8B


def _inputs(gpu, geom=QWEN3_8B):
    HQ, HKV, D = geom
    gen = torch.Generator(device=gpu).manual_seed(31)
    rn = lambda *shape: torch.randn(*shape, generator=gen, device=gpu, dtype=torch.float32).to(torch.bfloat16)
    q = torch.empty(B, HQ, S, D, device=gpu, dtype=torch.bfloat16)
    for b in range(B):  # one batch at a time: no 8 GB FP32 temporary
        q[b] = rn(HQ, S, D)
    k, v = rn(B, HKV, S, D), rn(B, HKV, S, D)
    gq, gk = (1.0 + 0.1 * rn(D).float()).to(torch.bfloat16), (1.0 + 0.1 * rn(D).float()).to(torch.bfloat16)
    cos, sin = (t.to(gpu) for t in rope_tables(S, D))
    return q, k, v, gq, gk, cos, sin


ROWS = torch.tensor([0, 1, 63, 64, 4095, 16383, 16384, 30000, S - 2, S - 1])


def test_max_size_attention_and_norm_rope(gpu):
    assert B * HQ * S * D < 2 ** 31 and B * HQ * S * D > 2 ** 31 - 2 ** 28
    q, k, v, gq, gk, cos, sin = _inputs(gpu)
    announce(f"max size B={B} S={S} Qwen3-8B: fused attention (query, fp32, causal)")
    out = torch.empty_like(q)
    kn = torch.empty_like(k)
    recs = list(launch_attention((q, k, v, gq, gk, cos, sin), out, causal=True, mode="query", kn=kn,
                                 norm_style="fp32"))
    torch.cuda.synchronize()
    assert any(r["kernel"].startswith("attn_") for r in recs), recs
    assert bool(torch.isfinite(out).all())
    last = [t[B - 1:B].cpu() for t in (q, k, v)]
    ref = oracle.oracle_rows_fp32(*last, gq.cpu(), gk.cpu(), cos.cpu(), sin.cpu(), ROWS, True)
    m = oracle.attention_gate(out[B - 1:B, :, ROWS.to(gpu)].cpu(), ref)
    assert m["pass"], m
    del out, kn
    announce(f"max size B={B} S={S} Qwen3-8B: Q+K norm+RoPE (fp32)")
    qn, kn = norm_rope(q, k, gq, gk, cos, sin, norm_style="fp32")
    torch.cuda.synchronize()
    for got, x, gam in ((qn, q, gq), (kn, k, gk)):
        xs = x[B - 1:B, :, ROWS.to(gpu)].cpu()
        ref = oracle.rope_fp32(oracle.norm_fp32(xs, gam.cpu()), cos.cpu()[ROWS], sin.cpu()[ROWS])
        m = oracle.norm_rope_gate(got[B - 1:B, :, ROWS.to(gpu)].cpu(), ref)
        assert m["pass"], m


def test_max_size_d256_general_and_factored(gpu):
    hq, hkv, d = GEMMA3_12B
    assert B * hq * S * d < 2 ** 31 and B * hq * S * d > 2 ** 31 - 2 ** 28
    q, k, v, gq, gk, cos, sin = _inputs(gpu, GEMMA3_12B)
    rows = ROWS.to(gpu)
    last = [t[B - 1:B].cpu() for t in (q, k, v)]
    announce(f"max size B={B} S={S} Gemma-3-12B: fused attention (query, fp32, causal)")
    out = torch.empty_like(q)
    kn = torch.empty_like(k)
    launch_attention((q, k, v, gq, gk, cos, sin), out, causal=True, mode="query", kn=kn, norm_style="fp32")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    ref = oracle.oracle_rows_fp32(*last, gq.cpu(), gk.cpu(), cos.cpu(), sin.cpu(), ROWS, True)
    m = oracle.attention_gate(out[B - 1:B, :, rows].cpu(), ref)
    assert m["pass"], m
    announce(f"max size B={B} S={S} Gemma-3-12B: factored no-RoPE attention (causal)")
    inv = torch.empty(q.shape[:-1], device=gpu, dtype=torch.float32)
    launch_factored_attention((q, k, v, gq, gk), out, inv, kn, causal=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    ref = oracle.oracle_rows_fp32(*last, gq.cpu(), gk.cpu(), None, None, ROWS, True)
    m = oracle.attention_gate(out[B - 1:B, :, rows].cpu(), ref)
    assert m["pass"], m
    inv_ref = oracle.rms_inverse(last[0][:, :, ROWS].float())[..., 0]
    assert torch.allclose(inv[B - 1:B, :, rows].cpu(), inv_ref, rtol=1e-6, atol=0)
