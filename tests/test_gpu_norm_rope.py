"""GPU parity of the row-preparation kernel (per-head Q/K RMSNorm + RoPE) against
the CPU FP32 oracle, on the same seeded BF16 inputs.

Gates: FP32 style within max-abs 1.6e-2 and mean-abs 2e-3 of the FP32 oracle
(north-star gate) and the reference metric; the HF and legacy styles match the
oracle's BF16-boundary restatement to within one BF16 ulp on a vanishing
fraction of elements (only an FP32 last-bit difference of the inverse RMS can
move a rounding).
"""
import pytest
import torch

import oracle
from helpers import announce, bf16_ulp
from kernelfuser_amd import QWEN3_8B, GEMMA3_12B, make_inputs, norm_rope, prepare_attention

pytestmark = pytest.mark.gpu


def _oracle_fp32(xs):
    return (oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin), oracle.norm_rope_fp32(xs.k, xs.gk, xs.cos, xs.sin))


def _oracle_chain(xs, style):
    """Oracle chain outputs and, per element, the magnitude max(|n_d|, |n_partner|)
    of the two normalised values the rotation combines."""
    norm = oracle.norm_hf_bf16 if style == "hf" else oracle.norm_legacy_bf16
    out = []
    for x, g in ((xs.q, xs.gq), (xs.k, xs.gk)):
        y = norm(x, g)
        half = y.shape[-1] // 2
        scale = torch.maximum(y.float().abs(), torch.cat([y[..., half:], y[..., :half]], -1).float().abs())
        out.append((oracle.rope_hf_bf16(y, xs.cos, xs.sin) if xs.cos is not None else y, scale))
    return out


@pytest.mark.parametrize("seed", [1701, 2803, 3907])
def test_config1_fp32_gate(gpu, seed):
    """Config 1: B=1, S=128, Qwen3-8B heads, theta=1e6; FP32 style passes the gate."""
    xs = make_inputs(1, 128, QWEN3_8B, seed)
    announce(f"norm_rope fp32 B=1 S=128 seed={seed}")
    qn, kn = norm_rope(*[t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin)], norm_style="fp32")
    torch.cuda.synchronize()
    rq, rk = _oracle_fp32(xs)
    for got, ref in ((qn, rq), (kn, rk)):
        m = oracle.norm_rope_gate(got.cpu(), ref)
        assert m["pass"], m


@pytest.mark.parametrize("style", ["hf", "legacy"])
@pytest.mark.parametrize("b,s,geom", [(1, 128, QWEN3_8B), (2, 33, QWEN3_8B), (1, 129, GEMMA3_12B)])
def test_bf16_chain_styles(gpu, style, b, s, geom):
    """HF / legacy rounding chains equal the oracle's restated chain (<= 1 ulp, rare)."""
    xs = make_inputs(b, s, geom, 4909)
    announce(f"norm_rope {style} B={b} S={s} geom={geom}")
    qn, kn = norm_rope(*[t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin)], norm_style=style)
    torch.cuda.synchronize()
    for got, (ref, scale) in zip((qn.cpu(), kn.cpu()), _oracle_chain(xs, style)):
        # A last-bit difference of the FP32 inverse RMS can flip one rounding of a
        # normalised value or RoPE product (one ulp of |n|), plus the final rounding.
        diff = (got.float() - ref.float()).abs()
        tol = bf16_ulp(scale) + bf16_ulp(ref)
        assert bool((diff <= tol).all()), float((diff / tol).max())
        assert float((diff > 0).float().mean()) < 2e-3


@pytest.mark.parametrize("b,s,geom", [(1, 33, QWEN3_8B), (1, 129, QWEN3_8B), (2, 64, GEMMA3_12B)])
def test_tails_and_d256_fp32(gpu, b, s, geom):
    xs = make_inputs(b, s, geom, 13109)
    announce(f"norm_rope fp32 tails B={b} S={s} geom={geom}")
    qn, kn = norm_rope(*[t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin)], norm_style="fp32")
    torch.cuda.synchronize()
    rq, rk = _oracle_fp32(xs)
    for got, ref in ((qn, rq), (kn, rk)):
        m = oracle.norm_rope_gate(got.cpu(), ref)
        assert m["pass"], m


def test_no_rope_norm_only(gpu):
    xs = make_inputs(1, 96, QWEN3_8B, 2909, rope=False)
    announce("norm_rope fp32 no-rope")
    qn, kn = norm_rope(*[t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk)], norm_style="fp32")
    torch.cuda.synchronize()
    for got, x, g in ((qn, xs.q, xs.gq), (kn, xs.k, xs.gk)):
        m = oracle.norm_rope_gate(got.cpu(), oracle.norm_fp32(x, g))
        assert m["pass"], m


def test_prepare_only_k_leaves_q(gpu):
    """prepare_attention(only_k=True) writes K rows only (rope:591-595)."""
    xs = make_inputs(1, 200, QWEN3_8B, 3907).to(gpu)
    qn = torch.full_like(xs.q, 7.0)
    kn = torch.empty_like(xs.k)
    announce("prepare only_k")
    prepare_attention(xs.reference7, qn, kn, only_k=True, rope=True, norm_style="fp32")
    torch.cuda.synchronize()
    assert bool((qn == 7.0).all())
    ref = oracle.norm_rope_fp32(xs.k.cpu(), xs.gk.cpu(), xs.cos.cpu(), xs.sin.cpu())
    assert oracle.norm_rope_gate(kn.cpu(), ref)["pass"]


@pytest.mark.parametrize("b,s", [(1, 512), (1, 2048)])
@pytest.mark.parametrize("style", ["fp32", "hf"])
def test_sweep_small_shapes_whole_tensor(gpu, b, s, style):
    """The two smaller bandwidth-sweep shapes (config 2), every element: the
    FP32 style passes the norm+RoPE gate against the FP32 oracle; the HF
    style passes the reference metric against it and equals the oracle's
    restated HF chain to one ulp on a vanishing fraction of elements."""
    xs = make_inputs(b, s, QWEN3_8B, 1909)
    announce(f"norm_rope {style} sweep shape B={b} S={s}")
    qn, kn = norm_rope(*[t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin)], norm_style=style)
    torch.cuda.synchronize()
    rq, rk = _oracle_fp32(xs)
    for got, ref in ((qn, rq), (kn, rk)):
        m = (oracle.norm_rope_gate if style == "fp32" else oracle.metric)(got.cpu(), ref)
        assert m["pass"], m
    if style == "hf":
        for got, (ref, scale) in zip((qn.cpu(), kn.cpu()), _oracle_chain(xs, style)):
            diff = (got.float() - ref.float()).abs()
            assert bool((diff <= bf16_ulp(scale) + bf16_ulp(ref)).all())
            assert float((diff > 0).float().mean()) < 2e-3


@pytest.mark.parametrize("b,s", [(1, 8192), (4, 2048), (8, 1024), (16, 512)])
def test_full_size_whole_tensor(gpu, b, s):
    """Bandwidth-sweep shapes, every element of Q and K against the FP32
    oracle (norm+RoPE gate), and the RoPE pair-norm invariant everywhere."""
    xs = make_inputs(b, s, QWEN3_8B, 1909)
    g = [t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin)]
    announce(f"norm_rope fp32 full size B={b} S={s} (whole tensor)")
    qn, kn = norm_rope(*g, norm_style="fp32")
    torch.cuda.synchronize()
    for got, ref in zip((qn, kn), _oracle_fp32(xs)):
        m = oracle.norm_rope_gate(got.cpu(), ref)
        assert m["pass"], m
    # pair-norm invariant on the whole tensor (rotation preserves |(y_i, y_i+64)|)
    d = 128
    nq = (g[0].float() * torch.rsqrt(g[0].float().square().mean(-1, keepdim=True) + 1e-6) * g[2].float())
    pre = nq[..., : d // 2].square() + nq[..., d // 2:].square()
    post = qn.float()[..., : d // 2].square() + qn.float()[..., d // 2:].square()
    assert bool(((post - pre).abs() <= pre * 2.0 ** -6 + 1e-3).all())


@pytest.mark.parametrize("style", ["fp32", "hf"])
@pytest.mark.parametrize("b,s,geom", [(1, 1, (3, 1, 128)), (1, 15, (3, 1, 128)), (3, 33, (1, 1, 128)),
                                      (1, 9, (3, 1, 256)), (2, 17, (5, 5, 128))])
def test_odd_heads_and_ragged_positions(gpu, style, b, s, geom):
    """The row kernel takes two heads and 256/(D/8) positions per workgroup.
    Odd head counts (the second head past a tensor's last) and S not a
    multiple of the block (positions past S) redo the last head / row and
    store exactly its bits: outputs match the oracle, and nothing outside the
    output tensors is written (they are views inside sentinel-filled buffers)."""
    xs = make_inputs(b, s, geom, 5151)
    q, k, gq, gk, cos, sin = (t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin))
    pad = 4096  # elements (8 KiB) on each side
    bufs = [torch.full((t.numel() + 2 * pad,), 7.0, dtype=torch.bfloat16, device=gpu) for t in (q, k)]
    qn, kn = (buf[pad:pad + t.numel()].view(t.shape) for buf, t in zip(bufs, (q, k)))
    announce(f"norm_rope {style} odd heads B={b} S={s} geom={geom}")
    norm_rope(q, k, gq, gk, cos, sin, norm_style=style, qn=qn, kn=kn)
    torch.cuda.synchronize()
    for buf in bufs:
        assert bool((buf[:pad] == 7.0).all()) and bool((buf[-pad:] == 7.0).all())
    if style == "fp32":
        for got, ref in zip((qn, kn), _oracle_fp32(xs)):
            m = oracle.norm_rope_gate(got.cpu(), ref)
            assert m["pass"], m
    else:
        for got, (ref, scale) in zip((qn.cpu(), kn.cpu()), _oracle_chain(xs, style)):
            diff = (got.float() - ref.float()).abs()
            assert bool((diff <= bf16_ulp(scale) + bf16_ulp(ref)).all())
    # K-only preparation of the same odd head count
    kn2 = torch.empty_like(k)
    prepare_attention((q, k, None, gq, gk, cos, sin), None, kn2, only_k=True, rope=True, norm_style=style)
    torch.cuda.synchronize()
    assert torch.equal(kn2, kn)


@pytest.mark.parametrize("b,s,geom", [(1, 33, (3, 1, 128)), (2, 17, (5, 5, 128)), (1, 9, (3, 1, 256)), (2, 200, QWEN3_8B)])
def test_in_place_outputs(gpu, b, s, geom):
    """Outputs may alias the inputs (qn=q, kn=k): a lane reads only its own
    rows before writing them, and lanes past S or past the last head write
    nothing, so the in-place result equals the out-of-place one bit for bit."""
    xs = make_inputs(b, s, geom, 6161)
    q, k, gq, gk, cos, sin = (t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin))
    announce(f"norm_rope in place B={b} S={s} geom={geom}")
    ref_q, ref_k = norm_rope(q, k, gq, gk, cos, sin, norm_style="fp32")
    qi, ki = q.clone(), k.clone()
    norm_rope(qi, ki, gq, gk, cos, sin, norm_style="fp32", qn=qi, kn=ki)
    kk = k.clone()
    prepare_attention((q, kk, None, gq, gk, cos, sin), None, kk, only_k=True, rope=True, norm_style="fp32")
    torch.cuda.synchronize()
    assert torch.equal(qi, ref_q) and torch.equal(ki, ref_k) and torch.equal(kk, ref_k)


def test_large_launch_four_heads_odd_and_in_place(gpu):
    """Q+K launches of at least 2^18 rows with S <= 4096 take four heads per
    workgroup: with B=10 and 7 Q and 7 K heads (70 heads per tensor, a partial
    last unit) and S = 1873 (a partial last block), the result passes the
    oracle gate, equals the in-place result bit for bit, and the launch
    record names the instance."""
    from kernelfuser_amd import _lib
    xs = make_inputs(10, 1873, (7, 7, 128), 7171)
    q, k, gq, gk, cos, sin = (t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin))
    announce("norm_rope four heads per workgroup, B=10, 7+7 heads, S=1873")
    qn, kn = norm_rope(q, k, gq, gk, cos, sin, norm_style="fp32")
    assert _lib.last_launches()[0]["kernel"] == "rows_kernel<128, 2, true, false, false, 4>"
    qi, ki = q.clone(), k.clone()
    norm_rope(qi, ki, gq, gk, cos, sin, norm_style="fp32", qn=qi, kn=ki)
    torch.cuda.synchronize()
    assert torch.equal(qi, qn) and torch.equal(ki, kn)
    for got, ref in zip((qn, kn), _oracle_fp32(xs)):
        m = oracle.norm_rope_gate(got.cpu(), ref)
        assert m["pass"], m


@pytest.mark.parametrize("style", ["hf", "legacy"])
def test_large_launch_four_heads_bf16_chains(gpu, style):
    """The four-heads-per-workgroup instances of the HF and legacy rounding
    chains (B=3, 7 Q and 7 K heads, S=1873: 78,666 rows, inside the band
    where these styles use four heads; a partial last unit of heads and a
    partial last block of positions) match the oracle's restated chain to
    one BF16 ulp, and write nothing outside the outputs (views inside
    sentinel-filled buffers)."""
    from kernelfuser_amd import _lib
    xs = make_inputs(3, 1873, (7, 7, 128), 8181)
    q, k, gq, gk, cos, sin = (t.to(gpu) for t in (xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin))
    pad = 4096
    bufs = [torch.full((t.numel() + 2 * pad,), 7.0, dtype=torch.bfloat16, device=gpu) for t in (q, k)]
    qn, kn = (buf[pad:pad + t.numel()].view(t.shape) for buf, t in zip(bufs, (q, k)))
    announce(f"norm_rope {style} four heads per workgroup, B=3, 7+7 heads, S=1873")
    norm_rope(q, k, gq, gk, cos, sin, norm_style=style, qn=qn, kn=kn)
    st = {"hf": 0, "legacy": 1}[style]
    assert _lib.last_launches()[0]["kernel"] == f"rows_kernel<128, {st}, true, false, false, 4>"
    torch.cuda.synchronize()
    for buf in bufs:
        assert bool((buf[:pad] == 7.0).all()) and bool((buf[-pad:] == 7.0).all())
    for got, (ref, scale) in zip((qn.cpu(), kn.cpu()), _oracle_chain(xs, style)):
        diff = (got.float() - ref.float()).abs()
        assert bool((diff <= bf16_ulp(scale) + bf16_ulp(ref)).all())
        assert float((diff > 0).float().mean()) < 2e-3
