"""GPU parity of the wide-wave attention kernel (attn_ww_kernel) against the
CPU FP32 oracle (src/e1_rope_publication_v1.py:295-302; no-RoPE / factored:
:736-742 and src/e1_qk_publication_v3.py:612-638), on shapes the shape-based
dispatch would send to other kernels: the kernel is forced through the
library's tuning overrides (kfmi_set_tuning), and every test checks from the
launch records that it ran.

Cases: ragged and tiny S (one key tile, a partial tile, tails past a 64-row
block), both causal modes, the FOLD (fp32) and scaled (hf, legacy,
prepared-Q, factored) softmax paths, GQA ratios 4 and 8, head counts that do
not spread over the 8 XCDs, the persistent long/short pairing (B=4, S=1000:
256 pairs), tensors followed by NaN (no read past S), inputs built to
overflow the lean softmax (a spiked key; huge V) so that the exact redo runs,
and one-tile items after a launch that left NaN bits in LDS.
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import QWEN3_8B, _lib, anchor, launch_attention, launch_factored_attention, make_inputs

pytestmark = pytest.mark.gpu

WIDE = "attn_ww_kernel"


def _launch(xs_gpu, causal, mode="query", norm_style="fp32", rope=True, kernel="wide", **tun):
    q = xs_gpu.q
    out = torch.empty_like(q)
    kn = torch.empty_like(xs_gpu.k)
    qn = torch.empty_like(q) if mode == "unfused" else None
    with _lib.tuning(attn_kernel=kernel, **tun):
        recs = list(launch_attention((q, xs_gpu.k, xs_gpu.v, xs_gpu.gq, xs_gpu.gk, xs_gpu.cos, xs_gpu.sin), out,
                                     causal=causal, mode=mode, rope=rope, qn=qn, kn=kn, norm_style=norm_style))
    torch.cuda.synchronize()
    return out.cpu(), recs


def _ran_wide(recs):
    assert any(r["kernel"].startswith(WIDE) for r in recs), recs


@pytest.mark.parametrize("b,s", [(1, 1), (1, 33), (1, 64), (1, 65), (1, 128), (1, 129), (2, 200), (1, 448)])
@pytest.mark.parametrize("causal", [True, False])
def test_wide_fp32_small_and_ragged(gpu, b, s, causal):
    xs = make_inputs(b, s, QWEN3_8B, 7101 + s)
    announce(f"wide query fp32 B={b} S={s} causal={causal}")
    out, recs = _launch(xs.to(gpu), causal)
    _ran_wide(recs)
    m = oracle.attention_gate(out, oracle.oracle_fp32(*xs.astuple(), causal))
    assert m["pass"], m


@pytest.mark.parametrize("style", ["hf", "legacy"])
@pytest.mark.parametrize("mode", ["query", "unfused"])
@pytest.mark.parametrize("s,causal", [(129, True), (300, False)])
def test_wide_scaled_softmax_styles(gpu, style, mode, s, causal):
    """Styles without the folded scale: logits scaled per score (HF and legacy
    prologues; mode 'unfused' runs the prepared-Q prologue)."""
    xs = make_inputs(1, s, QWEN3_8B, 7201)
    announce(f"wide {mode} {style} S={s} causal={causal}")
    out, recs = _launch(xs.to(gpu), causal, mode=mode, norm_style=style)
    _ran_wide(recs)
    m = oracle.metric(out, oracle.oracle_fp32(*xs.astuple(), causal))
    assert m["pass"], m


def test_wide_persistent_pairs_b4_s1000(gpu):
    """B=4, S=1000: 16 query blocks of 64 rows x 32 head quads = 256
    (long, short) units, the persistent form on 256 CUs; ragged last block."""
    xs = make_inputs(4, 1000, QWEN3_8B, 2909)
    announce("wide query fp32 B=4 S=1000 causal (persistent)")
    out, recs = _launch(xs.to(gpu), True)
    _ran_wide(recs)
    m = oracle.attention_gate(out, oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8))
    assert m["pass"], m


def test_wide_persistent_off_matches(gpu):
    """One item per workgroup (persistent pairing off) gives the same bits:
    each item's arithmetic does not depend on where it runs."""
    xs = make_inputs(4, 1000, QWEN3_8B, 2909)
    g = xs.to(gpu)
    announce("wide query fp32 B=4 S=1000 causal, persistent on/off")
    a, ra = _launch(g, True)
    b, rb = _launch(g, True, persistent=1)
    _ran_wide(ra)
    _ran_wide(rb)
    assert ra[-1]["grid"] != rb[-1]["grid"]
    assert torch.equal(a, b)


@pytest.mark.parametrize("geom,b,s", [((32, 4, 128), 1, 300), ((16, 4, 128), 2, 257), ((8, 2, 128), 1, 640)])
def test_wide_gqa_geometries(gpu, geom, b, s):
    """GQA ratio 8 (two head quads per KV head) and KV-head counts that do
    not fill the 8 XCDs (items in plain order)."""
    xs = make_inputs(b, s, geom, 7301)
    announce(f"wide query fp32 geom={geom} B={b} S={s} causal")
    out, recs = _launch(xs.to(gpu), True)
    _ran_wide(recs)
    m = oracle.attention_gate(out, oracle.oracle_fp32(*xs.astuple(), True))
    assert m["pass"], m


@pytest.mark.parametrize("s,causal", [(200, True), (129, False)])
def test_wide_factored_d128(gpu, s, causal):
    """The factored launch (qk:641-652) at D=128: Q's inverse RMS computed in
    the prologue and applied per score."""
    xs = make_inputs(1, s, QWEN3_8B, 7401, rope=False)
    g = xs.to(gpu)
    out = torch.empty_like(g.q)
    inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
    kn = torch.empty_like(g.k)
    announce(f"wide factored D=128 S={s} causal={causal}")
    with _lib.tuning(attn_kernel="wide"):
        recs = launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=causal)
    torch.cuda.synchronize()
    _ran_wide(recs)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, causal)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m
    inv_ref = oracle.rms_inverse(xs.q.float())[..., 0]
    assert torch.allclose(inv.cpu(), inv_ref, rtol=1e-6, atol=0)


GUARD_ELEMS = 64 * 1024


def _guarded(t, device):
    buf = torch.full((t.numel() + GUARD_ELEMS,), float("nan"), dtype=t.dtype, device=device)
    view = buf[: t.numel()].view(t.shape)
    view.copy_(t.to(device))
    return view


@pytest.mark.parametrize("b,s", [(4, 1000), (1, 33), (1, 129), (1, 3200)])
def test_wide_ragged_tiles_read_zeros(gpu, b, s):
    """K, V and the tables end where NaN begins: a tile copy past S would
    bring NaN into the stored rows."""
    xs = make_inputs(b, s, QWEN3_8B, 4949)
    q = xs.q.to(gpu)
    k, v = _guarded(xs.k, gpu), _guarded(xs.v, gpu)
    cos, sin = _guarded(xs.cos, gpu), _guarded(xs.sin, gpu)
    kn = _guarded(torch.zeros_like(xs.k), gpu)
    out = torch.full_like(q, float("nan"))
    announce(f"wide guard query fp32 B={b} S={s} causal")
    with _lib.tuning(attn_kernel="wide"):
        recs = launch_attention((q, k, v, xs.gq.to(gpu), xs.gk.to(gpu), cos, sin), out, causal=True, mode="query",
                                kn=kn, norm_style="fp32")
    torch.cuda.synchronize()
    _ran_wide(recs)
    assert bool(torch.isfinite(out).all()), "non-finite output rows"
    rows = torch.unique(torch.cat([torch.arange(0, s, 64), torch.arange(min(37, s - 1), s, 64),
                                   torch.arange(max(0, s - 4), s)]))
    m = oracle.attention_gate(out[:, :, rows.to(gpu)].cpu(), oracle.oracle_rows_fp32(*xs.astuple(), rows, True))
    assert m["pass"], m


@pytest.mark.parametrize("geom,b,s,causal,mode,style,tun", [
    ((64, 8, 128), 3, 64, False, "unfused", "legacy", {}),
    ((64, 8, 128), 1, 32, False, "unfused", "legacy", {}),
    ((64, 8, 128), 3, 64, True, "query", "hf", {}),
    (QWEN3_8B, 3, 64, False, "query", "fp32", {}),
    (QWEN3_8B, 2, 300, True, "query", "fp32", {"persistent": 1}),
])
def test_wide_one_tile_items_after_nan_in_lds(gpu, geom, b, s, causal, mode, style, tun):
    """Items of one key tile after a launch that left NaN bits in LDS.  The
    wide kernel's last iteration multiplies its second K buffer (scores that
    must give probabilities of 0), which an item of one tile never fills, and
    LDS keeps what earlier workgroups wrote: a wide launch on an all-NaN Q
    first stages NaN output rows through that region.  The NaN row sums must
    send such items to the exact redo; they used to pass the redo check,
    which the compiler had rewritten as a class test assuming no NaN, and the
    items returned NaN rows.  Cases: S <= 64 (one tile per item), and causal
    S=300 with one item per workgroup (block 0 holds one tile).  Three rounds
    each."""
    dirty = make_inputs(3, 700, (64, 8, 128), 8787).to(gpu)
    dirty.q.fill_(float("nan"))
    xs = make_inputs(b, s, geom, 8888 + s + b)
    g = xs.to(gpu)
    ref = oracle.oracle_fp32(*xs.astuple(), causal)
    gate = oracle.attention_gate if style == "fp32" else oracle.metric
    announce(f"wide one-tile items after NaN in LDS {geom} B={b} S={s} causal={causal} {mode} {style} {tun}")
    for _ in range(3):
        dirty_out, _ = _launch(dirty, False, mode="unfused", norm_style="legacy")
        assert not bool(torch.isfinite(dirty_out.float()).any())
        out, recs = _launch(g, causal, mode=mode, norm_style=style, **tun)
        _ran_wide(recs)
        m = gate(out, ref)
        assert m["pass"], m


def _spiked(s, key, k0, vscale, seed):
    g = torch.Generator().manual_seed(seed)
    q = 0.1 * torch.randn(1, 8, s, 128, generator=g)
    k = 0.1 * torch.randn(1, 2, s, 128, generator=g)
    v = vscale * torch.randn(1, 2, s, 128, generator=g)
    q[..., 0] = 8.0
    k[:, :, key, 0] = k0
    return tuple(t.to(torch.bfloat16) for t in (q, k, v))


@pytest.mark.parametrize("kernel", ["wide", "general"])
@pytest.mark.parametrize("causal", [True, False])
def test_lean_overflow_redo_spiked_key(gpu, kernel, causal):
    """One key's logit ~163 log2 units above the first tile's maximum:
    probabilities overflow on the lean path, so the item is redone exactly."""
    s, key = 700, 300
    q, k, v = _spiked(s, key, 160.0, 1.0, 4242)
    announce(f"{kernel} lean redo spiked key S={s} causal={causal}")
    with _lib.tuning(attn_kernel=kernel):
        out = anchor(q.to(gpu), k.to(gpu), v.to(gpu), None, None, causal)
        recs = _lib.last_launches()
    torch.cuda.synchronize()
    out = out.cpu()
    if kernel == "wide":
        _ran_wide(recs)
    assert torch.isfinite(out.float()).all()
    m = oracle.attention_gate(out, oracle.attention_fp32(q, k, v, causal))
    assert m["pass"], m


@pytest.mark.parametrize("kernel", ["wide", "general"])
def test_lean_overflow_redo_huge_v(gpu, kernel):
    """A key ~50 log2 units above the first tile's maximum keeps every row sum
    finite (about 2^50) but, with |V| ~ 1e24, overflows the lean path's
    accumulators; the exact softmax keeps them finite.  Compared relative to
    the scale of V."""
    s, key, vs = 700, 300, 1e24
    q, k, v = _spiked(s, key, 50.0, vs, 4343)
    announce(f"{kernel} lean redo huge V S={s} causal")
    with _lib.tuning(attn_kernel=kernel):
        out = anchor(q.to(gpu), k.to(gpu), v.to(gpu), None, None, True)
    torch.cuda.synchronize()
    out = out.cpu().float()
    assert torch.isfinite(out).all()
    ref = oracle.attention_fp32(q, k, v, True)
    m = oracle.attention_gate((out / vs).to(torch.bfloat16), ref / vs)
    assert m["pass"], m


def test_pingpong_still_runs_s4096_rows(gpu):
    """The ping-pong kernel forced at S=4096 (its shape-based choice too)
    beside the wide-kernel tests, on a row sample."""
    s = 4096
    xs = make_inputs(1, s, QWEN3_8B, 3909)
    announce("pingpong forced query fp32 B=1 S=4096 causal")
    out, recs = _launch(xs.to(gpu), True, kernel="pingpong")
    assert any(r["kernel"].startswith("attn_pp_kernel") for r in recs), recs
    rows = torch.unique(torch.cat([torch.arange(0, 4), torch.arange(0, s, 131), torch.arange(s - 4, s)]))
    m = oracle.attention_gate(out[:, :, rows], oracle.oracle_rows_fp32(*xs.astuple(), rows, True))
    assert m["pass"], m
