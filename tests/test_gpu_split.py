"""Split-KV execution of the general attention kernel at D = 256 (one
workgroup per CU): for causal shapes with fewer work items than CUs, the
longest query blocks' key ranges are split over two workgroups and merged by
the one finishing second.

Results are bit-identical from launch to launch (the merge runs in a fixed
order whichever half performs it), within a few ulp of the unsplit launch
(each half rounds its probabilities relative to its own running max), pass
the oracle gate, and stay correct over repeated launches and graph replays
(the merge counters re-arm themselves)."""
import pytest
import torch

import oracle
from helpers import announce, bf16_ulp
from kernelfuser_amd import attention_prefill, attention_workspace_bytes, make_inputs, prepare_attention

pytestmark = pytest.mark.gpu


def _run(xs, kn, causal, work, style="fp32"):
    out = torch.empty_like(xs.q)
    attention_prefill(xs.q, kn, xs.v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin, causal=causal, norm_style=style,
                      work=work)
    return out


@pytest.mark.parametrize("geom,b,s", [((16, 8, 256), 1, 1536), ((16, 8, 256), 1, 1900), ((8, 4, 256), 1, 2048),
                                      ((4, 2, 256), 1, 1000)])
def test_split_matches_unsplit(gpu, geom, b, s):
    hq, hkv, d = geom
    nbytes = attention_workspace_bytes(b, hq, hkv, s, d, True)
    assert nbytes > 0, "shape expected to split"
    xs = make_inputs(b, s, geom, 1212).to(gpu)
    kn = torch.empty_like(xs.k)
    prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="fp32")
    work = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    announce(f"split {geom} B={b} S={s} ({nbytes} B workspace)")
    ref_unsplit = _run(xs, kn, True, torch.empty(0, dtype=torch.uint8, device=gpu))
    first = _run(xs, kn, True, work)
    second = _run(xs, kn, True, work)  # counters must have re-armed
    torch.cuda.synchronize()
    pairs = nbytes // (2 * (d // 2 + 2) * 256 * 4)  # one counter per split (block, head) pair
    counters = work[:4 * pairs].view(torch.int32)
    assert int(counters.abs().sum()) == 0, counters.nonzero().flatten().tolist()[:8]  # re-armed
    assert torch.equal(first, second), float((first.float() - second.float()).abs().max())
    # each half rounds its probabilities to BF16 relative to its own running
    # max, so split rows differ from unsplit ones by a few ulp (a wrong merge
    # would be off by O(0.1))
    d_ = (first.float() - ref_unsplit.float()).abs()
    tol = 4 * bf16_ulp(torch.maximum(first.float().abs(), ref_unsplit.float().abs())) + 1e-3
    assert bool((d_ <= tol).all()), float((d_ / tol).max())
    rows = torch.unique(torch.cat([torch.arange(0, 3), torch.randint(0, s, (30,), generator=torch.Generator().manual_seed(s)),
                                   torch.arange(s - 130, s)]))
    ref = oracle.oracle_rows_fp32(*[t.cpu() for t in xs.astuple()], rows, True)
    assert oracle.attention_gate(first[:, :, rows.to(gpu)].cpu(), ref)["pass"]


def test_split_graph_replays(gpu):
    xs = make_inputs(1, 1536, (16, 8, 256), 1313).to(gpu)
    kn = torch.empty_like(xs.k)
    prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="hf")
    work = torch.zeros(attention_workspace_bytes(1, 16, 8, 1536, 256, True), dtype=torch.uint8, device=gpu)
    out = torch.empty_like(xs.q)
    fn = lambda: attention_prefill(xs.q, kn, xs.v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin, causal=True,
                                   norm_style="hf", work=work)
    announce("split graph replays")
    fn()
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        fn()  # eager launches between replays share the workspace
        torch.cuda.synchronize()
        assert torch.equal(out, eager)



def test_split_cached_workspace_per_stream(gpu):
    """With work=None each (device, stream) gets its own cached workspace, so
    split launches on two streams at once do not share counters or partials:
    both streams reproduce the single-stream result bit for bit."""
    xs = make_inputs(1, 1536, (16, 8, 256), 1515).to(gpu)
    kn = torch.empty_like(xs.k)
    prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="fp32")
    announce("split cached workspace on two streams")
    ref = _run(xs, kn, True, None)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.empty_like(xs.q) for _ in streams]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for _ in range(4):
        for st, out in zip(streams, outs):
            with torch.cuda.stream(st):
                attention_prefill(xs.q, kn, xs.v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin, causal=True,
                                  norm_style="fp32")
    torch.cuda.synchronize()
    for out in outs:
        bad = out != ref
        assert not bool(bad.any()), (int(bad.sum()), float((out.float() - ref.float()).abs().max()),
                                     bad.nonzero()[:4].tolist())


def test_workspace_serves_any_shape_sequence(gpu):
    """One zero-filled workspace serves any sequence of split shapes: the
    arrival counters sit in a region of the same size for every shape and no
    shape's partial results land in it.  A 12-pair plan (Hq=4, S=640) run on
    a workspace sized for a 96-pair plan (Hq=16, S=1536) leaves the larger
    plan's whole counter region at zero, and the larger shape then gives the
    same bits as on a fresh workspace."""
    small = make_inputs(1, 640, (4, 2, 256), 2121).to(gpu)
    large = make_inputs(1, 1536, (16, 8, 256), 2222).to(gpu)
    kn_s, kn_l = torch.empty_like(small.k), torch.empty_like(large.k)
    prepare_attention(small.reference7, None, kn_s, only_k=True, norm_style="fp32")
    prepare_attention(large.reference7, None, kn_l, only_k=True, norm_style="fp32")
    nb_s = attention_workspace_bytes(1, 4, 2, 640, 256, True)
    nb_l = attention_workspace_bytes(1, 16, 8, 1536, 256, True)
    per_pair = 2 * (256 // 2 + 2) * 256 * 4
    assert 0 < nb_s < nb_l and nb_l // per_pair == 96 and nb_s // per_pair == 12
    counter_region = nb_l - (nb_l // per_pair) * per_pair
    announce("split workspace reused from a 12-pair to a 96-pair plan")
    work = torch.zeros(nb_l, dtype=torch.uint8, device=gpu)
    for _ in range(2):
        _run(small, kn_s, True, work)
    torch.cuda.synchronize()
    assert int(work[:counter_region].count_nonzero()) == 0
    fresh = _run(large, kn_l, True, torch.zeros(nb_l, dtype=torch.uint8, device=gpu))
    reused = _run(large, kn_l, True, work)
    torch.cuda.synchronize()
    assert torch.equal(reused, fresh)
    assert int(work[:counter_region].count_nonzero()) == 0


def test_captured_split_keeps_its_workspace(gpu):
    """A launch captured with work=None gets a workspace of its own from the
    graph's memory pool, also when the capture comes before any eager launch
    on that stream (it still splits: its output equals the eager split
    output bit for bit, which differs from the unsplit one).  Growing the
    eager cache afterwards (a larger split shape on the same stream) must not
    disturb replays, which are compared bit for bit with eager results."""
    small = make_inputs(1, 2048, (8, 4, 256), 1717).to(gpu)
    large = make_inputs(1, 1536, (16, 8, 256), 1818).to(gpu)
    kn_s, kn_l = torch.empty_like(small.k), torch.empty_like(large.k)
    prepare_attention(small.reference7, None, kn_s, only_k=True, norm_style="fp32")
    prepare_attention(large.reference7, None, kn_l, only_k=True, norm_style="fp32")
    torch.cuda.synchronize()
    out = torch.empty_like(small.q)
    fn = lambda: attention_prefill(small.q, kn_s, small.v, out, gq=small.gq, cos=small.cos, sin=small.sin,
                                   causal=True, norm_style="fp32")
    announce("split capture before eager use, then cache growth")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            fn()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    unsplit = _run(small, kn_s, True, torch.empty(0, dtype=torch.uint8, device=gpu))
    split = _run(small, kn_s, True, None)
    torch.cuda.synchronize()
    assert not torch.equal(split, unsplit), "shape expected to split"
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, split), i
        big = _run(large, kn_l, True, None)  # grows this stream's cached workspace
        again = _run(small, kn_s, True, None)
        torch.cuda.synchronize()
        assert torch.equal(again, split), i
    ref = oracle.oracle_rows_fp32(*[t.cpu() for t in large.astuple()], torch.arange(1528, 1536), True)
    assert oracle.attention_gate(big[:, :, 1528:].cpu(), ref)["pass"]


@pytest.mark.parametrize("geom,b,s", [((8, 4, 256), 1, 2048), ((16, 8, 256), 1, 1536), ((4, 2, 256), 2, 1000)])
def test_factored_split_matches_unsplit(gpu, geom, b, s):
    """The factored no-RoPE launch (qk:641-652) on the split plan: its
    attention launch takes the same workspace.  With the cached workspace
    (work=None) the launch record shows the split, the output passes the
    oracle gate on the whole tensor and lies within a few ulp of the unsplit
    launch (an empty workspace), and INV (written by both halves of a split
    block, the same values) equals the oracle's."""
    from kernelfuser_amd import launch_factored_attention

    hq, hkv, d = geom
    assert attention_workspace_bytes(b, hq, hkv, s, d, True) > 0, "shape expected to split"
    xs = make_inputs(b, s, geom, 1313, rope=False)
    g = xs.to(gpu)
    announce(f"factored split {geom} B={b} S={s}")
    res = []
    for work in (None, torch.empty(0, dtype=torch.uint8, device=gpu)):
        out = torch.full_like(g.q, float("nan"))
        inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
        kn = torch.empty_like(g.k)
        recs = [r for r in launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=True, work=work)
                if r["kernel"].startswith("attn_")]
        res.append((out, inv, recs[0]["plan"]))
    torch.cuda.synchronize()
    (split, inv_s, plan_s), (unsplit, inv_u, plan_u) = res
    assert not plan_s.startswith("split=0") and plan_u.startswith("split=0"), (plan_s, plan_u)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True, head_chunk=8)
    m = oracle.attention_gate(split.cpu(), ref)
    assert m["pass"], m
    d_ = (split.float() - unsplit.float()).abs()
    tol = 4 * bf16_ulp(torch.maximum(split.float().abs(), unsplit.float().abs())) + 1e-3
    assert bool((d_ <= tol).all()), float((d_ / tol).max())
    inv_ref = oracle.rms_inverse(xs.q.float())[..., 0]
    assert torch.equal(inv_s, inv_u) and torch.allclose(inv_s.cpu(), inv_ref, rtol=1e-6, atol=0)
