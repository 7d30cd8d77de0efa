"""The allocation-free attention entry point, kfmi_launch_attention_bf16_noalloc.

It is kfmi_launch_attention_bf16 with the split-KV workspace taken from a
static per-GPU device array instead of a caller allocation.  Called through
the C ABI, its outputs (out and the KN scratch) must equal those of the
existing entry point given a zero-filled caller workspace, bit for bit (the
same kernels run the same split plan), on consecutive calls whose second
input is smaller (the array keeps the first call's contents).  A plan larger
than the array runs unsplit, bit for bit as the existing entry point given
no workspace.  Its callers include code under HIP graph capture: the first
test makes the process's first call of the entry point inside a capture
(the static array's address is resolved there) and replays the graph.
"""
import pytest
import torch

from helpers import announce
from kernelfuser_amd import GEMMA3_12B, QWEN3_8B, _lib, attention_workspace_bytes, make_inputs
from kernelfuser_amd._lib import MODE_FULL, MODE_QUERY, NORM_STYLES, ptr

pytestmark = pytest.mark.gpu


def _entry(name):
    lib = _lib.load()
    return lib, getattr(lib, name)


def _launch(xs, out, kn, causal, mode, noalloc, work=None):
    b, h, s, d = xs.q.shape
    stream = torch.cuda.current_stream(xs.q.device).cuda_stream
    args = [ptr(xs.q), ptr(xs.k), ptr(xs.v), ptr(xs.gq), ptr(xs.gk), ptr(xs.cos), ptr(xs.sin), ptr(out), None,
            ptr(kn), None, b, h, xs.k.shape[1], s, d, float(d) ** -0.5, 1e-6, int(causal), mode,
            NORM_STYLES["fp32"], 128, 64]
    if noalloc:
        lib, fn = _entry("kfmi_launch_attention_bf16_noalloc")
        rc = fn(*args, stream)
    else:
        lib, fn = _entry("kfmi_launch_attention_bf16")
        rc = fn(*args, ptr(work), 0 if work is None else work.numel(), stream)
    return rc, lib.kfmi_last_error().decode()


def _compare(xs, causal, mode):
    b, h, s, d = xs.q.shape
    nbytes = attention_workspace_bytes(b, h, xs.k.shape[1], s, d, causal)
    work = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=xs.q.device)
    outs = []
    for noalloc in (False, True):
        out = torch.full_like(xs.q, float("nan"))
        kn = torch.full_like(xs.k, float("nan"))
        rc, msg = _launch(xs, out, kn, causal, mode, noalloc, work)
        assert rc == 0, msg
        outs.append((out, kn))
    torch.cuda.synchronize()
    (o1, k1), (o2, k2) = outs
    assert bool(torch.isfinite(o1).all())
    assert torch.equal(o1, o2), float((o1.float() - o2.float()).abs().max())
    if mode == MODE_QUERY:
        assert torch.equal(k1, k2)
    return nbytes


def test_noalloc_first_use_inside_graph_capture(gpu):
    """The process's first calls of the entry point are recorded into a HIP
    graph: a split shape (Gemma-3-12B heads, B=1, S=1536: 96 split pairs,
    the counter fill recorded as a kernel node) and one that does not split
    (Qwen3-8B, B=1, S=1000).  Replays, with eager calls of the entry point
    and synchronisations between them, equal the eager results bit for bit."""
    split = make_inputs(1, 1536, GEMMA3_12B, 2525).to(gpu)
    plain = make_inputs(1, 1000, QWEN3_8B, 2626).to(gpu)
    assert attention_workspace_bytes(1, 16, 8, 1536, 256, True) > 0
    assert attention_workspace_bytes(1, 32, 8, 1000, 128, True) == 0
    cases = [(xs, torch.empty_like(xs.q), torch.empty_like(xs.k)) for xs in (split, plain)]
    announce("noalloc first use inside graph capture: Gemma-3-12B S=1536 (split), Qwen3-8B S=1000")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            rcs = [_launch(xs, out, kn, True, MODE_QUERY, True) for xs, out, kn in cases]
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    assert all(rc == 0 for rc, _ in rcs), rcs
    eager = []
    for xs, _, _ in cases:
        out, kn = torch.full_like(xs.q, float("nan")), torch.full_like(xs.k, float("nan"))
        rc, msg = _launch(xs, out, kn, True, MODE_QUERY, True)
        assert rc == 0, msg
        eager.append((out, kn))
    torch.cuda.synchronize()
    assert all(bool(torch.isfinite(o).all()) for o, _ in eager)
    for i in range(2):
        for _, out, kn in cases:
            out.fill_(float("nan"))
            kn.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for (_, out, kn), (eo, ek) in zip(cases, eager):
            assert torch.equal(out, eo) and torch.equal(kn, ek), i
        again = torch.empty_like(split.q)
        rc, msg = _launch(split, again, torch.empty_like(split.k), True, MODE_QUERY, True)  # eager, same array
        torch.cuda.synchronize()
        assert rc == 0 and torch.equal(again, eager[0][0]), (i, msg)


@pytest.mark.parametrize("mode", [MODE_QUERY, MODE_FULL])
def test_noalloc_matches_workspace_entry_twice(gpu, mode):
    """Gemma-3-4B heads at B=1, S=2048 (a 16 MiB split plan), then a smaller
    split input (Gemma-3-4B heads, B=1, S=1000), then a shape that does not
    split (Qwen3-8B, B=1, S=1000)."""
    first = make_inputs(1, 2048, (8, 4, 256), 2121).to(gpu)
    announce(f"noalloc mode={mode} Gemma-3-4B B=1 S=2048 causal")
    n1 = _compare(first, True, mode)
    assert n1 > 16 << 20
    second = make_inputs(1, 1000, (8, 4, 256), 2222).to(gpu)
    announce(f"noalloc mode={mode} Gemma-3-4B B=1 S=1000 causal (smaller, after the first)")
    assert 0 < _compare(second, True, mode) < n1
    third = make_inputs(1, 1000, QWEN3_8B, 2323).to(gpu)
    announce(f"noalloc mode={mode} Qwen3-8B B=1 S=1000 causal (no split)")
    assert _compare(third, True, mode) == 0


def test_noalloc_oversized_plan_runs_unsplit(gpu):
    """B=1, Hq=Hkv=84, S=384, D=256 splits two of its three query blocks per
    head (168 pairs, 45 MiB, more than the 36 MiB array): the call runs
    unsplit, bit for bit as the workspace entry point given no workspace."""
    xs = make_inputs(1, 384, (84, 84, 256), 2424).to(gpu)
    assert attention_workspace_bytes(1, 84, 84, 384, 256, True) > 36 << 20
    announce("noalloc oversized plan (unsplit)")
    res = []
    for noalloc in (True, False):
        out, kn = torch.full_like(xs.q, float("nan")), torch.full_like(xs.k, float("nan"))
        rc, msg = _launch(xs, out, kn, True, MODE_QUERY, noalloc, None)
        assert rc == 0, msg
        plan = [r["plan"] for r in _lib.last_launches() if r["kernel"].startswith("attn_")]
        res.append((out, kn, plan))
    torch.cuda.synchronize()
    (o1, k1, p1), (o2, k2, p2) = res
    assert p1 == p2 and p1[0].startswith("split=0"), (p1, p2)
    assert bool(torch.isfinite(o1).all())
    assert torch.equal(o1, o2) and torch.equal(k1, k2)


def test_noalloc_seeded_sequence_of_split_plans(gpu):
    """Twelve D=256 shapes drawn from a fixed seed (Gemma-3-4B and -12B heads,
    B in 1..2, S in 65..2100, mostly causal) run back to back: split plans of
    6-33 MiB in varying order of size, with unsplit shapes between them, so
    each call finds the array as a different plan left it.  Every call equals
    the workspace entry point bit for bit."""
    import random

    rng = random.Random(3131)
    for i in range(12):
        geom = rng.choice([(8, 4, 256), (16, 8, 256)])
        b = rng.choice([1, 1, 2])
        s = rng.randint(65, 2100)
        causal = rng.random() < 0.75
        assert attention_workspace_bytes(b, geom[0], geom[1], s, geom[2], causal) <= 36 << 20
        xs = make_inputs(b, s, geom, 3200 + i).to(gpu)
        announce(f"noalloc sequence {i}: {geom} B={b} S={s} causal={causal}")
        _compare(xs, causal, MODE_QUERY)
