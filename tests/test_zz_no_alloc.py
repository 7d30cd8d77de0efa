"""The allocation-free attention entry point, kfmi_launch_attention_bf16_noalloc.

It is kfmi_launch_attention_bf16 with the split-KV workspace taken from a
static per-GPU device array instead of a caller allocation.  Called through
the C ABI, its outputs (out and the KN scratch) must equal those of the
existing entry point given a zero-filled caller workspace, bit for bit (the
same kernels run the same split plan), on consecutive calls whose second
input is smaller (the array keeps the first call's contents).  A plan larger
than the array is refused before anything is launched.
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


@pytest.mark.parametrize("mode", [MODE_QUERY, MODE_FULL])
def test_noalloc_matches_workspace_entry_twice(gpu, mode):
    """Gemma-3-12B heads at B=1, S=2048 (a 32.5 MiB split plan), then a smaller
    split input (Gemma-3-4B heads, B=1, S=1000), then a shape that does not
    split (Qwen3-8B, B=1, S=1000)."""
    first = make_inputs(1, 2048, GEMMA3_12B, 2121).to(gpu)
    announce(f"noalloc mode={mode} Gemma-3-12B B=1 S=2048 causal")
    assert _compare(first, True, mode) > 30 << 20
    second = make_inputs(1, 1000, (8, 4, 256), 2222).to(gpu)
    announce(f"noalloc mode={mode} Gemma-3-4B B=1 S=1000 causal (smaller, after the first)")
    assert 0 < _compare(second, True, mode) < 30 << 20
    third = make_inputs(1, 1000, QWEN3_8B, 2323).to(gpu)
    announce(f"noalloc mode={mode} Qwen3-8B B=1 S=1000 causal (no split)")
    assert _compare(third, True, mode) == 0


def test_noalloc_refuses_oversized_plan(gpu):
    """B=1, Hq=128, Hkv=128, S=192, D=256 splits into 256 (block, head) pairs
    (65 MiB): refused with KFMI_EINVAL and a message, nothing written."""
    xs = make_inputs(1, 192, (128, 128, 256), 2424).to(gpu)
    assert attention_workspace_bytes(1, 128, 128, 192, 256, True) > 36 << 20
    out = torch.full_like(xs.q, 7.0)
    kn = torch.full_like(xs.k, 7.0)
    announce("noalloc oversized plan")
    rc, msg = _launch(xs, out, kn, True, MODE_QUERY, True)
    torch.cuda.synchronize()
    assert rc == _lib.KFMI_EINVAL and "exceeds the static scratch" in msg, (rc, msg)
    assert bool((out == 7.0).all()) and bool((kn == 7.0).all())
