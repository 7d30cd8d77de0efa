"""Rows past S are never read from memory beyond a tensor.

The attention kernels copy whole 64-row K/V tiles (and 128-row rotary-table
blocks) with buffer loads whose descriptor spans exactly one head's S rows;
the rows of a ragged last tile must arrive as zeros.  Here every tensor the
kernels read by tiles (KN or raw K, V, cos, sin) is a view at the START of an
allocation whose remainder is NaN, so the last head's tail is followed by NaN
instead of another head's finite rows.  A tile copy that read past its
descriptor would put 0 * NaN into P.V and the stored rows would be NaN.  The
guard is allocated memory, so no variant of the kernels can fault here.

Shapes: the general kernel's ragged grids (S=33, S=129, and B=4 S=1000
forced onto it), the ping-pong kernel's (B=4 S=1000, S=2970, S=3200), D=256 with the split-KV plan (S=1900,
Gemma-3-12B heads), mode 'full' (raw K tiles) and the factored path.
"""
import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import GEMMA3_12B, QWEN3_8B, _lib, launch_attention, launch_factored_attention, make_inputs

pytestmark = pytest.mark.gpu

GUARD_ELEMS = 64 * 1024  # 128 KiB of NaN after each tensor (a tile reads at most 32 KiB past S)


def guarded(t: torch.Tensor, device) -> torch.Tensor:
    """A contiguous copy of ``t`` at the start of a NaN-filled allocation."""
    buf = torch.full((t.numel() + GUARD_ELEMS,), float("nan"), dtype=t.dtype, device=device)
    view = buf[: t.numel()].view(t.shape)
    view.copy_(t.to(device))
    assert view.data_ptr() % 256 == 0
    return view


def _rows(s):
    """Two rows of every query block plus the last four rows."""
    return torch.unique(torch.cat([torch.arange(0, s, 128), torch.arange(min(61, s - 1), s, 128), torch.arange(max(0, s - 4), s)]))


def _check(out, ref_fn, s):
    assert bool(torch.isfinite(out).all()), "non-finite output rows"
    rows = _rows(s)
    m = oracle.attention_gate(out[:, :, rows.to(out.device)].cpu(), ref_fn(rows))
    assert m["pass"], m


@pytest.mark.parametrize("b,s,kernel", [(4, 1000, "auto"), (4, 1000, "general"), (1, 33, "auto"), (1, 129, "auto"),
                                          (1, 2970, "auto"), (1, 3200, "auto")])
@pytest.mark.parametrize("mode", ["query", "full"])
def test_qwen3_ragged_tiles_read_zeros(gpu, b, s, kernel, mode):
    xs = make_inputs(b, s, QWEN3_8B, 4949)
    q = xs.q.to(gpu)
    k = guarded(xs.k, gpu)
    v = guarded(xs.v, gpu)
    cos, sin = guarded(xs.cos, gpu), guarded(xs.sin, gpu)
    gq, gk = xs.gq.to(gpu), xs.gk.to(gpu)
    kn = guarded(torch.zeros_like(xs.k), gpu)
    out = torch.full_like(q, float("nan"))
    announce(f"guard {mode} fp32 B={b} S={s} causal kernel={kernel}")
    with _lib.tuning(attn_kernel=kernel):
        launch_attention((q, k, v, gq, gk, cos, sin), out, causal=True, mode=mode, kn=kn, norm_style="fp32")
    torch.cuda.synchronize()
    _check(out, lambda rows: oracle.oracle_rows_fp32(*xs.astuple(), rows, True), s)


@pytest.mark.parametrize("causal", [True, False])
def test_d256_split_ragged_tiles_read_zeros(gpu, causal):
    """Gemma-3-12B heads with RoPE, B=1, S=1900: 15 query blocks x 16 heads fit
    one workgroup per CU, so the causal launch splits its longest blocks."""
    b, s = 1, 1900
    xs = make_inputs(b, s, GEMMA3_12B, 5959)
    q = xs.q.to(gpu)
    v = guarded(xs.v, gpu)
    cos, sin = guarded(xs.cos, gpu), guarded(xs.sin, gpu)
    kn = guarded(torch.zeros_like(xs.k), gpu)
    out = torch.full_like(q, float("nan"))
    announce(f"guard D=256 query fp32 B={b} S={s} causal={causal}")
    launch_attention((q, xs.k.to(gpu), v, xs.gq.to(gpu), xs.gk.to(gpu), cos, sin), out, causal=causal,
                     mode="query", kn=kn, norm_style="fp32")
    torch.cuda.synchronize()
    _check(out, lambda rows: oracle.oracle_rows_fp32(*xs.astuple(), rows, causal), s)


@pytest.mark.parametrize("b,s", [(1, 1900), (2, 1000)])
def test_factored_ragged_tiles_read_zeros(gpu, b, s):
    xs = make_inputs(b, s, GEMMA3_12B, 6969, rope=False)
    q = xs.q.to(gpu)
    v = guarded(xs.v, gpu)
    kn = guarded(torch.zeros_like(xs.k), gpu)
    inv = torch.empty(q.shape[:-1], device=gpu, dtype=torch.float32)
    out = torch.full_like(q, float("nan"))
    announce(f"guard factored D=256 B={b} S={s} causal")
    launch_factored_attention((q, xs.k.to(gpu), v, xs.gq.to(gpu), xs.gk.to(gpu)), out, inv, kn, causal=True)
    torch.cuda.synchronize()

    def ref(rows):
        full = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, True)
        return full[:, :, rows]
    _check(out, ref, s)
