"""Per-workgroup clock stamps of the attention kernels (kfmi_clock_stamps,
kfmi_tuning.clock_stamps): every workgroup of a recording launch writes one
entry, up to KFMI_CLOCK_STAMPS_MAX; the shader clock each implies lies in a
physical range; and the launch's outputs are bit for bit those of the same
launch without stamps.  Covers the ping-pong kernel (persistent pairing),
the general kernel (plain, and the D=256 split plan, whose halves exit
through the publish-only and merging paths), the wide kernel, and a grid
larger than the array."""
import pytest
import torch

from helpers import announce
from kernelfuser_amd import GEMMA3_12B, QWEN3_8B, _lib, attention_workspace_bytes, launch_attention, make_inputs

pytestmark = pytest.mark.gpu


def _launch(xs, causal, kernel="auto", work=None):
    out = torch.full_like(xs.q, float("nan"))
    kn = torch.empty_like(xs.k)
    with _lib.tuning(attn_kernel=kernel):
        recs = list(launch_attention(xs.reference7, out, causal=causal, mode="query", kn=kn, norm_style="fp32",
                                     work=work))
    torch.cuda.synchronize()
    return out, [r for r in recs if r["kernel"].startswith("attn_")][0]


def _stamped(xs, causal, kernel="auto", work=None):
    plain, rec = _launch(xs, causal, kernel, work)
    with _lib.tuning(attn_kernel=kernel, clock_stamps=1):
        out = torch.full_like(xs.q, float("nan"))
        kn = torch.empty_like(xs.k)
        recs = list(launch_attention(xs.reference7, out, causal=causal, mode="query", kn=kn, norm_style="fp32",
                                     work=work))
    stamps = _lib.clock_stamps()
    rec2 = [r for r in recs if r["kernel"].startswith("attn_")][0]
    assert rec2["kernel"] == rec["kernel"] and rec2["grid"] == rec["grid"]
    assert torch.equal(out, plain), "stamps changed the results"
    return rec2, stamps


def _check(stamps, grid):
    assert len(stamps) == min(grid, _lib.CLOCK_STAMPS_MAX)
    assert all(t1 > t0 and r1 > r0 for t0, t1, r0, r1 in stamps)
    c = _lib.clock_summary(stamps)
    assert 0.3 < c["ghz_min"] <= c["ghz_median"] <= c["ghz_max"] < 3.5, c
    return c


@pytest.mark.parametrize("b,s,kernel", [(1, 4096, "pingpong"), (1, 2048, "general"), (4, 1000, "wide")])
def test_stamps_every_workgroup(gpu, b, s, kernel):
    xs = make_inputs(b, s, QWEN3_8B, 5151).to(gpu)
    announce(f"clock stamps {kernel} B={b} S={s} causal")
    rec, stamps = _stamped(xs, True, kernel)
    assert rec["kernel"].startswith({"pingpong": "attn_pp_kernel", "general": "attn_fwd_kernel",
                                     "wide": "attn_ww_kernel"}[kernel])
    _check(stamps, rec["grid"])


def test_stamps_split_halves(gpu):
    """Gemma-3-12B heads, B=1, S=1536: the split plan's halves end either
    after publishing their partial state or after merging both."""
    xs = make_inputs(1, 1536, GEMMA3_12B, 5252).to(gpu)
    nbytes = attention_workspace_bytes(1, 16, 8, 1536, 256, True)
    assert nbytes > 0
    work = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    announce("clock stamps general D=256 split B=1 S=1536 causal")
    rec, stamps = _stamped(xs, True, "auto", work)
    assert rec["plan"].startswith("split=") and not rec["plan"].startswith("split=0"), rec
    _check(stamps, rec["grid"])


def test_stamps_grid_larger_than_array(gpu):
    """B=4, S=4096, not causal, general kernel forced: 4096 workgroups; the
    first KFMI_CLOCK_STAMPS_MAX record."""
    xs = make_inputs(4, 4096, QWEN3_8B, 5353).to(gpu)
    announce("clock stamps general B=4 S=4096 non-causal (4096 workgroups)")
    rec, stamps = _stamped(xs, False, "general")
    assert rec["grid"] == 4096
    _check(stamps, rec["grid"])
