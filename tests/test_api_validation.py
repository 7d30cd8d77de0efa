"""Argument rules of the reference-signature ops, on CPU tensors (no GPU).

``optimized_attention`` raises ValueError before any launch for each rule of
src/e1_rope_publication_v1.py:695-719, in the reference's order; the
launchers raise 'Invalid fusion mode' / 'Missing scratch buffers'
(rope:668-672).  A valid call on CPU tensors stops at the device rule, so
each case below is checked against the message of the rule it breaks.
"""
import math

import pytest
import torch

import kernelfuser_amd as kf
from kernelfuser_amd.inputs import make_inputs


@pytest.fixture(scope="module")
def xs():
    return make_inputs(1, 16, (4, 2, 128), 3)


def _args(xs, **over):
    a = dict(q=xs.q, k=xs.k, v=xs.v, gq=xs.gq, gk=xs.gk, cos=xs.cos, sin=xs.sin)
    a.update(over)
    return a


def _call(a, **kw):
    return kf.optimized_attention(a["q"], a["k"], a["v"], a["gq"], a["gk"], a["cos"], a["sin"], **kw)


@pytest.mark.parametrize("kw,msg", [
    (dict(mode="full"), "mode"), (dict(mode="bad"), "mode"), (dict(bn=32), "bn"), (dict(bn=256), "bn"),
    (dict(norm_style="bf16"), "norm_style"),
])
def test_mode_bn_style(xs, kw, msg):
    with pytest.raises(ValueError, match=msg):
        _call(_args(xs), **kw)


def test_one_table_only(xs):
    with pytest.raises(ValueError, match="rotary tables"):
        _call(_args(xs, sin=None))


def test_requires_grad(xs):
    with pytest.raises(ValueError, match="forward-only"):
        _call(_args(xs, q=xs.q.clone().float().requires_grad_()))


@pytest.mark.parametrize("over", [
    lambda xs: dict(q=xs.q[0]),                                 # q not 4-D
    lambda xs: dict(v=xs.v[:, :, :8]),                          # k.shape != v.shape
])
def test_ranks_and_kv_shapes(xs, over):
    with pytest.raises(ValueError, match=r"Expected q \[B,Hq,S,D\]"):
        _call(_args(xs, **over(xs)))


@pytest.mark.parametrize("over", [
    lambda xs: dict(q=torch.zeros(1, 4, 16, 64, dtype=torch.bfloat16), k=torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16),
                    v=torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16)),     # D=64
    lambda xs: dict(k=torch.zeros(1, 3, 16, 128, dtype=torch.bfloat16),
                    v=torch.zeros(1, 3, 16, 128, dtype=torch.bfloat16)),    # Hq % Hkv
    lambda xs: dict(k=torch.zeros(2, 2, 16, 128, dtype=torch.bfloat16),
                    v=torch.zeros(2, 2, 16, 128, dtype=torch.bfloat16)),    # batch mismatch
    lambda xs: dict(k=xs.k[:, :, :8].contiguous(), v=xs.v[:, :, :8].contiguous()),  # sequence mismatch
    lambda xs: dict(q=xs.q[:, :, :0], k=xs.k[:, :, :0], v=xs.v[:, :, :0]),  # S = 0
])
def test_geometry(xs, over):
    with pytest.raises(ValueError, match="Expected D in"):
        _call(_args(xs, **over(xs)))


@pytest.mark.parametrize("over", [
    lambda xs: dict(gq=xs.gq[:64]), lambda xs: dict(gk=xs.gk[None]),
    lambda xs: dict(cos=xs.cos[:8], sin=xs.sin[:8]),
])
def test_gamma_and_tables(xs, over):
    with pytest.raises(ValueError, match="gamma"):
        _call(_args(xs, **over(xs)))


@pytest.mark.parametrize("over", [
    lambda xs: dict(), lambda xs: dict(q=xs.q.float()),
    lambda xs: dict(q=xs.q.transpose(2, 3).contiguous().transpose(2, 3)),
])
def test_device_dtype_contiguity(xs, over):
    # CPU tensors, FP32 or non-contiguous: the device/dtype/layout rule
    with pytest.raises(ValueError, match="contiguous BF16"):
        _call(_args(xs, **over(xs)))


def test_launcher_mode_and_scratch(xs):
    out = torch.empty_like(xs.q)
    with pytest.raises(ValueError, match="Invalid fusion mode"):
        kf.launch_attention(xs.reference7, out, mode="bad", kn=torch.empty_like(xs.k))
    with pytest.raises(ValueError, match="Missing scratch buffers"):
        kf.launch_attention(xs.reference7, out, mode="query")
    with pytest.raises(ValueError, match="Missing scratch buffers"):
        kf.launch_attention(xs.reference7, out, mode="unfused", kn=torch.empty_like(xs.k))
    # mode 'full' needs no scratch: on CPU tensors it reaches the library, whose
    # pointer/device checks reject host memory only after argument validation
    # (so no ValueError about scratch is raised here)


def test_norm_rope_rules(xs):
    with pytest.raises(ValueError, match="norm_style"):
        kf.norm_rope(xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin, norm_style="x")
    with pytest.raises(ValueError, match="rotary tables"):
        kf.norm_rope(xs.q, xs.k, xs.gq, xs.gk, xs.cos, None)
    with pytest.raises(ValueError, match="contiguous BF16"):
        kf.norm_rope(xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin)


@pytest.mark.parametrize("which", ["qn", "kn"])
@pytest.mark.parametrize("bad", ["short", "dtype", "strided", "other_shape"])
def test_norm_rope_output_buffers(xs, which, bad):
    """Caller-supplied outputs are checked (shape, BF16, device, contiguity)
    before anything else, so a too-small or strided buffer never reaches the
    kernel."""
    like = xs.q if which == "qn" else xs.k
    b, h, s, d = like.shape
    buf = {"short": torch.empty(b, h, s - 1, d, dtype=torch.bfloat16),
           "dtype": torch.empty_like(like, dtype=torch.float32),
           "strided": torch.empty(b, h, d, s, dtype=torch.bfloat16).transpose(2, 3),
           "other_shape": torch.empty(b, h + 1, s, d, dtype=torch.bfloat16)}[bad]
    with pytest.raises(ValueError, match=f"{which} must be a contiguous BF16 tensor shaped like"):
        kf.norm_rope(xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin, **{which: buf})
    # well-formed buffers pass this rule and stop at the device rule (CPU tensors)
    with pytest.raises(ValueError, match="one GPU device"):
        kf.norm_rope(xs.q, xs.k, xs.gq, xs.gk, xs.cos, xs.sin, **{which: torch.empty_like(like)})


def test_factored_rules(xs):
    with pytest.raises(ValueError, match="Expected"):
        kf.factored_qk_attention(xs.q, xs.k, xs.v[:, :1], xs.gq, xs.gk)
    with pytest.raises(ValueError, match="contiguous BF16"):
        kf.factored_qk_attention(xs.q, xs.k, xs.v, xs.gq, xs.gk)


def test_model_scale_and_tables():
    from kernelfuser_amd import model_scale, MODELS
    from kernelfuser_amd.ops import _position_table
    assert model_scale("Qwen3-8B", 128) == 1.0 / math.sqrt(128)
    assert model_scale("Gemma-3-27B", 128) == 1 / 16  # query_pre_attn_scalar 256 (rope:25-36)
    assert model_scale("Gemma-3-4B", 256) == 1 / 16
    assert set(MODELS) >= {"Qwen3-8B", "Gemma-3-12B", "Qwen3-30B-A3B"}
    q = torch.zeros(2, 4, 8, 128, dtype=torch.bfloat16)
    t = torch.arange(8 * 128, dtype=torch.float32).view(8, 128)
    for shaped in (t, t[None].expand(2, -1, -1), t[None, None].expand(2, 1, -1, -1)):
        got = _position_table(shaped, q)
        assert got.shape == (8, 128) and got.dtype == torch.bfloat16 and got.is_contiguous()
        assert torch.equal(got, t.to(torch.bfloat16))


def test_fused_rules(xs):
    import kernelfuser_amd as kf
    with pytest.raises(ValueError, match="norm_style"):
        kf.fused(xs.q, xs.k, xs.v, xs.gq, xs.gk, xs.cos, xs.sin, True, norm_style="legacy")
    with pytest.raises(ValueError, match="contiguous BF16"):
        kf.fused(xs.q, xs.k, xs.v, xs.gq, xs.gk, xs.cos, xs.sin, True)
    with pytest.raises(ValueError, match="Expected q"):
        kf.anchor(xs.q, xs.k, xs.v[:, :, :3], None, None, True)
