"""GPU parity of the fused-prologue GQA flash-attention prefill against the CPU
FP32 oracle (src/e1_rope_publication_v1.py:295-302) on the same seeded inputs.

Gates: attention max-abs <= 2e-2 plus the reference metric (finite,
allclose atol=rtol=.025, relative-L2 <= .025) for the FP32 prologue; the
reference metric alone for the HF prologue (the reference's own API checks,
src/e4_model_shapes_publication_v2.py:263-283, use the HF style).  Full-length
sequences (S=4096, 8192) are checked on a sample of query rows that always
includes the first and last rows.
"""
import pytest
import torch

import oracle
from helpers import announce, bf16_ulp
from kernelfuser_amd import QWEN3_8B, launch_attention, make_inputs, optimized_attention

pytestmark = pytest.mark.gpu


def _run(xs_gpu, causal, mode="query", bn=128, norm_style="fp32", rope=True):
    args = (xs_gpu.q, xs_gpu.k, xs_gpu.v, xs_gpu.gq, xs_gpu.gk) + ((xs_gpu.cos, xs_gpu.sin) if rope else ())
    out = optimized_attention(*args, causal=causal, mode=mode, bn=bn, norm_style=norm_style)
    torch.cuda.synchronize()
    return out.cpu()


def test_config3_s2048_causal_fp32(gpu):
    """Config 3: B=1, S=2048, Qwen3-8B, causal, theta=1e6."""
    xs = make_inputs(1, 2048, QWEN3_8B, 1909)
    announce("attention query fp32 B=1 S=2048 causal")
    out = _run(xs.to(gpu), True)
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.attention_gate(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("b,s", [(1, 2048), (4, 1000)])
def test_default_hf_style_configs_3_4(gpu, b, s):
    """The default norm_style ('hf', rope:680-681) at config 3 (B=1, S=2048) and
    the ragged config-4 case (B=4, S=1000), whole output, under the reference
    metric (rope:287-293) against the FP32 oracle."""
    xs = make_inputs(b, s, QWEN3_8B, 1909)
    announce(f"attention query hf B={b} S={s} causal")
    out = _run(xs.to(gpu), True, norm_style="hf")
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.metric(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("s", [4096, 8192])
def test_default_hf_style_long_whole_output(gpu, s):
    """The default 'hf' style on the ping-pong kernel (config 4 long shapes):
    the whole output under the reference metric against the FP32 oracle."""
    xs = make_inputs(1, s, QWEN3_8B, 3909)
    announce(f"attention query hf B=1 S={s} causal (whole output)")
    out = _run(xs.to(gpu), True, norm_style="hf")
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.metric(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("s", [33, 129])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("mode", ["query", "unfused"])
@pytest.mark.parametrize("bn", [64, 128])
def test_api_tails_hf(gpu, s, causal, mode, bn):
    """Public-API checks of the reference (e4:263-283): S in {33,129} x causal x
    {query, unfused} x BN {64,128}, Qwen3-8B RoPE with the HF style."""
    xs = make_inputs(1, s, QWEN3_8B, 9909)
    announce(f"attention {mode} hf S={s} causal={causal} bn={bn}")
    out = _run(xs.to(gpu), causal, mode=mode, bn=bn, norm_style="hf")
    ref = oracle.oracle_fp32(*xs.astuple(), causal)
    m = oracle.metric(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("s", [33, 129])
@pytest.mark.parametrize("causal", [False, True])
def test_api_tails_norope_legacy(gpu, s, causal):
    """The reference's no-RoPE API rows use Gemma-3-4B (8,4,256) with 'legacy'."""
    xs = make_inputs(1, s, (8, 4, 256), 9909, rope=False)
    announce(f"attention query legacy no-rope D=256 S={s} causal={causal}")
    out = _run(xs.to(gpu), causal, norm_style="legacy", rope=False)
    ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, causal)
    m = oracle.metric(out, ref)
    assert m["pass"], m


def test_ragged_b4_s1000(gpu):
    """Config 4 ragged case: B=4, S=1000 (non-multiple-of-64 tail), causal."""
    xs = make_inputs(4, 1000, QWEN3_8B, 2909)
    announce("attention query fp32 B=4 S=1000 causal")
    out = _run(xs.to(gpu), True)
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.attention_gate(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("s", [4096, 8192])
def test_long_causal_whole_output(gpu, s):
    """Config 4 long shapes, every row of every head, against the FP32 oracle
    (its SDPA run eight heads at a time to bound host memory)."""
    xs = make_inputs(1, s, QWEN3_8B, 3909)
    announce(f"attention query fp32 B=1 S={s} causal (whole output)")
    out = _run(xs.to(gpu), True)
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.attention_gate(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("s,kernel", [(2048, "attn_pp_kernel"), (3072, "attn_fwd_kernel")])
def test_noncausal_long_whole_output(gpu, s, kernel):
    """Non-causal prefill at B=1, whole output: S=2048 fills the CUs with
    exactly one round of ping-pong items (256), S=3072 would need 1.5 rounds
    and runs the general kernel (the shape-based dispatch's two sides)."""
    from kernelfuser_amd import _lib
    xs = make_inputs(1, s, QWEN3_8B, 4747)
    g = xs.to(gpu)
    out = torch.empty_like(g.q)
    kn = torch.empty_like(g.k)
    announce(f"attention query fp32 B=1 S={s} non-causal (whole output)")
    recs = list(launch_attention(g.reference7, out, causal=False, mode="query", kn=kn, norm_style="fp32"))
    torch.cuda.synchronize()
    if _lib.attention_kernel(1, 32, 8, s, 128, False, _lib.MODE_QUERY) == ("pingpong" if kernel == "attn_pp_kernel" else "general"):
        assert any(r["kernel"].startswith(kernel) for r in recs), recs
    ref = oracle.oracle_fp32(*xs.astuple(), False, head_chunk=8)
    m = oracle.attention_gate(out.cpu(), ref)
    assert m["pass"], m


@pytest.mark.parametrize("geom,b,s", [((32, 4, 128), 1, 3072), ((32, 8, 128), 3, 4096), ((8, 2, 128), 2, 3200)])
def test_pp_geometries_whole_output(gpu, geom, b, s):
    """Ping-pong kernel shapes off the Qwen3 grid: KV heads that do not
    spread evenly over the 8 XCDs (B*Hkv = 4: heads in plain order, one item
    per workgroup; ragged S=3200), and three block pairs per CU in the
    persistent loop (B=3, S=4096).  The whole output passes the oracle gate."""
    xs = make_inputs(b, s, geom, 5151)
    announce(f"attention query fp32 geometry={geom} B={b} S={s} causal (ping-pong, whole output)")
    out = _run(xs.to(gpu), True)
    ref = oracle.oracle_fp32(*xs.astuple(), True, head_chunk=8)
    m = oracle.attention_gate(out, ref)
    assert m["pass"], m


@pytest.mark.parametrize("b,s", [(1, 1900), (2, 1024)])
def test_two_slot_pairs_row_sample(gpu, b, s):
    """Causal D=128 grids that fill exactly one round of two workgroups per CU
    pair each CU's long query block with a short one (the second slot runs
    shortest first): R = 15 blocks at B=1, S=1900 (a ragged tail), and
    B=2, S=1024.  Two rows of every query block pass the oracle gate."""
    xs = make_inputs(b, s, QWEN3_8B, 3303)
    announce(f"attention query fp32 B={b} S={s} causal (two-slot pairs)")
    out = _run(xs.to(gpu), True)
    rows = torch.unique(torch.cat([torch.arange(0, s, 128), torch.arange(77, s, 128), torch.tensor([s - 1])]))
    ref = oracle.oracle_rows_fp32(*xs.astuple(), rows, True)
    m = oracle.attention_gate(out[:, :, rows], ref)
    assert m["pass"], m


@pytest.mark.parametrize("b,s,geom", [(1, 4096, QWEN3_8B), (2, 4096, QWEN3_8B), (1, 8192, QWEN3_8B),
                                      (1, 8192, (16, 8, 128)), (1, 4096, (64, 8, 128))])
def test_persistent_pairs_cover_every_block(gpu, b, s, geom):
    """Causal Qwen3 shapes whose (long, short) query-block pairs fill every CU
    equally run the ping-pong kernel persistently: one workgroup per CU loops
    over block pairs.  Every output element is written (the output starts as
    NaN), launches repeat bit for bit, and two rows of every query block pass
    the oracle gate."""
    from kernelfuser_amd import attention_prefill, prepare_attention
    # GQA ratios 4 (two head pairs per KV head), 2 (one) and 8 (four)
    xs = make_inputs(b, s, geom, 4101).to(gpu)
    kn = torch.empty_like(xs.k)
    prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="fp32")
    announce(f"attention persistent pairs B={b} S={s} geometry={geom}")
    outs = []
    for _ in range(2):
        out = torch.full_like(xs.q, float("nan"))
        attention_prefill(xs.q, kn, xs.v, out, gq=xs.gq, cos=xs.cos, sin=xs.sin, causal=True, norm_style="fp32")
        outs.append(out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(outs[0]).all())
    assert torch.equal(outs[0], outs[1])
    rows = torch.unique(torch.cat([torch.arange(0, s, 128), torch.arange(101, s, 128), torch.tensor([s - 1])]))
    ref = oracle.oracle_rows_fp32(*[t.cpu() for t in xs.astuple()], rows, True)
    m = oracle.attention_gate(outs[0][:, :, rows.to(gpu)].cpu(), ref)
    assert m["pass"], m


def test_noncausal_unfused_fp32(gpu):
    xs = make_inputs(2, 300, QWEN3_8B, 1701)
    announce("attention unfused fp32 B=2 S=300 non-causal")
    out = _run(xs.to(gpu), False, mode="unfused")
    ref = oracle.oracle_fp32(*xs.astuple(), False)
    m = oracle.attention_gate(out, ref)
    assert m["pass"], m


def test_gqa_head_mapping(gpu):
    """Each KV head's V is a distinct constant; Q head h must return the constant
    of KV head h // (Hq/Hkv) (rope:616)."""
    xs = make_inputs(1, 160, QWEN3_8B, 77)
    consts = torch.arange(1, 9, dtype=torch.float32) / 8.0
    xs.v = consts.view(1, 8, 1, 1).expand(1, 8, 160, 128).to(torch.bfloat16).contiguous()
    announce("attention GQA mapping")
    out = _run(xs.to(gpu), True)
    want = consts.repeat_interleave(4).view(1, 32, 1, 1).expand_as(out)
    assert float((out.float() - want).abs().max()) < 1e-2


def test_causal_row0_is_v0(gpu):
    xs = make_inputs(1, 70, QWEN3_8B, 78)
    announce("attention causal row 0")
    out = _run(xs.to(gpu), True)
    want = oracle.expand(xs.v.float(), 32)[:, :, 0]
    assert float((out[:, :, 0].float() - want).abs().max()) < 1e-2


def test_launch_attention_buffers(gpu):
    """launch_attention writes out and the K scratch; 'full' is refused, missing
    scratch raises ValueError (rope:668-672)."""
    xs = make_inputs(1, 96, QWEN3_8B, 5).to(gpu)
    out = torch.empty_like(xs.q)
    kn = torch.empty_like(xs.k)
    announce("launch_attention query")
    launch_attention(xs.reference7, out, causal=True, mode="query", kn=kn, norm_style="fp32")
    torch.cuda.synchronize()
    kref = oracle.norm_rope_fp32(xs.k.cpu(), xs.gk.cpu(), xs.cos.cpu(), xs.sin.cpu())
    assert oracle.norm_rope_gate(kn.cpu(), kref)["pass"]
    ref = oracle.oracle_fp32(*[t.cpu() for t in xs.astuple()], True)
    assert oracle.attention_gate(out.cpu(), ref)["pass"]
    with pytest.raises(ValueError):
        launch_attention(xs.reference7, out, mode="unfused", kn=kn)
    with pytest.raises(ValueError):
        launch_attention(xs.reference7, out, mode="bad", kn=kn)


@pytest.mark.parametrize("b,s,causal", [(1, 3000, True), (2, 3072, False), (1, 2970, True), (1, 1000, True)])
def test_vt_path_identical(gpu, b, s, causal):
    """The V^T scratch path of the ping-pong kernel (preparation writes V
    transposed per head, the kernel reads V^T rows) agrees with the row-major
    V path (the MFMA sums the same products of each 16-key step, possibly in
    another order, so results may differ in the last bit of a few outputs);
    shapes it does not apply to (S % 8 != 0, or short sequences, which run the
    general kernel) leave the scratch untouched.  S=3000 and 2970 also cover
    the ping-pong kernel's partial query block and partial key tile."""
    from kernelfuser_amd import uses_vt
    xs = make_inputs(b, s, QWEN3_8B, 606).to(gpu)
    out1, kn1 = torch.empty_like(xs.q), torch.empty_like(xs.k)
    out2, kn2 = torch.empty_like(xs.q), torch.empty_like(xs.k)
    vt = torch.full_like(xs.v, 3.0)
    announce(f"attention vt path B={b} S={s} causal={causal}")
    launch_attention(xs.reference7, out1, causal=causal, mode="query", kn=kn1, norm_style="fp32")
    launch_attention(xs.reference7, out2, causal=causal, mode="query", kn=kn2, norm_style="fp32", vt=vt)
    torch.cuda.synchronize()
    # one BF16 ulp, plus FP32 summation-order noise for outputs that cancel to ~0
    diff = (out1.float() - out2.float()).abs()
    tol = bf16_ulp(torch.maximum(out1.float().abs(), out2.float().abs())) * 1.01 + 1e-5
    assert bool((diff <= tol).all()), float((diff / tol).max())
    assert float((diff > 0).float().mean()) < 0.02
    assert torch.equal(kn1, kn2)
    if uses_vt(32, 8, s, 128, b, causal):
        assert torch.equal(vt, xs.v.transpose(2, 3).contiguous().view_as(vt))
    else:
        assert bool((vt == 3.0).all())
    rows = torch.unique(torch.cat([torch.arange(0, 4), torch.randint(0, s, (40,), generator=torch.Generator().manual_seed(s)),
                                   torch.arange(s - 70, s)]))
    ref = oracle.oracle_rows_fp32(*[t.cpu() for t in xs.astuple()], rows, causal)
    assert oracle.attention_gate(out2[:, :, rows.to(gpu)].cpu(), ref)["pass"]


def test_transpose_v_d256(gpu):
    from kernelfuser_amd import transpose_v
    v = (torch.randn(2, 3, 200, 256, generator=torch.Generator().manual_seed(3))).to(torch.bfloat16).to(gpu)
    vt = torch.empty_like(v)
    announce("transpose_v D=256 S=200")
    transpose_v(v, vt)
    torch.cuda.synchronize()
    assert torch.equal(vt.view(2, 3, 256, 200), v.transpose(2, 3))


@pytest.mark.parametrize("only_k,s", [(True, 1000), (False, 72), (True, 8)])
def test_prepare_writes_vt(gpu, only_k, s):
    """The preparation launch with a V^T output writes vt = V transposed per
    head and leaves its row outputs bit-identical to the launch without it."""
    from kernelfuser_amd import prepare_attention
    xs = make_inputs(2, s, QWEN3_8B, 707).to(gpu)
    qn1, kn1 = torch.empty_like(xs.q), torch.empty_like(xs.k)
    qn2, kn2 = torch.empty_like(xs.q), torch.empty_like(xs.k)
    vt = torch.full_like(xs.v, 3.0)
    announce(f"prepare with vt only_k={only_k} S={s}")
    prepare_attention(xs.reference7, qn1, kn1, only_k=only_k, norm_style="fp32")
    prepare_attention(xs.reference7, qn2, kn2, only_k=only_k, norm_style="fp32", vt=vt)
    torch.cuda.synchronize()
    assert torch.equal(kn1, kn2)
    if not only_k:
        assert torch.equal(qn1, qn2)
    assert torch.equal(vt.view(2, 8, 128, s), xs.v.transpose(2, 3))
    with pytest.raises(ValueError):  # D=128 needs S % 8 == 0 for V^T rows
        x2 = make_inputs(1, 12, QWEN3_8B, 1).to(gpu)
        prepare_attention(x2.reference7, None, torch.empty_like(x2.k), only_k=True, vt=torch.empty_like(x2.v))


@pytest.mark.parametrize("geom,b,s,causal,style,rope", [
    (QWEN3_8B, 1, 129, True, "hf", True), (QWEN3_8B, 2, 200, False, "fp32", True),
    ((8, 4, 256), 1, 65, True, "legacy", True), ((16, 8, 256), 1, 96, False, "fp32", False),
    ((32, 4, 128), 1, 70, True, "fp32", False),
])
def test_mode_full(gpu, geom, b, s, causal, style, rope):
    """mode='full' (one launch; Q and every K tile normalised inside attention,
    rope:619-635, :668-677) passes the oracle gate and stays close to
    mode='query': K may differ by one BF16 rounding (its row RMS is summed in
    another order), and for the FP32 style the query path folds the logit
    scale into Q before Q's single rounding while the general kernel rounds Q
    unscaled."""
    xs = make_inputs(b, s, geom, 808, rope=rope).to(gpu)
    out_f, out_q, kn = torch.empty_like(xs.q), torch.empty_like(xs.q), torch.empty_like(xs.k)
    announce(f"mode full {geom} B={b} S={s} causal={causal} {style} rope={rope}")
    launch_attention(xs.reference7, out_f, causal=causal, mode="full", rope=rope, norm_style=style)
    launch_attention(xs.reference7, out_q, causal=causal, mode="query", rope=rope, kn=kn, norm_style=style)
    torch.cuda.synchronize()
    cpu = [t.cpu() if t is not None else None for t in xs.astuple()]
    ref = oracle.oracle_fp32(*cpu, causal)  # every style is gated against the FP32 oracle
    assert oracle.attention_gate(out_f.cpu(), ref)["pass"]
    # the two modes are two numerical paths, each within the gate of the oracle
    d = (out_f.float() - out_q.float()).abs()
    assert float(d.max()) <= 2e-2, float(d.max())
    assert float(d.mean()) <= 1e-3, float(d.mean())


def test_launchers_return_their_kernels(gpu):
    """launch_attention / launch_factored_attention / prepare_attention return
    the launched kernels (instance, grid, block, registers, LDS, scratch) where
    the reference returns its kernel object (rope:674-677, qk:651)."""
    from kernelfuser_amd import launch_factored_attention, prepare_attention
    xs = make_inputs(1, 4096, QWEN3_8B, 31).to(gpu)
    out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
    announce("launch records B=1 S=4096 query")
    recs = launch_attention(xs.reference7, out, causal=True, mode="query", kn=kn, norm_style="fp32")
    assert [r["kernel"] for r in recs] == ["rows_kernel<128, 2, true, true, false, 2>",
                                           "attn_pp_kernel<true, 2, 2, false>"]
    assert recs[0]["block"] == 256 and recs[1]["block"] == 512 and recs[1]["grid"] == 256
    assert recs[1]["lds_bytes"] == 131072 and all(r["registers"] > 0 and r["scratch_bytes"] == 0 for r in recs)
    prep = prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="fp32")
    assert [r["kernel"] for r in prep] == [recs[0]["kernel"]]
    fx = make_inputs(1, 256, (8, 4, 256), 32, rope=False).to(gpu)
    inv = torch.empty(fx.q.shape[:-1], device=gpu, dtype=torch.float32)
    f = launch_factored_attention((fx.q, fx.k, fx.v, fx.gq, fx.gk), torch.empty_like(fx.q), inv,
                                  torch.empty_like(fx.k), causal=True)
    torch.cuda.synchronize()
    assert [r["kernel"].split("<")[0] for r in f] == ["rows_kernel", "attn_fwd_kernel"]


def test_launch_records_are_lazy_and_scoped(gpu):
    """The launchers' records are read from the library on first use; a handle
    read after a later call of the same thread raises rather than returning
    that call's kernels, and record_launches collects every call of a block."""
    from kernelfuser_amd import _lib, prepare_attention
    xs = make_inputs(1, 256, QWEN3_8B, 33).to(gpu)
    out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
    announce("lazy launch records B=1 S=256")
    with _lib.record_launches() as rec:
        first = launch_attention(xs.reference7, out, causal=True, mode="query", kn=kn, norm_style="fp32")
        assert len(first) == 2 and first[1]["kernel"].startswith("attn_fwd_kernel")
        stale = prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="fp32")
        prepare_attention(xs.reference7, None, kn, only_k=True, norm_style="fp32")
        with pytest.raises(RuntimeError):
            len(stale)
    torch.cuda.synchronize()
    assert [r["kernel"].split("<")[0] for r in rec.launches] == ["rows_kernel", "attn_fwd_kernel", "rows_kernel",
                                                                 "rows_kernel"]
    assert list(first) == rec.launches[:2]  # read before the next call, kept since
