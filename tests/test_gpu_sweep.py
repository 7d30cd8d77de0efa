"""Seeded sweep over the prologue's configuration space, each case checked on
its whole output against the CPU FP32 oracle (src/e1_rope_publication_v1.py:
295-302; no-RoPE factored: :736-742 and src/e1_qk_publication_v3.py:612-638).

The other GPU tests vary one or two settings around fixed shapes.  Here
cases drawn from a fixed seed mix them: a geometry of the reference's MODELS
table (rope:31-36), B, S from a list dense in tile and block edges, causal or
not, the launcher path ('query', 'unfused', 'full' or the factored launch),
the rounding style, RoPE on or off, and the attention kernel (by shape, or
forced to each kernel the geometry admits).  Draws: 40 short cases (B in
1..3, S from 1 to 700: one-tile items, partial tiles) and 30 long ones (B in
1..2, S from 777 to 4096: the dispatch thresholds, the persistent pairing, the
D=256 split plans), 20 short cases on geometries beyond the reference's
table (MHA and odd GQA ratios, general kernel only), and 16 D=256 causal
shapes with few heads, where the general kernel splits key ranges.  The case lists depend
only on the seeds, so every run checks the same cases.  Each test names its case before the GPU step and
checks from the launch records that a forced kernel ran.
"""
import random

import pytest
import torch

import oracle
from helpers import announce
from kernelfuser_amd import MODELS, _lib, launch_attention, launch_factored_attention, make_inputs

pytestmark = pytest.mark.gpu

S_CHOICES = [1, 2, 7, 31, 32, 33, 63, 64, 65, 96, 127, 128, 129, 191, 200, 255, 256, 257, 300, 383, 448,
             511, 513, 640, 700]
S_LONG = [777, 1000, 1023, 1024, 1025, 1500, 1536, 1900, 2047, 2048, 2049, 2945, 3000, 3072, 4095, 4096]
# geometries the boundary accepts beyond the reference's table: MHA (ratio 1)
# and odd GQA ratios, which only the general kernel serves
OFF_TABLE = {"MHA-8x128": (8, 8, 128), "MHA-5x128": (5, 5, 128), "MHA-4x256": (4, 4, 256),
             "GQA3-12q4kv-128": (12, 4, 128), "GQA3-24q8kv-128": (24, 8, 128), "GQA5-40q8kv-128": (40, 8, 128),
             "GQA3-6q2kv-256": (6, 2, 256), "GQA2-10q5kv-256": (10, 5, 256)}
GEOMETRIES = {**MODELS, **OFF_TABLE}
KERNEL_PREFIX = {"general": "attn_fwd_kernel", "pingpong": "attn_pp_kernel", "wide": "attn_ww_kernel"}


def _cases(n, seed, s_choices=S_CHOICES, b_choices=(1, 1, 2, 3), table=MODELS):
    rng = random.Random(seed)
    geoms = sorted(table.items())
    cases = []
    for i in range(n):
        name, (hq, hkv, d) = rng.choice(geoms)
        b = rng.choice(b_choices)
        s = rng.choice(s_choices)
        causal = rng.random() < 0.5
        path = rng.choice(["query", "query", "unfused", "full", "factored"])
        rope = path != "factored" and rng.random() < 0.75
        style = "factored" if path == "factored" else rng.choice(["fp32", "hf", "legacy"])
        kernels = ["auto", "general"]
        if path != "full" and d == 128 and (hq // hkv) % 2 == 0:
            kernels.append("pingpong")
        if path != "full" and d == 128 and (hq // hkv) % 4 == 0:
            kernels.append("wide")
        kernel = rng.choice(kernels)
        cid = f"{i:02d}-{name}-B{b}-S{s}-{'c' if causal else 'nc'}-{path}-{style}-{'rope' if rope else 'norope'}-{kernel}"
        cases.append(pytest.param(name, b, s, causal, path, style, rope, kernel, id=cid))
    return cases


@pytest.mark.parametrize("name,b,s,causal,path,style,rope,kernel", _cases(40, 4242))
def test_sweep_case_whole_output(gpu, name, b, s, causal, path, style, rope, kernel):
    _check_case(gpu, name, b, s, causal, path, style, rope, kernel)


@pytest.mark.parametrize("name,b,s,causal,path,style,rope,kernel", _cases(30, 9001, S_LONG, (1, 1, 2)))
def test_sweep_long_case_whole_output(gpu, name, b, s, causal, path, style, rope, kernel):
    _check_case(gpu, name, b, s, causal, path, style, rope, kernel)


@pytest.mark.parametrize("name,b,s,causal,path,style,rope,kernel", _cases(20, 5151, table=OFF_TABLE))
def test_sweep_off_table_case_whole_output(gpu, name, b, s, causal, path, style, rope, kernel):
    _check_case(gpu, name, b, s, causal, path, style, rope, kernel)


def _split_cases(n=16, seed=7373):
    rng = random.Random(seed)
    geoms = [(2, 1, 256), (4, 4, 256), (6, 2, 256), (8, 4, 256), (16, 8, 256), (4, 2, 256)]
    cases = []
    for i in range(n):
        geom = rng.choice(geoms)
        b = rng.choice([1, 1, 2])
        s = rng.randint(129, 2100)
        path = rng.choice(["query", "query", "unfused", "factored"])
        style = "factored" if path == "factored" else rng.choice(["fp32", "hf", "legacy"])
        rope = path != "factored"
        cases.append(pytest.param(geom, b, s, path, style, rope, id=f"{i:02d}-{geom[0]}q{geom[1]}kv-B{b}-S{s}-{path}-{style}"))
    return cases


@pytest.mark.parametrize("geom,b,s,path,style,rope", _split_cases())
def test_sweep_split_plan_whole_output(gpu, geom, b, s, path, style, rope):
    """D=256 causal grids with fewer query blocks than CUs: the general
    kernel cuts its longest blocks' key ranges in two and merges the halves
    (split-KV).  The launch record must show a split exactly when the shape
    has a workspace, and the whole output must pass the oracle's gate."""
    from kernelfuser_amd import attention_workspace_bytes
    recs = _check_case(gpu, geom, b, s, True, path, style, rope, "auto")
    n_split = int(recs[0]["plan"].split()[0].split("=")[1])
    assert (n_split > 0) == (attention_workspace_bytes(b, geom[0], geom[1], s, 256, True) > 0), recs[0]


def _check_case(gpu, name, b, s, causal, path, style, rope, kernel):
    geom = GEOMETRIES[name] if isinstance(name, str) else name
    xs = make_inputs(b, s, geom, 5000 + 7 * s + b, rope=rope)
    g = xs.to(gpu)
    out = torch.full_like(g.q, float("nan"))
    kn = torch.empty_like(g.k)
    announce(f"sweep {name} {geom} B={b} S={s} causal={causal} {path} {style} rope={rope} kernel={kernel}")
    with _lib.tuning(attn_kernel=kernel):
        if path == "factored":
            inv = torch.empty(g.q.shape[:-1], device=gpu, dtype=torch.float32)
            recs = list(launch_factored_attention((g.q, g.k, g.v, g.gq, g.gk), out, inv, kn, causal=causal))
        else:
            qn = torch.empty_like(g.q) if path == "unfused" else None
            recs = list(launch_attention(g.reference7, out, causal=causal, mode=path, rope=rope, qn=qn, kn=kn,
                                         norm_style=style))
    torch.cuda.synchronize()
    attn_recs = [r for r in recs if r["kernel"].startswith("attn_")]
    attn = [r["kernel"] for r in attn_recs]
    assert len(attn) == 1, recs
    if kernel != "auto":
        assert attn[0].startswith(KERNEL_PREFIX[kernel]), attn
    if path == "factored":
        ref = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, causal, head_chunk=8)
        inv_ref = oracle.rms_inverse(xs.q.float())[..., 0]
        assert torch.allclose(inv.cpu(), inv_ref, rtol=1e-6, atol=0)
    else:
        ref = oracle.oracle_fp32(*xs.astuple(), causal, head_chunk=8)
    gate = oracle.metric if style in ("hf", "legacy") else oracle.attention_gate
    m = gate(out.cpu(), ref)
    assert m["pass"], m
    return attn_recs
