"""Write the golden fixtures of this directory (run from the repository root:
``python tests/golden/make_golden.py``).

The reference holds no committed vectors for the attention-prologue path
(its in-runner gates compare against an FP32 oracle computed on the fly), so
these fixtures are produced by this repository's oracle restatement
(``oracle/``), itself pinned by ``tests/test_oracle_*.py``.  Each fixture
stores the seeded BF16 inputs as raw uint16 bits and the oracle outputs as
float32, at sizes small enough to keep the files a few tens of KiB:

* ``norm_rope_s16.npz``      B=1, S=16, Hq=4, Hkv=2, D=128, theta=1e6:
                             FP32 oracle qn/kn (rope:297-301) and the HF BF16
                             chain (rope:137-168) as BF16 bits.
* ``attention_s33.npz``      B=1, S=33, Hq=4, Hkv=2, D=128, causal: oracle_fp32
                             (rope:295-302).
* ``attention_norope_s17.npz`` B=1, S=17, Hq=4, Hkv=2, D=256, non-causal: the
                             no-RoPE refinement oracle (rope:736-742).
* ``factored_s17.npz``       same inputs: factored preparation (qk:592-609) and
                             factored attention (qk:612-638).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from kernelfuser_amd.inputs import make_inputs  # noqa: E402

HERE = Path(__file__).resolve().parent
SPECS = {
    "norm_rope_s16": dict(b=1, s=16, geom=(4, 2, 128), seed=1701, rope=True),
    "attention_s33": dict(b=1, s=33, geom=(4, 2, 128), seed=2803, rope=True, causal=True),
    "attention_norope_s17": dict(b=1, s=17, geom=(4, 2, 256), seed=3907, rope=False, causal=False),
    "factored_s17": dict(b=1, s=17, geom=(4, 2, 256), seed=3907, rope=False, causal=True),
}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def inputs_of(spec):
    return make_inputs(spec["b"], spec["s"], spec["geom"], spec["seed"], rope=spec["rope"])


def compute(name: str) -> dict:
    spec = SPECS[name]
    xs = inputs_of(spec)
    arrays = {f"in_{n}": bits(t) for n, t in zip(("q", "k", "v", "gq", "gk"), xs.astuple()[:5])}
    if spec["rope"]:
        arrays["in_cos"], arrays["in_sin"] = bits(xs.cos), bits(xs.sin)
    if name == "norm_rope_s16":
        arrays["qn_fp32"] = oracle.norm_rope_fp32(xs.q, xs.gq, xs.cos, xs.sin).numpy()
        arrays["kn_fp32"] = oracle.norm_rope_fp32(xs.k, xs.gk, xs.cos, xs.sin).numpy()
        arrays["qn_hf_bits"] = bits(oracle.rope_hf_bf16(oracle.norm_hf_bf16(xs.q, xs.gq), xs.cos, xs.sin))
        arrays["kn_hf_bits"] = bits(oracle.rope_hf_bf16(oracle.norm_hf_bf16(xs.k, xs.gk), xs.cos, xs.sin))
    elif name == "attention_s33":
        arrays["out_fp32"] = oracle.oracle_fp32(*xs.astuple(), spec["causal"]).numpy()
    elif name == "attention_norope_s17":
        arrays["out_fp32"] = oracle.refinement_oracle_norope(xs.q, xs.k, xs.v, xs.gq, xs.gk, spec["causal"]).numpy()
    elif name == "factored_s17":
        inv_q, kn = oracle.factored_prepare_fp32(xs.q, xs.k, xs.gq, xs.gk)
        arrays["inv_q_fp32"] = inv_q.numpy()
        arrays["kn_fp32"] = kn.numpy()
        arrays["out_fp32"] = oracle.factored_attention_fp32(xs.q, kn, xs.v, inv_q, spec["causal"]).numpy()
    return arrays


def main():
    torch.set_num_threads(1)
    for name in SPECS:
        np.savez_compressed(HERE / f"{name}.npz", **compute(name))
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main()
