"""The committed golden fixtures (``tests/golden/``) against the seeded input
generator and the oracle, on the CPU: inputs regenerate bit-exactly from
their seeds, and the oracle reproduces every stored output.  A change to
either shows up here before it can move a GPU parity result."""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(make_golden.SPECS))
def test_inputs_regenerate_bit_exactly(name):
    g = load(name)
    fresh = make_golden.compute(name)
    for key in (k for k in g if k.startswith("in_")):
        assert np.array_equal(g[key], fresh[key]), key


@pytest.mark.parametrize("name", sorted(make_golden.SPECS))
def test_oracle_reproduces_outputs(name):
    g = load(name)
    fresh = make_golden.compute(name)
    for key in (k for k in g if not k.startswith("in_")):
        if key.endswith("_bits"):
            assert np.array_equal(g[key], fresh[key]), key
        else:
            assert np.abs(g[key] - fresh[key]).max() <= 1e-6, key


def test_fixture_known_answers():
    """Facts the stored outputs must satisfy independently of the oracle code:
    causal row 0 equals V row 0 (per KV head); RoPE at position 0 is the
    identity, so qn row 0 equals the plain RMSNorm of q row 0."""
    a = load("attention_s33")
    v = torch.from_numpy(a["in_v"].view(np.int16)).view(torch.bfloat16).float().numpy()
    for h in range(4):
        assert np.array_equal(a["out_fp32"][0, h, 0], v[0, h // 2, 0])
    n = load("norm_rope_s16")
    q = torch.from_numpy(n["in_q"].view(np.int16)).view(torch.bfloat16).double().numpy()
    gq = torch.from_numpy(n["in_gq"].view(np.int16)).view(torch.bfloat16).double().numpy()
    row = q[0, :, 0]
    want = row / np.sqrt((row ** 2).mean(-1, keepdims=True) + 1e-6) * gq
    assert np.abs(n["qn_fp32"][0, :, 0] - want).max() < 1e-5
