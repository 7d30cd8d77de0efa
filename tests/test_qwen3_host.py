"""Host side of the Qwen3 prefill runner on CPU: the gates, and the reference
and noise-floor arms against HF's own eager attention on a tiny model."""
import pytest
import torch

from kernelfuser_amd import qwen3


@pytest.fixture(scope="module")
def tiny():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=97, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, rope_theta=1e6, rms_norm_eps=1e-6)
    cfg._attn_implementation = "eager"
    torch.manual_seed(5)
    return Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


def test_reference_and_floor_arms_match_hf_eager(tiny):
    ids = torch.randint(0, 97, (2, 24), generator=torch.Generator().manual_seed(1))
    base = qwen3.forward_logits(tiny, ids)
    for arm in ("reference", "floor"):
        saved = qwen3.patch(tiny, arm)
        got = qwen3.forward_logits(tiny, ids)
        qwen3.restore(saved)
        m = qwen3.quality(got, base, ids)
        assert m["relative_l2"] < 2e-2 and m["nll_abs_diff"] < 1e-2, (arm, m)
    assert torch.equal(qwen3.forward_logits(tiny, ids), base)  # restore put HF back


def test_quality_and_noise_floor_gate():
    g = torch.Generator().manual_seed(2)
    ref = torch.randn(1, 10, 50, generator=g) * 3
    ids = torch.randint(0, 50, (1, 10), generator=g)
    same = qwen3.quality(ref.clone(), ref, ids)
    assert same["pass"] and same["max_abs"] == 0 and same["top1_agreement"] == 1.0
    noisy = ref + 0.05 * torch.randn(ref.shape, generator=g)
    m = qwen3.quality(noisy, ref, ids)
    assert not m["allclose"] or m["max_abs"] <= 0.025 + 0.025 * ref.abs().max()
    floor = dict(m)
    assert qwen3.noise_floor_gate(m, floor)
    worse = dict(m, relative_l2=2 * m["relative_l2"] + 1e-3)
    assert not qwen3.noise_floor_gate(worse, floor)
    assert not qwen3.noise_floor_gate(dict(m, nll_abs_diff=0.1), floor)
    with pytest.raises(KeyError):
        qwen3.patch(None, "bogus")
