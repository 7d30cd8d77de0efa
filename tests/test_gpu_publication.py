"""Publication runner on the GPU, one short row (src/e1_rope_publication_v1.py:
353-413): every arm passes the FP32 gate on the three seeds, the fused and
separate arms launch this library's kernels, every pair is timed with its
retest, four traces are written and the row passes its gate."""
import pytest

from helpers import announce

pytestmark = pytest.mark.gpu


def test_publication_row(gpu, tmp_path):
    import torch
    from kernelfuser_amd import publication
    announce("publication row Qwen3-8B B=1 S=128 causal (with torch.compile)")
    math_sdp = torch.backends.cuda.math_sdp_enabled()
    torch.backends.cuda.enable_math_sdp(False)
    try:
        with torch.inference_mode():
            row = publication.run_row("Qwen3-8B", 1, 128, True, rounds=1, samples=2, launches=3,
                                      trace_dir=tmp_path, settle_ms=0.0)
    finally:
        torch.backends.cuda.enable_math_sdp(math_sdp)
    row["gpu_exclusivity"] = {"exclusive": None}
    assert not row["errors"], row["errors"]
    seeds = row["correctness"]["seeds"]
    assert [s["seed"] for s in seeds] == [1701, 2803, 3907] and row["correctness"]["pass"]
    assert all(s["fused"]["kernels"][-1].startswith("attn_fwd_kernel") for s in seeds)
    assert all(s["separate"]["kernels"][0].startswith("rows_kernel") for s in seeds)
    compiled = row["torchinductor_status"] == "compiled"
    assert compiled or row["torchinductor_status"].startswith("unavailable")
    pairs = {"separate_vs_fused", "vendor_vs_fused"} | ({"torch_compile_vs_fused"} if compiled else set())
    assert set(row["timing"]) == pairs
    assert all(set(p) == {"initial", "retest"} for p in row["timing"].values())
    assert row["speedup_vs_separate"] > 0 and row["speedup_vs_fastest"] > 0
    assert len(row["traces"]) == len(pairs) + 1 and all((tmp_path / "Qwen3-8B").exists() for _ in [0])
    assert publication.publication_gate(row, True)["pass"] == compiled
