"""The timing-validity guard on the GPU box: the selected device is found in
amd-smi's list by its PCI address, no foreign process is seen (the answer may
be unknown where the process list is not visible to this user), and the
refinement runner's receipt carries the run-level and per-row summaries."""
import shutil

import pytest
import torch

from helpers import announce
from kernelfuser_amd import exclusive

pytestmark = pytest.mark.gpu


def test_snapshot_finds_the_device(gpu):
    if shutil.which("amd-smi") is None:
        pytest.skip("amd-smi is not installed on this host")
    torch.zeros(1, device=gpu)
    announce("exclusivity snapshot")
    s = exclusive.gpu_snapshot(0)
    assert s.get("gpu") is not None, s
    assert s["exclusive"] in (True, None), s


def test_refine_receipt_records_exclusivity(gpu, tmp_path):
    from kernelfuser_amd import refine
    announce("refine main, one row, exclusivity summaries")
    rec = refine.main(["--grid", "rope", "--out", str(tmp_path / "r.json"), "--models", "Qwen3-8B",
                       "--sequences", "128", "--batches", "1", "--causal", "true", "--no-tails", "--launches", "5"])
    assert rec["status"] == "passed", rec["status"]
    assert rec["gpu_exclusivity"]["observations"] >= 2 and rec["gpu_exclusivity"]["exclusive"] in (True, None)
    assert all("gpu_exclusivity" in r for r in rec["rows"])
