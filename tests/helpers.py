"""Shared helpers of the test suite."""
import torch


def announce(msg: str) -> None:
    """Name the case before a GPU step (flushed), so a crash log identifies it."""
    print(f"[case] {msg}", flush=True)


def to_gpu(xs, device):
    return xs.to(device)


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of BF16 numbers at |x| (2^(e-7) for |x| in [2^e, 2^(e+1)))."""
    ax = x.float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(ax)) - 7)
