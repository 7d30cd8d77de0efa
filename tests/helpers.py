"""Shared helpers of the test suite."""
import numpy as np
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


def rne_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest BF16 (ties to even) by bit
    arithmetic, independently of torch's conversion; returns float32."""
    a = np.asarray(x, dtype=np.float32).copy()
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bf16_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
