"""Seeded synthetic inputs for the attention-prologue workloads.

Every tensor is drawn on the CPU with a seeded ``torch.Generator`` and rounded
to BF16, then copied to the device, so the CPU oracle and the GPU see
bit-identical inputs (CPU and GPU RNG streams differ).  The reference draws
its inputs on the GPU (src/e1_rope_publication_v1.py:172-183) with
Q/K/V = 0.5*N(0,1), gamma = 1 + 0.05*N(0,1) and theta = 1e4; the workloads
measured here use Q/K/V ~ N(0,1), gamma = 1 + 0.1*N(0,1), theta = 1e6.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

QWEN3_8B = (32, 8, 128)     # (Hq, Hkv, D)
GEMMA3_12B = (16, 8, 256)
THETA = 1e6


def rope_tables(s: int, d: int, theta: float = THETA, dtype=torch.bfloat16):
    """Split-half rotary tables ``[S,D]`` with duplicated halves, rounded once to
    ``dtype`` (table construction of rope:179-183): ``ang = pos * theta^(-2i/D)``."""
    pos = torch.arange(s, dtype=torch.float32)
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = pos[:, None] * inv[None, :]
    cos = torch.cat([torch.cos(ang), torch.cos(ang)], dim=1).to(dtype).contiguous()
    sin = torch.cat([torch.sin(ang), torch.sin(ang)], dim=1).to(dtype).contiguous()
    return cos, sin


@dataclass
class Inputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    gq: torch.Tensor
    gk: torch.Tensor
    cos: torch.Tensor | None
    sin: torch.Tensor | None

    def to(self, device) -> "Inputs":
        mv = lambda t: None if t is None else t.to(device, non_blocking=False).contiguous()
        return Inputs(*(mv(t) for t in self.astuple()))

    def astuple(self):
        return (self.q, self.k, self.v, self.gq, self.gk, self.cos, self.sin)

    @property
    def reference7(self):
        """The reference launchers' 7-tuple (rope:669), tables replaced by q/k when absent."""
        return (self.q, self.k, self.v, self.gq, self.gk,
                self.cos if self.cos is not None else self.q, self.sin if self.sin is not None else self.k)


def make_inputs(b: int, s: int, geometry=QWEN3_8B, seed: int = 1701, *, rope: bool = True,
                theta: float = THETA, qkv_std: float = 1.0, gamma_std: float = 0.1,
                with_v: bool = True, device="cpu") -> Inputs:
    """Q [B,Hq,S,D], K/V [B,Hkv,S,D] ~ qkv_std*N(0,1), gamma = 1 + gamma_std*N(0,1),
    all BF16; draw order q, k, v, gq, gk."""
    hq, hkv, d = geometry
    g = torch.Generator().manual_seed(int(seed))
    bf = torch.bfloat16
    q = (torch.randn((b, hq, s, d), generator=g) * qkv_std).to(bf)
    k = (torch.randn((b, hkv, s, d), generator=g) * qkv_std).to(bf)
    v = (torch.randn((b, hkv, s, d), generator=g) * qkv_std).to(bf) if with_v else torch.empty((b, hkv, s, d), dtype=bf)
    gq = (1 + gamma_std * torch.randn((d,), generator=g)).to(bf)
    gk = (1 + gamma_std * torch.randn((d,), generator=g)).to(bf)
    cos, sin = rope_tables(s, d, theta) if rope else (None, None)
    xs = Inputs(q, k, v, gq, gk, cos, sin)
    return xs if str(device) == "cpu" else xs.to(device)
