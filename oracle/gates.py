"""Correctness gates -- TEST INFRASTRUCTURE ONLY.

``metric`` restates the reference gate (src/e1_rope_publication_v1.py:287-293):
finite, ``allclose(atol=rtol=.025)`` and relative-L2 <= .025.  The two build
gates come from the north-star statement: norm+RoPE BF16 outputs within
max-abs 1.6e-2 and mean-abs 2e-3 of the FP32 oracle; attention outputs within
max-abs 2e-2.
"""
from __future__ import annotations

import torch

NORM_ROPE_MAX_ABS = 1.6e-2
NORM_ROPE_MEAN_ABS = 2e-3
ATTENTION_MAX_ABS = 2e-2


def metric(x: torch.Tensor, y: torch.Tensor) -> dict:
    """Reference gate (rope:287-293); ``y`` is the oracle."""
    a = x.detach().float().cpu()
    b = y.detach().float().cpu()
    finite = bool(torch.isfinite(a).all() and torch.isfinite(b).all())
    diff = a - b
    den = b.norm().clamp_min(1e-12)
    rl2 = float(diff.norm() / den) if finite else float('inf')
    close = bool(torch.allclose(a, b, atol=.025, rtol=.025)) if finite else False
    return {
        'max_abs': float(diff.abs().max()) if finite else float('inf'),
        'mean_abs': float(diff.abs().mean()) if finite else float('inf'),
        'relative_l2': rl2,
        'finite': finite,
        'pass': bool(finite and close and rl2 <= .025),
    }


def norm_rope_gate(x: torch.Tensor, y: torch.Tensor) -> dict:
    m = metric(x, y)
    m['gate'] = 'norm_rope max_abs<=1.6e-2 mean_abs<=2e-3'
    m['pass'] = bool(m['pass'] and m['max_abs'] <= NORM_ROPE_MAX_ABS and m['mean_abs'] <= NORM_ROPE_MEAN_ABS)
    return m


def attention_gate(x: torch.Tensor, y: torch.Tensor) -> dict:
    m = metric(x, y)
    m['gate'] = 'attention max_abs<=2e-2'
    m['pass'] = bool(m['pass'] and m['max_abs'] <= ATTENTION_MAX_ABS)
    return m
