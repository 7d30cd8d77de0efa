"""FP32 CPU restatement of the reference's oracle path -- TEST INFRASTRUCTURE ONLY.

Reference checkout: WenbinWang12/KernelFuser.  Every function below cites the
file:line of ``src/e1_rope_publication_v1.py`` (``rope``) or
``src/e1_qk_publication_v3.py`` (``qk``) whose arithmetic it restates.  All
tensors are CPU tensors; layout is BHSD contiguous (Q ``[B,Hq,S,D]``, K/V
``[B,Hkv,S,D]``), rotary tables ``[S,D]`` with duplicated halves.

Pinning status of each function (checks in ``tests/test_oracle_*.py``):

* ``rope_tables``          closed form cos/sin(pos * theta^(-2i/D)), duplicated halves.
* ``rms_inverse``/``norm_fp32``  constant-row closed form, scale invariance, brute force.
* ``rope_fp32``            position-0 identity, pair-norm preservation, R(-a)R(a)=I,
                           relative-position invariance, complex-multiplication form.
* ``norm_hf_bf16``/``rope_hf_bf16``/``norm_legacy_bf16``  step-by-step scalar
                           restatement with explicit RNE rounding (numpy, tiny inputs).
* ``attention_fp32``/``attention_rows_fp32``  float64 brute force on tiny inputs,
                           causal row 0 == v[0], constant V, q=0 prefix mean, GQA map.
* ``factored_*``           factoring identity against the unfused oracle.

No function here is "parity unpinned".
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

EPS = 1e-6  # rope:32, rope:558 (hard-coded 1e-6 in the kernels)
LOG2E = 1.4426950408889634  # rope:636


def rope_tables(S: int, D: int, theta: float, dtype=torch.bfloat16):
    """Split-half rotary tables ``[S,D]`` (rope:179-183).

    ``inv = 1/theta^(2i/D)``, ``ang = pos*inv``, ``cos = cat([cos(ang), cos(ang)])``,
    rounded once to ``dtype`` (the reference casts the tables to the activation
    dtype, rope:183).  The reference uses theta=10000; the build's configs use 1e6.
    """
    pos = torch.arange(S, dtype=torch.float32)
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = pos[:, None] * inv[None, :]
    cos = torch.cat([torch.cos(ang), torch.cos(ang)], dim=1).to(dtype)
    sin = torch.cat([torch.sin(ang), torch.sin(ang)], dim=1).to(dtype)
    return cos.contiguous(), sin.contiguous()


def rms_inverse(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """``rsqrt(mean(x^2) + eps)`` over the last dim in FP32 (rope:298, qk:600)."""
    xf = x.float()
    return torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)


def norm_fp32(x: torch.Tensor, g: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """FP32 RMSNorm ``x * rsqrt(mean x^2 + eps) * g`` (rope:298-299, rope:741)."""
    xf = x.float()
    return xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * g.float()


def _table_view(t: torch.Tensor, dtype) -> torch.Tensor:
    # rope:155-159: [S,D] or [B,S,D] tables broadcast over heads.
    t = t.to(dtype)
    if t.ndim == 2:
        return t[None, None]
    if t.ndim == 3:
        return t[:, None]
    return t


def rope_fp32(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """rotate-half RoPE with every operation in FP32 (rope:141-168, ``fp32=True``).

    The BF16 tables are upcast (rope:153-154) and only their first half is used
    for both output halves (rope:161), exactly as the reference oracle does.
    """
    xx = x.float()
    d = xx.shape[-1]
    half = d // 2
    cc = _table_view(cos, torch.float32)[..., :half]
    ss = _table_view(sin, torch.float32)[..., :half]
    a = xx[..., :half]
    b = xx[..., half:]
    y = torch.empty_like(xx)
    y[..., :half] = a * cc - b * ss
    y[..., half:] = b * cc + a * ss
    return y


def norm_rope_fp32(x, g, cos, sin, eps: float = EPS) -> torch.Tensor:
    """The norm+RoPE part of ``oracle_fp32`` (rope:297-301), FP32 result."""
    y = norm_fp32(x, g, eps)
    return rope_fp32(y, cos, sin) if cos is not None else y


# --- BF16-boundary chains (diagnostic contracts of the reference kernels) ---

def norm_hf_bf16(x: torch.Tensor, g: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """HF RMSNorm boundary (rope:137-139; kernel rope:559-561): round the
    normalised activation to BF16, then a BF16 multiply by BF16 gamma."""
    xf = x.float()
    xn = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    return (xn * g.to(torch.bfloat16)).to(torch.bfloat16)


def norm_legacy_bf16(x: torch.Tensor, g: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """``legacy`` boundary (rope:563): one BF16 cast of the FP32 product x*inv*g."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * g.float()).to(torch.bfloat16)


def rope_hf_bf16(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """rotate-half with HF's BF16 rounding points (rope:141-168, ``fp32=False``):
    each product and the add/subtract round to BF16."""
    bf = torch.bfloat16
    d = x.shape[-1]
    half = d // 2
    xx = x.to(bf)
    cc = _table_view(cos, bf)[..., :half]
    ss = _table_view(sin, bf)[..., :half]
    a = xx[..., :half]
    b = xx[..., half:]
    p0 = (a * cc).to(bf)
    p1 = (b * ss).to(bf)
    p2 = (b * cc).to(bf)
    p3 = (a * ss).to(bf)
    y = torch.empty_like(xx)
    y[..., :half] = (p0 - p1).to(bf)
    y[..., half:] = (p2 + p3).to(bf)
    return y


# --- attention ---

def expand(x: torch.Tensor, h: int) -> torch.Tensor:
    """GQA expansion by ``repeat_interleave`` (rope:170): KV head of Q head h is h // (Hq/Hkv)."""
    return x if x.shape[1] == h else x.repeat_interleave(h // x.shape[1], dim=1)


def attention_fp32(qn, kn, v, causal: bool, scale=None, head_chunk: int = 0) -> torch.Tensor:
    """FP32 SDPA with GQA expansion (rope:302).

    ``head_chunk>0`` loops over groups of Q heads to bound host memory at long S
    (one FP32 score matrix at S=8192 is 256 MiB per head).
    """
    qf, kf, vf = qn.float(), kn.float(), v.float()
    h = qf.shape[1]
    g = h // kf.shape[1]
    if head_chunk <= 0 or head_chunk >= h:
        return F.scaled_dot_product_attention(qf, expand(kf, h), expand(vf, h), is_causal=causal, scale=scale)
    out = torch.empty_like(qf)
    for h0 in range(0, h, head_chunk):
        h1 = min(h, h0 + head_chunk)
        kv = torch.arange(h0, h1) // g
        out[:, h0:h1] = F.scaled_dot_product_attention(
            qf[:, h0:h1], kf[:, kv], vf[:, kv], is_causal=causal, scale=scale)
    return out


def attention_rows_fp32(qn, kn, v, rows, causal: bool, scale=None) -> torch.Tensor:
    """Attention outputs for a subset of query ``rows`` only (all heads, all batches).

    Same math as ``attention_fp32`` (softmax(q k^T * scale) v, causal mask key<=query),
    evaluated explicitly so full-length sequences can be checked on a row sample.
    Returns ``[B,Hq,len(rows),D]`` FP32.
    """
    qf, kf, vf = qn.float(), kn.float(), v.float()
    B, H, S, D = qf.shape
    g = H // kf.shape[1]
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    rows = torch.as_tensor(rows, dtype=torch.long)
    out = torch.empty(B, H, len(rows), D, dtype=torch.float32)
    keys = torch.arange(S)
    for h in range(H):
        kh = h // g
        s = torch.matmul(qf[:, h, rows, :], kf[:, kh].transpose(-1, -2)) * sc
        if causal:
            s = s.masked_fill(keys[None, None, :] > rows[None, :, None], float('-inf'))
        p = torch.softmax(s, dim=-1)
        out[:, h] = torch.matmul(p, vf[:, kh])
    return out


def attention_bruteforce(qn, kn, v, causal: bool, scale=None) -> np.ndarray:
    """Float64 textbook attention with explicit loops over rows (tiny inputs only)."""
    q = np.asarray(qn.double().numpy())
    k = np.asarray(kn.double().numpy())
    vv = np.asarray(v.double().numpy())
    B, H, S, D = q.shape
    g = H // k.shape[1]
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    out = np.zeros((B, H, S, D))
    for b in range(B):
        for h in range(H):
            kh = h // g
            for i in range(S):
                n = i + 1 if causal else S
                s = (k[b, kh, :n] @ q[b, h, i]) * sc
                w = np.exp(s - s.max())
                out[b, h, i] = (w / w.sum()) @ vv[b, kh, :n]
    return out


def oracle_fp32(q, k, v, gq, gk, cos, sin, causal: bool, scale=None, eps: float = EPS,
                head_chunk: int = 0) -> torch.Tensor:
    """Independent FP32 oracle (rope:295-302): FP32 norm, FP32 RoPE, FP32 SDPA."""
    qn = norm_rope_fp32(q, gq, cos, sin, eps)
    kn = norm_rope_fp32(k, gk, cos, sin, eps)
    return attention_fp32(qn, kn, v, causal, scale, head_chunk)


def oracle_rows_fp32(q, k, v, gq, gk, cos, sin, rows, causal: bool, scale=None, eps: float = EPS):
    """``oracle_fp32`` restricted to a sample of query rows (same arithmetic)."""
    rows = torch.as_tensor(rows, dtype=torch.long)
    qs = q[:, :, rows]
    qn = norm_fp32(qs, gq, eps)
    if cos is not None:
        qn = rope_fp32(qn, cos[rows], sin[rows])
    kn = norm_rope_fp32(k, gk, cos, sin, eps)
    # Re-embed the sampled rows so the causal mask uses their true positions.
    qf, kf, vf = qn.float(), kn.float(), v.float()
    B, H, _, D = qf.shape
    S = kf.shape[2]
    g = H // kf.shape[1]
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    keys = torch.arange(S)
    out = torch.empty(B, H, len(rows), D)
    for h in range(H):
        kh = h // g
        s = torch.matmul(qf[:, h], kf[:, kh].transpose(-1, -2)) * sc
        if causal:
            s = s.masked_fill(keys[None, None, :] > rows[None, :, None], float('-inf'))
        out[:, h] = torch.matmul(torch.softmax(s, dim=-1), vf[:, kh])
    return out


def refinement_oracle_norope(q, k, v, gq, gk, causal: bool, eps: float = EPS, head_chunk: int = 0):
    """No-RoPE FP32 oracle (rope:736-742): FP32 RMSNorm of Q and K, then SDPA."""
    return attention_fp32(norm_fp32(q, gq, eps), norm_fp32(k, gk, eps), v, causal, None, head_chunk)


def factored_prepare_fp32(q, k, gq, gk, eps: float = EPS):
    """Factored preparation (qk:592-609) without rounding: FP32 ``inv_q`` ``[B,Hq,S]``
    and ``kn = k * inv_k * gk * gq`` (the kernel rounds kn once to BF16, qk:608)."""
    inv_q = rms_inverse(q, eps)[..., 0]
    kf = k.float()
    kn = kf * rms_inverse(k, eps) * gk.float() * gq.float()
    return inv_q, kn


def factored_attention_fp32(q, kn, v, inv_q, causal: bool, head_chunk: int = 0):
    """Factored scores ``(q_raw @ kn^T) * inv_q * D^-1/2`` then softmax @ V (qk:612-638).

    By the identity of results/RESULTS.md:104-112 this equals the unfused
    no-RoPE oracle in exact arithmetic.
    """
    qf = q.float() * inv_q.float()[..., None]
    return attention_fp32(qf, kn.float(), v.float(), causal, None, head_chunk)
