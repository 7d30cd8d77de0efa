"""Reference-signature ops of the RoPE-aware attention prologue on gfx950.

Each public function keeps the name, arguments, defaults and error behaviour of
the reference function it replaces (WenbinWang12/KernelFuser; ``rope`` =
src/e1_rope_publication_v1.py, ``qk`` = src/e1_qk_publication_v3.py) and runs
the hand-written gfx950 HIP kernels through the C ABI (``include/kfmi.h``).
There is no CPU or eager fallback: without the native library, or on another
GPU architecture, every op raises.

Differences from the reference, all deliberate:
  * ``norm_style`` also accepts ``'fp32'``: FP32 RMSNorm*gamma and RoPE with one
    final BF16 rounding (the FP32 semantics of rope:119-130).  ``'hf'`` stays the
    default of ``optimized_attention`` as in the reference.
  * The SM90 requirement (rope:718) becomes a gfx950 (MI355X) requirement.
  * Triton tuning knobs (``rows``, ``warps``, ``stages``, ``gather``) are accepted
    and ignored; ``bm``/``bn`` are tile hints -- results do not depend on them.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._lib import MODE_FULL, MODE_QUERY, MODE_UNFUSED, NORM_STYLES, PREP_ONLY_K, PREP_ROPE, ptr, stream_of

EPS = 1e-6  # rope:32; the reference kernels hard-code it (rope:558)

# Attention geometries (Hq, Hkv, D) of the reference's model table (rope:18-24).
MODELS = {
    "Qwen3-0.6B": (16, 8, 128), "Qwen3-1.7B": (32, 8, 128),
    "Qwen3-4B": (32, 8, 128), "Qwen3-8B": (32, 8, 128),
    "Qwen3-32B": (64, 8, 128), "Qwen3-30B-A3B": (32, 4, 128),
    "Gemma-3-4B": (8, 4, 256), "Gemma-3-12B": (16, 8, 256),
    "Gemma-3-27B": (32, 16, 128),
}

# Gemma-3 checkpoints set query_pre_attn_scalar = 256, also for the D=128
# 27B geometry; Qwen3 scales by D^-1/2 (rope:25-36).
MODEL_QUERY_PRE_ATTN_SCALAR = {"Gemma-3-4B": 256.0, "Gemma-3-12B": 256.0, "Gemma-3-27B": 256.0}


def model_scale(name: str, d: int) -> float:
    """Attention scale of a model (rope:34-36): query_pre_attn_scalar^-1/2 when
    the model sets one, else D^-1/2."""
    scalar = MODEL_QUERY_PRE_ATTN_SCALAR.get(name)
    return float(1.0 / math.sqrt(scalar if scalar is not None else d))


_arch_cache: dict[int, str] = {}


def device_arch(device: torch.device) -> str:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _arch_cache:
        _arch_cache[idx] = torch.cuda.get_device_properties(idx).gcnArchName
    return _arch_cache[idx]


def _style(norm_style: Optional[str], hf_norm: bool) -> int:
    style = norm_style if norm_style is not None else ("hf" if hf_norm else "legacy")
    if style not in NORM_STYLES:
        raise ValueError(f"norm_style must be one of {sorted(NORM_STYLES)}, got {style!r}")
    return NORM_STYLES[style]


# ---------------------------------------------------------------------------
# Split-KV workspace (see kfmi_attention_workspace_bytes).  Eager launches use
# one zero-filled buffer per (device, stream); launches that share it run in
# that stream's order, so they never overlap on it, and each launch leaves
# its counters at zero again.  The counter region has the same size for every
# shape, so the buffer serves any sequence of shapes that fit in it.  When a
# larger shape needs more, a new buffer
# replaces it in the cache; the old one stays referenced until the process
# ends, so nothing that ever held its address sees it freed.  A launch
# captured into a HIP graph never uses the cache: it gets its own buffer from
# the graph's private memory pool whose counter region (the first
# WORK_COUNTER_BYTES; the partials behind it are written before they are
# read) is zeroed by a fill that is part of the graph and runs before the
# launch on every replay, so replays, on whatever stream, never share a
# workspace with eager launches or with other graphs.
# ---------------------------------------------------------------------------

WORK_COUNTER_BYTES = 4096  # the workspace's arrival-counter region (include/kfmi.h)

_work_cache: dict[tuple[int, int], torch.Tensor] = {}
_work_retired: list[torch.Tensor] = []
_work_bytes_cache: dict[tuple, int] = {}


def attention_workspace_bytes(b: int, hq: int, hkv: int, s: int, d: int, causal: bool) -> int:
    """Workspace bytes with which attention splits the longest causal query
    blocks over two workgroups for this shape on the current device (0: it
    never splits).  Cached per (device, shape)."""
    key = (torch.cuda.current_device() if torch.cuda.is_available() else -1, b, hq, hkv, s, d, bool(causal))
    n = _work_bytes_cache.get(key)
    if n is None:
        n = int(_lib.load().kfmi_attention_workspace_bytes(b, hq, hkv, s, d, int(bool(causal))))
        if n < 0:
            raise ValueError("invalid attention shape")
        _work_bytes_cache[key] = n
    return n


def _workspace(device: torch.device, nbytes: int):
    """A workspace of at least nbytes on this device with zeroed counters:
    the current stream's cached one (zero-filled once) for eager launches, a
    new one from the graph's pool during capture; None when nbytes is 0."""
    if nbytes <= 0:
        return None
    if torch.cuda.is_current_stream_capturing():
        buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        buf[:WORK_COUNTER_BYTES].zero_()  # a fill kernel inside the graph, not a memset node
        return buf
    idx = device.index if device.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(torch.device("cuda", idx))
    key = (idx, stream.cuda_stream)
    buf = _work_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _work_retired.append(buf)
        # zero-filled on the stream the launches run on, so in their order
        buf = torch.zeros(max(nbytes, 0 if buf is None else 2 * buf.numel()), dtype=torch.uint8, device=device)
        _work_cache[key] = buf
    return buf


def _work_args(work, q, hkv, causal):
    """(pointer, bytes) of the split workspace: ``work=None`` uses the cached
    one when the shape splits; a tensor is used as given."""
    if work is None:
        b, h, s, d = q.shape
        work = _workspace(q.device, attention_workspace_bytes(b, h, hkv, s, d, causal))
    if work is None:
        return None, 0
    return work.data_ptr(), work.numel() * work.element_size()


# ---------------------------------------------------------------------------
# Low-level launchers (caller-preallocated buffers, no checks beyond the C ABI's)
# ---------------------------------------------------------------------------

def prepare_attention(inputs, qn, kn, *, only_k=False, rows=4, rope=True, hf_norm=True, norm_style=None, vt=None,
                      eps=EPS):
    """RMSNorm*gamma (+ rotate-half RoPE) of K rows into ``kn`` and, unless
    ``only_k``, of Q rows into ``qn`` in one launch (rope:652-658).

    ``inputs`` is the reference 7-tuple ``(q, k, v, gq, gk, cos, sin)``; with
    ``rope=False`` the table entries are ignored.  ``rows`` (Triton rows per
    program) is ignored.  ``vt`` (optional, D=128, S % 8 == 0): the same launch
    also writes V transposed per head into it (the V^T operand of
    ``attention_prefill``).  Returns the launched kernel's record (a lazy
    ``_lib.Launches``), where the reference returns its kernel object.
    """
    q, k, v, gq, gk, cos, sin = inputs
    b, h, s, d = q.shape
    flags = (PREP_ONLY_K if only_k else 0) | (PREP_ROPE if rope else 0)
    _lib.call("kfmi_prepare_bf16",
              None if only_k else ptr(q), ptr(k), ptr(v) if vt is not None else None,
              None if only_k else ptr(gq), ptr(gk),
              ptr(cos) if rope else None, ptr(sin) if rope else None,
              None if only_k else ptr(qn), ptr(kn), ptr(vt),
              b, h, k.shape[1], s, d, float(eps), _style(norm_style, hf_norm), flags, stream_of(k))
    return _lib.Launches()


def launch_attention(inputs, out, *, causal=False, mode="query", bm=64, bn=64, warps=4, stages=1,
                     gather=True, rope=True, hf_norm=True, qn=None, kn=None, norm_style=None, vt=None, work=None):
    """Preparation + attention launches of the reference launcher (rope:661-677).

    ``mode='query'``: K is prepared once into ``kn``; Q's norm (+RoPE) runs in the
    attention prologue.  ``mode='unfused'``: Q into ``qn`` and K into ``kn``, then
    plain attention.  ``mode='full'``: one launch; attention normalises (and
    rotates) Q in its prologue and each K tile as it uses it -- no scratch, same
    values as ``'query'``.  Scratch buffers must be preallocated for the other
    modes (rope:665-672).  Timings must include every launch, as this function
    issues them.

    ``vt`` (optional, shaped like V): scratch for V transposed per head.  When
    given and the shape runs the ping-pong kernel (``uses_vt``), the
    preparation launch also writes it and the attention kernel reads V^T rows
    (one 16-byte LDS read per V operand instead of two transposing reads);
    results are the same.  End to end it is slower on MI355X (the extra 2x V
    bytes of the preparation launch cost more than the LDS reads save: S=4096
    step 148.5 vs 144.0 us), so the allocating APIs do not use it; it serves
    callers that already keep V transposed.

    ``work``: split-KV workspace (a zero-filled tensor of at least
    ``attention_workspace_bytes`` bytes); ``None`` uses a cached one per device.

    Returns the launched kernels (``kfmi_last_launches``: instance, grid, block,
    registers, LDS and scratch per kernel) as a lazy ``_lib.Launches``, read
    from the library on first use and valid until the thread's next compute
    call, where the reference returns its attention kernel object
    (rope:674-677).
    """
    if mode not in ("full", "query", "unfused"):
        raise ValueError("Invalid fusion mode")
    if mode != "full" and (kn is None or (mode == "unfused" and qn is None)):
        raise ValueError("Missing scratch buffers")
    q, k, v, gq, gk, cos, sin = inputs
    b, h, s, d = q.shape
    wp, wb = _work_args(work, q, k.shape[1], causal)
    _lib.call("kfmi_launch_attention_bf16",
              ptr(q), ptr(k), ptr(v), ptr(gq), ptr(gk),
              ptr(cos) if rope else None, ptr(sin) if rope else None,
              ptr(out), ptr(qn), ptr(kn), ptr(vt),
              b, h, k.shape[1], s, d, float(d) ** -0.5, EPS, int(bool(causal)),
              {"query": MODE_QUERY, "unfused": MODE_UNFUSED, "full": MODE_FULL}[mode], _style(norm_style, hf_norm),
              _bm(bm), _bn(bn), wp, wb, stream_of(q))
    return _lib.Launches()


def attention_prefill(q, kn, v, out, *, gq=None, cos=None, sin=None, causal=False, fuse_q=True,
                      norm_style="fp32", bm=128, bn=64, scale=None, vt=None, eps=EPS, work=None):
    """The attention launch alone (attention_v2_kernel, rope:608-649) on a prepared
    ``kn``.  ``fuse_q=True``: raw ``q`` with its RMSNorm (``gq``) and, when both
    tables are given, RoPE in the prologue (FUSE_Q); ``fuse_q=False``: ``q`` is
    already prepared.  ``scale`` defaults to D^-1/2 (rope:676).  ``vt``: V
    transposed per head (see ``transpose_v``), read instead of ``v`` when the
    shape allows it (``uses_vt``)."""
    b, h, s, d = q.shape
    wp, wb = _work_args(work, q, kn.shape[1], causal)
    _lib.call("kfmi_attention_bf16", ptr(q), ptr(kn), ptr(v), ptr(vt), ptr(gq), ptr(cos), ptr(sin), ptr(out),
              b, h, kn.shape[1], s, d, float(d) ** -0.5 if scale is None else float(scale), float(eps),
              int(bool(causal)), int(bool(fuse_q)), NORM_STYLES[norm_style], _bm(bm), _bn(bn), wp, wb, stream_of(q))


def transpose_v(v, vt):
    """``vt[b,h,d,s] = v[b,h,s,d]`` (S % 8 == 0): the V^T scratch that
    ``launch_attention`` fills itself when given ``vt``."""
    b, h, s, d = v.shape
    _lib.call("kfmi_transpose_v_bf16", ptr(v), ptr(vt), b * h, s, d, stream_of(v))


def launch_factored_attention(inputs, out, inv, kn, *, causal=False, bm=64, bn=64, work=None):
    """No-RoPE factored launch (qk:641-652): ``kn = bf16(k*inv_k*gk*gq)`` and FP32
    ``inv`` ``[B,Hq,S]`` (Q's inverse RMS, applied to the scores) are written to the
    caller's buffers, then factored attention writes ``out``.  ``inputs`` uses the
    reference five-tensor order ``(q, k, v, gq, gk)``.  Returns the launched
    kernels, as ``launch_attention`` does (the reference returns its kernel
    object, qk:651).  ``work``: the split-KV workspace, as for
    ``launch_attention`` (``None`` uses the cached one when the shape splits).
    """
    q, k, v, gq, gk = inputs[:5]
    b, h, s, d = q.shape
    wp, wb = _work_args(work, q, k.shape[1], causal)
    _lib.call("kfmi_launch_factored_attention_bf16",
              ptr(q), ptr(k), ptr(v), ptr(gq), ptr(gk), ptr(out), ptr(inv), ptr(kn),
              b, h, k.shape[1], s, d, EPS, int(bool(causal)), _bm(bm), _bn(bn), wp, wb, stream_of(q))
    return _lib.Launches()


def prepare_factored(inputs, inv, kn):
    """The factored preparation alone (qk:592-609): ``inv`` for every Q row and
    ``kn`` for every K row, one launch."""
    q, k, v, gq, gk = inputs[:5]
    b, h, s, d = q.shape
    _lib.call("kfmi_factored_prepare_bf16", ptr(q), ptr(k), ptr(gq), ptr(gk), ptr(inv), ptr(kn),
              b, h, k.shape[1], s, d, EPS, stream_of(q))


def factored_attention(q, kn, v, inv, out, *, causal=False, bm=64, bn=64, compute_inv=False, work=None):
    """The factored attention launch alone (qk:612-638) on raw ``q`` and prepared
    ``kn``; ``compute_inv=True`` derives Q's inverse RMS in the prologue (and
    writes it to ``inv`` when given) instead of reading ``inv``.  ``work``: the
    split-KV workspace, as for ``launch_attention``."""
    b, h, s, d = q.shape
    wp, wb = _work_args(work, q, kn.shape[1], causal)
    _lib.call("kfmi_factored_attention_bf16", ptr(q), ptr(kn), ptr(v), ptr(inv), ptr(out),
              b, h, kn.shape[1], s, d, EPS, int(bool(causal)), int(bool(compute_inv)), _bm(bm), _bn(bn),
              wp, wb, stream_of(q))


def _bm(bm):
    return int(bm) if int(bm) % 32 == 0 and 32 <= int(bm) <= 256 else 128


def _bn(bn):
    return int(bn) if int(bn) in (32, 64, 128) else 64


# ---------------------------------------------------------------------------
# Validated, allocating API
# ---------------------------------------------------------------------------

def _check_device(tensors, device):
    if any((not t.is_cuda) or t.device != device or t.dtype != torch.bfloat16 or not t.is_contiguous()
           for t in tensors):
        raise ValueError("Inputs must be contiguous BF16 tensors on one GPU device")
    if not device_arch(device).startswith("gfx950"):
        raise ValueError(f"This implementation targets gfx950 (MI355X); device is {device_arch(device)}")


def optimized_attention(q, k, v, gq, gk, cos=None, sin=None, *, causal=False, mode="query", bn=128,
                        gather=False, norm_style="hf"):
    """Forward BF16 attention with Q/K RMSNorm (+ optional split-half RoPE) fused
    into the prologue (rope:680-726).

    ``mode='query'`` prepares K once and fuses Q's norm (and RoPE when both
    tables are given) into the attention prologue; ``mode='unfused'`` prepares Q
    and K, then runs the same attention.  ``norm_style``: ``'hf'`` rounds at HF's
    BF16 op boundaries, ``'legacy'`` casts x*inv*gamma once, ``'fp32'`` keeps the
    whole prologue in FP32 with one final rounding.  Forward only; projections,
    KV caches and backward are out of scope.  Every argument error raises
    ``ValueError`` before anything is launched (rope:695-719).
    """
    if mode not in ("query", "unfused") or bn not in (64, 128):
        raise ValueError("mode must be 'query' or 'unfused' and bn must be 64 or 128")
    if norm_style not in NORM_STYLES:
        raise ValueError("norm_style must be 'hf', 'legacy' or 'fp32'")
    if (cos is None) != (sin is None):
        raise ValueError("Pass both rotary tables (cos and sin) or neither")
    rotary = cos is not None
    tensors = (q, k, v, gq, gk) + ((cos, sin) if rotary else ())
    if any(t.requires_grad for t in tensors):
        raise ValueError("optimized_attention is forward-only")
    if q.ndim != 4 or k.ndim != 4 or k.shape != v.shape:
        raise ValueError("Expected q [B,Hq,S,D] and k, v [B,Hkv,S,D]")
    b, h, s, d = q.shape
    if (d not in (128, 256) or min(b, h, s) < 1 or k.shape[0] != b or tuple(k.shape[2:]) != (s, d)
            or k.shape[1] < 1 or h % k.shape[1]):
        raise ValueError("Expected D in (128, 256), matching batch and sequence, and Hq a multiple of Hkv")
    if (tuple(gq.shape) != (d,) or tuple(gk.shape) != (d,)
            or (rotary and (tuple(cos.shape) != (s, d) or tuple(sin.shape) != (s, d)))):
        raise ValueError("Expected gamma vectors [D] and optional rotary tables [S,D]")
    _check_device(tensors, q.device)
    if max(q.numel(), k.numel()) >= 2 ** 31:
        raise ValueError("Tensors must have fewer than 2**31 elements")
    return torch.ops.kfmi.optimized_attention(q, k, v, gq, gk, cos, sin, bool(causal), mode, int(bn), norm_style)


def _position_table(t, q):
    """[S,D], [B,S,D] or [B,1,S,D] rotary table -> contiguous [S,D] of q's dtype.
    All rows of the isolated workloads share positions, so the first broadcast
    slice is exact (rope:193-200)."""
    if t.ndim == 4:
        t = t[:, 0]
    if t.ndim == 3:
        t = t[0]
    return t.to(q.dtype).contiguous()


def _fused_checks(q, k, v, gq, gk, cos, sin):
    if q.ndim != 4 or k.ndim != 4 or k.shape != v.shape:
        raise ValueError("Expected q [B,Hq,S,D] and k, v [B,Hkv,S,D]")
    b, h, s, d = q.shape
    if d not in (128, 256) or k.shape[0] != b or tuple(k.shape[2:]) != (s, d) or h % k.shape[1]:
        raise ValueError("Expected D in (128, 256), matching batch and sequence, and Hq a multiple of Hkv")
    tensors = (q, k, v) + tuple(t for t in (gq, gk, cos, sin) if t is not None)
    _check_device(tensors, q.device)


def fused(q, k, v, gq, gk, cos, sin, causal, eps=EPS, scale=None, norm_style="qwen3"):
    """Fused Q/K RMSNorm + rotate-half RoPE + attention with explicit ``eps`` and
    ``scale`` (the older API, rope:185-203; ``scale=None`` is D^-1/2).

    The HF/Qwen3 rounding chain (``norm_style='qwen3'``, the reference's only
    style here; ``'hf'`` is accepted as its name in this package) is applied to
    both Q and K.  The reference recomputes K's norm+RoPE for every key tile
    inside one kernel; here K is prepared once (one launch) and Q's
    norm+RoPE runs in the attention prologue -- the same values, since a K row
    prepared once or per tile is the same function of the same inputs.
    Tables may be [S,D], [B,S,D] or [B,1,S,D] (the first broadcast slice is
    used, rope:193-200)."""
    if norm_style not in ("qwen3", "hf"):
        raise ValueError("fused implements the HF/Qwen3 norm_style only")
    cos, sin = _position_table(cos, q), _position_table(sin, q)
    _fused_checks(q, k, v, gq, gk, cos, sin)
    b, h, s, d = q.shape
    if tuple(cos.shape) != (s, d) or tuple(sin.shape) != (s, d):
        raise ValueError("Expected rotary tables of S rows")
    out, kn = torch.empty_like(q), torch.empty_like(k)
    with torch.cuda.device(q.device):
        prepare_attention((q, k, v, gq, gk, cos, sin), None, kn, only_k=True, rope=True, norm_style="hf", eps=eps)
        attention_prefill(q, kn, v, out, gq=gq, cos=cos, sin=sin, causal=causal, fuse_q=True, norm_style="hf",
                          scale=scale, eps=eps)
    return out


def anchor(q, k, v, cos, sin, causal, scale=None):
    """Attention on already prepared Q/K (the reference's FUSED=False launch,
    rope:205-208); the tables are unused."""
    _fused_checks(q, k, v, None, None, None, None)
    out = torch.empty_like(q)
    with torch.cuda.device(q.device):
        attention_prefill(q, k, v, out, causal=causal, fuse_q=False, scale=scale)
    return out


def separate(q, k, v, gq, gk, cos, sin, causal, eps=EPS, scale=None, norm_style="qwen3"):
    """Separate preparation of Q and K (HF/Qwen3 chain, one launch) followed by
    ``anchor`` (rope:210-212)."""
    if norm_style not in ("qwen3", "hf"):
        raise ValueError("separate implements the HF/Qwen3 norm_style only")
    cos, sin = _position_table(cos, q), _position_table(sin, q)
    _fused_checks(q, k, v, gq, gk, cos, sin)
    qn, kn = torch.empty_like(q), torch.empty_like(k)
    with torch.cuda.device(q.device):
        prepare_attention((q, k, v, gq, gk, cos, sin), qn, kn, only_k=False, rope=True, norm_style="hf", eps=eps)
    return anchor(qn, kn, v, cos, sin, causal, scale)


def norm_rope(q, k, gq, gk, cos=None, sin=None, *, norm_style="fp32", qn=None, kn=None):
    """Isolated per-head Q/K RMSNorm (+ rotate-half RoPE): one launch over every Q
    and K row (the ``only_k=False`` preparation of rope:652-658).  Returns
    ``(qn, kn)``, allocating them unless given."""
    if norm_style not in NORM_STYLES:
        raise ValueError("norm_style must be 'hf', 'legacy' or 'fp32'")
    if (cos is None) != (sin is None):
        raise ValueError("Pass both rotary tables (cos and sin) or neither")
    if q.ndim != 4 or k.ndim != 4 or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
        raise ValueError("Expected q [B,Hq,S,D] and k [B,Hkv,S,D]")
    b, h, s, d = q.shape
    if d not in (128, 256) or h % k.shape[1]:
        raise ValueError("Expected D in (128, 256) and Hq a multiple of Hkv")
    if tuple(gq.shape) != (d,) or tuple(gk.shape) != (d,) or (cos is not None and (
            tuple(cos.shape) != (s, d) or tuple(sin.shape) != (s, d))):
        raise ValueError("Expected gamma vectors [D] and optional rotary tables [S,D]")
    for name, out, like in (("qn", qn, q), ("kn", kn, k)):
        if out is not None and (out.shape != like.shape or out.dtype != torch.bfloat16
                                or out.device != like.device or not out.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous BF16 tensor shaped like its input on the same device")
    tensors = (q, k, gq, gk) + ((cos, sin) if cos is not None else ())
    _check_device(tensors, q.device)
    if qn is None and kn is None:
        return torch.ops.kfmi.norm_rope(q, k, gq, gk, cos, sin, norm_style)
    qn = torch.empty_like(q) if qn is None else qn
    kn = torch.empty_like(k) if kn is None else kn
    _norm_rope_into(q, k, gq, gk, cos, sin, qn, kn, norm_style)
    return qn, kn


def _norm_rope_into(q, k, gq, gk, cos, sin, qn, kn, norm_style):
    b, h, s, d = q.shape
    rope = cos is not None
    _lib.call("kfmi_prepare_bf16", ptr(q), ptr(k), None, ptr(gq), ptr(gk), ptr(cos), ptr(sin), ptr(qn), ptr(kn), None,
              b, h, k.shape[1], s, d, EPS, NORM_STYLES[norm_style], PREP_ROPE if rope else 0, stream_of(q))


def factored_qk_attention(q, k, v, gq, gk, *, causal=False):
    """Allocating form of ``launch_factored_attention``: returns ``(out, inv, kn)``."""
    if q.ndim != 4 or k.ndim != 4 or k.shape != v.shape:
        raise ValueError("Expected q [B,Hq,S,D] and k, v [B,Hkv,S,D]")
    b, h, s, d = q.shape
    if (d not in (128, 256) or k.shape[0] != b or tuple(k.shape[2:]) != (s, d) or h % k.shape[1]
            or tuple(gq.shape) != (d,) or tuple(gk.shape) != (d,)):
        raise ValueError("Expected D in (128, 256), matching shapes, gamma vectors [D] and valid GQA")
    _check_device((q, k, v, gq, gk), q.device)
    return torch.ops.kfmi.factored_attention(q, k, v, gq, gk, bool(causal))


# ---------------------------------------------------------------------------
# torch.library custom ops (graph-capturable: no host sync, launches on the
# current stream; fake kernels give shapes to tracing)
# ---------------------------------------------------------------------------

@torch.library.custom_op("kfmi::optimized_attention", mutates_args=(), device_types="cuda")
def _optimized_attention_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gq: torch.Tensor,
                            gk: torch.Tensor, cos: Optional[torch.Tensor], sin: Optional[torch.Tensor],
                            causal: bool, mode: str, bn: int, norm_style: str) -> torch.Tensor:
    out = torch.empty_like(q)
    kn = torch.empty_like(k)
    qn = torch.empty_like(q) if mode == "unfused" else None
    rotary = cos is not None
    xs = (q, k, v, gq, gk, cos if rotary else q, sin if rotary else k)
    with torch.cuda.device(q.device):
        launch_attention(xs, out, causal=causal, mode=mode, bm=128, bn=bn, rope=rotary, qn=qn, kn=kn,
                         norm_style=norm_style)
    return out


def uses_vt(hq: int, hkv: int, s: int, d: int, b: int = 1, causal: bool = True) -> bool:
    """Whether launch_attention (mode 'query' or 'unfused') makes use of a
    ``vt`` scratch for this shape on the current device: when the library
    runs its ping-pong kernel for it (``kfmi_attention_kernel``) and V^T rows
    are 16-byte aligned (S % 8 == 0)."""
    return s % 8 == 0 and _lib.attention_kernel(b, hq, hkv, s, d, causal, MODE_QUERY) == "pingpong"


@_optimized_attention_op.register_fake
def _(q, k, v, gq, gk, cos, sin, causal, mode, bn, norm_style):
    return torch.empty_like(q)


@torch.library.custom_op("kfmi::norm_rope", mutates_args=(), device_types="cuda")
def _norm_rope_op(q: torch.Tensor, k: torch.Tensor, gq: torch.Tensor, gk: torch.Tensor,
                  cos: Optional[torch.Tensor], sin: Optional[torch.Tensor],
                  norm_style: str) -> tuple[torch.Tensor, torch.Tensor]:
    qn = torch.empty_like(q)
    kn = torch.empty_like(k)
    with torch.cuda.device(q.device):
        _norm_rope_into(q, k, gq, gk, cos, sin, qn, kn, norm_style)
    return qn, kn


@_norm_rope_op.register_fake
def _(q, k, gq, gk, cos, sin, norm_style):
    return torch.empty_like(q), torch.empty_like(k)


@torch.library.custom_op("kfmi::factored_attention", mutates_args=(), device_types="cuda")
def _factored_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gq: torch.Tensor, gk: torch.Tensor,
                 causal: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    out = torch.empty_like(q)
    kn = torch.empty_like(k)
    inv = torch.empty(q.shape[:-1], device=q.device, dtype=torch.float32)
    with torch.cuda.device(q.device):
        launch_factored_attention((q, k, v, gq, gk), out, inv, kn, causal=causal, bm=128, bn=64)
    return out, inv, kn


@_factored_op.register_fake
def _(q, k, v, gq, gk, causal):
    return (torch.empty_like(q), torch.empty(q.shape[:-1], device=q.device, dtype=torch.float32),
            torch.empty_like(k))


def attention_flops(b: int, hq: int, s: int, d: int, causal: bool) -> int:
    """Algorithmic FLOPs of QK^T and PV: 4*B*Hq*D*pairs, pairs = S(S+1)/2 causal, S^2 otherwise."""
    pairs = s * (s + 1) // 2 if causal else s * s
    return 4 * b * hq * d * pairs


def norm_rope_bytes(b: int, hq: int, hkv: int, s: int, d: int, rope: bool = True) -> int:
    """Algorithmic HBM bytes of one Q+K norm+RoPE pass: BF16 read+write of every
    row, the cos/sin half-tables and both gamma vectors."""
    return 4 * b * s * (hq + hkv) * d + (2 * s * d if rope else 0) + 4 * d


def k_prep_bytes(b: int, hkv: int, s: int, d: int, rope: bool = True) -> int:
    return 4 * b * s * hkv * d + (2 * s * d if rope else 0) + 2 * d

