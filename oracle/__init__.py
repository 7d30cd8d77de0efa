"""CPU FP32 oracle for the RoPE-aware attention prologue -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``kernelfuser_amd``) imports this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or, for the CPU baseline, as the
eager FP32 path that is timed beside the GPU).

Every function restates an algorithm of the reference checkout
(WenbinWang12/KernelFuser) and cites the file:line it follows.  The pins that
check the restatement itself (closed forms, invariants, brute force on tiny
inputs, planted-mistake tests) live in ``tests/test_oracle_*.py``.
"""
from .fp32 import (  # noqa: F401
    EPS,
    rope_tables,
    rms_inverse,
    norm_fp32,
    rope_fp32,
    norm_rope_fp32,
    norm_hf_bf16,
    rope_hf_bf16,
    norm_legacy_bf16,
    attention_fp32,
    attention_rows_fp32,
    attention_bruteforce,
    oracle_fp32,
    oracle_rows_fp32,
    refinement_oracle_norope,
    factored_prepare_fp32,
    factored_attention_fp32,
    expand,
)
from .gates import metric, norm_rope_gate, attention_gate  # noqa: F401
