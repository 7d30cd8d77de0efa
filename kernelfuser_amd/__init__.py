"""kernelfuser_amd -- MI355X (gfx950) RoPE-aware attention prologue.

Hand-written gfx950 HIP kernels behind a C ABI (``include/kfmi.h``), exposed as
PyTorch-ROCm ops with the signatures of KernelFuser's attention-prologue path:

* ``optimized_attention``  (src/e1_rope_publication_v1.py:680-726)
* ``launch_attention`` / ``prepare_attention``  (rope:652-677)
* ``launch_factored_attention``  (src/e1_qk_publication_v3.py:641-652)
* ``norm_rope``  isolated per-head Q/K RMSNorm + RoPE
* ``fused`` / ``anchor`` / ``separate``, ``model_scale``  (the older API, rope:25-36, :185-212)

Build the native library with ``python -m kernelfuser_amd.build``.
"""
from .ops import (  # noqa: F401
    EPS,
    MODEL_QUERY_PRE_ATTN_SCALAR,
    MODELS,
    anchor,
    fused,
    model_scale,
    separate,
    attention_flops,
    attention_workspace_bytes,
    attention_prefill,
    factored_attention,
    factored_qk_attention,
    k_prep_bytes,
    launch_attention,
    launch_factored_attention,
    norm_rope,
    norm_rope_bytes,
    optimized_attention,
    prepare_attention,
    prepare_factored,
    transpose_v,
    uses_vt,
)
from .inputs import GEMMA3_12B, QWEN3_8B, Inputs, make_inputs, rope_tables  # noqa: F401

__all__ = [
    "EPS", "MODELS", "MODEL_QUERY_PRE_ATTN_SCALAR", "model_scale", "fused", "anchor", "separate",
    "optimized_attention", "attention_prefill", "launch_attention", "prepare_attention",
    "launch_factored_attention", "prepare_factored", "factored_attention", "factored_qk_attention",
    "norm_rope", "uses_vt", "attention_workspace_bytes", "transpose_v", "attention_flops", "norm_rope_bytes", "k_prep_bytes", "make_inputs", "rope_tables",
    "Inputs", "QWEN3_8B", "GEMMA3_12B",
]
