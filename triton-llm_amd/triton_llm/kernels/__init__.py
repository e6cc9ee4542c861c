"""Attention-path kernels of triton_llm on the gfx950 HIP library.

Exports the reference's hot-path names (triton_llm/kernels/__init__.py:6-31 of
ziliangpeng/triton-llm: ``attention``, ``attention_gqa``, ``precompute_cos_sin``,
``apply_rope``) plus the additive batched entry points of this build
(flash prefill, KV-cache append, split-K decode) and the model's projection
``gemm`` (rocBLAS-backed).  The reference's other kernels (add, gelu,
layer_norm, rms_norm, softmax, swiglu, embedding) are outside this library's
scope.
"""

from .attention import attention
from .attention_gqa import attention_gqa
from .rope import apply_rope, precompute_cos_sin, precompute_cos_sin_device
from .flash import flash_attention, flash_attention_strided
from .gemm import gemm
from .decode import (
    allocate_kv_cache,
    attention_decode,
    decode_step,
    decode_workspace,
    rope_kv_append,
)

__all__ = [
    "attention",
    "attention_gqa",
    "precompute_cos_sin",
    "precompute_cos_sin_device",
    "apply_rope",
    "flash_attention",
    "flash_attention_strided",
    "allocate_kv_cache",
    "rope_kv_append",
    "attention_decode",
    "decode_step",
    "decode_workspace",
    "gemm",
]
