"""Attention-path kernels of triton_llm on the gfx950 HIP library.

Exports the reference's hot-path names (triton_llm/kernels/__init__.py:6-31 of
ziliangpeng/triton-llm: ``attention``, ``attention_gqa``, ``precompute_cos_sin``,
``apply_rope``) plus the additive batched entry points of this build
(flash prefill, KV-cache append, split-K decode) and the model step's other
layers: the projection ``gemm``, ``rms_norm`` (plus the fused
``add_rms_norm``), ``swiglu`` and ``add``, and on-device next-token
``sample`` / ``sample_rows`` (the models' ``_sample``).  The reference's gelu,
layer_norm, softmax and embedding kernels (GPT-2 and host-side pieces) are
outside this library's scope.
"""

from .attention import attention
from .attention_gqa import attention_gqa
from .rope import apply_rope, precompute_cos_sin, precompute_cos_sin_device
from .flash import flash_attention, flash_attention_strided
from .gemm import gemm, gemm_grouped
from .rms_norm import add_rms_norm, rms_norm
from .swiglu import swiglu
from .add import add
from .sample import sample, sample_rows
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
    "gemm_grouped",
    "rms_norm",
    "add_rms_norm",
    "swiglu",
    "add",
    "sample",
    "sample_rows",
]
