"""Grouped-query attention (GQA) on the gfx950 HIP library.

Same entry point, arguments, validation order and error types as the
reference's ``attention_gqa`` (triton_llm/kernels/attention_gqa.py:149-269 of
ziliangpeng/triton-llm):

    O = softmax(Q @ K^T * sm_scale) @ V,  kv_head = q_head // (n_head // n_kv_head)

with rows grouped by head (Q ``(n_head * seq_q, d_k)``, K/V
``(n_kv_head * seq_k, d_k)``) and bottom-right causal alignment
(key j visible to query i iff j <= seq_k - seq_q + i, attention_gqa.py:97).

Dispatch (all HIP, no CPU path):
  * seq_q == 1 and d_k in (64, 128): split-K decode kernel (tl_attention_decode)
    -- the shape the models' decode step produces;
  * otherwise: flash prefill kernel (tl_attention_fwd; MFMA for d_k 64/128).
Inputs may be float32 (the reference's dtype), float16 or gpu.bfloat16; the
output has the input dtype.  Like the reference, nothing is synchronised.
"""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from ._common import launch, check_status, default_scale, same_dtype, shared_workspace, vp
from triton_llm import _lib

DECODE_D = (64, 128)
# Largest head size the library computes (its generic kernel keeps a query
# row and an accumulator row of d_k floats in LDS).  The reference accepts
# any power of two; above this one this build raises.
MAX_D = 4096


def attention_gqa(
    q_dev: "gpu.DeviceTensor",
    k_dev: "gpu.DeviceTensor",
    v_dev: "gpu.DeviceTensor",
    n_head: int,
    n_kv_head: int,
    causal: bool = True,
    sm_scale: float | None = None,
) -> "gpu.DeviceTensor":
    """GPU-resident GQA attention. No sync, no host copies."""
    # --- Input validation (same checks and order as attention_gqa.py:188-233) ---
    if n_head <= 0:
        raise ValueError(f"n_head must be > 0, got {n_head}")
    if n_kv_head <= 0:
        raise ValueError(f"n_kv_head must be > 0, got {n_kv_head}")
    if n_head % n_kv_head != 0:
        raise ValueError(
            f"n_head ({n_head}) must be divisible by n_kv_head ({n_kv_head})"
        )
    if len(q_dev.shape) != 2 or len(k_dev.shape) != 2 or len(v_dev.shape) != 2:
        raise ValueError(
            f"All inputs must be 2D, got q.ndim={len(q_dev.shape)}, k.ndim={len(k_dev.shape)}, v.ndim={len(v_dev.shape)}"
        )
    if q_dev.shape[0] % n_head != 0:
        raise ValueError(
            f"Query shape[0] ({q_dev.shape[0]}) must be divisible by n_head ({n_head})"
        )
    if k_dev.shape[0] % n_kv_head != 0:
        raise ValueError(
            f"Key shape[0] ({k_dev.shape[0]}) must be divisible by n_kv_head ({n_kv_head})"
        )

    d_k = q_dev.shape[1]
    seq_q = q_dev.shape[0] // n_head
    seq_k = k_dev.shape[0] // n_kv_head

    if k_dev.shape != (n_kv_head * seq_k, d_k):
        raise ValueError(
            f"K shape {k_dev.shape} != expected ({n_kv_head * seq_k}, {d_k})"
        )
    if v_dev.shape != (n_kv_head * seq_k, d_k):
        raise ValueError(
            f"V shape {v_dev.shape} != expected ({n_kv_head * seq_k}, {d_k})"
        )
    code = same_dtype(q_dev, k_dev, v_dev)
    out_dtype = q_dev.dtype

    if seq_q == 0:
        return gpu.allocate((0, d_k), out_dtype)
    if seq_k == 0:
        # The reference's tests require zeros here (test_attention_gqa.py:297).
        return gpu.zeros((n_head * seq_q, d_k), out_dtype)

    if d_k <= 0 or (d_k & (d_k - 1)) != 0:
        raise ValueError(
            f"d_k ({d_k}) must be a positive power of 2"
        )
    if d_k > MAX_D:
        raise ValueError(f"d_k ({d_k}) > {MAX_D} is not supported by the HIP kernels")

    if sm_scale is None:
        sm_scale = default_scale(d_k)

    o_dev = gpu.allocate((n_head * seq_q, d_k), out_dtype)
    if seq_q == 1 and d_k in DECODE_D:
        _decode_one(q_dev, k_dev, v_dev, o_dev, n_head, n_kv_head, seq_k, d_k, sm_scale, code)
    else:
        q_str = _lib.strides(n_head * seq_q * d_k, seq_q * d_k, d_k)
        kv_str = _lib.strides(n_kv_head * seq_k * d_k, seq_k * d_k, d_k)
        lib = gpu.runtime()
        ws_bytes = lib.tl_attention_fwd_workspace_bytes_split(1, n_head, n_kv_head, seq_q, seq_k, d_k,
                                                              1 if causal else 0, code)
        ws = shared_workspace("attention_gqa.prefill", ws_bytes)
        launch(lib.tl_attention_fwd, vp(q_dev), vp(k_dev), vp(v_dev), vp(o_dev), vp(ws), ws_bytes,
            1, n_head, n_kv_head, seq_q, seq_k, d_k,
            q_str, kv_str, kv_str, q_str,
            float(sm_scale), 1 if causal else 0, code, None,
            what="attention_gqa")
    return o_dev


def _decode_one(q_dev, k_dev, v_dev, o_dev, n_head, n_kv_head, seq_k, d_k, sm_scale, code):
    """seq_q == 1: every query row sees all seq_k keys (causal or not).

    The length goes to the kernel by value (``cache_lens`` NULL, ``len_add``
    = seq_k) and the split-K partials use a workspace kept across calls, so
    a decode step uploads nothing, waits for nothing and, once the output
    block is cached, allocates nothing."""
    lib = gpu.runtime()
    split = lib.tl_decode_split_size(1, n_kv_head, seq_k)
    ws_bytes = lib.tl_attention_decode_workspace_bytes(1, n_head, seq_k, d_k, split)
    ws = shared_workspace("attention_gqa.decode", ws_bytes)
    qo = _lib.strides(n_head * d_k, d_k)
    kv = _lib.strides(n_kv_head * seq_k * d_k, seq_k * d_k, d_k)
    launch(lib.tl_attention_decode, vp(q_dev), vp(k_dev), vp(v_dev), None, seq_k, vp(o_dev), vp(ws), ws.nbytes,
        1, n_head, n_kv_head, seq_k, d_k, qo, kv, kv, qo,
        float(sm_scale), split, code, None,
        what="attention_gqa(decode)")
