"""Batched flash attention forward (additive API, the prefill hot path).

``flash_attention(q, k, v)`` with q ``(batch, n_head, seq_q, d_k)`` and k/v
``(batch, n_kv_head, seq_k, d_k)`` device tensors (float32 / float16 /
gpu.bfloat16), bottom-right causal alignment and GQA head mapping exactly as
``attention_gqa`` (attention_gqa.py:76, :97 of the reference), for many
sequences in one launch.  The reference handles batch = 1 only and launches
one program per (row, head) (attention_gqa.py:247).

``flash_attention_strided`` takes explicit {batch, head, seq} element strides,
so it reads K/V straight out of a ``(batch, n_kv_head, max_ctx, d_k)`` cache
and Q/O in any row-major layout with a contiguous head dimension, e.g. the
``(seq, n_head * d_k)`` rows a QKV projection writes, removing the host
transposes of smollm2_triton/model.py:320-348.
"""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from triton_llm import _lib
from ._common import launch, check_status, contiguous_strides, default_scale, same_dtype, scratch, vp
from .attention_gqa import MAX_D


def flash_workspace_bytes(batch: int, n_kv_head: int, seq_k: int, d_k: int, dtype, *,
                          n_head: int | None = None, seq_q: int | None = None,
                          causal: bool = True) -> int:
    """Workspace bytes of a flash call.  Given ``n_head`` and ``seq_q`` too,
    the size that also lets a causal call split its costliest tiles' key
    ranges over two workgroups (tl_attention_fwd_workspace_bytes_split);
    otherwise the minimum."""
    lib = gpu.runtime()
    code = gpu.dtype_code(dtype)
    if n_head is None or seq_q is None:
        return lib.tl_attention_fwd_workspace_bytes(batch, n_kv_head, seq_k, d_k, code)
    return lib.tl_attention_fwd_workspace_bytes_split(batch, n_head, n_kv_head, seq_q, seq_k, d_k,
                                                      1 if causal else 0, code)


def flash_attention_strided(q, k, v, out, *, batch, n_head, n_kv_head, seq_q, seq_k, d_k,
                            q_strides, k_strides, v_strides, o_strides, causal=True,
                            sm_scale=None, workspace=None):
    """Launch the flash kernel on raw layouts given by element strides."""
    if n_head <= 0 or n_kv_head <= 0 or n_head % n_kv_head:
        raise ValueError(f"n_head ({n_head}) must be a positive multiple of n_kv_head ({n_kv_head})")
    if not (d_k > 0 and (d_k & (d_k - 1)) == 0 and d_k <= MAX_D):
        raise ValueError(f"d_k ({d_k}) must be a power of 2 <= {MAX_D}")
    code = same_dtype(q, k, v, out)
    if batch == 0 or seq_q == 0:
        return out
    if seq_k == 0:
        raise ValueError("seq_k must be >= 1")
    if sm_scale is None:
        sm_scale = default_scale(d_k)
    lib = gpu.runtime()
    if workspace is None:  # the shared workspace, large enough to split
        ws_bytes = lib.tl_attention_fwd_workspace_bytes_split(batch, n_head, n_kv_head, seq_q, seq_k,
                                                              d_k, 1 if causal else 0, code)
        ws = scratch(ws_bytes, None, key="flash")
    else:
        # a caller's workspace must hold the minimum (which may be 0) and is
        # always passed on: the call splits if it holds more
        need = lib.tl_attention_fwd_workspace_bytes(batch, n_kv_head, seq_k, d_k, code)
        if workspace.nbytes < need:
            raise ValueError(f"workspace holds {workspace.nbytes} bytes, {need} required")
        ws = workspace
    launch(lib.tl_attention_fwd, vp(q), vp(k), vp(v), vp(out), vp(ws), ws.nbytes if ws is not None else 0,
        batch, n_head, n_kv_head, seq_q, seq_k, d_k,
        _lib.strides(*q_strides), _lib.strides(*k_strides), _lib.strides(*v_strides),
        _lib.strides(*o_strides), float(sm_scale), 1 if causal else 0, code, None,
        what="flash_attention")
    return out


def flash_attention(q, k, v, causal: bool = True, sm_scale: float | None = None, out=None,
                    workspace=None):
    """O = softmax(Q K^T * sm_scale [+ causal mask]) V for contiguous 4-D tensors."""
    if len(q.shape) != 4 or len(k.shape) != 4 or k.shape != v.shape:
        raise ValueError(f"expected q (B,Hq,Sq,D) and k/v (B,Hkv,Sk,D), got {q.shape}, {k.shape}, {v.shape}")
    batch, n_head, seq_q, d_k = q.shape
    kb, n_kv, seq_k, kd = k.shape
    if kb != batch or kd != d_k:
        raise ValueError(f"q {q.shape} and k {k.shape} disagree on batch or d_k")
    if n_kv <= 0 or n_head % n_kv:
        raise ValueError(f"n_head ({n_head}) must be a positive multiple of n_kv_head ({n_kv})")
    same_dtype(q, k, v)
    if out is None:
        out = gpu.allocate(q.shape, q.dtype)
    elif out.shape != q.shape:
        raise ValueError(f"out shape {out.shape} != q shape {q.shape}")
    qs = contiguous_strides(q.shape)[:3]
    ks = contiguous_strides(k.shape)[:3]
    return flash_attention_strided(
        q, k, v, out, batch=batch, n_head=n_head, n_kv_head=n_kv, seq_q=seq_q, seq_k=seq_k,
        d_k=d_k, q_strides=qs, k_strides=ks, v_strides=ks, o_strides=qs, causal=causal,
        sm_scale=sm_scale, workspace=workspace,
    )
