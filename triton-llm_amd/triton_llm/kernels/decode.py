"""Batched decode over a GPU-resident, preallocated KV cache (additive API).

The reference keeps its KV cache on the host and, every decode step, applies
RoPE on the GPU, copies the new K/V to the host, writes them at position
``prev_seq`` and re-uploads the whole valid prefix before calling
``attention_gqa(..., causal=False)`` (smollm2_triton/model.py:289-314;
gpt2_triton/model.py:332-349; cache layout :219-225).  Here the cache lives in
HBM as ``(batch, n_kv_head, max_ctx, d_k)`` per K and V and is updated in place:

* :func:`allocate_kv_cache` -- the preallocated cache (cf. ``_init_cache_gpu``,
  smollm2_triton/model.py:190-225, batched);
* :func:`rope_kv_append` -- RoPE on q/k fused with the cache write at
  ``cache_lens[b] + s`` (one kernel);
* :func:`attention_decode` -- split-K decode + log-sum-exp combine over
  ``cache_lens[b] + len_add`` positions;
* :func:`decode_workspace` -- a reusable split-K workspace;
* :func:`decode_step` -- append then attend over ``cache_lens[b] + 1``
  positions, the reference's per-layer decode sequence in two launches.

``cache_lens`` is an int32 device array of tokens already cached per sequence;
it is not modified (the caller advances it, as the model advances
``_cache_len``).  Nothing here synchronises.
"""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from triton_llm import _lib
from ._common import launch, check_status, default_scale, same_dtype, scratch, vp


def allocate_kv_cache(batch: int, n_kv_head: int, max_ctx: int, d_k: int, dtype=np.float32,
                      zero: bool = True):
    """(k_cache, v_cache), each ``(batch, n_kv_head, max_ctx, d_k)`` on the GPU."""
    if batch <= 0 or n_kv_head <= 0 or max_ctx <= 0 or d_k <= 0:
        raise ValueError(
            f"cache dims must be positive, got batch={batch} n_kv_head={n_kv_head} "
            f"max_ctx={max_ctx} d_k={d_k}"
        )
    gpu.dtype_code(dtype)
    alloc = gpu.zeros if zero else gpu.allocate
    shape = (batch, n_kv_head, max_ctx, d_k)
    return alloc(shape, dtype), alloc(shape, dtype)


def _check_cache(k_cache, v_cache):
    if len(k_cache.shape) != 4 or k_cache.shape != v_cache.shape:
        raise ValueError(
            f"k_cache/v_cache must be matching 4-D (batch, n_kv_head, max_ctx, d_k), "
            f"got {k_cache.shape} and {v_cache.shape}"
        )
    return k_cache.shape


def _check_lens(lens, batch):
    if gpu.dtype_name(lens.dtype) != "int32" or lens.shape != (batch,):
        raise ValueError(f"cache_lens must be int32 of shape ({batch},), got {gpu.dtype_name(lens.dtype)} {lens.shape}")


def rope_kv_append(q_dev, k_new, v_new, k_cache, v_cache, cache_lens,
                   cos_dev=None, sin_dev=None):
    """Rotate q (in place) and k_new, write k/v into the cache at ``cache_lens[b] + s``.

    q_dev: ``(batch, n_new, n_head, d_k)`` or ``(batch, n_head, d_k)`` (n_new = 1),
    or None; k_new / v_new: ``(batch, n_new, n_kv_head, d_k)`` or
    ``(batch, n_kv_head, d_k)``.  cos/sin: float32 ``(rows, d_k // 2)`` tables,
    or None for no RoPE (GPT-2).  Positions past the cache (or the table) are
    skipped by the kernel; callers are expected to keep ``cache_lens[b] +
    n_new <= max_ctx`` as the reference model does (model.py:262-268).
    """
    batch, n_kv, max_ctx, d_k = _check_cache(k_cache, v_cache)
    if len(k_new.shape) == 3:
        n_new = 1
    elif len(k_new.shape) == 4:
        n_new = k_new.shape[1]
    else:
        raise ValueError(f"k_new must be 3-D or 4-D, got {k_new.shape}")
    kv_shape = (batch, n_new, n_kv, d_k)
    if int(np.prod(k_new.shape)) != int(np.prod(kv_shape)) or k_new.shape[0] != batch or k_new.shape[-1] != d_k:
        raise ValueError(f"k_new shape {k_new.shape} does not match cache {k_cache.shape}")
    if v_new.shape != k_new.shape:
        raise ValueError(f"v_new shape {v_new.shape} != k_new shape {k_new.shape}")
    n_head = 0
    if q_dev is not None:
        if q_dev.shape[0] != batch or q_dev.shape[-1] != d_k:
            raise ValueError(f"q shape {q_dev.shape} does not match cache {k_cache.shape}")
        n_head = int(np.prod(q_dev.shape)) // (batch * n_new * d_k)
        if n_head * batch * n_new * d_k != int(np.prod(q_dev.shape)) or n_head % n_kv:
            raise ValueError(f"q shape {q_dev.shape} is not (batch, n_new, n_head, d_k)")
    _check_lens(cache_lens, batch)
    tensors = [k_new, v_new, k_cache, v_cache] + ([q_dev] if q_dev is not None else [])
    code = same_dtype(*tensors)
    rope_rows = 0
    if (cos_dev is None) != (sin_dev is None):
        raise ValueError("cos_dev and sin_dev must both be given or both be None")
    if cos_dev is not None:
        if cos_dev.shape != sin_dev.shape or len(cos_dev.shape) != 2 or cos_dev.shape[1] != d_k // 2:
            raise ValueError(f"cos/sin tables must be (rows, {d_k // 2}), got {cos_dev.shape}")
        rope_rows = cos_dev.shape[0]
    kv_str = _lib.strides(n_new * n_kv * d_k, n_kv * d_k, d_k)
    q_str = _lib.strides(n_new * n_head * d_k, n_head * d_k, d_k)
    c_str = _lib.strides(n_kv * max_ctx * d_k, max_ctx * d_k, d_k)
    launch(gpu.runtime().tl_rope_kv_append, vp(q_dev), vp(k_new), vp(v_new), vp(k_cache), vp(v_cache), vp(cache_lens),
        vp(cos_dev), vp(sin_dev), rope_rows, batch, n_new, n_head, n_kv, max_ctx, d_k,
        q_str, kv_str, kv_str, c_str, c_str, code, None,
        what="rope_kv_append")
    return q_dev


def decode_workspace_bytes(batch: int, n_head: int, n_kv_head: int, max_ctx: int, d_k: int,
                           split: int = 0) -> tuple[int, int]:
    """(bytes, split) of the split-K workspace for these dims."""
    lib = gpu.runtime()
    if split == 0:
        split = lib.tl_decode_split_size(batch, n_kv_head, max_ctx)
    return lib.tl_attention_decode_workspace_bytes(batch, n_head, max_ctx, d_k, split), split


def decode_workspace(batch: int, n_head: int, n_kv_head: int, max_ctx: int, d_k: int,
                     split: int = 0):
    """A split-K workspace for these dims, reusable by consecutive calls on
    the library stream (calls that overlap in time need one each)."""
    nbytes, _ = decode_workspace_bytes(batch, n_head, n_kv_head, max_ctx, d_k, split)
    return gpu.allocate((max(nbytes, 1),), np.uint8)


def attention_decode(q_dev, k_cache, v_cache, cache_lens, n_head: int, n_kv_head: int,
                     sm_scale: float | None = None, len_add: int = 0, out=None,
                     workspace=None, split: int = 0):
    """One query token per sequence over the cache: returns ``(batch, n_head, d_k)``.

    Sequence b attends to positions ``[0, cache_lens[b] + len_add)`` (clamped to
    max_ctx); query head h reads KV head ``h // (n_head // n_kv_head)``.
    """
    batch, n_kv, max_ctx, d_k = _check_cache(k_cache, v_cache)
    if n_kv != n_kv_head:
        raise ValueError(f"cache has {n_kv} KV heads, n_kv_head={n_kv_head}")
    if n_head <= 0 or n_head % n_kv_head:
        raise ValueError(f"n_head ({n_head}) must be a positive multiple of n_kv_head ({n_kv_head})")
    if int(np.prod(q_dev.shape)) != batch * n_head * d_k:
        raise ValueError(f"q shape {q_dev.shape} is not (batch={batch}, n_head={n_head}, d_k={d_k})")
    if d_k not in (64, 128):
        raise ValueError(f"decode supports d_k in (64, 128), got {d_k}")
    _check_lens(cache_lens, batch)
    code = same_dtype(q_dev, k_cache, v_cache)
    if sm_scale is None:
        sm_scale = default_scale(d_k)
    if out is None:
        out = gpu.allocate((batch, n_head, d_k), q_dev.dtype)
    elif int(np.prod(out.shape)) != batch * n_head * d_k or gpu.dtype_name(out.dtype) != gpu.dtype_name(q_dev.dtype):
        raise ValueError(f"out must hold (batch, n_head, d_k) of the input dtype, got {out.shape}")
    ws_bytes, split = decode_workspace_bytes(batch, n_head, n_kv_head, max_ctx, d_k, split)
    ws = scratch(ws_bytes, workspace, key="decode")
    qo = _lib.strides(n_head * d_k, d_k)
    c_str = _lib.strides(n_kv * max_ctx * d_k, max_ctx * d_k, d_k)
    launch(gpu.runtime().tl_attention_decode, vp(q_dev), vp(k_cache), vp(v_cache), vp(cache_lens), int(len_add), vp(out), vp(ws),
        ws.nbytes if ws is not None else 0,
        batch, n_head, n_kv_head, max_ctx, d_k, qo, c_str, c_str, qo,
        float(sm_scale), split, code, None,
        what="attention_decode")
    return out


def decode_step(q_dev, k_new, v_new, k_cache, v_cache, cache_lens, n_head: int, n_kv_head: int,
                cos_dev=None, sin_dev=None, sm_scale: float | None = None, out=None,
                workspace=None, split: int = 0):
    """RoPE + append of the new token, then attention over ``cache_lens[b] + 1`` positions.

    The same results as ``rope_kv_append`` followed by ``attention_decode``
    with ``len_add=1`` (q rotated in place, cache row ``cache_lens[b]``
    written, the output returned), in one library call
    (``tl_attention_decode_append``): with a small cache the workgroups that
    stream each (sequence, KV head) write its token first, so the step is a
    single launch.  q_dev: ``(batch, n_head, d_k)``; k_new / v_new:
    ``(batch, n_kv_head, d_k)``.
    """
    batch, n_kv, max_ctx, d_k = _check_cache(k_cache, v_cache)
    if n_kv != n_kv_head:
        raise ValueError(f"cache has {n_kv} KV heads, n_kv_head={n_kv_head}")
    if n_head <= 0 or n_head % n_kv_head:
        raise ValueError(f"n_head ({n_head}) must be a positive multiple of n_kv_head ({n_kv_head})")
    if int(np.prod(q_dev.shape)) != batch * n_head * d_k or q_dev.shape[0] != batch or q_dev.shape[-1] != d_k:
        raise ValueError(f"q shape {q_dev.shape} is not (batch={batch}, n_head={n_head}, d_k={d_k})")
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if int(np.prod(t.shape)) != batch * n_kv * d_k or t.shape[0] != batch or t.shape[-1] != d_k:
            raise ValueError(f"{name} shape {t.shape} is not (batch={batch}, n_kv_head={n_kv}, d_k={d_k})")
    if d_k not in (64, 128):
        raise ValueError(f"decode supports d_k in (64, 128), got {d_k}")
    _check_lens(cache_lens, batch)
    code = same_dtype(q_dev, k_new, v_new, k_cache, v_cache)
    rope_rows = 0
    if (cos_dev is None) != (sin_dev is None):
        raise ValueError("cos_dev and sin_dev must both be given or both be None")
    if cos_dev is not None:
        if cos_dev.shape != sin_dev.shape or len(cos_dev.shape) != 2 or cos_dev.shape[1] != d_k // 2:
            raise ValueError(f"cos/sin tables must be (rows, {d_k // 2}), got {cos_dev.shape}")
        rope_rows = cos_dev.shape[0]
    if sm_scale is None:
        sm_scale = default_scale(d_k)
    if out is None:
        out = gpu.allocate((batch, n_head, d_k), q_dev.dtype)
    elif int(np.prod(out.shape)) != batch * n_head * d_k or gpu.dtype_name(out.dtype) != gpu.dtype_name(q_dev.dtype):
        raise ValueError(f"out must hold (batch, n_head, d_k) of the input dtype, got {out.shape}")
    ws_bytes, split = decode_workspace_bytes(batch, n_head, n_kv_head, max_ctx, d_k, split)
    ws = scratch(ws_bytes, workspace, key="decode")
    qo = _lib.strides(n_head * d_k, d_k)
    kv = _lib.strides(n_kv * d_k, d_k)
    c_str = _lib.strides(n_kv * max_ctx * d_k, max_ctx * d_k, d_k)
    launch(gpu.runtime().tl_attention_decode_append, vp(q_dev), vp(k_new), vp(v_new), vp(k_cache), vp(v_cache),
           vp(cache_lens), vp(cos_dev), vp(sin_dev), rope_rows, vp(out), vp(ws),
           ws.nbytes if ws is not None else 0,
           batch, n_head, n_kv_head, max_ctx, d_k, qo, kv, kv, c_str, c_str, qo,
           float(sm_scale), split, code, None,
           what="decode_step")
    return out
