"""GPU-resident KV cache and the attention sub-block of the cached forward pass.

Reference behaviour replaced:

* ``_init_cache_gpu`` (smollm2_triton/model.py:190-225) keeps each layer's
  cache as host NumPy arrays ``(n_kv_head, max_seq, d_k)``;
* per layer, ``_forward_cached`` (model.py:286-347) rotates q/k with
  ``apply_rope``, then for decode copies k/v to the host, writes the cache
  row, re-uploads the whole valid prefix and calls ``attention_gqa``; for
  prefill it copies q/k/v to the host to transpose them head-major, uploads
  them, copies k/v back into the host cache, and transposes the output back
  through the host.

Here the cache stays on the GPU in the decode kernels' layout
``(1, n_kv_head, max_seq, d_k)`` and one call runs the whole sub-block on the
projection outputs in place:

* decode (``seq == 1``): ``tl_rope_kv_append`` (RoPE of q and k at position
  ``cache_len``, k/v written into the cache) and ``tl_attention_decode`` over
  ``cache_len + 1`` positions -- no host copies;
* prefill (``seq > 1`` into an empty cache): the same append for all ``seq``
  rows, then ``tl_attention_fwd`` reading q as ``(seq, n_head, d_k)`` rows
  and K/V straight from the cache, writing the output in the
  ``(seq, n_head * d_k)`` layout the output projection consumes -- no host
  transposes.

The validation and its messages follow model.py:197-214 and :256-268.
"""

from __future__ import annotations

import ctypes

import numpy as np

from triton_llm import gpu
from triton_llm.kernels.decode import allocate_kv_cache, decode_step, decode_workspace, rope_kv_append
from triton_llm.kernels.flash import flash_attention_strided, flash_workspace_bytes

__all__ = ["GpuKVCache", "check_step"]


def check_step(prev_seq: int, seq: int, max_seq: int) -> int:
    """The checks of a cached forward step (model.py:256-268); returns the
    cache length after the step."""
    if prev_seq > 0 and seq > 1:
        raise ValueError(f"Decode mode requires seq=1, got seq={seq}. ")
    total_after = prev_seq + seq
    if total_after > max_seq:
        raise ValueError(
            f"Total sequence length {total_after} exceeds "
            f"pre-allocated cache size ({max_seq})"
        )
    return total_after


class GpuKVCache:
    """Per-layer K/V caches on the GPU plus the cached attention sub-block.

    ``kv_cache_dev[i]`` is ``{"k": DeviceTensor, "v": DeviceTensor}``, each
    ``(1, n_kv_head, max_seq, d_k)``, zero-filled like the reference's
    ``np.zeros``.  ``cache_len`` counts the cached tokens (the reference's
    ``_cache_len``); :meth:`advance` moves it after all layers of a step ran,
    as model.py:353 does.
    """

    def __init__(self, n_layer: int, n_head: int, n_kv_head: int, d_k: int,
                 max_seq: int | None = None, max_position_embeddings: int | None = None,
                 dtype=np.float32):
        if max_seq is None:
            if max_position_embeddings is None:
                raise ValueError("give max_seq or max_position_embeddings")
            max_seq = max_position_embeddings
        elif max_seq <= 0:
            raise ValueError(f"max_seq must be a positive integer, got {max_seq}")
        elif max_position_embeddings is not None and max_seq > max_position_embeddings:
            raise ValueError(
                f"max_seq ({max_seq}) cannot exceed model's "
                f"max_position_embeddings ({max_position_embeddings})"
            )
        if n_layer <= 0 or n_kv_head <= 0 or n_head <= 0 or n_head % n_kv_head:
            raise ValueError(f"bad head counts: n_layer={n_layer} n_head={n_head} n_kv_head={n_kv_head}")
        self.n_layer, self.n_head, self.n_kv_head, self.d_k = n_layer, n_head, n_kv_head, d_k
        self.max_seq = int(max_seq)
        self.dtype = dtype
        self.kv_cache_dev = []
        for _ in range(n_layer):
            k, v = allocate_kv_cache(1, n_kv_head, self.max_seq, d_k, dtype=dtype)
            self.kv_cache_dev.append({"k": k, "v": v})
        self._cache_len = 0
        self._lens = gpu.zeros((1,), np.int32)  # cache_len on the device, read by the kernels
        # 0 .. max_seq on the device: advance() and reset() copy the new length
        # from here (a stream-ordered device copy, no host synchronisation)
        self._len_table = gpu.to_device(np.arange(self.max_seq + 1, dtype=np.int32))
        self._decode_ws = decode_workspace(1, n_head, n_kv_head, self.max_seq, d_k)
        # room to split a full-length prompt's costliest tiles (shorter
        # prompts split as far as it allows)
        wsb = flash_workspace_bytes(1, n_kv_head, self.max_seq, d_k, dtype, n_head=n_head,
                                    seq_q=self.max_seq)
        self._prefill_ws = gpu.allocate((wsb,), np.uint8) if wsb else None

    @property
    def cache_len(self) -> int:
        return self._cache_len

    def _set_lens(self, n: int):
        src = ctypes.c_void_p(self._len_table.ptr.value + 4 * n)
        gpu.check_error(gpu.runtime().tl_memcpy_dtod(self._lens.ptr, src, 4))

    def reset(self):
        """Forget the cached tokens (the cache rows are overwritten as it refills)."""
        self._cache_len = 0
        self._set_lens(0)

    def advance(self, seq: int):
        """Count ``seq`` more cached tokens (after every layer of the step).
        Stream-ordered: no host synchronisation."""
        self._cache_len = check_step(self._cache_len, seq, self.max_seq)
        self._set_lens(self._cache_len)

    def attention(self, layer: int, q_dev, k_dev, v_dev, cos_dev=None, sin_dev=None,
                  sm_scale: float | None = None):
        """Attention sub-block of one layer for the step's ``seq`` new tokens.

        q_dev ``(seq, n_head * d_k)``, k_dev / v_dev ``(seq, n_kv_head * d_k)``:
        the projection outputs, in the cache's dtype.  q_dev is rotated in
        place.  cos/sin: RoPE tables ``(rows, d_k // 2)`` float32, or None (no
        RoPE).  Returns the attention output ``(seq, n_head * d_k)``.
        """
        H, Hkv, D = self.n_head, self.n_kv_head, self.d_k
        if not 0 <= layer < self.n_layer:
            raise ValueError(f"layer {layer} out of range [0, {self.n_layer})")
        if len(q_dev.shape) != 2 or q_dev.shape[1] != H * D:
            raise ValueError(f"q must be (seq, {H * D}), got {q_dev.shape}")
        seq = q_dev.shape[0]
        for name, t in (("k", k_dev), ("v", v_dev)):
            if tuple(t.shape) != (seq, Hkv * D):
                raise ValueError(f"{name} must be ({seq}, {Hkv * D}), got {t.shape}")
        prev = self._cache_len
        total_after = check_step(prev, seq, self.max_seq)
        if cos_dev is not None and seq and prev + seq > cos_dev.shape[0]:
            # apply_rope's check (rope.py:194-198): the kernel would skip rows
            # past the table, leaving q unrotated and the cache row unwritten.
            raise ValueError(
                f"position_offset ({prev}) + seq_len ({seq}) "
                f"exceeds cos/sin table size ({cos_dev.shape[0]})"
            )
        cache = self.kv_cache_dev[layer]
        out = gpu.allocate((seq, H * D), q_dev.dtype)
        if seq == 0:
            return out
        if seq == 1 and prev > 0:
            decode_step(gpu.view(q_dev, (1, H, D)), gpu.view(k_dev, (1, Hkv, D)), gpu.view(v_dev, (1, Hkv, D)),
                        cache["k"], cache["v"], self._lens, H, Hkv, cos_dev, sin_dev,
                        sm_scale=sm_scale, out=out, workspace=self._decode_ws)
            return out
        # Prefill into an empty cache (prev == 0; a single token is a prefill too).
        q4 = gpu.view(q_dev, (1, seq, H, D))
        rope_kv_append(q4, gpu.view(k_dev, (1, seq, Hkv, D)), gpu.view(v_dev, (1, seq, Hkv, D)),
                       cache["k"], cache["v"], self._lens, cos_dev, sin_dev)
        c_str = (Hkv * self.max_seq * D, self.max_seq * D, D)
        qo_str = (seq * H * D, D, H * D)  # (b, head, row) strides of (seq, H, D) rows
        flash_attention_strided(q_dev, cache["k"], cache["v"], out, batch=1, n_head=H, n_kv_head=Hkv,
                                seq_q=seq, seq_k=total_after, d_k=D, q_strides=qo_str,
                                k_strides=c_str, v_strides=c_str, o_strides=qo_str, causal=True,
                                sm_scale=sm_scale, workspace=self._prefill_ws)
        return out
