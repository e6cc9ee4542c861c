"""Restatements of the model step's non-attention layers (test infrastructure only).

* :func:`rms_norm_ref` -- triton_llm/kernels/rms_norm.py:40-56:
  ``rms = sqrt(sum(x^2) / N + eps)``, ``y = (x / rms) * w`` per row.
* :func:`swiglu_ref`   -- triton_llm/kernels/swiglu.py:38-57: ``silu(g) * u``
  with ``sigmoid = 1/(1+e)`` for ``g >= 0`` and ``e/(1+e)`` otherwise,
  ``e = exp(-|g|)``.
* :func:`add_ref`      -- triton_llm/kernels/add.py:41-51.
* :func:`decoder_layer_ref` -- one SmolLM2 / Llama decoder layer
  (smollm2_triton/model.py:276-365): RMSNorm, q/k/v projections, RoPE,
  cache write, GQA attention (causal for a prompt into an empty cache,
  over the cache prefix for one decoded token), o projection, residual,
  RMSNorm, gate/up, SwiGLU, down, residual.

All in float64 and rounded once to float32, except where the kernel's
rounding point matters (noted).  Pinned in tests/test_oracle.py by
invariants: RMSNorm of a row is unchanged by scaling the row (eps aside)
and has unit RMS before the weight; SwiGLU is 0 at g = 0, tends to u * g
for large g and to 0 for very negative g; the decoder layer with zero
weights returns its input; and the reference's cached == full-recompute
invariant (tests/test_smollm2_model.py:95-165): a whole S-token prompt gives,
row for row, what an (S-k)-token prefill followed by k one-token decode steps
gives, for one layer and for a two-layer stack's logits.  Mistakes planted in
the RoPE positions, the cache write or the causal flag break that invariant
(tested).
"""

from __future__ import annotations

import numpy as np

from oracle import attention as oa
from oracle import rope as orope


def rms_norm_ref(x, w, eps: float = 1e-5) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    rms = np.sqrt(np.sum(x * x, axis=-1, keepdims=True) / x.shape[-1] + eps)
    return ((x / rms) * np.asarray(w, dtype=np.float64)).astype(np.float32)


def silu_ref(g) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    e = np.exp(-np.abs(g))
    return g * np.where(g >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def swiglu_ref(g, u) -> np.ndarray:
    return (silu_ref(g) * np.asarray(u, dtype=np.float64)).astype(np.float32)


def add_ref(x, y) -> np.ndarray:
    return (np.asarray(x, dtype=np.float64) + np.asarray(y, dtype=np.float64)).astype(np.float32)


def positions(prev: int, seq: int) -> np.ndarray:
    """RoPE positions of a step's new tokens: the model applies RoPE with
    position_offset = prev_seq (smollm2_triton/model.py:296-297, :332-333)."""
    return np.arange(prev, prev + seq)


def write_cache(cache, k, v, prev: int) -> None:
    """k, v (seq, n_kv, D) into the (n_kv, max_seq, D) caches at rows
    [prev, prev + seq) (smollm2_triton/model.py:301-302, :338-339)."""
    seq = k.shape[0]
    cache["k"][:, prev:prev + seq] = k.transpose(1, 0, 2)
    cache["v"][:, prev:prev + seq] = v.transpose(1, 0, 2)


def causal_flag(prev: int) -> bool:
    """A prompt into an empty cache is causal (model.py:341-343); a decoded
    token attends to the whole prefix with causal=False (model.py:310-314)."""
    return prev == 0


def decoder_layer_ref(h, w, cache, prev: int, cos, sin, n_head: int, n_kv: int, eps: float = 1e-5):
    """h (seq, E) float32; w: dict of float32 arrays ln1 (E,), q (E, H*D),
    k (E, Hkv*D), v (E, Hkv*D), o (H*D, E), ln2 (E,), gate (E, I), up (E, I),
    down (I, E); cache: dict k/v (Hkv, max_seq, D) float32, updated in place at
    [prev, prev + seq).  Returns the layer output (seq, E) float32."""
    seq, E = h.shape
    D = w["q"].shape[1] // n_head
    x = rms_norm_ref(h, w["ln1"], eps)
    q = (x.astype(np.float64) @ w["q"]).astype(np.float32).reshape(seq, n_head, D)
    k = (x.astype(np.float64) @ w["k"]).astype(np.float32).reshape(seq, n_kv, D)
    v = (x.astype(np.float64) @ w["v"]).astype(np.float32).reshape(seq, n_kv, D)
    pos = positions(prev, seq)
    q = orope.rotate(q, cos[pos][:, None], sin[pos][:, None])
    k = orope.rotate(k, cos[pos][:, None], sin[pos][:, None])
    write_cache(cache, k, v, prev)
    kf = cache["k"][:, :prev + seq].reshape(-1, D)
    vf = cache["v"][:, :prev + seq].reshape(-1, D)
    att = oa.attention_gqa_ref(q.transpose(1, 0, 2).reshape(-1, D), kf, vf, n_head, n_kv,
                               causal=causal_flag(prev))
    att = att.reshape(n_head, seq, D).transpose(1, 0, 2).reshape(seq, n_head * D)
    h1 = add_ref((att.astype(np.float64) @ w["o"]).astype(np.float32), h)
    x2 = rms_norm_ref(h1, w["ln2"], eps)
    g = (x2.astype(np.float64) @ w["gate"]).astype(np.float32)
    u = (x2.astype(np.float64) @ w["up"]).astype(np.float32)
    a = swiglu_ref(g, u)
    return add_ref((a.astype(np.float64) @ w["down"]).astype(np.float32), h1)
