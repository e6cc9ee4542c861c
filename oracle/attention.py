"""Attention restatements (test infrastructure only).

* :func:`attention_ref`      -- triton_llm/kernels/attention.py:141-216
  (one head; scale 1/sqrt(d) applied to q before the dot, :71; top-left
  causal j <= i, :85-100; non-causal masks nothing, :101-113).
* :func:`attention_gqa_ref`  -- triton_llm/kernels/attention_gqa.py:149-269
  (rows grouped by head; kv = h // group, :76; q * sm_scale, :83;
  bottom-right causal j <= seq_k - seq_q + i, :97; zeros when seq_k = 0 as
  tests/test_attention_gqa.py:297 requires).
* :func:`attention_bhsd`     -- the same math batched over (b, KV group) and
  blockwise over query tiles so long sequences fit in memory; this is also
  the CPU baseline's computation.
* :func:`decode_ref`         -- one query token per sequence against a cache
  prefix, the reference's decode call attention_gqa(q, K[:L], V[:L],
  causal=False) (smollm2_triton/model.py:305-314).
* :func:`kv_append_ref`      -- RoPE on q / k_new at position len and the
  cache write at [:, len] (smollm2_triton/model.py:296-302, :336-339).

Fully masked query rows (possible only when seq_q > seq_k under causal
masking) give NaN, as the reference kernel's 0/0 does.
"""

from __future__ import annotations

import numpy as np

from .numerics import from_storage
from .rope import rotate


def _softmax_rows(scores):
    with np.errstate(invalid="ignore"):
        m = scores.max(axis=-1, keepdims=True)
        e = np.exp(scores - m)
        return e / e.sum(axis=-1, keepdims=True)


def attention_ref(q, k, v, causal: bool = True, compute_dtype=np.float32):
    """attention.py:141 -- q (seq_q, d), k/v (seq_k, d) -> (seq_q, d) float32."""
    q = np.asarray(q, dtype=compute_dtype)
    k = np.asarray(k, dtype=compute_dtype)
    v = np.asarray(v, dtype=compute_dtype)
    seq_q, d = q.shape
    seq_k = k.shape[0]
    if seq_q == 0 or seq_k == 0:
        return np.empty((seq_q, d), dtype=np.float32)
    if causal and seq_q != seq_k:
        raise ValueError("causal requires seq_q == seq_k")
    scale = compute_dtype(1.0) / np.sqrt(compute_dtype(d))
    s = (q * scale) @ k.T
    if causal:
        s = np.where(np.tril(np.ones((seq_q, seq_k), dtype=bool)), s, -np.inf)
    return (_softmax_rows(s) @ v).astype(np.float32)


def _bottom_right_mask(seq_q: int, seq_k: int, q0: int = 0, q1: int | None = None):
    q1 = seq_q if q1 is None else q1
    qi = np.arange(q0, q1)[:, None]
    kj = np.arange(seq_k)[None, :]
    return kj <= qi + (seq_k - seq_q)


def attention_gqa_ref(q_flat, k_flat, v_flat, n_head: int, n_kv_head: int,
                      causal: bool = True, sm_scale: float | None = None,
                      compute_dtype=np.float32):
    """attention_gqa.py:149 -- flat head-grouped rows in, (n_head*seq_q, d) out."""
    q_flat = np.asarray(q_flat, dtype=compute_dtype)
    k_flat = np.asarray(k_flat, dtype=compute_dtype)
    v_flat = np.asarray(v_flat, dtype=compute_dtype)
    d = q_flat.shape[1]
    seq_q = q_flat.shape[0] // n_head
    seq_k = k_flat.shape[0] // n_kv_head
    if seq_q == 0:
        return np.empty((0, d), dtype=np.float32)
    if seq_k == 0:
        return np.zeros((n_head * seq_q, d), dtype=np.float32)
    group = n_head // n_kv_head
    scale = compute_dtype(1.0 / np.sqrt(d) if sm_scale is None else sm_scale)
    q3 = q_flat.reshape(n_head, seq_q, d)
    k3 = k_flat.reshape(n_kv_head, seq_k, d)
    v3 = v_flat.reshape(n_kv_head, seq_k, d)
    mask = _bottom_right_mask(seq_q, seq_k) if causal else None
    out = np.empty((n_head, seq_q, d), dtype=np.float32)
    for h in range(n_head):
        kv = h // group
        s = (q3[h] * scale) @ k3[kv].T
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        out[h] = _softmax_rows(s) @ v3[kv]
    return out.reshape(n_head * seq_q, d)


def attention_bhsd(q, k, v, causal: bool = True, sm_scale: float | None = None,
                   block_q: int = 512, rows=None, compute_dtype=np.float32,
                   dtype: str = "float32"):
    """Batched GQA attention, q (B, Hq, Sq, D), k/v (B, Hkv, Sk, D) -> (B, Hq, Sq, D).

    Work is done per (b, KV head) with the group's query heads stacked into one
    matmul, blockwise over ``block_q`` query rows (memory O(block_q * Sk)).
    ``rows``: optional sorted array of query indices to evaluate (others are
    left as NaN) -- used to check long sequences on a sample of rows.
    ``dtype``: storage type of q/k/v (bfloat16 arrays hold uint16 bits).
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    B, Hq, Sq, D = q.shape
    _, Hkv, Sk, _ = k.shape
    group = Hq // Hkv
    scale = compute_dtype(1.0 / np.sqrt(D) if sm_scale is None else sm_scale)
    out = np.full((B, Hq, Sq, D), np.nan, dtype=np.float32)
    row_sets = [np.asarray(rows)] if rows is not None else [
        np.arange(i, min(Sq, i + block_q)) for i in range(0, Sq, block_q)
    ]
    off = Sk - Sq
    for b in range(B):
        for hk in range(Hkv):
            kk = from_storage(k[b, hk], dtype).astype(compute_dtype, copy=False)
            vv = from_storage(v[b, hk], dtype).astype(compute_dtype, copy=False)
            for r in row_sets:
                if len(r) == 0:
                    continue
                kmax = Sk if not causal else int(min(Sk, max(0, r.max() + off + 1)))
                if kmax == 0:
                    continue
                qq = from_storage(q[b, hk * group:(hk + 1) * group][:, r], dtype).astype(compute_dtype, copy=False)
                s = (qq * scale) @ kk[:kmax].T  # (group, len(r), kmax)
                if causal:
                    m = np.arange(kmax)[None, :] <= (r[:, None] + off)
                    s = np.where(m[None], s, -np.inf)
                out[b, hk * group:(hk + 1) * group][:, r] = _softmax_rows(s) @ vv[:kmax]
    return out


def decode_ref(q, k_cache, v_cache, ctx_lens, sm_scale: float | None = None,
               compute_dtype=np.float32, batches=None, dtype: str = "float32"):
    """q (B, Hq, D), caches (B, Hkv, max_ctx, D), ctx_lens (B,) -> (B, Hq, D).

    Sequence b attends to cache positions [0, ctx_lens[b]); zeros if empty.
    ``batches``: optional subset of sequence indices to evaluate.
    ``dtype``: storage type of the inputs (bfloat16 arrays hold uint16 bits).
    """
    q = np.asarray(q)
    B, Hq, D = q.shape
    Hkv = k_cache.shape[1]
    group = Hq // Hkv
    scale = compute_dtype(1.0 / np.sqrt(D) if sm_scale is None else sm_scale)
    out = np.full((B, Hq, D), np.nan, dtype=np.float32)
    for b in (range(B) if batches is None else batches):
        L = int(ctx_lens[b])
        if L <= 0:
            out[b] = 0.0
            continue
        for hk in range(Hkv):
            kk = from_storage(k_cache[b, hk, :L], dtype).astype(compute_dtype, copy=False)
            vv = from_storage(v_cache[b, hk, :L], dtype).astype(compute_dtype, copy=False)
            qq = from_storage(q[b, hk * group:(hk + 1) * group], dtype).astype(compute_dtype, copy=False)
            s = (qq * scale) @ kk.T
            out[b, hk * group:(hk + 1) * group] = _softmax_rows(s) @ vv
    return out


def kv_append_ref(q, k_new, v_new, k_cache, v_cache, cache_lens, cos=None, sin=None,
                  round_fn=None):
    """Float-valued restatement of RoPE + append for one new token per sequence.

    q (B, Hq, D), k_new/v_new (B, Hkv, D) float32 values; caches
    (B, Hkv, max_ctx, D) float32 values (copied, not modified).  Returns
    (q_rot, k_cache', v_cache').  ``round_fn`` rounds rotated values to the
    storage type (identity for float32).
    """
    round_fn = round_fn or (lambda x: x)
    q = np.array(q, dtype=np.float32)
    kc = np.array(k_cache, dtype=np.float32)
    vc = np.array(v_cache, dtype=np.float32)
    B = q.shape[0]
    for b in range(B):
        pos = int(cache_lens[b])
        kb = np.asarray(k_new[b], dtype=np.float32)
        if cos is not None:
            q[b] = round_fn(rotate(q[b], cos[pos], sin[pos]))
            kb = round_fn(rotate(kb, cos[pos], sin[pos]))
        kc[b, :, pos] = kb
        vc[b, :, pos] = np.asarray(v_new[b], dtype=np.float32)
    return q, kc, vc
