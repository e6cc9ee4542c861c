"""Restatement of next-token sampling (test infrastructure only).

* :func:`sample_ref` -- SmolLM2._sample (smollm2_triton/model.py:566-584;
  GPT-2's copy is gpt2_triton/model.py:424-438): greedy ``np.argmax`` for
  ``temperature <= 1e-6``; otherwise fp32 ``exp(x / T - max(x / T))``
  promoted to fp64 and normalised, top-k filter through ``np.argpartition``
  (``top_k`` capped at the vocabulary) and renormalised, and
  ``np.random.choice(V, p=p)``.  The draw is made explicit: NumPy's legacy
  ``choice`` with ``p`` takes ``u = random_sample()`` and returns
  ``searchsorted(cdf / cdf[-1], u, side="right")``, so ``sample_ref(...,
  u)`` is the reference's token for that ``u``.
* :func:`kept_mask` -- the entries the device kernel keeps for a top_k
  filter: every logit at or above the k-th largest (ties with the k-th all
  kept; ``argpartition`` keeps exactly k of them, which ones being
  unspecified).
* :func:`sample_kept_ref` -- the inverse CDF over :func:`kept_mask`'s
  entries: the device's tie rule; equal to :func:`sample_ref` whenever no
  logit ties the k-th (pinned in tests/test_oracle.py).
* :func:`crossing_margin` -- how far ``u`` is from the nearest CDF step, so
  tests can tell a real mismatch from a draw that sits on a boundary within
  fp32 ``exp`` rounding.

Pinned in tests/test_oracle.py against the library routines it restates:
``np.random.choice`` with the same seed (both filtered and unfiltered),
``np.argmax`` (first maximum, NaN first), and the empirical distribution of
many draws against the normalised probabilities.
"""

from __future__ import annotations

import numpy as np


def probs_ref(logits, temperature: float, top_k: int) -> np.ndarray:
    """The reference's final probability vector (fp64, sums to 1)."""
    logits = np.asarray(logits, dtype=np.float32)
    scaled = logits / temperature  # fp32: the Python float is weak (NEP 50)
    logits_stable = scaled - np.max(scaled)
    probs = np.exp(logits_stable).astype(np.float64)
    probs = probs / np.sum(probs)
    if top_k > 0:
        top_k = min(top_k, len(probs))
        indices = np.argpartition(probs, -top_k)[-top_k:]
        filtered = np.zeros_like(probs)
        filtered[indices] = probs[indices]
        filtered /= filtered.sum()
        probs = filtered
    return probs


def sample_ref(logits, temperature: float, top_k: int, u: float) -> int:
    """Token the reference picks for the uniform draw ``u`` in [0, 1)."""
    logits = np.asarray(logits, dtype=np.float32)
    if temperature > 1e-6:
        p = probs_ref(logits, temperature, top_k)
        cdf = p.cumsum()
        cdf /= cdf[-1]
        return int(cdf.searchsorted(u, side="right"))
    return int(np.argmax(logits))


def kept_mask(logits, top_k: int) -> np.ndarray:
    """Entries kept by the device's top_k filter (all logits >= the k-th)."""
    x = np.asarray(logits, dtype=np.float32)
    if top_k <= 0 or top_k >= x.size:
        return np.ones(x.shape, bool)
    kth = np.sort(x)[::-1][top_k - 1]
    return x >= kth


def sample_kept_ref(logits, temperature: float, top_k: int, u: float) -> int:
    """Token for draw ``u`` when every logit >= the k-th largest is kept."""
    x = np.asarray(logits, dtype=np.float32)
    if not temperature > 1e-6:
        return int(np.argmax(x))
    cdf = kept_probs(x, temperature, top_k).cumsum()
    cdf /= cdf[-1]
    return int(cdf.searchsorted(u, side="right"))


def kept_probs(logits, temperature: float, top_k: int) -> np.ndarray:
    """Normalised probabilities over :func:`kept_mask`'s entries."""
    x = np.asarray(logits, dtype=np.float32)
    scaled = x / temperature
    p = np.exp(scaled - np.max(scaled)).astype(np.float64) * kept_mask(x, top_k)
    return p / p.sum()


def crossing_margin(logits, temperature: float, top_k: int, u: float, keep_ties: bool = False) -> float:
    """Distance from ``u`` to the nearest step of the CDF (the reference's,
    or with ``keep_ties`` the device rule's)."""
    p = kept_probs(logits, temperature, top_k) if keep_ties else probs_ref(logits, temperature, top_k)
    cdf = p.cumsum()
    cdf /= cdf[-1]
    return float(np.min(np.abs(cdf - u)))
