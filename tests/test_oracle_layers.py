"""The decoder-layer oracle against the reference model's cached == full
recompute invariant (CPU).

tests/test_smollm2_model.py:95-165 of the reference checks that a full
forward and a cached prefill give the same logits, and that one decoded
token's logits equal the full forward's last row.  Here the same invariant
pins oracle/layers.py decoder_layer_ref: an S-token prompt through a fresh
cache equals, row for row, an (S - k)-token prefill followed by k one-token
decode steps -- for one layer and for a two-layer stack's final logits
(final RMSNorm + lm_head).  Then each plausible mistake is planted in the
oracle (wrong RoPE positions, a transposed cache write, the wrong causal
flag) and the invariant must catch it.
"""

import numpy as np
import pytest

from oracle import attention as oa
from oracle import layers as ol
from oracle import rope as orope
from oracle.gemm import gemm_ref

E, HQ, HKV, D, I, MAX_SEQ = 64, 4, 2, 16, 128, 32


def _weights(rng, n_layer):
    mk = lambda *s, scale=1.0: (scale * rng.standard_normal(s)).astype(np.float32)  # noqa: E731
    return [{"ln1": 1.0 + mk(E, scale=0.1), "ln2": 1.0 + mk(E, scale=0.1),
             "q": mk(E, HQ * D, scale=E ** -0.5), "k": mk(E, HKV * D, scale=E ** -0.5),
             "v": mk(E, HKV * D, scale=E ** -0.5), "o": mk(HQ * D, E, scale=(HQ * D) ** -0.5),
             "gate": mk(E, I, scale=E ** -0.5), "up": mk(E, I, scale=E ** -0.5),
             "down": mk(I, E, scale=I ** -0.5)} for _ in range(n_layer)]


def _cache():
    return {"k": np.zeros((HKV, MAX_SEQ, D), np.float32), "v": np.zeros((HKV, MAX_SEQ, D), np.float32)}


def _stack(h, layers, caches, prev, cos, sin, head=None):
    for w, c in zip(layers, caches):
        h = ol.decoder_layer_ref(h, w, c, prev, cos, sin, HQ, HKV)
    if head is None:
        return h
    ln_f, lm = head
    return gemm_ref(ol.rms_norm_ref(h, ln_f), lm)


def _full_vs_cached(n_layer, S, k, seed=0, head=False):
    """max |full - cached| over all S rows of the stack's output."""
    rng = np.random.default_rng(seed)
    layers = _weights(rng, n_layer)
    cos, sin = orope.precompute_cos_sin(MAX_SEQ, D, 1e4)
    h = rng.standard_normal((S, E)).astype(np.float32)
    hd = None
    if head:
        hd = (1.0 + 0.1 * rng.standard_normal(E).astype(np.float32),
              (E ** -0.5 * rng.standard_normal((E, 97))).astype(np.float32))
    full = _stack(h, layers, [_cache() for _ in layers], 0, cos, sin, hd)
    caches = [_cache() for _ in layers]
    rows = [_stack(h[:S - k], layers, caches, 0, cos, sin, hd)]
    for t in range(S - k, S):
        rows.append(_stack(h[t:t + 1], layers, caches, t, cos, sin, hd))
    cached = np.concatenate(rows, axis=0)
    assert cached.shape == full.shape
    return float(np.max(np.abs(full.astype(np.float64) - cached)))


@pytest.mark.parametrize("S,k", [(9, 1), (9, 4), (12, 11)])
def test_one_layer_full_equals_prefill_then_decode(S, k):
    assert _full_vs_cached(1, S, k) < 1e-5


@pytest.mark.parametrize("S,k", [(5, 1), (10, 3)])
def test_two_layer_logits_full_equals_prefill_then_decode(S, k):
    # the reference's atol/rtol is 1e-5 (test_smollm2_model.py:122-125, :158-161)
    assert _full_vs_cached(2, S, k, seed=7, head=True) < 1e-5


def test_invariant_catches_wrong_rope_positions(monkeypatch):
    """Decode steps rotating at position 0..seq-1 instead of prev..prev+seq-1."""
    monkeypatch.setattr(ol, "positions", lambda prev, seq: np.arange(seq))
    assert _full_vs_cached(1, 9, 3) > 1e-2


def test_invariant_catches_a_transposed_cache_write(monkeypatch):
    """k/v written as (seq, n_kv) rows without the head-major transpose."""
    def bad_write(cache, k, v, prev):
        seq = k.shape[0]
        cache["k"][:, prev:prev + seq] = k.reshape(HKV, seq, D)
        cache["v"][:, prev:prev + seq] = v.reshape(HKV, seq, D)
    monkeypatch.setattr(ol, "write_cache", bad_write)
    assert _full_vs_cached(1, 9, 3) > 1e-2


@pytest.mark.parametrize("flag", [lambda prev: False, lambda prev: True])
def test_invariant_catches_the_wrong_causal_flag(monkeypatch, flag):
    """A non-causal prompt sees later tokens the prefill of S - k does not;
    a causal decode step over the prefix is the same as a non-causal one
    (bottom-right alignment, one query row), so only the prompt flag
    matters -- and S - k >= 2 rows make it visible."""
    monkeypatch.setattr(ol, "causal_flag", flag)
    err = _full_vs_cached(1, 9, 3)
    if flag(0):
        assert err < 1e-5  # causal everywhere is the reference's semantics too
    else:
        assert err > 1e-2


def test_invariant_catches_a_dropped_prefix_in_decode(monkeypatch):
    """Decode attending only to the new token (cache prefix dropped)."""
    real = oa.attention_gqa_ref

    def only_last(q, k, v, nh, nkv, causal=True, sm_scale=None):
        sk = k.shape[0] // nkv
        sq = q.shape[0] // nh
        if sq == 1 and sk > 1:
            k = k.reshape(nkv, sk, -1)[:, -1:].reshape(nkv, -1)
            v = v.reshape(nkv, sk, -1)[:, -1:].reshape(nkv, -1)
        return real(q, k, v, nh, nkv, causal=causal, sm_scale=sm_scale)
    monkeypatch.setattr(ol.oa, "attention_gqa_ref", only_last)
    assert _full_vs_cached(1, 9, 3) > 1e-2
