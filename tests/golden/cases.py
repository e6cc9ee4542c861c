"""Input recipes of the reference's own kernel tests, replayed exactly.

The reference's tests (tests/test_attention.py, tests/test_attention_gqa.py,
tests/test_rope.py of ziliangpeng/triton-llm) store no fixtures; each draws
its inputs from the legacy global NumPy stream (``np.random.seed(s)`` then
``randn`` in a fixed order).  That stream (MT19937 + Box-Muller legacy
gaussian) is stable across NumPy versions, so the same inputs are recreated
here case by case.  Each generator names the reference lines whose draw order
it follows.  Expected outputs live in reference_cases.npz (make_golden.py).
"""

from __future__ import annotations

import hashlib

import numpy as np

# (N, d_k) cases of tests/test_attention.py:41-51, drawn in this order after
# np.random.seed(42), q, k, v per case (:53-58).
ATTN_CASES = [(1, 64), (4, 64), (16, 64), (32, 64), (128, 64), (777, 64), (1024, 64), (16, 32), (16, 128)]

# (n_head, n_kv_head, d_k, seq) of tests/test_attention_gqa.py:126-131.
GQA_REDUCED = [(9, 3, 64, 8), (15, 5, 64, 8), (32, 8, 64, 16), (6, 2, 128, 8)]

# (seq_len, d_k, n_rows) of tests/test_rope.py:47-54.
ROPE_CASES = [(8, 64, 576), (128, 64, 1024), (512, 64, 2048), (16, 64, 144), (32, 64, 32)]


def _randn(*shape):
    return np.random.randn(*shape).astype(np.float32)


def attention_cases():
    """test_attention.py:37-67 -- list of (name, q, k, v, causal)."""
    out = []
    np.random.seed(42)
    for n, d in ATTN_CASES:
        q, k, v = _randn(n, d), _randn(n, d), _randn(n, d)
        out.append((f"attn_n{n}_d{d}", q, k, v, True))
    return out


def attention_causal_perturb():
    """test_attention.py:81-92 -- (q, k, v, k_perturbed)."""
    np.random.seed(42)
    n, d = 16, 64
    q, k, v = _randn(n, d), _randn(n, d), _randn(n, d)
    kp = k.copy()
    kp[-1, :] = _randn(d)
    return q, k, v, kp


def attention_noncausal():
    """test_attention.py:157-163 -- one query against 8 keys."""
    np.random.seed(42)
    return _randn(1, 64), _randn(8, 64), _randn(8, 64)


def gqa_equivalence():
    """test_attention_gqa.py:101-109."""
    np.random.seed(42)
    return _randn(4 * 16, 64), _randn(4 * 16, 64), _randn(4 * 16, 64), 4, 4


def gqa_reduced():
    """test_attention_gqa.py:125-137 -- list of (name, q, k, v, n_head, n_kv)."""
    np.random.seed(42)
    out = []
    for nh, nkv, d, s in GQA_REDUCED:
        q, k, v = _randn(nh * s, d), _randn(nkv * s, d), _randn(nkv * s, d)
        out.append((f"gqa_{nh}_{nkv}_d{d}_s{s}", q, k, v, nh, nkv))
    return out


def gqa_rope():
    """test_attention_gqa.py:157-171 -- q, k, v before RoPE (9 / 3 heads, seq 8, theta 1e5)."""
    np.random.seed(42)
    return _randn(9 * 8, 64), _randn(3 * 8, 64), _randn(3 * 8, 64)


def gqa_causal():
    """test_attention_gqa.py:195-233 -- (q, k, v, k_pert) for 6/2 heads seq 8,
    then (q2, k2, v2) with seq_q = 2, seq_k = 8 from the continuing stream."""
    np.random.seed(42)
    nh, nkv, d, s = 6, 2, 64, 8
    q, k, v = _randn(nh * s, d), _randn(nkv * s, d), _randn(nkv * s, d)
    kp = k.copy()
    for h in range(nkv):
        kp[h * s + (s - 1), :] = _randn(d)
    q2, k2, v2 = _randn(nh * 2, d), _randn(nkv * 8, d), _randn(nkv * 8, d)
    return (q, k, v, kp), (q2, k2, v2)


def gqa_noncausal():
    """test_attention_gqa.py:246-255 -- 9 / 3 heads, seq_q 1, seq_k 16."""
    np.random.seed(42)
    return _randn(9, 64), _randn(3 * 16, 64), _randn(3 * 16, 64)


def rope_cases():
    """test_rope.py:45-61 -- list of (name, x, seq_len, table_rows); theta 1e5."""
    np.random.seed(42)
    out = []
    for seq, d, n_rows in ROPE_CASES:
        x = _randn(n_rows, d)
        out.append((f"rope_s{seq}_d{d}_r{n_rows}", x, seq, max(seq, 128)))
    return out


def rope_theta_cases():
    """test_rope.py:320-330 -- list of (theta, x), seq 8, 16 rows, table 16."""
    np.random.seed(7)
    return [(t, _randn(16, 64)) for t in (10000.0, 100000.0, 500000.0)]


def rope_offset():
    """test_rope.py:117-127 -- x (16, 64), seq 16, offset 8, table 64 rows."""
    np.random.seed(3)
    return _randn(16, 64)


def rope_multidim():
    """test_rope.py:347-352 -- x (2, 9, 8, 64), table 16 rows, default theta."""
    np.random.seed(9)
    return _randn(2, 9, 8, 64)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]
