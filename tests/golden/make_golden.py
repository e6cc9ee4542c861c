"""Write reference_cases.npz: expected outputs for the reference tests' inputs.

Inputs come from cases.py (the reference tests' own seeded streams).  Expected
outputs are computed here in float64 straight from the definitions --
softmax(q k^T * scale + mask) v with an explicit exp / sum, and the half-split
rotation with float64 cos/sin -- independently of the oracle package, so the
fixtures pin both the oracle (tests/test_golden.py) and the HIP kernels
(tests/test_gpu_*.py).  Each entry stores a digest of its inputs so a change
in the regenerated inputs is detected.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.golden import cases  # noqa: E402

OUT = os.path.join(HERE, "reference_cases.npz")


def softmax_attn_f64(q, k, v, scale, visible):
    """softmax over visible keys in float64; rows with no visible key -> NaN."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    s = (q @ k.T) * scale
    s = np.where(visible, s, -np.inf)
    with np.errstate(invalid="ignore"):
        m = s.max(axis=1, keepdims=True)
        e = np.exp(s - m)
        return (e / e.sum(axis=1, keepdims=True)) @ v


def mha_f64(q, k, v, causal):
    n, d = q.shape
    sk = k.shape[0]
    vis = np.ones((n, sk), dtype=bool)
    if causal:
        vis = np.arange(sk)[None, :] <= np.arange(n)[:, None]
    return softmax_attn_f64(q, k, v, 1.0 / np.sqrt(d), vis)


def gqa_f64(q, k, v, nh, nkv, causal):
    d = q.shape[1]
    sq = q.shape[0] // nh
    sk = k.shape[0] // nkv
    g = nh // nkv
    vis = np.ones((sq, sk), dtype=bool)
    if causal:
        vis = np.arange(sk)[None, :] <= (np.arange(sq)[:, None] + sk - sq)
    out = []
    for h in range(nh):
        kv = h // g
        out.append(softmax_attn_f64(q[h * sq:(h + 1) * sq], k[kv * sk:(kv + 1) * sk],
                                    v[kv * sk:(kv + 1) * sk], 1.0 / np.sqrt(d), vis))
    return np.concatenate(out, axis=0)


def rope_f64(x, seq_len, theta, offset=0):
    x = x.astype(np.float64)
    n, d = x.shape
    half = d // 2
    pos = (np.arange(n) % seq_len + offset).astype(np.float64)
    inv = theta ** (-2.0 * np.arange(half) / d)
    ang = pos[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    xe, xo = x[:, :half], x[:, half:]
    return np.concatenate([xe * c - xo * s, xe * s + xo * c], axis=1)


def build() -> dict:
    out: dict[str, np.ndarray] = {}

    def put(name, value, *inputs):
        out[name] = np.asarray(value, dtype=np.float32)
        out["digest__" + name] = np.array(cases.digest(*inputs))

    for name, q, k, v, causal in cases.attention_cases():
        put(name, mha_f64(q, k, v, causal), q, k, v)
    q, k, v, kp = cases.attention_causal_perturb()
    put("attn_perturb_ref", mha_f64(q, k, v, True), q, k, v)
    put("attn_perturb_out", mha_f64(q, kp, v, True), q, kp, v)
    q, k, v = cases.attention_noncausal()
    put("attn_noncausal", mha_f64(q, k, v, False), q, k, v)
    eye = np.eye(8, 64, dtype=np.float32)
    put("attn_identity", mha_f64(eye, eye, eye, True), eye)

    q, k, v, nh, nkv = cases.gqa_equivalence()
    put("gqa_equivalence", gqa_f64(q, k, v, nh, nkv, True), q, k, v)
    for name, q, k, v, nh, nkv in cases.gqa_reduced():
        put(name, gqa_f64(q, k, v, nh, nkv, True), q, k, v)
    (q, k, v, kp), (q2, k2, v2) = cases.gqa_causal()
    put("gqa_causal_ref", gqa_f64(q, k, v, 6, 2, True), q, k, v)
    put("gqa_causal_pert", gqa_f64(q, kp, v, 6, 2, True), q, kp, v)
    put("gqa_causal_sq2_sk8", gqa_f64(q2, k2, v2, 6, 2, True), q2, k2, v2)
    q, k, v = cases.gqa_noncausal()
    put("gqa_noncausal", gqa_f64(q, k, v, 9, 3, False), q, k, v)
    q, k, v = cases.gqa_rope()
    qr = rope_f64(q, 8, 100000.0).astype(np.float32)
    kr = rope_f64(k, 8, 100000.0).astype(np.float32)
    put("gqa_rope", gqa_f64(qr, kr, v, 9, 3, True), q, k, v)

    # Large RoPE cases are covered bit-exactly against the oracle instead.
    for name, x, seq, _rows in cases.rope_cases():
        if x.shape[0] <= 256:
            put(name, rope_f64(x, seq, 100000.0), x)
    for theta, x in cases.rope_theta_cases():
        put(f"rope_theta_{int(theta)}", rope_f64(x, 8, theta), x)
    x = cases.rope_multidim()
    put("rope_multidim", rope_f64(x.reshape(-1, 64), 8, 100000.0).reshape(x.shape), x)
    x = cases.rope_offset()
    put("rope_offset8", rope_f64(x, 16, 100000.0, offset=8), x)
    return out


if __name__ == "__main__":
    data = build()
    np.savez_compressed(OUT, **data)
    size = os.path.getsize(OUT)
    print(f"wrote {OUT}: {len([k for k in data if not k.startswith('digest__')])} cases, {size / 1024:.0f} KiB")
