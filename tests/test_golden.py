"""The oracle against the committed golden vectors of the reference's own test
cases (inputs replayed from the reference tests' seeded streams, outputs in
float64 from the definitions).  CPU only."""

import os

import numpy as np
import pytest

from oracle import attention as oa
from oracle import rope as orope
from tests.golden import cases

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.npz"))


def expect(name, *inputs):
    assert str(GOLDEN["digest__" + name]) == cases.digest(*inputs), f"inputs of {name} changed"
    return GOLDEN[name]


def test_golden_file_covers_reference_cases():
    names = {k for k in GOLDEN.files if not k.startswith("digest__")}
    assert len(names) >= 30
    for n, d in cases.ATTN_CASES:
        assert f"attn_n{n}_d{d}" in names


@pytest.mark.parametrize("idx", range(len(cases.ATTN_CASES)))
def test_attention_cases(idx):
    name, q, k, v, causal = cases.attention_cases()[idx]
    np.testing.assert_allclose(oa.attention_ref(q, k, v, causal), expect(name, q, k, v), atol=1e-5)


def test_attention_noncausal_and_perturb():
    q, k, v = cases.attention_noncausal()
    np.testing.assert_allclose(oa.attention_ref(q, k, v, False), expect("attn_noncausal", q, k, v), atol=1e-5)
    q, k, v, kp = cases.attention_causal_perturb()
    a = expect("attn_perturb_ref", q, k, v)
    b = expect("attn_perturb_out", q, kp, v)
    np.testing.assert_allclose(a[:-1], b[:-1], atol=1e-6)  # the golden itself is causal
    np.testing.assert_allclose(oa.attention_ref(q, kp, v), b, atol=1e-5)


def test_gqa_cases():
    q, k, v, nh, nkv = cases.gqa_equivalence()
    np.testing.assert_allclose(oa.attention_gqa_ref(q, k, v, nh, nkv), expect("gqa_equivalence", q, k, v), atol=1e-5)
    for name, q, k, v, nh, nkv in cases.gqa_reduced():
        np.testing.assert_allclose(oa.attention_gqa_ref(q, k, v, nh, nkv), expect(name, q, k, v), atol=1e-5)
    (q, k, v, kp), (q2, k2, v2) = cases.gqa_causal()
    np.testing.assert_allclose(oa.attention_gqa_ref(q, kp, v, 6, 2), expect("gqa_causal_pert", q, kp, v), atol=1e-5)
    np.testing.assert_allclose(oa.attention_gqa_ref(q2, k2, v2, 6, 2), expect("gqa_causal_sq2_sk8", q2, k2, v2), atol=1e-5)
    q, k, v = cases.gqa_noncausal()
    np.testing.assert_allclose(oa.attention_gqa_ref(q, k, v, 9, 3, causal=False),
                               expect("gqa_noncausal", q, k, v), atol=1e-5)


def test_gqa_with_rope():
    q, k, v = cases.gqa_rope()
    cos, sin = orope.precompute_cos_sin(64, 64, 100000.0)
    qr = orope.apply_rope(q, cos, sin, 8)
    kr = orope.apply_rope(k, cos, sin, 8)
    np.testing.assert_allclose(oa.attention_gqa_ref(qr, kr, v, 9, 3), expect("gqa_rope", q, k, v), atol=1e-5)


def test_rope_cases():
    for name, x, seq, rows in cases.rope_cases():
        if "digest__" + name not in GOLDEN.files:
            continue
        cos, sin = orope.precompute_cos_sin(rows, 64, 100000.0)
        np.testing.assert_allclose(orope.apply_rope(x, cos, sin, seq), expect(name, x), atol=1e-5)
    for theta, x in cases.rope_theta_cases():
        cos, sin = orope.precompute_cos_sin(16, 64, theta)
        np.testing.assert_allclose(orope.apply_rope(x, cos, sin, 8), expect(f"rope_theta_{int(theta)}", x), atol=1e-5)
    x = cases.rope_offset()
    cos, sin = orope.precompute_cos_sin(64, 64, 100000.0)
    np.testing.assert_allclose(orope.apply_rope(x, cos, sin, 16, 8), expect("rope_offset8", x), atol=1e-5)
    x = cases.rope_multidim()
    cos, sin = orope.precompute_cos_sin(16, 64, 100000.0)
    got = orope.apply_rope(x.reshape(-1, 64), cos, sin, 8).reshape(x.shape)
    np.testing.assert_allclose(got, expect("rope_multidim", x), atol=1e-5)
