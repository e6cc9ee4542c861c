"""The reference's own kernel tests, replayed on the HIP path.

Inputs come from the reference tests' seeded streams (tests/golden/cases.py);
expected values from the float64 golden file and from the oracle.  Tolerance
is the reference's own (atol 1e-4; tests/test_attention.py:64,
tests/test_attention_gqa.py:115, tests/test_rope.py:65 use 1e-4).
"""

import os

import numpy as np
import pytest

from oracle import attention as oa
from oracle import rope as orope
from tests import _helpers as H
from tests.golden import cases
from triton_llm import gpu
from triton_llm.kernels import attention, precompute_cos_sin

pytestmark = pytest.mark.gpu

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.npz"))
ATOL = 1e-4


def check(name, got, tol=ATOL):
    exp = GOLDEN[name]
    err = H.max_abs(got, exp)
    H.report(name, err, tol)
    assert got.shape == exp.shape
    assert err <= tol, f"{name}: max_abs {err:.3e}"


# ---- allocator (tests/test_gpu_allocator.py) ---------------------------------

def test_allocator_roundtrip_dtypes_and_cleanup():
    arr = np.random.randn(4, 8).astype(np.float32)
    back = gpu.to_host(gpu.to_device(arr))
    assert back.shape == arr.shape and np.array_equal(arr, back)
    for dt in (np.float32, np.float64, np.float16, np.int32):
        a = np.arange(9, dtype=dt).reshape(3, 3)
        b = gpu.to_host(gpu.to_device(a))
        assert b.dtype == dt and np.array_equal(a, b)
    bits = np.array([0x3F80, 0xC000, 0x7FC0], np.uint16)
    t = gpu.to_device(bits, gpu.bfloat16)
    assert gpu.dtype_name(t.dtype) == "bfloat16" and np.array_equal(gpu.to_host(t), bits)
    empty = gpu.to_device(np.empty((0, 64), np.float32))
    assert gpu.to_host(empty).shape == (0, 64)
    z = gpu.zeros((5, 7), np.float32)
    assert np.all(gpu.to_host(z) == 0)
    dev = gpu.to_device(np.ones((10,), np.float32))
    del dev


# ---- attention (tests/test_attention.py) --------------------------------------

@pytest.mark.parametrize("idx", range(len(cases.ATTN_CASES)))
def test_attention_correctness(idx):
    name, q, k, v, causal = cases.attention_cases()[idx]
    out = attention(q, k, v)
    check(name, out)
    np.testing.assert_allclose(out, oa.attention_ref(q, k, v), atol=ATOL)


def test_attention_causal_mask():
    q, k, v, kp = cases.attention_causal_perturb()
    ref = attention(q, k, v)
    out = attention(q, kp, v)
    assert np.allclose(out[:-1], ref[:-1], atol=1e-5)
    check("attn_perturb_out", out)


def test_attention_identity_and_single_token():
    eye = np.eye(8, 64, dtype=np.float32)
    check("attn_identity", attention(eye, eye, eye))
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(attention(q, k, v), v, atol=ATOL)


def test_attention_non_causal():
    q, k, v = cases.attention_noncausal()
    out = attention(q, k, v, causal=False)
    assert out.shape == (1, 64) and not np.any(np.isnan(out))
    check("attn_noncausal", out)


# ---- attention_gqa (tests/test_attention_gqa.py) ------------------------------

def test_gqa_equivalence():
    q, k, v, nh, nkv = cases.gqa_equivalence()
    check("gqa_equivalence", H.attention_gqa_cpu(q, k, v, nh, nkv))


def test_gqa_reduced_kv():
    for name, q, k, v, nh, nkv in cases.gqa_reduced():
        check(name, H.attention_gqa_cpu(q, k, v, nh, nkv))


def test_gqa_with_rope():
    q, k, v = cases.gqa_rope()
    cos, sin = precompute_cos_sin(64, 64, theta=100000.0)
    q_rope = H.apply_rope_cpu(q, cos, sin, seq_len=8)
    k_rope = H.apply_rope_cpu(k, cos, sin, seq_len=8)
    out = H.attention_gqa_cpu(q_rope, k_rope, v, 9, 3)
    check("gqa_rope", out)
    np.testing.assert_allclose(out, oa.attention_gqa_ref(q_rope, k_rope, v, 9, 3), atol=ATOL)


def test_gqa_causal():
    (q, k, v, kp), (q2, k2, v2) = cases.gqa_causal()
    ref = H.attention_gqa_cpu(q, k, v, 6, 2).reshape(6, 8, 64)
    out = H.attention_gqa_cpu(q, kp, v, 6, 2).reshape(6, 8, 64)
    assert np.allclose(out[:, :-1], ref[:, :-1], atol=1e-5)
    check("gqa_causal_sq2_sk8", H.attention_gqa_cpu(q2, k2, v2, 6, 2))


def test_gqa_non_causal_decode():
    q, k, v = cases.gqa_noncausal()
    out = H.attention_gqa_cpu(q, k, v, 9, 3, causal=False)
    assert out.shape == (9, 64) and not np.any(np.isnan(out))
    check("gqa_noncausal", out)


def test_gqa_empty():
    k_some = np.random.randn(2 * 8, 64).astype(np.float32)
    out = H.attention_gqa_cpu(np.empty((0, 64), np.float32), k_some, k_some, 4, 2, causal=False)
    assert out.shape == (0, 64)
    q_some = np.random.randn(4 * 4, 64).astype(np.float32)
    out2 = H.attention_gqa_cpu(q_some, np.empty((0, 64), np.float32), np.empty((0, 64), np.float32), 4, 2, causal=False)
    assert out2.shape == (16, 64) and np.all(out2 == 0.0)
    e = np.empty((0, 64), np.float32)
    assert H.attention_gqa_cpu(e, e, e, 4, 2, causal=False).shape == (0, 64)


# ---- rope (tests/test_rope.py) -- bit-exact against the oracle ----------------

def test_rope_correctness_bitexact():
    for name, x, seq, rows in cases.rope_cases():
        cos, sin = precompute_cos_sin(rows, 64, theta=100000.0)
        out = H.apply_rope_cpu(x, cos, sin, seq_len=seq)
        np.testing.assert_array_equal(out, orope.apply_rope(x, cos, sin, seq))
        if name in GOLDEN.files:
            check(name, out)


def test_rope_identity_offset_single_theta_multidim():
    np.random.seed(1)
    x = np.random.randn(32, 64).astype(np.float32)
    cos, sin = precompute_cos_sin(1, 64, theta=100000.0)
    np.testing.assert_array_equal(H.apply_rope_cpu(x, cos, sin, seq_len=1), x)
    x = cases.rope_offset()
    cos, sin = precompute_cos_sin(64, 64, theta=100000.0)
    check("rope_offset8", H.apply_rope_cpu(x, cos, sin, seq_len=16, position_offset=8))
    for theta, x in cases.rope_theta_cases():
        cos, sin = precompute_cos_sin(16, 64, theta=theta)
        check(f"rope_theta_{int(theta)}", H.apply_rope_cpu(x, cos, sin, seq_len=8))
    x = cases.rope_multidim()
    cos, sin = precompute_cos_sin(16, 64)
    out = H.apply_rope_cpu(x, cos, sin, seq_len=8)
    assert out.shape == (2, 9, 8, 64)
    check("rope_multidim", out)
    cos, sin = precompute_cos_sin(8, 64)
    e = H.apply_rope_cpu(np.empty((0, 64), np.float32), cos, sin, seq_len=1)
    assert e.shape == (0, 64) and e.dtype == np.float32
