"""RMSNorm, the fused residual add + RMSNorm, SwiGLU and add against the
oracle (oracle/layers.py), on the reference's own cases (tests/test_rms_norm.py,
test_swiglu.py, test_add.py of the reference: seeded shapes incl. model
widths and non-powers of two, constant / zero / large rows, empty inputs,
shape errors) plus 16-bit storage.  Tolerances: the reference's
allclose(atol 1e-4, rtol 1e-4) for fp32; 16-bit outputs within their
rounding (rtol 8e-3, atol 1e-2).  The fused add + RMSNorm must equal add then
RMSNorm bit for bit.
"""

import numpy as np
import pytest

from oracle import layers as ol
from oracle import numerics as on
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import add, add_rms_norm, rms_norm, swiglu

pytestmark = pytest.mark.gpu


def rms_norm_cpu(x, w, eps=1e-5, dtype="float32"):
    x2 = x.reshape(-1, x.shape[-1])
    out = gpu.allocate(x2.shape, H.GPU_DTYPES[dtype])
    rms_norm(H.upload(x2, dtype), H.upload(w, dtype), out, eps)
    return H.download(out).reshape(x.shape)


@pytest.mark.parametrize("M,N", [(8, 64), (16, 128), (32, 576), (16, 960), (8, 2048), (16, 777), (4, 1), (3, 3072),
                                 (2, 8192), (2, 8193), (2, 10000)])
def test_rms_norm_reference_cases(M, N):
    np.random.seed(42)
    x = np.random.randn(M, N).astype(np.float32)
    w = np.random.randn(N).astype(np.float32)
    out = rms_norm_cpu(x, w)
    assert np.allclose(out, ol.rms_norm_ref(x, w), atol=1e-4, rtol=1e-4)


def test_rms_norm_edge_cases():
    w = np.random.randn(576).astype(np.float32)
    for x in (np.full((4, 576), 3.25, np.float32), np.zeros((4, 576), np.float32),
              1000.0 * np.random.randn(4, 576).astype(np.float32), np.random.randn(4, 16, 576).astype(np.float32)):
        assert np.allclose(rms_norm_cpu(x, w), ol.rms_norm_ref(x, w), atol=1e-4, rtol=1e-4)
    out = gpu.allocate((0, 576), np.float32)
    assert rms_norm(gpu.allocate((0, 576), np.float32), gpu.to_device(np.ones(576, np.float32)), out) is out
    with pytest.raises(AssertionError):
        rms_norm_cpu(np.ones((8, 576), np.float32), np.ones(64, np.float32))
    with pytest.raises(ValueError):
        rms_norm(gpu.to_device(np.ones(64, np.float32)), gpu.to_device(np.ones(64, np.float32)),
                 gpu.allocate((64,), np.float32))
    with pytest.raises(ValueError, match="N > 0"):
        rms_norm(gpu.allocate((3, 0), np.float32), gpu.allocate((0,), np.float32), gpu.allocate((3, 0), np.float32))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_rms_norm_16bit(dtype):
    rng = np.random.default_rng(4)
    x = on.to_storage(rng.standard_normal((7, 960), dtype=np.float32), dtype)
    w = on.to_storage(rng.standard_normal(960, dtype=np.float32), dtype)
    got = on.from_storage(rms_norm_cpu(x, w, dtype=dtype), dtype)
    np.testing.assert_allclose(got, ol.rms_norm_ref(on.from_storage(x, dtype), on.from_storage(w, dtype)),
                               rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_add_rms_norm_equals_add_then_rms_norm(dtype):
    rng = np.random.default_rng(5)
    a = on.to_storage(rng.standard_normal((5, 960), dtype=np.float32), dtype)
    b = on.to_storage(rng.standard_normal((5, 960), dtype=np.float32), dtype)
    w = on.to_storage(rng.standard_normal(960, dtype=np.float32), dtype)
    gd = H.GPU_DTYPES[dtype]
    a_d, b_d, w_d = H.upload(a, dtype), H.upload(b, dtype), H.upload(w, dtype)
    h1, y1 = gpu.allocate((5, 960), gd), gpu.allocate((5, 960), gd)
    add_rms_norm(a_d, b_d, h1, w_d, y1)
    h2 = add(a_d, b_d)
    y2 = rms_norm(h2, w_d, gpu.allocate((5, 960), gd))
    np.testing.assert_array_equal(H.download(h1), H.download(h2))
    np.testing.assert_array_equal(H.download(y1), H.download(y2))
    # and the residual updated in place (h is a)
    add_rms_norm(a_d, b_d, a_d, w_d, y1)
    np.testing.assert_array_equal(H.download(a_d), H.download(h2))
    np.testing.assert_array_equal(H.download(y1), H.download(y2))


@pytest.mark.parametrize("N", [1536, 2560, 8192, 777, 1])
def test_swiglu_reference_cases(N):
    np.random.seed(42)
    g = np.random.randn(N).astype(np.float32)
    u = np.random.randn(N).astype(np.float32)
    out = H.download(swiglu(gpu.to_device(g), gpu.to_device(u)))
    assert np.allclose(out, ol.swiglu_ref(g, u), atol=1e-4, rtol=1e-4)


def test_swiglu_edge_cases():
    g = np.array([0.0, 50.0, -50.0, 88.0, -100.0, 1e-8, -1e-8], np.float32)
    u = np.array([1.0, 2.0, 3.0, 0.5, 7.0, 1.0, 1.0], np.float32)
    out = H.download(swiglu(gpu.to_device(g), gpu.to_device(u)))
    assert np.all(np.isfinite(out)) and np.allclose(out, ol.swiglu_ref(g, u), atol=1e-4, rtol=1e-4)
    multi = np.random.randn(4, 16, 1536).astype(np.float32)
    up = np.random.randn(4, 16, 1536).astype(np.float32)
    o = H.download(swiglu(gpu.to_device(multi), gpu.to_device(up)))
    assert o.shape == multi.shape and np.allclose(o, ol.swiglu_ref(multi, up), atol=1e-4, rtol=1e-4)
    assert swiglu(gpu.allocate((0,), np.float32), gpu.allocate((0,), np.float32)).shape == (0,)
    with pytest.raises(ValueError):
        swiglu(gpu.allocate((8,), np.float32), gpu.allocate((9,), np.float32))
    bf = on.to_storage(np.random.randn(1536).astype(np.float32), "bfloat16")
    ub = on.to_storage(np.random.randn(1536).astype(np.float32), "bfloat16")
    got = on.from_storage(H.download(swiglu(H.upload(bf, "bfloat16"), H.upload(ub, "bfloat16"))), "bfloat16")
    np.testing.assert_allclose(got, ol.swiglu_ref(on.from_storage(bf, "bfloat16"), on.from_storage(ub, "bfloat16")),
                               rtol=8e-3, atol=1e-2)


def test_add_reference_cases():
    np.random.seed(42)
    for shape in [(1024,), (1000,), (4, 576), (3, 5, 7), (1,)]:
        x = np.random.randn(*shape).astype(np.float32)
        y = np.random.randn(*shape).astype(np.float32)
        out = H.download(add(gpu.to_device(x), gpu.to_device(y)))
        np.testing.assert_array_equal(out, x + y)  # one fp32 add: exact
    big = 1e30 * np.ones(8, np.float32)
    np.testing.assert_array_equal(H.download(add(gpu.to_device(big), gpu.to_device(-big))), np.zeros(8, np.float32))
    assert add(gpu.allocate((0, 3), np.float32), gpu.allocate((0, 3), np.float32)).shape == (0, 3)
    with pytest.raises(AssertionError):
        add(gpu.allocate((4,), np.float32), gpu.allocate((5,), np.float32))
