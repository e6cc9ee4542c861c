"""Host-side behaviour of the drop-in Python API that needs no GPU: the
reference's validation errors (same types, same order), backend selection,
and the loud failure when no HIP device is present."""

import ctypes

import numpy as np
import pytest

from triton_llm import gpu
from triton_llm import _lib
from triton_llm.kernels import attention, attention_gqa, apply_rope, precompute_cos_sin
from triton_llm.kernels import attention_decode, flash_attention, rope_kv_append


def fake(shape, dtype=np.float32):
    """A DeviceTensor that points nowhere (validation must fail before use)."""
    return gpu.DeviceTensor(ctypes.c_void_p(None), shape, dtype, 0, defer_free=False)


def has_device():
    n = ctypes.c_int(0)
    try:
        _lib.load().tl_device_count(ctypes.byref(n))
    except Exception:
        return False
    return n.value > 0


# ---- rope (reference tests/test_rope.py:253-309, rope.py:179-203) ----------

def test_apply_rope_validation():
    cos, sin = fake((8, 32)), fake((8, 32))
    with pytest.raises(ValueError):
        apply_rope(fake((64,)), cos, sin, seq_len=1)  # 1-D input
    with pytest.raises(ValueError):
        apply_rope(fake((4, 63)), fake((8, 31)), fake((8, 31)), seq_len=1)  # odd d_k
    with pytest.raises(ValueError):
        apply_rope(fake((4, 64)), fake((8, 64)), sin, seq_len=1)  # bad cos shape
    with pytest.raises(ValueError):
        apply_rope(fake((4, 64)), cos, sin, seq_len=0)
    with pytest.raises(ValueError):
        apply_rope(fake((4, 64)), fake((4, 32)), fake((4, 32)), seq_len=4, position_offset=1)
    with pytest.raises(ValueError):
        apply_rope(fake((4, 64)), cos, sin, seq_len=1, position_offset=-1)
    with pytest.raises(ValueError):
        apply_rope(fake((5, 64)), cos, sin, seq_len=2)
    with pytest.raises(ValueError):
        apply_rope(fake((4, 64)), fake((8, 32), np.float16), fake((8, 32), np.float16), seq_len=1)
    # n_rows == 0 returns the input untouched, before the seq_len checks
    x = fake((0, 64))
    assert apply_rope(x, cos, sin, seq_len=0) is x


def test_precompute_cos_sin_validation_and_values():
    with pytest.raises(ValueError):
        precompute_cos_sin(0, 64)
    with pytest.raises(ValueError):
        precompute_cos_sin(8, 63)
    with pytest.raises(ValueError):
        precompute_cos_sin(8, 64, theta=0)
    cos, sin = precompute_cos_sin(16, 64, 100000.0)
    assert cos.shape == (16, 32) and cos.dtype == np.float32
    assert np.allclose(cos[0], 1.0) and np.allclose(sin[0], 0.0)


# ---- attention_gqa (attention_gqa.py:188-233) ------------------------------

@pytest.mark.parametrize("args,msg", [
    (((4, 64), (4, 64), (4, 64), 0, 1), "n_head must be > 0"),
    (((4, 64), (4, 64), (4, 64), 2, 0), "n_kv_head must be > 0"),
    (((4, 64), (4, 64), (4, 64), 3, 2), "divisible by n_kv_head"),
    (((4, 64, 1), (4, 64), (4, 64), 2, 1), "must be 2D"),
    (((5, 64), (4, 64), (4, 64), 2, 1), "divisible by n_head"),
    (((4, 64), (5, 64), (5, 64), 2, 2), "divisible by n_kv_head"),
    (((4, 64), (4, 32), (4, 64), 2, 1), "K shape"),
    (((4, 64), (4, 64), (2, 64), 2, 1), "V shape"),
])
def test_attention_gqa_validation(args, msg):
    qs, ks, vs, nh, nkv = args
    with pytest.raises(ValueError, match=msg):
        attention_gqa(fake(qs), fake(ks), fake(vs), nh, nkv)


def test_attention_gqa_rejects_non_pow2_and_mixed_dtypes():
    with pytest.raises(ValueError, match="power of 2"):
        attention_gqa(fake((4, 48)), fake((4, 48)), fake((4, 48)), 2, 2)
    with pytest.raises(ValueError, match="share one dtype"):
        attention_gqa(fake((4, 64)), fake((4, 64), np.float16), fake((4, 64)), 2, 2)


# ---- attention (attention.py:166-180) ---------------------------------------

def test_attention_asserts():
    z = np.zeros
    with pytest.raises(AssertionError):
        attention(z((4,)), z((4, 8)), z((4, 8)))
    with pytest.raises(AssertionError):
        attention(z((4, 8)), z((3, 8)), z((4, 8)))
    with pytest.raises(AssertionError):
        attention(z((2, 8)), z((4, 8)), z((4, 8)), causal=True)
    with pytest.raises(AssertionError):
        attention(z((4, 12)), z((4, 12)), z((4, 12)))
    out = attention(z((0, 8)), z((0, 8)), z((0, 8)))
    assert out.shape == (0, 8) and out.dtype == np.float32


# ---- additive batched API ----------------------------------------------------

def test_decode_api_validation():
    kc = fake((2, 2, 16, 64), gpu.bfloat16)
    lens = fake((2,), np.int32)
    with pytest.raises(ValueError, match="KV heads"):
        attention_decode(fake((2, 4, 64), gpu.bfloat16), kc, kc, lens, 4, 1)
    with pytest.raises(ValueError, match="int32"):
        attention_decode(fake((2, 4, 64), gpu.bfloat16), kc, kc, fake((2,), np.int64), 4, 2)
    with pytest.raises(ValueError, match="share one dtype"):
        attention_decode(fake((2, 4, 64), np.float16), kc, kc, lens, 4, 2)
    with pytest.raises(ValueError, match="d_k in"):
        kc32 = fake((2, 2, 16, 32), gpu.bfloat16)
        attention_decode(fake((2, 4, 32), gpu.bfloat16), kc32, kc32, lens, 4, 2)
    with pytest.raises(ValueError, match="both be given"):
        rope_kv_append(None, fake((2, 2, 64), gpu.bfloat16), fake((2, 2, 64), gpu.bfloat16), kc, kc, lens,
                       fake((16, 32)), None)


def test_flash_api_validation():
    with pytest.raises(ValueError):
        flash_attention(fake((1, 4, 8, 64)), fake((1, 3, 8, 64)), fake((1, 3, 8, 64)))
    with pytest.raises(ValueError):
        flash_attention(fake((1, 4, 8, 64)), fake((2, 2, 8, 64)), fake((2, 2, 8, 64)))


# ---- runtime / backend -------------------------------------------------------

def test_bfloat16_dtype_tag():
    assert gpu.dtype_name(gpu.bfloat16) == "bfloat16"
    assert gpu.dtype_name(np.uint16) == "uint16"
    assert gpu.dtype_code(gpu.bfloat16) == _lib.DTYPE_BF16
    with pytest.raises(ValueError):
        gpu.dtype_code(np.uint16)
    assert np.empty((2, 2), dtype=gpu.bfloat16).reshape(4).dtype.metadata == gpu.bfloat16.metadata


def test_view_checks_element_count():
    t = fake((4, 8))
    v = gpu.view(t, (32,))
    assert v.shape == (32,) and v.ptr is t.ptr and not v._defer_free
    with pytest.raises(ValueError, match="element count mismatch"):
        gpu.view(t, (31,))


def test_cuda_backend_rejected(monkeypatch):
    monkeypatch.setenv("GPU_BACKEND", "cuda")
    with pytest.raises(RuntimeError, match="HIP-only"):
        gpu._detect_backend()
    monkeypatch.setenv("GPU_BACKEND", "metal")
    with pytest.raises(RuntimeError, match="only 'hip'"):
        gpu._detect_backend()
    monkeypatch.setenv("GPU_BACKEND", "hip")
    assert gpu._detect_backend() == "hip"


@pytest.mark.skipif(has_device(), reason="a HIP device is present")
def test_no_device_fails_loudly(monkeypatch):
    monkeypatch.setattr(gpu, "_initialized", False)
    with pytest.raises(RuntimeError, match="No supported GPU runtime found"):
        gpu.allocate((4,))
