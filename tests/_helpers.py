"""NumPy-in / NumPy-out wrappers over the GPU entry points, for tests.

Counterpart of the reference's tests/_kernel_helpers.py (:53-115): move data
to the GPU, call the entry point through the C ABI, synchronise, copy back.
Storage dtypes: 'float32', 'float16', 'bfloat16' (bf16 carried as uint16 bits).
"""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from triton_llm.kernels.attention_gqa import attention_gqa as _attention_gqa
from triton_llm.kernels.rope import apply_rope as _apply_rope

GPU_DTYPES = {"float32": np.float32, "float16": np.float16, "bfloat16": gpu.bfloat16}


def upload(storage: np.ndarray, dtype: str = "float32"):
    return gpu.to_device(np.ascontiguousarray(storage), GPU_DTYPES[dtype])


def download(t) -> np.ndarray:
    gpu.synchronize()
    out = gpu.to_host(t)
    if gpu.dtype_name(t.dtype) == "bfloat16":
        return out.view(np.uint16)
    return out


def apply_rope_cpu(x, cos, sin, seq_len, position_offset=0, dtype="float32"):
    """reference _kernel_helpers.apply_rope_cpu, extended to 16-bit storage."""
    orig = x.shape
    if x.ndim > 2:
        x = x.reshape(-1, orig[-1])
    x_dev = upload(x, dtype)
    cos_dev = gpu.to_device(np.require(cos, np.float32, ["C_CONTIGUOUS"]))
    sin_dev = gpu.to_device(np.require(sin, np.float32, ["C_CONTIGUOUS"]))
    _apply_rope(x_dev, cos_dev, sin_dev, seq_len=seq_len, position_offset=position_offset)
    return download(x_dev).reshape(orig)


def attention_gqa_cpu(q, k, v, n_head, n_kv_head, causal=True, dtype="float32", sm_scale=None):
    """reference _kernel_helpers.attention_gqa_cpu, extended to 16-bit storage."""
    o = _attention_gqa(upload(q, dtype), upload(k, dtype), upload(v, dtype), n_head, n_kv_head,
                       causal=causal, sm_scale=sm_scale)
    return download(o)


def set_override(monkeypatch, name: str, value) -> None:
    """Set (or, for None, clear) one of the library's test-only environment
    overrides and have the library re-read them now (it reads them in
    tl_init, not per launch).  monkeypatch restores the variable after the
    test, and the autouse fixture in conftest re-reads it then."""
    if value is None:
        monkeypatch.delenv(name, raising=False)
    else:
        monkeypatch.setenv(name, str(value))
    gpu.reload_overrides()


def max_abs(a, b) -> float:
    """Largest |a - b| over the broadcast arrays, NaN-strict.

    A NaN on one side only makes the error +inf, so a partly-NaN result can
    never pass a tolerance.  NaN on both sides at the same position counts as
    agreement (fully masked rows are NaN by definition), and equal
    infinities count as zero error.
    """
    a, b = np.broadcast_arrays(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64))
    if a.size == 0:
        return 0.0
    nan_a, nan_b = np.isnan(a), np.isnan(b)
    if np.any(nan_a != nan_b):
        return float("inf")
    keep = ~nan_a
    a, b = a[keep], b[keep]
    if a.size == 0:
        return 0.0
    diff = np.abs(a - b)
    diff[a == b] = 0.0  # inf == inf
    return float(diff.max())


def report(name: str, err: float, tol: float) -> None:
    print(f"[{'PASS' if err <= tol else 'FAIL'}] {name}: max_abs={err:.3e} tol={tol:.0e}", flush=True)
