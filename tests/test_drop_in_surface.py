"""The drop-in surface (CPU, no GPU touched).

1. Every name the unchanged SmolLM2 model imports
   (smollm2_triton/model.py:13-19 of the reference) resolves in this package
   with the reference's parameter names, order and defaults (reference
   signatures: kernels/gemm.py:53-57, add.py:54-58, rms_norm.py:68-73,
   rope.py:73-77, :126-130, :153-159, swiglu.py:70-74,
   attention_gqa.py:149-157; GPT-2's attention: attention.py:141).
2. ``attention_gqa``'s decode call (one query token, the call the model makes
   once per layer per token, model.py:310-314) uploads nothing, waits for
   nothing and, after warm-up, allocates nothing: the reference's "no sync"
   contract (attention_gqa.py:158, :269).  A stand-in runtime records every
   C-ABI call; host-only sizing functions go to the real library.
"""

import ctypes
import importlib
import inspect

import numpy as np
import pytest

from triton_llm import _lib, gpu

REQ = inspect.Parameter.empty  # a required parameter

# (module, name) -> [(parameter, default or REQ), ...]
SMOLLM2_IMPORTS = {
    ("triton_llm.kernels.gemm", "gemm"): [("h_dev", REQ), ("w_dev", REQ), ("out_dev", None)],
    ("triton_llm.kernels.add", "add"): [("x_dev", REQ), ("y_dev", REQ), ("out_dev", None)],
    ("triton_llm.kernels.rms_norm", "rms_norm"): [("x_dev", REQ), ("w_dev", REQ), ("out_dev", REQ), ("eps", 1e-5)],
    ("triton_llm.kernels.rope", "precompute_cos_sin_device"): [("max_seq_len", REQ), ("d_k", REQ), ("theta", 100000.0)],
    ("triton_llm.kernels.rope", "apply_rope"): [("x_dev", REQ), ("cos_dev", REQ), ("sin_dev", REQ), ("seq_len", REQ),
                                                ("position_offset", 0)],
    ("triton_llm.kernels.swiglu", "swiglu"): [("gate_dev", REQ), ("up_dev", REQ), ("out_dev", None)],
    ("triton_llm.kernels.attention_gqa", "attention_gqa"): [("q_dev", REQ), ("k_dev", REQ), ("v_dev", REQ),
                                                            ("n_head", REQ), ("n_kv_head", REQ), ("causal", True),
                                                            ("sm_scale", None)],
    ("triton_llm.kernels.rope", "precompute_cos_sin"): [("max_seq_len", REQ), ("d_k", REQ), ("theta", 100000.0)],
    ("triton_llm.kernels.attention", "attention"): [("q", REQ), ("k", REQ), ("v", REQ), ("causal", True)],
}


@pytest.mark.parametrize("mod,name", sorted(SMOLLM2_IMPORTS))
def test_model_imports_resolve_with_the_reference_parameters(mod, name):
    fn = getattr(importlib.import_module(mod), name)
    params = list(inspect.signature(fn).parameters.values())
    want = SMOLLM2_IMPORTS[(mod, name)]
    got = [(p.name, p.default) for p in params[:len(want)]]
    assert got == want, f"{mod}.{name}: {got} != {want}"
    # anything this build adds after the reference's parameters is optional
    for p in params[len(want):]:
        assert p.default is not inspect.Parameter.empty, f"{name}.{p.name} added without a default"
    # and the package-level export the reference's kernels/__init__.py:6-16 offers
    if name != "precompute_cos_sin_device":
        import triton_llm.kernels as k
        assert getattr(k, name) is fn


class RecordingRuntime:
    """Stands in for the loaded HIP library: counts calls, hands out fake
    device addresses, launches nothing.  Host-only queries are answered by
    the real library."""

    HOST_ONLY = ("tl_decode_split_size", "tl_attention_decode_workspace_bytes",
                 "tl_attention_fwd_workspace_bytes", "tl_attention_fwd_workspace_bytes_split",
                 "tl_error_string")

    def __init__(self):
        self.real = _lib.load()
        self.calls = []
        self.next_addr = 1 << 40
        self.decode_args = None

    def _rec(self, name):
        self.calls.append(name)

    def tl_malloc(self, ref, nbytes):
        self._rec("tl_malloc")
        ref._obj.value = self.next_addr
        self.next_addr += (nbytes + 4095) // 4096 * 4096
        return 0

    def tl_attention_decode(self, *args):
        self._rec("tl_attention_decode")
        self.decode_args = args
        return 0

    def __getattr__(self, name):
        if name in self.HOST_ONLY:
            return getattr(self.real, name)
        if name.startswith("tl_"):
            return lambda *a: (self._rec(name), 0)[1]
        raise AttributeError(name)


@pytest.fixture
def recording(monkeypatch):
    rt = RecordingRuntime()
    monkeypatch.setattr(gpu, "_rt", rt)
    monkeypatch.setattr(gpu, "_initialized", True)
    monkeypatch.setattr(gpu, "_pool", {})
    monkeypatch.setattr(gpu, "_pool_bytes", 0)
    from triton_llm.kernels import _common
    monkeypatch.setattr(_common, "_shared", {})
    yield rt
    # blocks handed to the stand-in must not reach the real library later
    gpu._pool.clear()
    _common._shared.clear()


def _fake(shape, dtype):
    nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return gpu.DeviceTensor(ctypes.c_void_p(1 << 20), shape, dtype, nbytes, defer_free=False)


@pytest.mark.parametrize("dtype", [np.float32, gpu.bfloat16])
def test_attention_gqa_decode_uploads_waits_and_allocates_nothing(recording, dtype):
    from triton_llm.kernels import attention_gqa

    H, Hkv, D = 9, 3, 64
    for step, L in enumerate((100, 101, 102, 103)):
        q = _fake((H, D), dtype)
        k, v = _fake((Hkv * L, D), dtype), _fake((Hkv * L, D), dtype)
        recording.calls.clear()
        o = attention_gqa(q, k, v, H, Hkv, causal=False)
        assert o.shape == (H, D)
        args = recording.decode_args
        assert args[3] is None and args[4] == L  # length by value: cache_lens NULL, len_add = seq_k
        if step >= 2:  # warm-up done: the output block comes from the cache
            assert recording.calls == ["tl_attention_decode"], recording.calls
        for banned in ("tl_memcpy_htod", "tl_memcpy_dtoh", "tl_synchronize", "tl_free"):
            assert banned not in recording.calls, recording.calls
        del o  # the model drops each step's output


def test_block_cache_reuses_and_bounds(recording, monkeypatch):
    a = gpu.allocate((1000,), np.float32)
    addr = a.data_ptr()
    del a
    assert gpu.cached_bytes() == 4096
    b = gpu.allocate((1024,), np.float32)  # same 256-byte-rounded size
    assert b.data_ptr() == addr and recording.calls.count("tl_malloc") == 1
    c = gpu.allocate((1025,), np.float32)  # another size: a new block
    assert c.data_ptr() != addr and recording.calls.count("tl_malloc") == 2
    assert gpu.allocate((0,), np.float32).data_ptr() == 0
    monkeypatch.setattr(gpu, "POOL_MAX_BLOCK", 1024)
    del b
    assert "tl_free" in recording.calls  # too large for the cache: returned to HIP
    gpu.empty_cache()
    assert gpu.cached_bytes() == 0


def test_kv_cache_rejects_positions_past_the_rope_table(recording):
    """apply_rope's ValueError (rope.py:194-198) before any launch: the
    kernel would otherwise skip the rows past the table silently."""
    from triton_llm.kv_cache import GpuKVCache

    H, Hkv, D = 4, 2, 64
    cache = GpuKVCache(1, H, Hkv, D, max_seq=16)
    cos, sin = _fake((4, D // 2), np.float32), _fake((4, D // 2), np.float32)
    q, k, v = _fake((5, H * D), np.float32), _fake((5, Hkv * D), np.float32), _fake((5, Hkv * D), np.float32)
    recording.calls.clear()
    with pytest.raises(ValueError, match=r"position_offset \(0\) \+ seq_len \(5\) exceeds cos/sin table size \(4\)"):
        cache.attention(0, q, k, v, cos, sin)
    assert not any(c.startswith("tl_rope") or c.startswith("tl_attention") for c in recording.calls)


def test_kv_cache_advance_is_a_device_copy(recording):
    """The cache length the kernels read moves by a stream-ordered device
    copy from a table of lengths: advance() and reset() upload nothing and
    never synchronise (the model advances once per generated token)."""
    from triton_llm.kv_cache import GpuKVCache

    copies = []

    def dtod(dst, src, n):
        copies.append((dst.value, src.value, n))
        return 0

    cache = GpuKVCache(2, 4, 2, 64, max_seq=32)
    recording.tl_memcpy_dtod = dtod
    table = cache._len_table.ptr.value
    recording.calls.clear()
    cache.advance(5)
    cache.advance(1)
    cache.reset()
    assert copies == [(cache._lens.ptr.value, table + 4 * 5, 4), (cache._lens.ptr.value, table + 4 * 6, 4),
                      (cache._lens.ptr.value, table, 4)]
    for banned in ("tl_memcpy_htod", "tl_memcpy_dtoh", "tl_synchronize"):
        assert banned not in recording.calls, recording.calls
    assert cache.cache_len == 0
