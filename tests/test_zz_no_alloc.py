"""tl_attention_decode_noalloc, the decode entry point that allocates
nothing, against tl_attention_decode (the existing entry point, same
kernels) and the oracle.  The file name makes pytest collect it last.

Both are called through the C ABI on the same inputs; the outputs must be
bitwise equal (same partition, same kernels), and within the decode
tolerance (2e-2 for bf16/fp16, 2e-3 for fp32) of the oracle.  Two calls in a
row, the second on a smaller problem, so the second reuses the static scratch
the first left behind.  A problem larger than the static scratch is refused
with TL_ERR_INVALID before any device work.
"""

import numpy as np
import pytest

from oracle import attention as oa
from oracle import inputs as oi
from oracle import numerics as on
from tests import _helpers as H
from triton_llm import _lib, gpu

pytestmark = pytest.mark.gpu

TOL = {"float32": 2e-3, "float16": 2e-2, "bfloat16": 2e-2}
CODE = {"float32": _lib.DTYPE_F32, "float16": _lib.DTYPE_F16, "bfloat16": _lib.DTYPE_BF16}


@pytest.fixture
def shares_path(monkeypatch):
    """Small caches would take the pair path, which writes no partials; the
    equal-shares path is the one whose partials live in the static scratch."""
    H.set_override(monkeypatch, "TRITON_LLM_HIP_DECODE_SHARES", 1)


def _run_both(cfg):
    dt = cfg.dtype
    B, Hq, Hkv, D, C = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.d_k, cfg.max_ctx
    print(f"[case] noalloc {cfg.name} B={B} Hq={Hq} Hkv={Hkv} D={D} ctx={C} {dt}", flush=True)
    d = oi.make_decode(cfg, fill="nan")
    q, kc, vc = H.upload(d["q"], dt), H.upload(d["k_cache"], dt), H.upload(d["v_cache"], dt)
    lens = gpu.to_device(d["lens"])
    lib = gpu.runtime()
    split = lib.tl_decode_split_size(B, Hkv, C)
    need = lib.tl_attention_decode_workspace_bytes(B, Hq, C, D, split)
    assert need <= _lib_max_bytes()
    ws = gpu.allocate((need,), np.uint8)
    qo = _lib.strides(Hq * D, D)
    cs = _lib.strides(Hkv * C * D, C * D, D)
    o_ref = gpu.allocate((B, Hq, D), q.dtype)
    o_new = gpu.allocate((B, Hq, D), q.dtype)
    st = lib.tl_attention_decode(q.ptr, kc.ptr, vc.ptr, lens.ptr, 0, o_ref.ptr, ws.ptr, need,
                                 B, Hq, Hkv, C, D, qo, cs, cs, qo, float(cfg.scale), split, CODE[dt], None)
    assert st == 0, st
    st = lib.tl_attention_decode_noalloc(q.ptr, kc.ptr, vc.ptr, lens.ptr, 0, o_new.ptr,
                                         B, Hq, Hkv, C, D, qo, cs, cs, qo, float(cfg.scale), split,
                                         CODE[dt], None)
    assert st == 0, st
    got_ref, got_new = H.download(o_ref), H.download(o_new)
    np.testing.assert_array_equal(got_new, got_ref)  # same kernels, same partition: bit-equal
    exp = oa.decode_ref(d["q"], d["k_cache"], d["v_cache"], d["lens"], sm_scale=cfg.scale, dtype=dt)
    err = H.max_abs(on.from_storage(got_new, dt), exp)
    H.report(f"noalloc {cfg.name}", err, TOL[dt])
    assert err <= TOL[dt]


def _lib_max_bytes():
    return _lib.noalloc_scratch_bytes()


def test_noalloc_scratch_size_is_the_header_limit():
    assert _lib_max_bytes() == 32 << 20  # TL_DECODE_NOALLOC_SCRATCH_BYTES


def test_noalloc_matches_decode_on_two_calls_second_smaller(shares_path):
    big = oi.scaled(oi.CONFIGS["4"], batch=16, max_ctx=4096, lo=1, hi=4095, seed=31)
    small = oi.scaled(oi.CONFIGS["2"], batch=3, max_ctx=300, lo=0, hi=299, seed=32)
    _run_both(big)
    _run_both(small)


@pytest.mark.parametrize("dtype,d_k", [("float32", 64), ("bfloat16", 128)])
def test_noalloc_dtypes(shares_path, dtype, d_k):
    cfg = oi.Config("noalloc-dt", "decode", dtype, 5, 8, 2, d_k, 33, 1 / np.sqrt(d_k),
                    max_ctx=700, lo=0, hi=699)
    _run_both(cfg)


def test_noalloc_pair_mode_default_path():
    """No override: a small 16-bit d_k 64 cache takes pair mode (one
    workgroup per (sequence, KV head) that writes the finished output, no
    partials), twice in a row, the second call smaller."""
    _run_both(oi.Config("noalloc-pair", "decode", "bfloat16", 6, 12, 4, 64, 34, 0.125,
                        max_ctx=1024, lo=0, hi=1023))
    _run_both(oi.Config("noalloc-pair2", "decode", "float16", 2, 6, 2, 64, 35, 0.125,
                        max_ctx=256, lo=0, hi=255))


def test_noalloc_refuses_problems_past_the_scratch():
    lib = gpu.runtime()
    B, Hq, Hkv, C, D, split = 64, 24, 8, 65536, 128, 64
    assert lib.tl_attention_decode_workspace_bytes(B, Hq, C, D, split) > _lib_max_bytes()
    null = None
    qo = _lib.strides(Hq * D, D)
    cs = _lib.strides(Hkv * C * D, C * D, D)
    # refused on the sizes alone: no pointer is touched, no kernel launched
    st = lib.tl_attention_decode_noalloc(null, null, null, null, 1, null, B, Hq, Hkv, C, D,
                                         qo, cs, cs, qo, 0.1, split, _lib.DTYPE_BF16, None)
    assert st == 1
