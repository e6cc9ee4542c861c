"""RoPE in place and the fused RoPE + KV-cache append: bit-exact against the
oracle in every storage dtype; untouched cache positions must stay bitwise
unchanged."""

import numpy as np
import pytest

from oracle import numerics as on
from oracle import rope as orope
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import precompute_cos_sin, rope_kv_append

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("d_k", [64, 128])
def test_rope_inplace_bitexact(dtype, d_k):
    rng = np.random.default_rng(d_k)
    seq, rows, off = 48, 48 * 5, 100
    cos, sin = precompute_cos_sin(off + seq, d_k, 5e5)
    x = on.to_storage(rng.standard_normal((rows, d_k), dtype=np.float32), dtype)
    got = H.apply_rope_cpu(x, cos, sin, seq_len=seq, position_offset=off, dtype=dtype)
    pos = np.arange(rows) % seq + off
    exp = orope.apply_rope_storage(x, cos, sin, pos, dtype)
    np.testing.assert_array_equal(got.view(np.uint8), exp.view(np.uint8))


def _make_cache(rng, B, Hkv, C, D, dtype, lens):
    kc = on.to_storage(rng.standard_normal((B, Hkv, C, D), dtype=np.float32), dtype)
    vc = on.to_storage(rng.standard_normal((B, Hkv, C, D), dtype=np.float32), dtype)
    return kc, vc


@pytest.mark.parametrize("dtype,rope", [("bfloat16", True), ("float16", False), ("float32", True), ("bfloat16", False)])
def test_decode_append_bitexact(dtype, rope):
    rng = np.random.default_rng(7)
    B, Hq, Hkv, C, D = 5, 6, 2, 40, 64
    lens = np.array([0, 1, 17, 38, 39], np.int32)
    kc, vc = _make_cache(rng, B, Hkv, C, D, dtype, lens)
    q = on.to_storage(rng.standard_normal((B, Hq, D), dtype=np.float32), dtype)
    kn = on.to_storage(rng.standard_normal((B, Hkv, D), dtype=np.float32), dtype)
    vn = on.to_storage(rng.standard_normal((B, Hkv, D), dtype=np.float32), dtype)
    cos, sin = precompute_cos_sin(C, D, 1e4) if rope else (None, None)

    q_d, kn_d, vn_d = H.upload(q, dtype), H.upload(kn, dtype), H.upload(vn, dtype)
    kc_d, vc_d = H.upload(kc, dtype), H.upload(vc, dtype)
    lens_d = gpu.to_device(lens)
    cos_d = gpu.to_device(cos) if rope else None
    sin_d = gpu.to_device(sin) if rope else None
    rope_kv_append(q_d, kn_d, vn_d, kc_d, vc_d, lens_d, cos_d, sin_d)
    q_g, kc_g, vc_g = H.download(q_d), H.download(kc_d), H.download(vc_d)

    q_e, kc_e, vc_e = q.copy(), kc.copy(), vc.copy()
    for b in range(B):
        p = int(lens[b])
        if rope:
            q_e[b] = orope.apply_rope_storage(q[b], cos, sin, p, dtype)
            kc_e[b, :, p] = orope.apply_rope_storage(kn[b], cos, sin, p, dtype)
        else:
            kc_e[b, :, p] = kn[b]
        vc_e[b, :, p] = vn[b]
    np.testing.assert_array_equal(q_g.view(np.uint8), q_e.view(np.uint8))
    np.testing.assert_array_equal(kc_g.view(np.uint8), kc_e.view(np.uint8))
    np.testing.assert_array_equal(vc_g.view(np.uint8), vc_e.view(np.uint8))


def test_prefill_fill_multi_token_bitexact():
    """n_new > 1 tokens per sequence (prefill into the cache at offset lens[b])."""
    rng = np.random.default_rng(8)
    dtype = "bfloat16"
    B, S, Hq, Hkv, C, D = 3, 33, 9, 3, 80, 64
    lens = np.array([0, 5, 47], np.int32)
    kc, vc = _make_cache(rng, B, Hkv, C, D, dtype, lens)
    q = on.to_storage(rng.standard_normal((B, S, Hq, D), dtype=np.float32), dtype)
    kn = on.to_storage(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), dtype)
    vn = on.to_storage(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), dtype)
    cos, sin = precompute_cos_sin(C, D, 1e4)
    q_d, kc_d, vc_d = H.upload(q, dtype), H.upload(kc, dtype), H.upload(vc, dtype)
    rope_kv_append(q_d, H.upload(kn, dtype), H.upload(vn, dtype), kc_d, vc_d, gpu.to_device(lens),
                   gpu.to_device(cos), gpu.to_device(sin))
    q_g, kc_g, vc_g = H.download(q_d), H.download(kc_d), H.download(vc_d)
    q_e, kc_e, vc_e = q.copy(), kc.copy(), vc.copy()
    for b in range(B):
        pos = lens[b] + np.arange(S)
        q_e[b] = orope.apply_rope_storage(q[b], cos, sin, pos[:, None], dtype)
        kc_e[b, :, pos] = orope.apply_rope_storage(kn[b], cos, sin, pos[:, None], dtype)
        vc_e[b, :, pos] = vn[b]
    np.testing.assert_array_equal(q_g, q_e)
    np.testing.assert_array_equal(kc_g, kc_e)
    np.testing.assert_array_equal(vc_g, vc_e)


def test_append_past_capacity_is_not_written():
    """A position >= max_ctx is skipped by the kernel (no out-of-bounds write)."""
    dtype = "float32"
    B, Hkv, C, D = 2, 1, 8, 64
    kc = np.zeros((B, Hkv, C, D), np.float32)
    kn = np.ones((B, Hkv, D), np.float32)
    kc_d, vc_d = H.upload(kc, dtype), H.upload(kc, dtype)
    lens = gpu.to_device(np.array([8, 3], np.int32))
    rope_kv_append(None, H.upload(kn, dtype), H.upload(kn, dtype), kc_d, vc_d, lens)
    got = H.download(kc_d)
    assert np.all(got[0] == 0)
    assert np.all(got[1, :, 3] == 1) and np.all(np.delete(got[1], 3, axis=1) == 0)


def _append_case(B, S, Hq, Hkv, C, D, dtype, lens, theta, seed):
    """Run rope_kv_append on (B, S, ., D) token rows and return GPU and oracle
    (q, k_cache, v_cache), all as storage bits."""
    rng = np.random.default_rng(seed)
    kc, vc = _make_cache(rng, B, Hkv, C, D, dtype, lens)
    q = on.to_storage(rng.standard_normal((B, S, Hq, D), dtype=np.float32), dtype)
    kn = on.to_storage(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), dtype)
    vn = on.to_storage(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), dtype)
    cos, sin = precompute_cos_sin(C, D, theta) if theta else (None, None)
    q_d, kc_d, vc_d = H.upload(q, dtype), H.upload(kc, dtype), H.upload(vc, dtype)
    rope_kv_append(q_d, H.upload(kn, dtype), H.upload(vn, dtype), kc_d, vc_d, gpu.to_device(lens),
                   gpu.to_device(cos) if theta else None, gpu.to_device(sin) if theta else None)
    got = (H.download(q_d), H.download(kc_d), H.download(vc_d))
    q_e, kc_e, vc_e = q.copy(), kc.copy(), vc.copy()
    for b in range(B):
        pos = lens[b] + np.arange(S)
        if theta:
            q_e[b] = orope.apply_rope_storage(q[b], cos, sin, pos[:, None], dtype)
            kc_e[b, :, pos] = orope.apply_rope_storage(kn[b], cos, sin, pos[:, None], dtype)
        else:
            kc_e[b, :, pos] = kn[b]
        vc_e[b, :, pos] = vn[b]
    return got, (q_e, kc_e, vc_e)


def _assert_bits(got, exp):
    for g, e, name in zip(got, exp, ("q", "k_cache", "v_cache")):
        diff = int(np.count_nonzero(g.view(np.uint8) != e.view(np.uint8)))
        assert diff == 0, f"{name}: {diff} bytes differ"


@pytest.mark.parametrize("cfg", ["5a", "3"])
def test_prompt_append_at_config_size_bitexact(cfg):
    """The S-token append GpuKVCache runs before prefill attention, at the
    config's full prompt: q rotated in place, k rotated and v copied into an
    empty cache (positions 0..S-1); every bit of q and of both caches,
    including the untouched rest of the cache, against the oracle."""
    B, S, Hq, Hkv, D, theta = {"5a": (1, 8192, 24, 8, 128, 5e5), "3": (4, 2048, 9, 3, 64, 1e4)}[cfg]
    print(f"[case] prompt append {cfg} B={B} S={S} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    got, exp = _append_case(B, S, Hq, Hkv, S + 64, D, "bfloat16", np.zeros(B, np.int32), theta, 11)
    _assert_bits(got, exp)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("B,S,Hq,Hkv,D", [
    (2, 300, 7, 1, 64),     # row groups that cut across the q / k / v kinds
    (3, 1, 10, 5, 128),     # decode-sized: one row per thread
    (1, 2000, 3, 3, 8),     # fp32: one 16-byte chunk per half row
    (2, 40, 4, 2, 12),      # half = 6: not a multiple of the 16-byte chunk, scalar kernel
    (2, 40, 4, 2, 2),       # half = 1: scalar kernel
])
def test_append_vector_and_scalar_paths_bitexact(dtype, B, S, Hq, Hkv, D):
    lens = np.array([5, 0, 9][:B], np.int32)
    got, exp = _append_case(B, S, Hq, Hkv, S + 16, D, dtype, lens, 1e4, S + D)
    _assert_bits(got, exp)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("d_k,stride", [(64, 64), (64, 72), (64, 68), (10, 10), (128, 136)])
def test_rope_inplace_vector_and_scalar_paths(dtype, d_k, stride):
    """apply_rope's kernel through the C ABI on rows with a padded stride: 16-byte
    chunks when d_k / 2 and the row stride are multiples of 16 bytes, the
    scalar kernel otherwise (d_k 10; bf16 stride 68); padding untouched."""
    from triton_llm import _lib
    rng = np.random.default_rng(d_k + stride)
    seq, rows, off = 37, 37 * 4, 3
    cos, sin = precompute_cos_sin(off + seq, d_k, 1e4)
    x = on.to_storage(rng.standard_normal((rows, stride), dtype=np.float32), dtype)
    x_d = H.upload(x, dtype)
    code = {"float32": _lib.DTYPE_F32, "bfloat16": _lib.DTYPE_BF16}[dtype]
    cos_d, sin_d = gpu.to_device(cos), gpu.to_device(sin)
    st = gpu.runtime().tl_rope_inplace(x_d.ptr, cos_d.ptr, sin_d.ptr, rows, stride, d_k, seq, off, code, None)
    assert st == 0
    got = H.download(x_d)
    exp = x.copy()
    exp[:, :d_k] = orope.apply_rope_storage(x[:, :d_k], cos, sin, np.arange(rows) % seq + off, dtype)
    np.testing.assert_array_equal(got.view(np.uint8), exp.view(np.uint8))
