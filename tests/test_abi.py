"""The C-ABI library: it loads, exports every function include/triton_llm_hip.h
declares, and its host-only entry points (workspace sizing, argument checks)
behave -- no kernel launch, no GPU needed."""

import ctypes
import os
import re

import pytest

from triton_llm import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "triton_llm_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tl_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    declared = header_functions()
    assert len(declared) >= 20
    assert sorted(_lib.SIGNATURES) == declared


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in header_functions():
        assert hasattr(lib, name), name


def test_workspace_queries():
    lib = _lib.load()
    # fp32 reads V in place; the 16-bit MFMA path stages V^T: B * Hkv * D * round_up(Sk, 128) * 2.
    assert lib.tl_attention_fwd_workspace_bytes(1, 8, 8192, 128, _lib.DTYPE_F32) == 0
    assert lib.tl_attention_fwd_workspace_bytes(1, 8, 8192, 128, _lib.DTYPE_BF16) == 8 * 128 * 8192 * 2
    # d_k 64 reads V in place: no V^T copy
    assert lib.tl_attention_fwd_workspace_bytes(2, 3, 100, 64, _lib.DTYPE_F16) == 0
    assert lib.tl_attention_fwd_workspace_bytes(2, 3, 100, 128, _lib.DTYPE_F16) == 2 * 3 * 128 * 128 * 2
    assert lib.tl_attention_fwd_workspace_bytes(1, 1, 100, 32, _lib.DTYPE_BF16) == 0  # generic path
    # Key-split region: only causal 16-bit MFMA calls with seq_k >= seq_q and few
    # tiles; otherwise the minimum.  (Planned for 256 CUs when no device is visible.)
    fwd, split = lib.tl_attention_fwd_workspace_bytes, lib.tl_attention_fwd_workspace_bytes_split
    BF, F16, F32 = _lib.DTYPE_BF16, _lib.DTYPE_F16, _lib.DTYPE_F32
    base = fwd(1, 8, 2048, 128, BF)
    ll = split(1, 24, 8, 2048, 2048, 128, 1, BF)  # Llama-3.2-3B heads, a 2048-token prompt
    assert ll > base and split(1, 24, 8, 2048, 2048, 128, 1, F16) == ll
    # after the V copy (256-aligned): 64 bytes of arrival words per split tile
    # (256-aligned), then two partial slots of 8 waves x (64 KiB / 4 + 512) bytes
    slot = 8 * (4 * 4 * 1024 + 512)
    extra = ll - base
    tiles = extra // (2 * slot)
    assert tiles > 0 and extra == ((tiles * 64 + 255) // 256) * 256 + tiles * 2 * slot
    assert split(1, 24, 8, 2048, 2048, 128, 0, BF) == base                # not causal
    assert split(1, 24, 8, 2048, 2048, 128, 1, F32) == 0                  # fp32 kernel
    assert split(1, 24, 8, 2048, 1024, 128, 1, BF) == fwd(1, 8, 1024, 128, BF)  # seq_q > seq_k
    assert split(2, 9, 3, 2048, 2048, 64, 1, BF) > 0                      # d_k 64, batch 2: split
    assert split(4, 9, 3, 2048, 2048, 64, 1, BF) > 0                      # config 3: one list, split
    assert split(32, 15, 5, 512, 512, 64, 1, BF) == 0                     # many tiles: balanced
    assert split(1, 24, 8, 8192, 8192, 128, 1, BF) == fwd(1, 8, 8192, 128, BF)  # balanced: 5a
    split = lib.tl_decode_split_size(64, 8, 16384)
    assert split % 16 == 0 and 64 <= split <= 4096
    assert lib.tl_decode_split_size(8, 12, 1024) == 64  # short caches: one-iteration floor
    ws = lib.tl_attention_decode_workspace_bytes(64, 24, 16384, 128, split)
    # A (sequence, head) spans at most ceil(max_ctx / split) + 1 workgroup shares.
    rows = 64 * 24 * ((16384 + split - 1) // split + 1)
    assert ws >= rows * (128 + 2) * 4
    assert lib.tl_attention_decode_workspace_bytes(0, 24, 16384, 128, split) == 0


def test_argument_errors_return_invalid_without_launching():
    lib = _lib.load()
    null = ctypes.c_void_p(None)
    s3 = _lib.strides(0, 0, 0)
    # NULL tensors -> TL_ERR_INVALID (1) before any HIP call.
    st = lib.tl_attention_fwd(null, null, null, null, null, 0, 1, 2, 1, 4, 4, 64,
                              s3, s3, s3, s3, 0.125, 1, _lib.DTYPE_BF16, None)
    assert st == 1
    # n_head not a multiple of n_kv_head.
    st = lib.tl_attention_decode(null, null, null, null, 0, null, null, 0, 1, 3, 2, 16, 64,
                                 s3, s3, s3, s3, 0.125, 0, _lib.DTYPE_BF16, None)
    assert st == 1
    # Empty work is a successful no-op.
    assert lib.tl_rope_inplace(null, null, null, 0, 64, 64, 1, 0, _lib.DTYPE_F32, None) == 0
    assert lib.tl_rope_inplace(null, null, null, 4, 64, 63, 1, 0, _lib.DTYPE_F32, None) == 1
    assert lib.tl_rope_kv_append(null, null, null, null, null, null, null, null, 0, 0, 1, 1, 1, 8, 64,
                                 s3, s3, s3, s3, s3, _lib.DTYPE_F32, None) == 0


def test_decode_pair_mode_needs_16_byte_row_slices():
    """A small 16-bit d_k 64 cache runs in pair mode, where 8 lanes read a
    128-byte key row with 16-byte loads: a row stride that is a multiple of
    4 elements but not of 8 is refused (TL_ERR_UNSUPPORTED) before any HIP
    call, while an aligned-pointer check would otherwise pass."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x100000)
    batch, n_head, n_kv, max_ctx, d_k = 2, 3, 1, 64, 64
    ws = lib.tl_attention_decode_workspace_bytes(batch, n_head, max_ctx, d_k, 16)
    q_st = _lib.strides(n_head * d_k, d_k, 1)
    for row in (68, 76):
        kv_st = _lib.strides(n_kv * max_ctx * row, max_ctx * row, row)
        st = lib.tl_attention_decode(fake, fake, fake, None, 1, fake, fake, ws, batch, n_head, n_kv, max_ctx,
                                     d_k, q_st, kv_st, kv_st, q_st, 0.125, 16, _lib.DTYPE_BF16, None)
        assert st == 801, st


def test_error_string():
    assert _lib.error_string(0) == "success"
    assert isinstance(_lib.error_string(1), str)


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setenv("TRITON_LLM_HIP_LIB", "/nonexistent/libtriton_llm_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback|There is no CPU fallback"):
        _lib.load()
