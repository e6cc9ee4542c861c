"""Host-only calls into the C ABI: workspace sizing, split sizes, error
strings and argument errors of every compute entry point (NULL or fake
pointers, shapes and strides each check refuses, unknown dtypes).  None of
them reaches a HIP call.  Prints one JSON list of the results.

Run by tests/test_asan_host.py twice: against the AddressSanitizer build of
the library's host code (ASan runtime preloaded) and against the product
library, whose results must agree.  Not collected by pytest itself."""

import ctypes
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "triton-llm_amd"))

from triton_llm import _lib  # noqa: E402

lib = _lib.load()
null = ctypes.c_void_p(None)
fake = ctypes.c_void_p(0x100000)  # never dereferenced: every call below is refused first
BF16, F16, F32, BAD = _lib.DTYPE_BF16, _lib.DTYPE_F16, _lib.DTYPE_F32, 99
out = []


def rec(name, value):
    out.append([name, value if not isinstance(value, bytes) else value.decode()])


def s3(a, b, c):
    return _lib.strides(a, b, c)


# ---- workspace sizing and split sizes (pure host arithmetic) ----
for args in [(1, 8, 8192, 128, BF16), (1, 8, 8192, 128, F32), (2, 3, 100, 64, F16), (2, 3, 100, 128, F16),
             (1, 1, 100, 32, BF16), (0, 8, 8192, 128, BF16), (1, 8, 0, 128, BF16), (64, 8, 1 << 20, 128, BF16),
             (1, 8, 8192, 4096, BF16), (1, 8, 8192, 8192, BF16), (-1, 8, 16, 128, BF16), (1, 8, 16, 128, BAD)]:
    rec(f"fwd_ws{args}", lib.tl_attention_fwd_workspace_bytes(*args))
for args in [(64, 8, 16384), (8, 12, 1024), (1, 1, 1), (0, 8, 16384), (4096, 64, 1 << 20), (-3, 8, 100)]:
    rec(f"split{args}", lib.tl_decode_split_size(*args))
for args in [(64, 24, 16384, 128, 256), (8, 12, 1024, 64, 64), (0, 24, 16384, 128, 256), (1, 1, 1, 64, 16),
             (32, 15, 8192, 64, 0), (32, 15, 8192, 64, -16), (4096, 64, 1 << 20, 128, 16)]:
    rec(f"dec_ws{args}", lib.tl_attention_decode_workspace_bytes(*args))
for args in [(1, 3072, 3072, BF16), (64, 8192, 3072, BF16), (2048, 3072, 8192, F32), (0, 1, 1, F32),
             (1, 1, 1 << 30, F32), (-1, 4, 4, BF16), (4, 4, 4, BAD)]:
    rec(f"gemm_ws{args}", lib.tl_gemm_workspace_bytes(*args))
for count, ns in [(3, [3072, 1024, 1024]), (2, [8192, 8192]), (4, [16, 32, 48, 64]), (0, [1]), (5, [1] * 5),
                  (2, [0, 16]), (2, [-8, 16])]:
    arr = (ctypes.c_int * len(ns))(*ns)
    for m, k in [(1, 3072), (64, 3072), (2048, 3072)]:
        rec(f"grouped_ws{(m, k, count, ns)}", lib.tl_gemm_grouped_workspace_bytes(m, k, count, arr, BF16))
for args in [(1, 49152), (64, 128256), (0, 10), (3, 0), (1, 1 << 24), (-2, 100)]:
    rec(f"sample_ws{args}", lib.tl_sample_workspace_bytes(*args))
rec("sample_max_vocab", lib.tl_sample_max_vocab())
for code in [0, 1, 2, 3, 100, 801, -1, 123456]:
    rec(f"error_string({code})", lib.tl_error_string(code))

# ---- argument errors: refused before any HIP call ----
z = s3(0, 0, 0)
rec("fwd null", lib.tl_attention_fwd(null, null, null, null, null, 0, 1, 2, 1, 4, 4, 64, z, z, z, z, 0.125, 1,
                                     BF16, None))
good = s3(4 * 8 * 64, 8 * 64, 64)
for name, (b, hq, hkv, sq, sk, d, dt) in {
        "fwd group": (1, 3, 2, 8, 8, 64, BF16), "fwd d_k 0": (1, 2, 1, 8, 8, 0, BF16),
        "fwd d_k 8192": (1, 2, 1, 8, 8, 8192, BF16),
        "fwd dtype": (1, 2, 1, 8, 8, 64, BAD), "fwd neg batch": (-1, 2, 1, 8, 8, 64, BF16),
        "fwd seq_k 0": (1, 2, 1, 8, 0, 64, BF16)}.items():
    rec(name, lib.tl_attention_fwd(fake, fake, fake, fake, None, 0, b, hq, hkv, sq, sk, d, good, good, good, good,
                                   0.125, 1, dt, None))
rec("fwd missing workspace", lib.tl_attention_fwd(fake, fake, fake, fake, None, 0, 1, 2, 1, 8, 8, 128,
                                                  s3(8 * 128 * 2, 8 * 128, 128), s3(8 * 128, 8 * 128, 128),
                                                  s3(8 * 128, 8 * 128, 128), s3(8 * 128 * 2, 8 * 128, 128),
                                                  0.125, 1, BF16, None))
rec("dec group", lib.tl_attention_decode(null, null, null, null, 0, null, null, 0, 1, 3, 2, 16, 64, z, z, z, z,
                                         0.125, 0, BF16, None))
q_st = s3(3 * 64, 64, 1)
for row in (68, 76):
    kv = s3(64 * row, 64 * row, row)
    ws = lib.tl_attention_decode_workspace_bytes(2, 3, 64, 64, 16)
    rec(f"dec pair row {row}", lib.tl_attention_decode(fake, fake, fake, None, 1, fake, fake, ws, 2, 3, 1, 64, 64,
                                                        q_st, kv, kv, q_st, 0.125, 16, BF16, None))
kv = s3(64 * 64, 64 * 64, 64)
rec("dec small workspace", lib.tl_attention_decode(fake, fake, fake, None, 1, fake, fake, 16, 2, 3, 1, 64, 64,
                                                    q_st, kv, kv, q_st, 0.125, 16, BF16, None))
rec("dec split 5", lib.tl_attention_decode(fake, fake, fake, None, 1, fake, fake, 1 << 30, 2, 3, 1, 64, 64,
                                           q_st, kv, kv, q_st, 0.125, 5, BF16, None))
rec("dec dtype", lib.tl_attention_decode(fake, fake, fake, None, 1, fake, fake, 1 << 30, 2, 3, 1, 64, 64,
                                         q_st, kv, kv, q_st, 0.125, 16, BAD, None))
rec("dec noalloc group", lib.tl_attention_decode_noalloc(null, null, null, null, 0, null, 1, 3, 2, 16, 64, z, z, z,
                                                         z, 0.125, 0, BF16, None))
rec("dec noalloc too big", lib.tl_attention_decode_noalloc(fake, fake, fake, None, 1, fake, 4096, 64, 8, 1 << 20,
                                                           128, s3(64 * 128, 128, 1), s3(8 << 27, 1 << 27, 128),
                                                           s3(8 << 27, 1 << 27, 128), s3(64 * 128, 128, 1), 0.125,
                                                           256, BF16, None))
kvn = s3(2 * 64, 64, 1)
rec("dec_append null k_new", lib.tl_attention_decode_append(fake, null, fake, fake, fake, fake, None, None, 0, fake,
                                                            fake, 1 << 30, 2, 3, 1, 64, 64, q_st, kvn, kvn, kv, kv,
                                                            q_st, 0.125, 16, BF16, None))
rec("dec_append null lens", lib.tl_attention_decode_append(fake, fake, fake, fake, fake, null, None, None, 0, fake,
                                                           fake, 1 << 30, 2, 3, 1, 64, 64, q_st, kvn, kvn, kv, kv,
                                                           q_st, 0.125, 16, BF16, None))
rec("dec_append cos only", lib.tl_attention_decode_append(fake, fake, fake, fake, fake, fake, fake, None, 8, fake,
                                                          fake, 1 << 30, 2, 3, 1, 64, 64, q_st, kvn, kvn, kv, kv,
                                                          q_st, 0.125, 16, BF16, None))
rec("dec_append group", lib.tl_attention_decode_append(fake, fake, fake, fake, fake, fake, None, None, 0, fake,
                                                       fake, 1 << 30, 2, 3, 2, 64, 64, q_st, kvn, kvn, kv, kv,
                                                       q_st, 0.125, 16, BF16, None))
rec("dec_append empty", lib.tl_attention_decode_append(null, null, null, null, null, null, None, None, 0, null,
                                                       null, 0, 0, 3, 1, 64, 64, z, z, z, z, z, z, 0.125, 16, BF16,
                                                       None))
rec("rope empty", lib.tl_rope_inplace(null, null, null, 0, 64, 64, 1, 0, F32, None))
rec("rope odd d", lib.tl_rope_inplace(null, null, null, 4, 64, 63, 1, 0, F32, None))
rec("rope null", lib.tl_rope_inplace(null, null, null, 4, 64, 64, 1, 0, F32, None))
rec("rope dtype", lib.tl_rope_inplace(fake, fake, fake, 4, 64, 64, 1, 0, BAD, None))
rec("append empty", lib.tl_rope_kv_append(null, null, null, null, null, null, null, null, 0, 0, 1, 1, 1, 8, 64,
                                          z, z, z, z, z, F32, None))
rec("append null", lib.tl_rope_kv_append(null, null, null, null, null, null, null, null, 1, 1, 1, 1, 1, 8, 64,
                                         z, z, z, z, z, F32, None))
rec("gemm null", lib.tl_gemm(null, null, null, 4, 4, 4, 4, 4, 4, None, 0, F32, None))
rec("gemm lda", lib.tl_gemm(fake, fake, fake, 4, 4, 8, 4, 4, 4, None, 0, F32, None))
rec("gemm dtype", lib.tl_gemm(fake, fake, fake, 4, 4, 4, 4, 4, 4, None, 0, BAD, None))
rec("gemm empty", lib.tl_gemm(null, null, null, 0, 4, 4, 4, 4, 4, None, 0, F32, None))
ns = (ctypes.c_int * 3)(16, 16, 16)
ptrs = (ctypes.c_void_p * 3)(0x100000, 0x100000, 0x100000)
lds = (ctypes.c_int64 * 3)(16, 16, 16)
rec("grouped count 5", lib.tl_gemm_grouped(fake, 4, 16, 16, 5, ptrs, ptrs, ns, lds, lds, None, 0, F32, None))
rec("grouped null b", lib.tl_gemm_grouped(fake, 4, 16, 16, 3, None, ptrs, ns, lds, lds, None, 0, F32, None))
rec("grouped dtype", lib.tl_gemm_grouped(fake, 4, 16, 16, 3, ptrs, ptrs, ns, lds, lds, None, 0, BAD, None))
rec("rms null", lib.tl_rms_norm(null, null, null, 4, 64, 1e-5, F32, None))
rec("rms dtype", lib.tl_rms_norm(fake, fake, fake, 4, 64, 1e-5, BAD, None))
rec("add_rms null", lib.tl_add_rms_norm(null, null, null, null, null, 4, 64, 1e-5, F32, None))
rec("swiglu null", lib.tl_swiglu(null, null, null, 64, F32, None))
rec("add null", lib.tl_add(null, null, null, 64, F32, None))
rec("add dtype", lib.tl_add(fake, fake, fake, 64, BAD, None))
u = (ctypes.c_double * 2)(0.5, 0.5)
tok = (ctypes.c_int32 * 2)()
rec("sample null", lib.tl_sample(null, 2, 100, 100, 1.0, 0, u, tok, null, 0, F32, None))
rec("sample vocab", lib.tl_sample(fake, 2, lib.tl_sample_max_vocab() + 1, 1 << 30, 1.0, 0, u, tok, fake, 1 << 30,
                                  F32, None))
rec("sample stride", lib.tl_sample(fake, 2, 100, 50, 1.0, 0, u, tok, fake, 1 << 30, F32, None))
rec("sample small ws", lib.tl_sample(fake, 2, 100, 100, 1.0, 0, u, tok, fake, 8, F32, None))
rec("sample dtype", lib.tl_sample(fake, 2, 100, 100, 1.0, 0, u, tok, fake, 1 << 30, BAD, None))
rec("sample_row null", lib.tl_sample_row(null, 100, 1.0, 0, 0.5, tok, null, 0, F32, None))
rec("sample_row vocab 0", lib.tl_sample_row(fake, 0, 1.0, 0, 0.5, tok, fake, 1 << 30, F32, None))

if os.environ.get("LD_PRELOAD"):
    # the sanitizer is really in this process
    rec("asan_runtime", hasattr(ctypes.CDLL(None), "__asan_init"))
print(json.dumps(out))
