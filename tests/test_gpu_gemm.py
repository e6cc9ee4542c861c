"""The model's projection GEMM against the oracle (oracle/gemm.py), on the
reference's own cases (tests/test_gemm.py of the reference: seeded shapes,
non-block-aligned shapes, empty dimensions, mismatched K) and on the
projection shapes of SmolLM2-360M and Llama-3.2-3B for one decoded token,
a few tokens (the hand-written streaming kernel, up to 8 rows) and prompts
(the hand-written MFMA kernel; the simple FMA kernel for rows that are not
16-byte aligned).  Tolerances: fp32 2e-3 max-abs (the reference's own
bar is allclose(rtol 1e-2, atol 5e-2)); 16-bit outputs within their
rounding, rtol 8e-3 + atol 1e-2.
"""

import ctypes
import time

import numpy as np
import pytest

from oracle import numerics as on
from oracle.gemm import gemm_ref
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import gemm, gemm_grouped

pytestmark = pytest.mark.gpu


def gemm_cpu(a, b, dtype="float32"):
    return H.download(gemm(H.upload(a, dtype), H.upload(b, dtype)))


@pytest.mark.parametrize("M,K,N", [(64, 128, 32), (128, 256, 128), (256, 512, 256), (65, 130, 33), (100, 200, 150)])
def test_gemm_reference_cases(M, K, N):
    np.random.seed(42)
    a = np.random.randn(M, K).astype(np.float32)
    b = np.random.randn(K, N).astype(np.float32)
    out = gemm_cpu(a, b)
    assert np.allclose(out, a @ b, rtol=1e-2, atol=5e-2)
    err = H.max_abs(out, gemm_ref(a, b))
    H.report(f"gemm {M}x{K}@{K}x{N}", err, 2e-3)
    assert err <= 2e-3


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("M", [1, 3, 8, 37])
@pytest.mark.parametrize("K,N", [(960, 960), (960, 320), (960, 2560), (2560, 960), (3072, 1024), (8192, 3072)])
def test_gemm_projection_shapes(dtype, M, K, N):
    rng = np.random.default_rng(K * 7 + N + M)
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    b = on.to_storage(rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K), dtype)
    got = on.from_storage(gemm_cpu(a, b, dtype), dtype)
    exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
    if dtype == "float32":
        err = H.max_abs(got, exp)
        H.report(f"{dtype} {M}x{K}@{K}x{N}", err, 2e-3)
        assert err <= 2e-3
    else:
        np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("K,N", [(960, 49152), (576, 49152), (1024, 65536), (1040, 65536)])
def test_gemm_lm_head_shapes(dtype, M, K, N):
    """The lm_head of a decoded token: so many column tiles that K is one
    slice (960, 576, 1024), stored straight to C with no reduce pass; 1040 just
    past one slice takes the reduce.  Also into a strided C (ldc > N)."""
    rng = np.random.default_rng(K + M)
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    b = on.to_storage(rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K), dtype)
    exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
    got = on.from_storage(gemm_cpu(a, b, dtype), dtype)
    tol = (2e-3, 0.0) if dtype == "float32" else (1e-2, 8e-3)
    np.testing.assert_allclose(got, exp, atol=tol[0], rtol=tol[1])
    # strided C through the C ABI: row stride N + 64, padding left untouched
    lib = gpu.runtime()
    code = gpu.dtype_code(H.GPU_DTYPES[dtype])
    ldc = N + 64
    pad = np.full((M, ldc), 7.0, np.float32)
    c_dev = H.upload(on.to_storage(pad, dtype), dtype)
    a_dev, b_dev = H.upload(a, dtype), H.upload(b, dtype)
    nws = lib.tl_gemm_workspace_bytes(M, N, K, code)
    ws = gpu.zeros((max(nws, 1),), np.uint8)
    assert lib.tl_gemm(a_dev.ptr, b_dev.ptr, c_dev.ptr, M, N, K, K, N, ldc, ws.ptr, nws, code, None) == 0
    c = on.from_storage(H.download(c_dev), dtype)
    np.testing.assert_allclose(c[:, :N], exp, atol=tol[0], rtol=tol[1])
    assert (c[:, N:] == 7.0).all()


@pytest.mark.parametrize("M,K,N", [(1, 130, 33), (2, 7, 40), (5, 1000, 100), (8, 4100, 260)])
def test_gemm_few_rows_odd_shapes(M, K, N):
    """Few-row products on shapes the streaming kernel handles partly (a
    ragged last K-slice or column tile) or not at all (N not a multiple of
    the 16-byte chunk: the simple FMA kernel), against the oracle."""
    rng = np.random.default_rng(M * 1000 + K + N)
    a = rng.standard_normal((M, K), dtype=np.float32)
    b = rng.standard_normal((K, N), dtype=np.float32)
    err = H.max_abs(gemm_cpu(a, b), gemm_ref(a, b))
    H.report(f"few rows {M}x{K}@{K}x{N}", err, 2e-3)
    assert err <= 2e-3


def test_gemm_edge_cases():
    # K = 0: zeros of shape (M, N) (the reference only checks the shape)
    out = gemm_cpu(np.zeros((10, 0), np.float32), np.zeros((0, 10), np.float32))
    assert out.shape == (10, 10) and not out.any()
    assert gemm_cpu(np.zeros((0, 20), np.float32), np.ones((20, 10), np.float32)).shape == (0, 10)
    assert gemm_cpu(np.ones((10, 20), np.float32), np.zeros((20, 0), np.float32)).shape == (10, 0)
    with pytest.raises(AssertionError):
        gemm(gpu.to_device(np.ones((10, 20), np.float32)), gpu.to_device(np.ones((30, 10), np.float32)))
    with pytest.raises(AssertionError):
        gemm(gpu.to_device(np.ones((10, 20), np.float32)), gpu.to_device(np.ones((20, 10), np.float32)),
             out_dev=gpu.allocate((10, 11), np.float32))
    # a given output is written in place
    a, b = np.random.randn(33, 17).astype(np.float32), np.random.randn(17, 5).astype(np.float32)
    out = gpu.allocate((33, 5), np.float32)
    assert gemm(gpu.to_device(a), gpu.to_device(b), out_dev=out) is out
    assert H.max_abs(H.download(out), gemm_ref(a, b)) <= 2e-3


def test_gemm_reference_performance_bound():
    """The reference's performance test: 512x1024 @ 1024x512 under 50 ms
    per call including the copies."""
    a = np.random.randn(512, 1024).astype(np.float32)
    b = np.random.randn(1024, 512).astype(np.float32)
    for _ in range(3):
        gemm_cpu(a, b)
    t0 = time.perf_counter()
    for _ in range(10):
        gemm_cpu(a, b)
    assert (time.perf_counter() - t0) / 10 * 1e3 < 50


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("M,K,N", [(128, 3072, 1024), (300, 960, 2560), (517, 2560, 960), (2048, 3072, 3072),
                                   (64, 8192, 3072), (9, 136, 200)])
def test_gemm_prompt_shapes_mfma(dtype, M, K, N):
    """Prompt-sized products on the matrix-core kernel: the models' projection
    shapes, ragged tiles in M and N, K not a multiple of the LDS stage."""
    print(f"[case] gemm mfma {dtype} {M}x{K}@{K}x{N}", flush=True)
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    b = on.to_storage(rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K), dtype)
    got = on.from_storage(gemm_cpu(a, b, dtype), dtype)
    exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
    if dtype == "float32":
        err = H.max_abs(got, exp)
        H.report(f"mfma {dtype} {M}x{K}@{K}x{N}", err, 2e-3)
        assert err <= 2e-3
    else:
        np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("M,K,Ns", [(1900, 136, (16456,)), (2048, 264, (16384,)), (2000, 72, (8192, 8200))])
def test_gemm_prompt_huge_tiles(dtype, M, K, Ns):
    """16-bit products with at least two 256 x 256 tiles per CU (520, 512 and
    520 such tiles here) take the eight-wave 256 x 256 tile kernel: ragged M
    and N, K tails inside a 32-k stage, and the grouped form."""
    print(f"[case] gemm huge {dtype} {M}x{K} -> {Ns}", flush=True)
    rng = np.random.default_rng(M + K + sum(Ns))
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    bs = [on.to_storage(rng.standard_normal((K, n), dtype=np.float32) / np.sqrt(K), dtype) for n in Ns]
    a_dev = H.upload(a, dtype)
    if len(Ns) == 1:
        outs = [gemm(a_dev, H.upload(bs[0], dtype))]
    else:
        outs = gemm_grouped(a_dev, [H.upload(b, dtype) for b in bs])
    for b, o in zip(bs, outs):
        got = on.from_storage(H.download(o), dtype)
        exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
        np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype,M,K,Ns", [("float32", 2048, 3072, (3072,)), ("float32", 1900, 3000, (3000,)),
                                          ("float32", 300, 3072, (3072, 1024, 1024)), ("float32", 2048, 8200, (3068,))])
def test_gemm_prompt_split_k(dtype, M, K, Ns):
    """fp32 products whose whole tiles would leave some CUs a tile more than
    others run K in slices (fp32 partials, one reduce pass): ragged M and N,
    a K tail in the last slice, the grouped form.  The workspace query
    reports the partials, so these shapes do take the split path."""
    print(f"[case] gemm split-k {dtype} {M}x{K} -> {Ns}", flush=True)
    lib = gpu.runtime()
    code = gpu.dtype_code(H.GPU_DTYPES[dtype])
    n_arr = (ctypes.c_int * len(Ns))(*Ns)
    assert lib.tl_gemm_grouped_workspace_bytes(M, K, len(Ns), n_arr, code) >= 2 * M * sum(Ns) * 4
    rng = np.random.default_rng(M + K + sum(Ns))
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    bs = [on.to_storage(rng.standard_normal((K, n), dtype=np.float32) / np.sqrt(K), dtype) for n in Ns]
    a_dev = H.upload(a, dtype)
    if len(Ns) == 1:
        outs = [gemm(a_dev, H.upload(bs[0], dtype))]
    else:
        outs = gemm_grouped(a_dev, [H.upload(b, dtype) for b in bs])
    for b, o in zip(bs, outs):
        got = on.from_storage(H.download(o), dtype)
        exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
        if dtype == "float32":
            err = H.max_abs(got, exp)
            H.report(f"split-k {dtype} {M}x{K}@{K}x{b.shape[1]}", err, 2e-3)
            assert err <= 2e-3
        else:
            np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("M,K,Ns", [(2048, 960, (960, 320, 320)), (2048, 960, (960,)), (2048, 960, (320,)),
                                   (2000, 2560, (960,)), (1999, 964, (2560, 2560))])
def test_gemm_prompt_fp32_64_row_plans(M, K, Ns):
    """fp32 prompt products with few 128-row tiles per CU (SmolLM2-360M's
    projections at a 2048-token prompt) run 64-row tiles, whole-K or with K
    split in 2-4: the grouped q/k/v, o / down with their splits, ragged M and
    a K tail inside a 16-k stage."""
    print(f"[case] gemm fp32 64-row {M}x{K} -> {Ns}", flush=True)
    rng = np.random.default_rng(M + 5 * K + sum(Ns))
    a = rng.standard_normal((M, K), dtype=np.float32)
    bs = [rng.standard_normal((K, n), dtype=np.float32) / np.float32(np.sqrt(K)) for n in Ns]
    a_dev = gpu.to_device(a)
    if len(Ns) == 1:
        outs = [gemm(a_dev, gpu.to_device(bs[0]))]
    else:
        outs = gemm_grouped(a_dev, [gpu.to_device(b) for b in bs])
    for b, o in zip(bs, outs):
        err = H.max_abs(H.download(o), gemm_ref(a, b))
        H.report(f"fp32 64-row {M}x{K}@{K}x{b.shape[1]}", err, 2e-3)
        assert err <= 2e-3


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("M,K,Ns", [(9, 3072, (3072,)), (33, 3072, (3072, 1024, 1024)), (64, 8192, (3072,)),
                                    (130, 3072, (3072, 1024)), (17, 3000, (3000,))])
def test_gemm_few_rows_split_k(dtype, M, K, Ns):
    """A batch of decoded tokens (9 to a few hundred rows): the MFMA product
    has only a few dozen tiles of C, so K is split until about one item per
    CU runs, two for fp32 (fp32 partials in the workspace, one reduce pass rounding to the
    output type); ragged M, a K tail, slices past K, the grouped form.  The
    workspace query reports the partials, so these shapes take the split path."""
    print(f"[case] gemm few-rows split-k {dtype} {M}x{K} -> {Ns}", flush=True)
    lib = gpu.runtime()
    code = gpu.dtype_code(H.GPU_DTYPES[dtype])
    n_arr = (ctypes.c_int * len(Ns))(*Ns)
    assert lib.tl_gemm_grouped_workspace_bytes(M, K, len(Ns), n_arr, code) >= 2 * M * sum(Ns) * 4
    rng = np.random.default_rng(M + K + sum(Ns))
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    bs = [on.to_storage(rng.standard_normal((K, n), dtype=np.float32) / np.sqrt(K), dtype) for n in Ns]
    a_dev = H.upload(a, dtype)
    if len(Ns) == 1:
        outs = [gemm(a_dev, H.upload(bs[0], dtype))]
    else:
        outs = gemm_grouped(a_dev, [H.upload(b, dtype) for b in bs])
    for b, o in zip(bs, outs):
        got = on.from_storage(H.download(o), dtype)
        exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
        if dtype == "float32":
            err = H.max_abs(got, exp)
            H.report(f"few-rows split-k {dtype} {M}x{K}@{K}x{b.shape[1]}", err, 2e-3)
            assert err <= 2e-3
        else:
            np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("M", [9, 63, 64, 65])
def test_gemm_row_tile_boundaries(dtype, M):
    """Around the switch from 64-row to 128-row tiles (64 / 65 rows), with a K
    tail in every dtype (1000 = 15 stages of 64 k + 40, or 62 of 16 + 8) and
    column counts that are not whole tiles, grouped and single."""
    print(f"[case] gemm row-tile boundary {dtype} M={M}", flush=True)
    K, Ns = 1000, (1000, 200)
    rng = np.random.default_rng(M)
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    bs = [on.to_storage(rng.standard_normal((K, n), dtype=np.float32) / np.sqrt(K), dtype) for n in Ns]
    a_dev = H.upload(a, dtype)
    outs = gemm_grouped(a_dev, [H.upload(b, dtype) for b in bs]) + [gemm(a_dev, H.upload(bs[1], dtype))]
    for b, o in zip(bs + [bs[1]], outs):
        got = on.from_storage(H.download(o), dtype)
        exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
        if dtype == "float32":
            err = H.max_abs(got, exp)
            H.report(f"row-tile boundary {dtype} {M}x{K}@{K}x{b.shape[1]}", err, 2e-3)
            assert err <= 2e-3
        else:
            assert np.all(np.isfinite(got))
            np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype,M", [("float32", 2048), ("float32", 40), ("bfloat16", 64)])
def test_gemm_prompt_split_k_without_workspace_runs_whole(dtype, M):
    """The C ABI with no workspace for a shape its plan would split: the
    product runs with whole-K tiles instead (no failure, same result)."""
    lib = gpu.runtime()
    K, N = 3072, 3072
    code = gpu.dtype_code(H.GPU_DTYPES[dtype])
    assert lib.tl_gemm_workspace_bytes(M, N, K, code) > 0
    rng = np.random.default_rng(5 + M)
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    b = on.to_storage(rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K), dtype)
    a_dev, b_dev = H.upload(a, dtype), H.upload(b, dtype)
    c_dev = gpu.allocate((M, N), H.GPU_DTYPES[dtype])
    assert lib.tl_gemm(a_dev.ptr, b_dev.ptr, c_dev.ptr, M, N, K, K, N, N, None, 0, code, None) == 0
    got = on.from_storage(H.download(c_dev), dtype)
    exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
    if dtype == "float32":
        err = H.max_abs(got, exp)
        H.report(f"split-k shape {M} rows, no workspace", err, 2e-3)
        assert err <= 2e-3
    else:
        np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("dtype,K", [("bfloat16", 136), ("float16", 72), ("float32", 132), ("float32", 20)])
def test_gemm_strided_operands_keep_padding_out(dtype, K):
    """Row strides past the logical sizes, with NaN in every padding element:
    lda = K + 8 (the last LDS stage reads past K into the padding, which must
    not reach C), ldb = N + 8, ldc = N + 4 (padding of C left untouched)."""
    M, N = 150, 200
    print(f"[case] gemm strided {dtype} K={K}", flush=True)
    rng = np.random.default_rng(K)
    a = rng.standard_normal((M, K), dtype=np.float32)
    b = rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)
    a_pad = np.full((M, K + 8), np.nan, np.float32)
    a_pad[:, :K] = a
    b_pad = np.full((K, N + 8), np.nan, np.float32)
    b_pad[:, :N] = b
    a_s, b_s = on.to_storage(a_pad, dtype), on.to_storage(b_pad, dtype)
    ldc = N + 4
    c_dev = H.upload(on.to_storage(np.full((M, ldc), 3.0, np.float32), dtype), dtype)
    lib = gpu.runtime()
    code = gpu.dtype_code(H.GPU_DTYPES[dtype])
    st = lib.tl_gemm(H.upload(a_s, dtype).ptr, H.upload(b_s, dtype).ptr, c_dev.ptr, M, N, K, K + 8, N + 8, ldc,
                     None, 0, code, None)
    assert st == 0
    c = on.from_storage(H.download(c_dev), dtype)
    exp = gemm_ref(on.from_storage(a_s, dtype)[:, :K], on.from_storage(b_s, dtype)[:, :N])
    if dtype == "float32":
        err = H.max_abs(c[:, :N], exp)
        H.report(f"strided {dtype} K={K}", err, 2e-3)
        assert err <= 2e-3
    else:  # output rounding of 16-bit C; NaN anywhere fails
        np.testing.assert_allclose(c[:, :N], exp, rtol=8e-3, atol=1e-2)
    assert (c[:, N:] == 3.0).all()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("M", [1, 3, 8, 37, 300])
@pytest.mark.parametrize("K,Ns", [(3072, (3072, 1024, 1024)), (960, (2560, 2560)), (576, (576, 192, 192)),
                                  (100, (40, 0, 24))])
def test_gemm_grouped_matches_each_product(dtype, M, K, Ns):
    """q/k/v (and gate/up) in one launch: every output against the oracle.
    Few-row products share one K-slice plan and one reduce; prompts share one
    MFMA tile space; a zero-width group is skipped; (100, (40, 0, 24)) has
    rows that are not 16-byte aligned (the simple kernel, one grid layer per
    group)."""
    print(f"[case] gemm_grouped {dtype} M={M} K={K} N={Ns}", flush=True)
    rng = np.random.default_rng(M + K + sum(Ns))
    a = on.to_storage(rng.standard_normal((M, K), dtype=np.float32), dtype)
    bs = [on.to_storage(rng.standard_normal((K, n), dtype=np.float32) / np.sqrt(K), dtype) for n in Ns]
    outs = gemm_grouped(H.upload(a, dtype), [H.upload(b, dtype) for b in bs])
    for b, o in zip(bs, outs):
        got = on.from_storage(H.download(o), dtype)
        exp = gemm_ref(on.from_storage(a, dtype), on.from_storage(b, dtype))
        assert got.shape == exp.shape
        if dtype == "float32":
            err = H.max_abs(got, exp)
            H.report(f"grouped {dtype} {M}x{K}@{K}x{b.shape[1]}", err, 2e-3)
            assert err <= 2e-3
        else:
            np.testing.assert_allclose(got, exp, rtol=8e-3, atol=1e-2)


def test_gemm_few_rows_mixed_shapes_share_workspace():
    """Few-row products of different tilings, one after another and repeated,
    through the one module-wide workspace: each comes out right whatever ran
    before it."""
    rng = np.random.default_rng(5)
    shapes = [(1, 3072, 5120), (4, 8192, 3072), (1, 3072, 5120), (2, 3072, 16384), (8, 1000, 100), (1, 8192, 3072)]
    cases = []
    for M, K, N in shapes:
        a = rng.standard_normal((M, K), dtype=np.float32)
        b = (rng.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
        cases.append((gpu.to_device(a), gpu.to_device(b), gemm_ref(a, b)))
    for rep in range(3):
        outs = [gemm(a, b) for a, b, _ in cases]
        for (M, K, N), out, (_, _, exp) in zip(shapes, outs, cases):
            err = H.max_abs(out.to_numpy(), exp)
            H.report(f"mixed shapes rep {rep} {M}x{K}@{K}x{N}", err, 2e-3)
            assert err <= 2e-3


def test_gemm_zero_k_strided_output_keeps_padding():
    """K = 0 writes zeros into the (M, N) view only: a strided C (ldc > N)
    keeps its padding columns, through the C ABI, for the single and the
    grouped entry points."""
    lib = gpu.runtime()
    M, N, ldc = 5, 40, 56
    print("[case] gemm K=0 strided", flush=True)
    c_dev = gpu.to_device(np.full((M, ldc), 7.0, np.float32))
    a_dev = gpu.allocate((M, 1), np.float32)
    b_dev = gpu.allocate((1, N), np.float32)
    assert lib.tl_gemm(a_dev.ptr, b_dev.ptr, c_dev.ptr, M, N, 0, 1, N, ldc, None, 0, 0, None) == 0
    c = c_dev.to_numpy()
    assert not c[:, :N].any() and (c[:, N:] == 7.0).all()
    c2 = gpu.to_device(np.full((M, ldc), 7.0, np.float32))
    ns = (ctypes.c_int * 2)(N, 8)
    bs = (ctypes.c_void_p * 2)(b_dev.ptr.value, b_dev.ptr.value)
    cs = (ctypes.c_void_p * 2)(c_dev.ptr.value, c2.ptr.value)
    lds_b = (ctypes.c_int64 * 2)(N, 8)
    lds_c = (ctypes.c_int64 * 2)(ldc, ldc)
    c_dev.from_numpy(np.full((M, ldc), 7.0, np.float32))
    assert lib.tl_gemm_grouped(a_dev.ptr, M, 0, 1, 2, bs, cs, ns, lds_b, lds_c, None, 0, 0, None) == 0
    c, c2h = c_dev.to_numpy(), c2.to_numpy()
    assert not c[:, :N].any() and (c[:, N:] == 7.0).all()
    assert not c2h[:, :8].any() and (c2h[:, 8:] == 7.0).all()
