"""Dense projection GEMM (the model's ``gemm``) on the HIP library.

``gemm(h_dev, w_dev, out_dev=None)`` keeps the reference's signature, shape
asserts and empty-dimension handling (triton_llm/kernels/gemm.py:53-108): h
``(M, K)``, w ``(K, N)``, out ``(M, N)``, all row-major on the GPU, no sync.
The reference is fp32 only; float16 and bfloat16 are accepted as well, with
fp32 accumulation.  ``K == 0`` gives zeros (the reference leaves the fresh
output unwritten).  ``tl_gemm`` streams the weights with a hand-written
kernel for up to 8 rows (a decoded token) and runs larger products on the
matrix cores with a hand-written MFMA kernel.
"""

from __future__ import annotations

import ctypes

from triton_llm import gpu
from ._common import launch, same_dtype, shared_workspace, vp

# Workspace of the few-row path, kept across calls and grown on demand: every
# call runs on the library stream, so consecutive calls are ordered and may
# share it (hipMalloc per call would cost more than the product).
def _workspace(nbytes: int):
    return shared_workspace("gemm", nbytes)


def gemm(h_dev: "gpu.DeviceTensor", w_dev: "gpu.DeviceTensor",
         out_dev: "gpu.DeviceTensor | None" = None, workspace=None) -> "gpu.DeviceTensor":
    """GPU-resident GEMM. No sync, no host copies.  ``workspace``: optional
    device buffer of at least ``tl_gemm_workspace_bytes`` (the few-row path's
    K-slice partials, or a split-K fp32 prompt's partials); a module-wide
    buffer is used when omitted."""
    M, K = h_dev.shape
    K2, N = w_dev.shape
    assert K == K2, f"gemm shape mismatch: ({M},{K}) x ({K2},{N})"
    if out_dev is not None:
        assert out_dev.shape == (M, N), f"out_dev shape mismatch: expected ({M},{N}), got {out_dev.shape}"
    code = same_dtype(h_dev, w_dev) if out_dev is None else same_dtype(h_dev, w_dev, out_dev)
    if out_dev is None:
        out_dev = gpu.allocate((M, N), h_dev.dtype)
    if M == 0 or N == 0:
        return out_dev
    lib = gpu.runtime()
    need = lib.tl_gemm_workspace_bytes(M, N, K, code)
    if workspace is not None and need and workspace.nbytes < need:
        raise ValueError(f"workspace holds {workspace.nbytes} bytes, {need} required")
    ws = workspace if workspace is not None else _workspace(need)
    launch(lib.tl_gemm, vp(h_dev), vp(w_dev), vp(out_dev), M, N, K, K, N, N, vp(ws),
           ws.nbytes if ws is not None else 0, code, None, what="gemm")
    return out_dev


def gemm_grouped(h_dev: "gpu.DeviceTensor", w_devs, out_devs=None, workspace=None):
    """``[h @ w for w in w_devs]`` in one launch (up to four weights sharing
    ``h``): the q/k/v or gate/up projections of a layer.  Each ``w`` is
    ``(K, N_g)``; returns the list of ``(M, N_g)`` outputs (``out_devs`` if
    given).  Same checks and semantics as :func:`gemm` per product.  No sync."""
    M, K = h_dev.shape
    w_devs = list(w_devs)
    if not 1 <= len(w_devs) <= 4:
        raise ValueError(f"gemm_grouped takes 1 to 4 weights, got {len(w_devs)}")
    for w in w_devs:
        assert w.shape[0] == K, f"gemm shape mismatch: ({M},{K}) x {w.shape}"
    if out_devs is None:
        out_devs = [gpu.allocate((M, w.shape[1]), h_dev.dtype) for w in w_devs]
    else:
        out_devs = list(out_devs)
        for w, o in zip(w_devs, out_devs, strict=True):
            assert o.shape == (M, w.shape[1]), f"out_dev shape mismatch: expected ({M},{w.shape[1]}), got {o.shape}"
    code = same_dtype(h_dev, *w_devs, *out_devs)
    if M == 0:
        return out_devs
    n = len(w_devs)
    ns = (ctypes.c_int * n)(*[int(w.shape[1]) for w in w_devs])
    lib = gpu.runtime()
    need = lib.tl_gemm_grouped_workspace_bytes(M, K, n, ns, code)
    if workspace is not None and need and workspace.nbytes < need:
        raise ValueError(f"workspace holds {workspace.nbytes} bytes, {need} required")
    ws = workspace if workspace is not None else _workspace(need)
    bs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in w_devs])
    cs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in out_devs])
    lds = (ctypes.c_int64 * n)(*[int(w.shape[1]) for w in w_devs])
    launch(lib.tl_gemm_grouped, vp(h_dev), M, K, K, n, bs, cs, ns, lds, lds, vp(ws),
           ws.nbytes if ws is not None else 0, code, None, what="gemm_grouped")
    return out_devs
