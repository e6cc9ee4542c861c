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

import numpy as np

from triton_llm import gpu
from ._common import launch, check_status, same_dtype, vp

# Workspace of the few-row path, kept across calls and grown on demand: every
# call runs on the library stream, so consecutive calls are ordered and may
# share it (hipMalloc per call would cost more than the product).
_shared_ws: "gpu.DeviceTensor | None" = None


def _workspace(nbytes: int):
    global _shared_ws
    if nbytes == 0:
        return None
    if _shared_ws is None or _shared_ws.nbytes < nbytes:
        _shared_ws = gpu.allocate((max(nbytes, 1 << 20),), np.uint8)
    return _shared_ws


def gemm(h_dev: "gpu.DeviceTensor", w_dev: "gpu.DeviceTensor",
         out_dev: "gpu.DeviceTensor | None" = None, workspace=None) -> "gpu.DeviceTensor":
    """GPU-resident GEMM. No sync, no host copies.  ``workspace``: optional
    device buffer of at least ``tl_gemm_workspace_bytes`` for the few-row
    (decoded token) path; a module-wide buffer is used when omitted."""
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
