"""Next-token sampling on the HIP library.

Replaces the reference's host-side ``_sample`` (smollm2_triton/model.py:566-584,
gpt2_triton/model.py:424-438), which needs the logits row downloaded first:

* :func:`sample` -- ``sample(logits_dev, temperature, top_k, row=-1) -> int``,
  the reference's method on a device logits tensor ``(..., vocab)``; ``row``
  picks the flattened row (``-1``: the last, i.e. ``logits[0, -1, :]`` of a
  ``(1, seq, vocab)`` prompt).  Greedy argmax for ``temperature <= 1e-6``;
  otherwise one uniform draw from NumPy's global stream -- the draw
  ``np.random.choice`` itself would take -- so ``np.random.seed(s)`` makes
  runs repeatable as the reference's server does (scripts/serve_model.py:391).
  The draw goes to the device as a kernel argument (``tl_sample_row``).
  ``top_k <= 0`` keeps every entry, ``top_k`` beyond the vocabulary is capped.
* :func:`sample_rows` -- one token per row of ``(rows, vocab)`` logits into a
  device int32 tensor, with caller-supplied draws or draws from NumPy's
  stream; no synchronisation.

Where the reference's ``np.random.choice`` raises ``ValueError`` (NaN in the
probabilities: a NaN or +inf logit, or every logit -inf) :func:`sample`
raises the same; :func:`sample_rows` writes -1 for such rows.
Ties with the k-th largest logit are all kept by the top_k filter
(``argpartition`` keeps exactly k of them, which ones being unspecified).
"""

from __future__ import annotations

import ctypes

import numpy as np

from triton_llm import gpu
from ._common import check_status, vp

__all__ = ["sample", "sample_rows", "max_vocab"]

_GREEDY_T = 1e-6  # model.py:569


class _Buffers:
    """Device buffers reused across calls (copies and kernels are ordered on
    the library stream, so reuse cannot overtake a pending kernel): the token
    of :func:`sample` and the sampler's workspace."""

    def __init__(self):
        self.tok = None
        self.ws = None

    def token(self):
        if self.tok is None:
            self.tok = gpu.allocate((1,), np.int32)
        return self.tok

    def workspace(self, rows: int, vocab: int):
        need = int(gpu.runtime().tl_sample_workspace_bytes(rows, vocab))
        if need == 0:
            raise ValueError(f"sampling {rows} rows of vocab {vocab} is not supported "
                             f"(rows <= 65535, vocab <= {max_vocab()})")
        if self.ws is None or self.ws.nbytes < need:
            self.ws = gpu.allocate((need,), np.uint8)
        return self.ws


_bufs = _Buffers()


def max_vocab() -> int:
    """Largest vocabulary the device sampler accepts."""
    return int(gpu.runtime().tl_sample_max_vocab())


def _flat_rows(logits_dev) -> tuple[int, int]:
    if len(logits_dev.shape) < 1 or logits_dev.shape[-1] <= 0:
        raise ValueError(f"logits must be (..., vocab) with vocab > 0, got {logits_dev.shape}")
    vocab = int(logits_dev.shape[-1])
    return int(np.prod(logits_dev.shape[:-1], dtype=np.int64)), vocab


def _launch(ptr: int, rows: int, vocab: int, row_stride: int, itemsize_dtype, temperature: float, top_k: int,
            u_dev, tok_dev) -> None:
    t = float(np.float32(temperature)) if temperature > _GREEDY_T else 0.0
    k = int(top_k) if top_k > 0 else 0
    k = min(k, vocab)
    ws = _bufs.workspace(rows, vocab)
    status = gpu.runtime().tl_sample(ctypes.c_void_p(ptr), rows, vocab, row_stride, t, k,
                                     vp(u_dev) if t > 0.0 else ctypes.c_void_p(None), vp(tok_dev),
                                     vp(ws), ws.nbytes, gpu.dtype_code(itemsize_dtype), None)
    check_status(status, "sample")


def sample(logits_dev: "gpu.DeviceTensor", temperature: float, top_k: int, row: int = -1) -> int:
    """Sample one token from row ``row`` of device logits ``(..., vocab)``."""
    rows, vocab = _flat_rows(logits_dev)
    if rows == 0:
        raise ValueError("logits hold no rows")
    if not -rows <= row < rows:
        raise IndexError(f"row {row} out of range for {rows} rows")
    row %= rows
    tok_dev = _bufs.token()
    greedy = not temperature > _GREEDY_T
    u = 0.0 if greedy else float(np.random.random_sample())  # greedy consumes no draw
    t = 0.0 if greedy else float(np.float32(temperature))
    k = min(int(top_k), vocab) if top_k > 0 else 0
    ws = _bufs.workspace(1, vocab)
    ptr = logits_dev.data_ptr() + row * vocab * logits_dev.dtype.itemsize
    check_status(gpu.runtime().tl_sample_row(ctypes.c_void_p(ptr), vocab, t, k, u, vp(tok_dev), vp(ws), ws.nbytes,
                                             gpu.dtype_code(logits_dev.dtype), None), "sample")
    tok = int(tok_dev.to_numpy()[0])
    if tok < 0:
        raise ValueError("probabilities contain NaN")
    return tok


def sample_rows(logits_dev: "gpu.DeviceTensor", temperature: float, top_k: int, uniforms=None,
                out_dev: "gpu.DeviceTensor | None" = None) -> "gpu.DeviceTensor":
    """One token per row of ``(rows, vocab)`` logits, as int32 on the device.

    ``uniforms``: None (draw ``rows`` values from NumPy's global stream), a
    host array of ``rows`` floats in [0, 1), or a float64 DeviceTensor of
    ``rows`` entries.  Rows whose probabilities are undefined get -1.
    """
    rows, vocab = _flat_rows(logits_dev)
    if out_dev is None:
        out_dev = gpu.allocate((rows,), np.int32)
    elif out_dev.dtype != np.int32 or out_dev.size != rows:
        raise ValueError(f"out_dev must be int32 with {rows} entries, got {out_dev.dtype} {out_dev.shape}")
    if rows == 0:
        return out_dev
    greedy = not temperature > _GREEDY_T
    u_dev = None
    if not greedy:
        if isinstance(uniforms, gpu.DeviceTensor):
            if uniforms.dtype != np.float64 or uniforms.size != rows:
                raise ValueError(f"uniforms must be float64 with {rows} entries")
            u_dev = uniforms
        else:
            u = np.random.random_sample(rows) if uniforms is None else np.asarray(uniforms, np.float64).ravel()
            if u.size != rows:
                raise ValueError(f"uniforms must hold {rows} values, got {u.size}")
            u_dev = gpu.to_device(u)
    _launch(logits_dev.data_ptr(), rows, vocab, vocab, logits_dev.dtype, temperature, top_k, u_dev, out_dev)
    return out_dev
