"""Shared host-side helpers for the kernel wrappers (no GPU work on import)."""

from __future__ import annotations

import ctypes
import math

import numpy as np

from triton_llm import gpu
from triton_llm import _lib

LOG2E = 1.4426950408889634


def contiguous_strides(shape) -> tuple[int, ...]:
    """Element strides of a C-contiguous array of ``shape``."""
    out = []
    acc = 1
    for s in reversed(shape):
        out.append(acc)
        acc *= int(s)
    return tuple(reversed(out))


def check_status(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"GPU runtime error (hip): {status} ({_lib.error_string(status)}) in {what}")


# ---- launchers: a wrapper call's C-ABI launches, replayable without Python
# validation (serving loops, benchmarks) ---------------------------------------
_recording: list | None = None


def launch(fn, *args, what: str) -> None:
    """Issue one C-ABI launch, or record it while :func:`record` runs."""
    if _recording is not None:
        _recording.append((fn, args, what))
        return
    check_status(fn(*args), what)


class Launcher:
    """The C-ABI launches one wrapper call made, replayed with the same
    arguments: no Python validation, no shape logic, one ctypes call per
    kernel launch.  It holds the recorded call's result and every buffer
    allocated or handed out as a shared workspace while recording; buffers
    the caller passed in must stay alive as long as the launcher is used."""

    def __init__(self, calls, keep):
        self.calls = calls
        self._keep = keep  # the call's result and the buffers it used

    def __call__(self) -> None:
        for fn, args, what in self.calls:
            st = fn(*args)
            if st:
                check_status(st, what)


def record(thunk) -> Launcher:
    """Run ``thunk`` (wrapper calls) recording instead of issuing their
    launches; returns a :class:`Launcher` that issues them."""
    global _recording
    prev, _recording = _recording, []
    held: list = []
    gpu._keepers.append(held)
    try:
        result = thunk()
        calls = _recording
    finally:
        _recording = prev
        gpu._keepers.remove(held)
    return Launcher(calls, (result, held))


def same_dtype(*tensors) -> int:
    """Dtype code shared by all tensors; ValueError if they differ."""
    names = {gpu.dtype_name(t.dtype) for t in tensors}
    if len(names) != 1:
        raise ValueError(f"inputs must share one dtype, got {sorted(names)}")
    return gpu.dtype_code(tensors[0].dtype)


def is_pow2(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def default_scale(d_k: int) -> float:
    return 1.0 / math.sqrt(d_k)


def vp(t) -> ctypes.c_void_p:
    """Raw pointer argument of a DeviceTensor (NULL for None)."""
    if t is None:
        return ctypes.c_void_p(None)
    return t.ptr if isinstance(t.ptr, ctypes.c_void_p) else ctypes.c_void_p(t.ptr)


def scratch(nbytes: int, workspace=None, key: str = "scratch"):
    """Return a workspace of at least ``nbytes``: the caller's (ValueError if
    too small), else the shared one kept for ``key``."""
    if nbytes == 0:
        return None
    if workspace is not None:
        if workspace.nbytes < nbytes:
            raise ValueError(f"workspace holds {workspace.nbytes} bytes, {nbytes} required")
        return workspace
    return shared_workspace(key, nbytes)


# Workspaces kept across calls, one per purpose, grown on demand.  Every call
# runs on the library stream, so consecutive calls are ordered and may share
# one buffer; allocating per call would cost a hipMalloc (and the free a
# device synchronisation) each time.
_shared: dict[str, "gpu.DeviceTensor"] = {}


def shared_workspace(key: str, nbytes: int):
    """A device buffer of at least ``nbytes`` kept for ``key`` (None for 0).
    Grows to the next power of two (at least 1 MiB) when too small."""
    if nbytes == 0:
        return None
    ws = _shared.get(key)
    if ws is None or ws.nbytes < nbytes:
        size = max(1 << 20, 1 << (int(nbytes) - 1).bit_length())
        _shared.pop(key, None)
        ws = gpu.allocate((size,), np.uint8)
        _shared[key] = ws
    gpu.keep_alive(ws)  # a recorded launch using it outlives a later growth
    return ws
