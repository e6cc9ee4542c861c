"""
GPU memory allocator (ctypes + HIP runtime), MI355X / gfx950 only.

Same public surface as the reference allocator (triton_llm/gpu.py of
ziliangpeng/triton-llm: ``DeviceTensor`` :184-227, ``allocate`` :230,
``to_device`` :239, ``to_host`` :247, ``synchronize`` :252, ``view`` :266,
``check_error`` :179), without PyTorch.  Differences by design:

* HIP only.  ``GPU_BACKEND`` may be unset or ``hip``; ``cuda`` raises, as the
  reference raises for a backend whose runtime is absent (gpu.py:57-71).
* Every call goes through ``libtriton_llm_hip.so`` (tl_malloc / tl_free /
  tl_memcpy_* / tl_synchronize), which issues copies with ``hipMemcpyAsync`` on
  the library's single stream -- the same stream every kernel of this package
  is launched on -- so kernels and copies stay in issue order without device
  synchronisation.  ``to_host`` waits for that stream before returning.
* bfloat16 is a first-class storage dtype: ``gpu.bfloat16`` is a uint16 NumPy
  dtype tagged with metadata, and host arrays of it hold raw bf16 bit patterns.
* Freed blocks are cached for reuse.  ``hipFree`` waits for the whole
  device, so the reference's free-on-``__del__`` puts a device
  synchronisation into every call that drops a temporary.  Here a dropped
  tensor's block (up to ``POOL_MAX_BLOCK`` bytes, ``POOL_MAX_BYTES`` in all)
  goes to a free list keyed by its rounded size, and the next ``allocate`` of
  that size takes it without ``hipMalloc``.  Reuse is safe because every
  kernel and copy of this package runs on the one library stream: work that
  used the block is ordered before any work that uses it again.  Blocks are
  uninitialised either way.  ``empty_cache()`` returns the cached blocks to
  HIP, and an allocation that fails empties the cache and tries once more.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

from . import _lib

# Kept for callers that used the reference's constants.
CUDA_MEMCPY_HOST_TO_DEVICE = 1
CUDA_MEMCPY_DEVICE_TO_HOST = 2
CUDA_SUCCESS = 0

HIP_LIBRARIES = [_lib.library_path()]

bfloat16 = np.dtype(np.uint16, metadata={"triton_llm.dtype": "bfloat16"})

_SUPPORTED_COMPUTE = {"float32": _lib.DTYPE_F32, "float16": _lib.DTYPE_F16, "bfloat16": _lib.DTYPE_BF16}


def dtype_name(dtype) -> str:
    """Canonical dtype name; ``'bfloat16'`` for the tagged uint16 dtype."""
    dt = np.dtype(dtype)
    if dt.metadata and dt.metadata.get("triton_llm.dtype") == "bfloat16":
        return "bfloat16"
    return dt.name


def dtype_code(dtype) -> int:
    """C-ABI dtype code for a compute dtype; ValueError for anything else."""
    name = dtype_name(dtype)
    if name not in _SUPPORTED_COMPUTE:
        raise ValueError(f"unsupported dtype {name}; expected float32, float16 or bfloat16")
    return _SUPPORTED_COMPUTE[name]


def _detect_backend() -> str:
    """Backend selection (reference gpu.py:47-86), HIP only."""
    env = os.environ.get("GPU_BACKEND", "").lower().strip()
    if env == "cuda":
        raise RuntimeError(
            "GPU_BACKEND=cuda was set, but this build of triton_llm is HIP-only "
            "(MI355X / gfx950); no CUDA runtime is used."
        )
    if env not in ("", "hip"):
        raise RuntimeError(f"Unknown GPU_BACKEND={env!r}; only 'hip' is supported.")
    return "hip"


_initialized = False
_backend = None
_rt = None


def _initialize():
    """Load the HIP library and create its stream on first use."""
    global _initialized, _backend, _rt
    if _initialized:
        return
    _backend = _detect_backend()
    lib = _lib.load()
    count = ctypes.c_int(0)
    err = lib.tl_device_count(ctypes.byref(count))
    if err != 0 or count.value == 0:
        raise RuntimeError(
            "No supported GPU runtime found. A ROCm (HIP) device is required "
            f"(hipGetDeviceCount status {err}, devices {count.value})."
        )
    device = int(os.environ.get("TRITON_LLM_DEVICE", "0"))
    check_error(lib.tl_init(device))
    _rt = lib
    _initialized = True


def reload_overrides():
    """Make the library re-read its test-only environment overrides
    (TRITON_LLM_HIP_MAX_CUS, TRITON_LLM_HIP_DECODE_SHARES,
    TRITON_LLM_HIP_PREFILL_W64, TRITON_LLM_HIP_PREFILL_ONE_LIST,
    TRITON_LLM_HIP_PREFILL_NO_SPLIT), which it reads
    in tl_init, never per launch.  Does nothing before the first GPU use."""
    if _initialized:
        check_error(_rt.tl_init(int(os.environ.get("TRITON_LLM_DEVICE", "0"))))


def runtime():
    """The loaded HIP library (initialising on first use)."""
    _initialize()
    return _rt


def check_error(err):
    if err != CUDA_SUCCESS:
        raise RuntimeError(f"GPU runtime error ({_backend or 'hip'}): {err} ({_lib.error_string(err)})")


# ---- block cache -------------------------------------------------------------

POOL_MAX_BLOCK = 256 << 20  # larger blocks go straight back to hipFree
POOL_MAX_BYTES = 2 << 30    # most bytes held in freed blocks
_POOL_ALIGN = 256
_pool: dict[int, list[int]] = {}
_pool_bytes = 0
_pool_lock = threading.Lock()


def _block_size(nbytes: int) -> int:
    return (nbytes + _POOL_ALIGN - 1) // _POOL_ALIGN * _POOL_ALIGN


def _take_block(size: int):
    """A cached block of exactly ``size`` bytes (address), or None."""
    global _pool_bytes
    with _pool_lock:
        blocks = _pool.get(size)
        if blocks:
            _pool_bytes -= size
            return blocks.pop()
    return None


def _release_block(addr: int, size: int) -> None:
    """Keep a dropped tensor's block for reuse, or hand it back to HIP."""
    global _pool_bytes
    with _pool_lock:
        if size <= POOL_MAX_BLOCK and _pool_bytes + size <= POOL_MAX_BYTES:
            _pool.setdefault(size, []).append(addr)
            _pool_bytes += size
            return
    _rt.tl_free(ctypes.c_void_p(addr))


def empty_cache() -> None:
    """Return every cached free block to HIP (hipFree)."""
    global _pool_bytes
    with _pool_lock:
        blocks = [a for lst in _pool.values() for a in lst]
        _pool.clear()
        _pool_bytes = 0
    for addr in blocks:
        _rt.tl_free(ctypes.c_void_p(addr))


def cached_bytes() -> int:
    """Bytes held in cached free blocks."""
    return _pool_bytes


class DeviceTensor:
    """Wrapper for a GPU device pointer with automatic cleanup (reference gpu.py:184).

    An owning tensor's block goes back to the block cache when the tensor is
    dropped (see the module docstring); a view (``defer_free=False``) owns
    nothing.
    """

    def __init__(self, ptr, shape, dtype, nbytes, defer_free=True):
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(nbytes)
        self._defer_free = defer_free

    def __del__(self):
        if getattr(self, "_defer_free", False) and self.ptr and self.ptr.value is not None:
            try:
                if _rt is not None:
                    _release_block(self.ptr.value, _block_size(self.nbytes))
            except Exception:
                pass

    def __repr__(self):
        return f"DeviceTensor(shape={self.shape}, dtype={dtype_name(self.dtype)}, ptr={self.data_ptr():#x})"

    def to_numpy(self):
        _initialize()
        host = np.empty(self.shape, dtype=self.dtype)
        check_error(_rt.tl_memcpy_dtoh(host.ctypes.data_as(ctypes.c_void_p), self.ptr, self.nbytes))
        return host

    def from_numpy(self, arr: np.ndarray):
        _initialize()
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"from_numpy: {arr.nbytes} bytes into a {self.nbytes}-byte tensor")
        check_error(_rt.tl_memcpy_htod(self.ptr, arr.ctypes.data_as(ctypes.c_void_p), self.nbytes))

    def data_ptr(self):
        return self.ptr.value or 0

    @property
    def ndim(self):
        return len(self.shape)

    @property
    def size(self):
        return int(np.prod(self.shape)) if self.shape else 1


# Keep-alive lists of the active graph captures and launcher recordings
# (kernels._common.record): a recorded launch holds raw pointers, so every
# buffer allocated or handed out as a shared workspace while one is active is
# held by it until the graph or launcher itself is dropped; otherwise a freed
# buffer could be reused while a replay still writes into it.
_keepers: list[list] = []


def keep_alive(obj) -> None:
    """Hold ``obj`` for every active capture / launcher recording."""
    for k in _keepers:
        k.append(obj)


def allocate(shape, dtype=np.float32):
    """Allocate (uninitialised) memory on the GPU: a cached block of the same
    rounded size if one is free, else ``hipMalloc``."""
    _initialize()
    shape = tuple(int(s) for s in shape)
    nbytes = int(np.prod(shape) * np.dtype(dtype).itemsize)
    if nbytes == 0:
        return DeviceTensor(ctypes.c_void_p(), shape, dtype, 0)
    size = _block_size(nbytes)
    addr = _take_block(size)
    if addr is not None:
        t = DeviceTensor(ctypes.c_void_p(addr), shape, dtype, nbytes)
    else:
        ptr = ctypes.c_void_p()
        err = _rt.tl_malloc(ctypes.byref(ptr), size)
        if err != CUDA_SUCCESS and _pool_bytes:
            empty_cache()  # out of memory with blocks cached: give them back, try once more
            err = _rt.tl_malloc(ctypes.byref(ptr), size)
        check_error(err)
        t = DeviceTensor(ptr, shape, dtype, nbytes)
    if _keepers:
        keep_alive(t)
    return t


def zeros(shape, dtype=np.float32):
    """Allocate and zero-fill (a stream-ordered fill kernel)."""
    t = allocate(shape, dtype)
    if t.nbytes:
        check_error(_rt.tl_memset(t.ptr, 0, t.nbytes))
    return t


def to_device(arr: np.ndarray, dtype=None):
    """Copy a NumPy array to the GPU.

    ``dtype`` may retag the bytes, e.g. ``to_device(bits_u16, gpu.bfloat16)``.
    """
    _initialize()
    arr = np.ascontiguousarray(arr)
    dt = np.dtype(dtype) if dtype is not None else arr.dtype
    if dt.itemsize != arr.dtype.itemsize:
        raise ValueError(f"cannot retag {arr.dtype} as {dtype_name(dt)}: itemsize differs")
    tensor = allocate(arr.shape, dt)
    tensor.from_numpy(arr)
    return tensor


def to_host(tensor: DeviceTensor):
    """Copy a DeviceTensor back to NumPy (waits for the library stream)."""
    return tensor.to_numpy()


def synchronize():
    """Wait for all work on the library stream and the device."""
    _initialize()
    check_error(_rt.tl_synchronize())


def view(tensor: DeviceTensor, new_shape: tuple) -> DeviceTensor:
    """Zero-copy reshape; the view does not own the memory (reference gpu.py:266)."""
    n_elems = int(np.prod(tensor.shape))
    n_new = int(np.prod(new_shape))
    if n_elems != n_new:
        raise ValueError(
            f"Cannot view {tensor.shape} ({n_elems} elements) as "
            f"{new_shape} ({n_new} elements) — element count mismatch"
        )
    return DeviceTensor(tensor.ptr, new_shape, tensor.dtype, tensor.nbytes, defer_free=False)


class Graph:
    """An executable HIP graph recorded by :func:`capture`; ``replay()``
    runs the recorded launches again on the library stream (same pointers,
    same sizes).  No sync.  Holds every buffer allocated, or handed out as a
    shared workspace, during the capture."""

    def __init__(self):
        self.exec = ctypes.c_void_p()
        self.keep: list = []

    def replay(self):
        _initialize()
        if not self.exec.value:
            raise RuntimeError("graph was not captured")
        check_error(_rt.tl_graph_launch(self.exec, None))

    def __del__(self):
        try:
            if self.exec.value and _rt is not None:
                _rt.tl_graph_destroy(self.exec)
        except Exception:
            pass


class capture:
    """``with gpu.capture() as g: <launches>`` records the launches on the
    library stream into ``g`` instead of running them; ``g.replay()`` runs
    them.  Inside, only stream-ordered launches, device copies and fills
    (``zeros``, ``tl_memset``: a fill kernel) are legal: no host copies, no
    synchronize.  Allocations are legal but are not recorded, so make them
    (or warm the block cache) before capturing."""

    def __enter__(self) -> Graph:
        _initialize()
        self.graph = Graph()
        check_error(_rt.tl_graph_capture_begin(None))
        _keepers.append(self.graph.keep)
        return self.graph

    def __exit__(self, exc_type, exc, tb):
        _keepers.remove(self.graph.keep)
        err = _rt.tl_graph_capture_end(None, ctypes.byref(self.graph.exec))
        if exc_type is None:
            check_error(err)
        return False


def copy_(dst: DeviceTensor, src: DeviceTensor):
    """Device-to-device copy of ``src`` into ``dst`` (same byte size), stream ordered."""
    _initialize()
    if dst.nbytes != src.nbytes:
        raise ValueError(f"copy_: {src.nbytes} bytes into {dst.nbytes}")
    check_error(_rt.tl_memcpy_dtod(dst.ptr, src.ptr, src.nbytes))
