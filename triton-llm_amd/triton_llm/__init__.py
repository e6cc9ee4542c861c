"""triton_llm -- MI355X (gfx950) attention path for the triton-llm inference stack.

Drop-in for the reference package's allocator (``triton_llm.gpu``) and its
attention-path kernels (``triton_llm.kernels``); the kernels are hand-written
HIP in ``libtriton_llm_hip.so``, reached through ctypes.  No PyTorch, no
Triton, no CPU fallback.
"""

from . import gpu

__all__ = ["gpu"]
