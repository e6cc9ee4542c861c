"""CPU oracle for the triton-llm attention path -- TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference's algorithms (ziliangpeng/triton-llm):
  * attention       -- triton_llm/kernels/attention.py:18-216
  * attention_gqa   -- triton_llm/kernels/attention_gqa.py:21-269
  * RoPE + tables   -- triton_llm/kernels/rope.py:25-222
  * KV-cache append -- smollm2_triton/model.py:219-225, :296-308, :336-339
  * decode over the cache -- smollm2_triton/model.py:305-314
plus the seeded input recipe of the benchmark configurations.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker or the reported CPU
baseline -- never as the computation that is shipped or measured.  The
product (``triton_llm``) never imports it.

Parity pinning: every function here is checked in tests/test_oracle.py
against properties the mathematics fixes independently of this code
(brute-force fp64 loops on small inputs, closed forms such as Q=K=V=I and
uniform attention, causal-perturbation invariance, the GQA head map, the
rotation's norm preservation and pairing, float64 cos/sin, exhaustive bf16
rounding, and the length draws quoted for the benchmark configurations).
"""

from . import attention, inputs, numerics, rope  # noqa: F401
