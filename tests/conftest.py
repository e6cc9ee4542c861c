"""pytest configuration: paths and the ``gpu`` marker.

Tests marked ``gpu`` need an MI355X (gfx950) and the built HIP library; the
rest run on any CPU (oracle pinning, host-side validation, ABI surface).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "triton-llm_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and libtriton_llm_hip.so")


def pytest_runtest_logstart(nodeid, location):
    # With TL_TRACE_TESTS set, name each test before it runs so a fault that
    # ends the process still identifies its case in the captured output.
    if os.environ.get("TL_TRACE_TESTS"):
        print(f"\n[start] {nodeid}", flush=True)


@pytest.fixture(autouse=True)
def _library_overrides_follow_env():
    """The HIP library reads its test overrides (TRITON_LLM_HIP_MAX_CUS,
    TRITON_LLM_HIP_DECODE_SHARES, TRITON_LLM_HIP_PREFILL_W64,
    TRITON_LLM_HIP_PREFILL_ONE_LIST, TRITON_LLM_HIP_PREFILL_NO_SPLIT) in tl_init,
    not per launch.  Tests set them
    with tests._helpers.set_override; this fixture is set up before
    monkeypatch and so torn down after it, and re-reads the restored
    environment, so no override outlives its test."""
    yield
    if "triton_llm.gpu" in sys.modules:
        sys.modules["triton_llm.gpu"].reload_overrides()
