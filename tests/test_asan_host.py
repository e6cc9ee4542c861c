"""The library's host code under AddressSanitizer (CPU only, no GPU).

The host pass of every source is rebuilt with -fsanitize=address
(triton_llm._build.build_host_asan: host-only, no device code), loaded into
a Python process with the ASan runtime preloaded, and driven through the
host-only paths of the C ABI: workspace sizing, split sizes, error strings
and the argument errors of every compute entry point
(tests/asan_host_calls.py).  The run must report no ASan error, and every
result must equal the product library's for the same calls."""

import json
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "triton-llm_amd"))

from triton_llm import _build, _lib  # noqa: E402

SCRIPT = os.path.join(ROOT, "tests", "asan_host_calls.py")


def run_calls(env):
    res = subprocess.run([sys.executable, SCRIPT], env=env, capture_output=True, text=True, timeout=600)
    return res


def test_host_entry_points_under_asan(tmp_path):
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")
    rt = _build.asan_runtime()
    if rt is None:
        pytest.skip("no shared ASan runtime in this toolchain")
    lib = _build.build_host_asan(str(tmp_path))
    env = dict(os.environ)
    env["LD_PRELOAD"] = rt + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:exitcode=23"
    env["TRITON_LLM_HIP_LIB"] = lib
    asan = run_calls(env)
    assert "AddressSanitizer" not in asan.stderr, asan.stderr[-4000:]
    assert asan.returncode == 0, asan.stderr[-4000:]
    got = json.loads(asan.stdout.strip().splitlines()[-1])
    assert got[-1] == ["asan_runtime", True]

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("product library not built")
    env = dict(os.environ)
    env.pop("TRITON_LLM_HIP_LIB", None)
    plain = run_calls(env)
    assert plain.returncode == 0, plain.stderr[-4000:]
    want = json.loads(plain.stdout.strip().splitlines()[-1])
    assert got[:-1] == want
    assert len(want) > 100
