"""Build libtriton_llm_hip.so (gfx950) from triton-llm_amd/csrc.

Each ``.hip`` source is compiled to an object in parallel with hipcc, then the
objects are linked into ``triton_llm/_lib/libtriton_llm_hip.so`` in-tree, so
the built library travels with the source tree.

Run as ``python -m triton_llm._build`` (with ``triton-llm_amd`` on sys.path) or
call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import re
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)  # triton-llm_amd/
CSRC_DIR = os.path.join(ROOT_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libtriton_llm_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops is disabled for every device compile: packed fp32 forms
# have produced silently wrong results on the target boxes.  The host pass
# warns that it does not know the feature; that warning is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Extra flags per source.  tl_prefill_w64.hip builds its MFMA builtins in VGPR
# form: its S products are read by VALU code, while its O accumulators live in
# AGPRs through inline assembly (at one wave per SIMD the compiler would
# otherwise give every MFMA AGPR operands and copy S out for the softmax).
FILE_FLAGS: dict[str, list[str]] = {
    "tl_prefill_w64.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}

# Only the HIP runtime is linked (hipcc adds it); every kernel is this library's own.
LINK_LIBS: list[str] = []


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build the HIP library")
    return path


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip")
    )


# Instructions that read or write m0 without naming it.
_M0_IMPLICIT = re.compile(r"\b(s_movrel|v_movrel|s_sendmsg|ds_gws|ds_read_addtid|ds_write_addtid|v_interp|"
                          r"s_ttracedata)")
_M0_NAMED = re.compile(r"\bm0\b")


def check_m0(asm_text: str, source: str) -> int:
    """Reject a kernel that issues the inline-asm LDS-DMA (csrc/tl_common.h
    lds_dma16, which writes m0) and in which compiler-generated code reads
    or writes m0 too.  m0 is a reserved register, so the asm cannot declare
    it clobbered; this check, run on every build, is what makes that asm
    safe: no value of the compiler's lives in m0 around it.  Returns the
    number of kernels that issue the DMA."""
    funcs: dict[str, list] = {}  # name -> [issues the asm DMA, compiler m0 uses]
    name, in_asm = None, False
    for line in asm_text.splitlines():
        m = re.match(r"\s*\.type\s+([^,\s]+)\s*,\s*@function", line)
        if m:
            name, in_asm = m.group(1), False
            funcs[name] = [False, []]
            continue
        if name is None:
            continue
        if ";;#ASMSTART" in line:
            in_asm = True
            continue
        if ";;#ASMEND" in line:
            in_asm = False
            continue
        code = line.split(";", 1)[0]
        if in_asm:
            funcs[name][0] = funcs[name][0] or code.rstrip().endswith(" lds")
        elif _M0_NAMED.search(code) or _M0_IMPLICIT.search(code) or code.rstrip().endswith(" lds"):
            funcs[name][1].append(code.strip())
    bad = [f"{n}: {uses[:3]}" for n, (dma, uses) in funcs.items() if dma and uses]
    if bad:
        raise RuntimeError(f"{os.path.basename(source)}: compiler-generated code uses m0 in kernels that issue "
                           f"the inline-asm LDS-DMA (which writes m0):\n  " + "\n  ".join(bad))
    return sum(1 for dma, _ in funcs.values() if dma)


def _compile_one(src: str, obj: str) -> None:
    # -save-temps=obj leaves the device assembly next to the object (in the
    # build's temporary directory) for check_m0.
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-save-temps=obj", "-c", src,
           "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True, cwd=os.path.dirname(obj))
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    stem = os.path.splitext(os.path.basename(src))[0]
    asm = os.path.join(os.path.dirname(obj), f"{stem}-hip-amdgcn-amd-amdhsa-{OFFLOAD_ARCH}.s")
    if not os.path.exists(asm):
        raise RuntimeError(f"device assembly {asm} missing: cannot check m0 use")
    with open(asm) as f:
        n_dma = check_m0(f.read(), src)
    with open(src) as f:
        calls_dma = "lds_dma16(" in f.read()
    if calls_dma and n_dma == 0:
        raise RuntimeError(f"{os.path.basename(src)} calls lds_dma16 but check_m0 found no kernel issuing it: "
                           "the guard no longer recognises the DMA")


def build(verbose: bool = True, jobs: int | None = None) -> str:
    """Compile every csrc/*.hip for gfx950 and link the shared library."""
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with tempfile.TemporaryDirectory(prefix="tl_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in srcs]
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = [ex.submit(_compile_one, s, o) for s, o in zip(srcs, objs)]
            for f in futs:
                f.result()
        tmp_lib = LIB_PATH + ".tmp"
        cmd = [_hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib,
               *LINK_LIBS]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        os.replace(tmp_lib, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def build_host_asan(out_dir: str, jobs: int | None = None) -> str:
    """A CPU-only AddressSanitizer build of the library's host code, for
    tests that drive the entry points' argument checks and workspace sizing
    (which return before any HIP call).  Host-only compile (no device code:
    the device binary embedded is empty, so no kernel can be launched from
    this build); the sanitizer applies to the host pass only.  Returns the
    library path.  Needs the ASan runtime preloaded into the process that
    loads it (see asan_runtime())."""
    os.makedirs(out_dir, exist_ok=True)
    empty_fb = os.path.join(out_dir, "empty.hipfb")
    open(empty_fb, "wb").close()
    host_flags = ["--offload-host-only", "-O1", "-g", "-std=c++17", "-fPIC",
                  "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
                  "-Xclang", "-fcuda-include-gpubinary", "-Xclang", empty_fb]
    srcs = sources()
    objs = [os.path.join(out_dir, os.path.basename(s) + ".o") for s in srcs]

    def one(src, obj):
        res = subprocess.run([_hipcc(), *host_flags, "-c", src, "-o", obj], capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"host ASan compile failed for {os.path.basename(src)}:\n{res.stderr}")

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs or min(len(srcs), 8)) as ex:
        for f in [ex.submit(one, s, o) for s, o in zip(srcs, objs)]:
            f.result()
    lib = os.path.join(out_dir, "libtriton_llm_hip_asan.so")
    res = subprocess.run([_hipcc(), "--offload-host-only", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
                          *objs, "-o", lib, *LINK_LIBS], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host ASan link failed:\n{res.stderr}")
    return lib


def asan_runtime() -> str | None:
    """Path of the compiler's shared ASan runtime, or None."""
    clang = os.path.join(os.path.dirname(os.path.realpath(_hipcc())), "..", "llvm", "bin", "clang")
    for c in (clang, "/opt/rocm/llvm/bin/clang"):
        if os.path.exists(c):
            res = subprocess.run([c, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
            path = res.stdout.strip()
            if res.returncode == 0 and os.path.isabs(path) and os.path.exists(path):
                return path
    return None


if __name__ == "__main__":
    build()
