"""Benchmark of the MI355X attention path on one GPU.

Default run: every configuration of BASELINE.json, each timed on its own with
inputs resident in HBM --
  1   GPT-2 causal prefill fp32 (B1 H12 D64 S128);
  2   GPT-2 decode fp16 (B8 H12 D64, cache 1024);
  3   SmolLM2-135M GQA causal prefill bf16 (B4 Hq9 Hkv3 D64 S2048);
  4   SmolLM2-360M GQA decode bf16 (B32 Hq15 Hkv5 D64, cache 8192);
  5a  Llama-3.2-3B GQA causal prefill bf16 (B1 Hq24 Hkv8 D128 S8192);
  5b  Llama-3.2-3B GQA decode bf16 (B64 Hq24 Hkv8 D128, cache 16384);
a decode step is RoPE + KV append + split-K attention.  ``value`` is 5b's
decode-step HBM throughput (GB/s), the headline; 5a is repeated in the
``prefill`` object and every config sits in ``configs``, each with its
``roofline`` (HIP events on the library stream around the attention call) and
``cpu_baseline`` (the NumPy oracle of the same attention, a bounded number of
passes on this host's cores).

``append-5a`` and ``append-3`` time the fused RoPE + KV append at those
prefill configs' full prompts (what the GPU-resident cache runs before
prefill attention), HBM-bound, with the oracle's NumPy append as the CPU
baseline.  ``5a-2048`` (5a's attention at a 2048-token prompt) and ``3-b1``
(config 3 at batch 1) time shapes on which the flash kernel splits its
longest tiles' key ranges over two workgroups.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--config all|5|append|1|2|3|4|5a|5b|append-5a|append-3|5a-2048|3-b1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "triton-llm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode attn HBM GB/s + prefill attn TFLOP/s (% MI355X roofline), 1 GPU"
HBM_PEAK_GBS = 8000.0
PEAK_TFLOPS = {"bfloat16": 2516.6, "float16": 2516.6, "float32": 157.3}
DT_SHORT = {"bfloat16": "bf16", "float16": "fp16", "float32": "fp32"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Events:
    """HIP event pairs on the library stream (via the C ABI)."""

    def __init__(self, lib, n):
        import ctypes

        self.lib = lib
        self.ev = []
        for _ in range(n):
            p = ctypes.c_void_p()
            assert lib.tl_event_create(ctypes.byref(p)) == 0
            self.ev.append(p)

    def record(self, i):
        assert self.lib.tl_event_record(self.ev[i], None) == 0

    def ms(self, i, j):
        import ctypes

        out = ctypes.c_float()
        assert self.lib.tl_event_synchronize(self.ev[j]) == 0
        assert self.lib.tl_event_elapsed_ms(ctypes.byref(out), self.ev[i], self.ev[j]) == 0
        return float(out.value)

    def close(self):
        for e in self.ev:
            self.lib.tl_event_destroy(e)


def profile_traffic(name):
    """HBM bytes per launch recorded in profiles/<name> (rocprofv3 FETCH_SIZE +
    WRITE_SIZE runs of this bench, scaled by a copy-kernel calibration), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def clock_ramp(step, ramp_ms):
    """Run ``step(i)`` untimed until ``ramp_ms`` of wall time has passed (at
    most 2000 calls).  The GPU's shader clock climbs over the first tens of
    milliseconds of sustained load; this puts the warm-up and timed steps at
    the clock the GPU holds under a serving load, whatever --warmup is.  The
    ramp's steps are the same work as the timed ones and are never timed.
    Returns (calls, ms)."""
    from triton_llm import gpu

    if ramp_ms <= 0:
        return 0, 0.0
    t0 = time.perf_counter()
    n = 0
    while n < 2000:
        step(n)
        n += 1
        if n % 4 == 0:
            gpu.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= ramp_ms:
                break
    gpu.synchronize()
    return n, (time.perf_counter() - t0) * 1e3


def time_calls(lib, calls, steps, warmup, ramp_ms):
    """Run calls[i % len(calls)] (zero-argument launchers or graph replays)
    for a clock ramp, ``warmup`` untimed steps, then exactly ``steps`` timed
    steps enqueued back to back between two events on the library stream
    (synchronised on both sides).  Returns (ms per step, ramp (calls, ms),
    host wall ms per step)."""
    from triton_llm import gpu

    n = len(calls)
    ramp = clock_ramp(lambda i: calls[i % n](), ramp_ms)
    for i in range(warmup):
        calls[i % n]()
    gpu.synchronize()
    ev = Events(lib, 2)
    t0 = time.perf_counter()
    ev.record(0)
    for i in range(steps):
        calls[i % n]()
    ev.record(1)
    ms = ev.ms(0, 1) / steps
    gpu.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev.close()
    return ms, ramp, wall


def cpu_threads():
    n = os.environ.get("OMP_NUM_THREADS") or os.environ.get("OPENBLAS_NUM_THREADS")
    try:
        return int(n) if n else len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


def cpu_host():
    """What the CPU baseline ran on: cores the process may use, the thread
    settings and NumPy's BLAS."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except Exception:
        affinity = os.cpu_count()
    blas = None
    try:
        cfg = np.show_config(mode="dicts")
        b = cfg.get("Build Dependencies", {}).get("blas", {})
        blas = f"{b.get('name')} {b.get('version')}".strip()
    except Exception:
        pass
    return {"affinity_cores": affinity, "blas": blas,
            "threads_env": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS")}}


# ---------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------

def bench_decode(cfg, steps, warmup, replicas=1, cpu=True, split=0, cpu_budget_s=10.0, ramp_ms=0.0):
    from oracle import attention as oa
    from oracle import inputs as oi
    from oracle import numerics as on
    from triton_llm import gpu
    from triton_llm.kernels import attention_decode, decode_step
    from triton_llm.kernels.decode import decode_workspace, decode_workspace_bytes

    dt = cfg.dtype
    gdt = {"bfloat16": gpu.bfloat16, "float16": np.float16, "float32": np.float32}[dt]
    t0 = time.perf_counter()
    data = oi.make_decode(cfg, fill="zero")
    log(f"{cfg.name}: inputs generated in {time.perf_counter() - t0:.1f}s")
    lens = data["lens"]
    B, Hq, Hkv, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.d_k
    cos, sin = oi.rope_tables(cfg)
    caches = []
    for _ in range(replicas):  # rotate replicas so small caches are not served from MALL
        caches.append((gpu.to_device(data["k_cache"], gdt), gpu.to_device(data["v_cache"], gdt)))
    q = gpu.to_device(data["q"], gdt)
    kn = gpu.to_device(data["k_new"], gdt)
    vn = gpu.to_device(data["v_new"], gdt)
    lens_d = gpu.to_device(lens)
    cos_d = gpu.to_device(cos) if cos is not None else None
    sin_d = gpu.to_device(sin) if sin is not None else None
    out = gpu.allocate((B, Hq, D), gdt)
    ws_bytes, split = decode_workspace_bytes(B, Hq, Hkv, cfg.max_ctx, D, split)
    ws = decode_workspace(B, Hq, Hkv, cfg.max_ctx, D, split)
    lib = gpu.runtime()

    def attend(i):
        kc, vc = caches[i % replicas]
        attention_decode(q, kc, vc, lens_d, Hq, Hkv, sm_scale=cfg.scale, len_add=1, out=out,
                         workspace=ws, split=split)

    def step(i):
        # RoPE + append + attention: one tl_attention_decode_append call
        kc, vc = caches[i % replicas]
        decode_step(q, kn, vn, kc, vc, lens_d, Hq, Hkv, cos_d, sin_d, sm_scale=cfg.scale, out=out,
                    workspace=ws, split=split)

    # One eager step per replica fills the workspace and block caches.  Each
    # replica's step (RoPE + append + attention) and its attention call alone
    # are then recorded as launchers: the same C-ABI launches, replayed
    # without the wrappers' Python validation, so the small configs' steps
    # are not timed behind their host launch cost.  The same steps recorded
    # as HIP graphs give a second figure.
    from triton_llm.kernels._common import record

    for i in range(replicas):
        step(i)
    gpu.synchronize()
    step_calls = [record(lambda i=i: step(i)) for i in range(replicas)]
    attn_calls = [record(lambda i=i: attend(i)) for i in range(replicas)]
    step_med, ramp, wall_ms = time_calls(lib, step_calls, steps, warmup, ramp_ms)
    attn_med, _, _ = time_calls(lib, attn_calls, steps, warmup, 0.0)
    graphs = []
    for i in range(replicas):
        with gpu.capture() as g:
            step(i)
        graphs.append(g.replay)
    graph_ms, _, _ = time_calls(lib, graphs, steps, warmup, 0.0)

    e = 4 if dt == "float32" else 2
    step_bytes = oi.decode_bytes(cfg, lens)
    attn_bytes = int(np.sum(2 * Hkv * (lens.astype(np.int64) + 1) * D * e)) + B * Hq * D * 2 * e
    res = {
        "value": step_bytes / (step_med * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": step_med,
        "wall_ms_per_step": wall_ms,
        "timing": f"{steps} steps enqueued back to back between two events (C-ABI launches recorded "
                  f"from the wrappers), cycling over {replicas} cache replica(s)",
        "graph_ms_per_step": graph_ms,
        "clock_ramp": {"calls": ramp[0], "ms": round(ramp[1], 1)},
        "split": split,
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_split_kernel + decode_combine_kernel (tl_attention_decode)",
            "achieved": attn_bytes / (attn_med * 1e-3) / 1e9,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": attn_bytes / (attn_med * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "traffic": profile_traffic(f"decode_split_kernel_{cfg.name}.md"),
            "algorithmic_bytes": attn_bytes,
            "kernel_ms": attn_med,
        },
    }
    if cpu:
        res["cpu_baseline"] = cpu_decode_baseline(cfg, data, oa, on, budget_s=cpu_budget_s)
    return res


# ---------------------------------------------------------------------------
# projections (tl_gemm): the model step's plain GEMMs
# ---------------------------------------------------------------------------

GEMM_MODELS = {
    # name: (n_embd, q, kv, intermediate) -- projection widths of the model
    "smollm2-360m": (960, 960, 320, 2560),
    "llama3.2-3b": (3072, 3072, 1024, 8192),
}
FP32_PEAK_TFLOPS = 157.3


def rocblas_calls(lib, shapes, x, w, out, M, dt):
    """Zero-argument launchers of rocblas_gemm_ex for each projection
    C (M, N) = X (M, K) . W (K, N), row-major, run as the column-major
    C^T = W^T X^T on the library stream, fp32 accumulation.  A measurement
    reference point only (bench.py --gemm --gemm-rocblas)."""
    import ctypes

    rb = ctypes.CDLL("librocblas.so")
    lib.tl_default_stream.restype = ctypes.c_void_p
    handle = ctypes.c_void_p()
    if rb.rocblas_create_handle(ctypes.byref(handle)) != 0:
        raise RuntimeError("rocblas_create_handle failed")
    if rb.rocblas_set_stream(handle, ctypes.c_void_p(lib.tl_default_stream())) != 0:
        raise RuntimeError("rocblas_set_stream failed")
    code = 151 if dt == "float32" else 168  # rocblas_datatype_f32_r / _bf16_r
    one, zero = ctypes.c_float(1.0), ctypes.c_float(0.0)
    calls = []
    for name, (K, N) in shapes.items():
        a, b, c = x[K].ptr.value, w[name].ptr.value, out[name].ptr.value

        def call(a=a, b=b, c=c, K=K, N=N):
            st = rb.rocblas_gemm_ex(handle, 111, 111, N, M, K, ctypes.byref(one), ctypes.c_void_p(b), code, N,
                                    ctypes.c_void_p(a), code, K, ctypes.byref(zero), ctypes.c_void_p(c), code, N,
                                    ctypes.c_void_p(c), code, N, 151, 0, 0, 0)
            if st != 0:
                raise RuntimeError(f"rocblas_gemm_ex failed: {st}")
        calls.append(call)
    return calls


def bench_gemm(steps, warmup, cpu=True, models=("llama3.2-3b", "smollm2-360m"), prompt=2048, batch_rows=64,
               vs_rocblas=False):
    """Time the projections of one layer (q, k, v, o, gate, up, down) of each
    model for one decoded token (M = 1, weight-bandwidth bound), for a batch
    of decoded tokens (M = batch_rows, one per sequence of a batched decode
    step: still weight-bandwidth bound) and for a prompt (M = prompt, MFMA
    bound), fp32 as the reference runs them and bf16,
    two ways: seven gemm calls, and the grouped form a layer step uses
    (gemm_grouped for q/k/v and for gate/up, gemm for o and down: four
    launches, plus a split-K reduce each for few rows).  Each layer's launches
    are recorded once and replayed back to back between two events.  For
    M = 1 and batch_rows the weights rotate over copies totalling >= 1 GB so
    each layer reads them from HBM, not MALL.  The CPU baseline is NumPy float32 matmul
    on the host (a bounded sample: one pass per shape, M = 1 and 128)."""
    from triton_llm import gpu
    from triton_llm.kernels import gemm, gemm_grouped
    from triton_llm.kernels._common import record

    lib = gpu.runtime()
    rows = []
    for model in models:
        e, q, kv, inter = GEMM_MODELS[model]
        shapes = {"q": (e, q), "k": (e, kv), "v": (e, kv), "o": (q, e), "gate": (e, inter), "up": (e, inter),
                  "down": (inter, e)}
        for dt, gdt, esz, peak in (("float32", np.float32, 4, FP32_PEAK_TFLOPS),
                                   ("bfloat16", gpu.bfloat16, 2, PEAK_TFLOPS["bfloat16"])):
            rng = np.random.default_rng(len(model))

            def host(shape):
                x = rng.standard_normal(shape, dtype=np.float32)
                return (x.view(np.uint32) >> 16).astype(np.uint16) if dt == "bfloat16" else x

            layer_w = sum(K * N for K, N in shapes.values()) * esz
            w0 = {name: gpu.to_device(host(shape), gdt) for name, shape in shapes.items()}
            for M in (1, batch_rows, prompt):
                reps = max(1, int(np.ceil(1e9 / layer_w))) if M <= batch_rows else 1
                W = [w0]
                for _ in range(reps - 1):
                    copy = {}
                    for name, (K, N) in shapes.items():
                        copy[name] = gpu.allocate((K, N), gdt)
                        gpu.copy_(copy[name], w0[name])
                    W.append(copy)
                x = {d: gpu.to_device(host((M, d)), gdt) for d in {e, q, inter}}
                out = {name: gpu.allocate((M, N), gdt) for name, (K, N) in shapes.items()}

                def separate(r):
                    for name, (K, N) in shapes.items():
                        gemm(x[K], W[r][name], out_dev=out[name])

                def grouped(r):
                    gemm_grouped(x[e], [W[r]["q"], W[r]["k"], W[r]["v"]], [out["q"], out["k"], out["v"]])
                    gemm(x[q], W[r]["o"], out_dev=out["o"])
                    gemm_grouped(x[e], [W[r]["gate"], W[r]["up"]], [out["gate"], out["up"]])
                    gemm(x[inter], W[r]["down"], out_dev=out["down"])

                flops = sum(2 * M * K * N for K, N in shapes.values())
                nbytes = layer_w + sum((M * K + M * N) * esz for K, N in shapes.values())
                for form, fn in (("seven gemm calls", separate), ("grouped", grouped)):
                    for r in range(reps):
                        fn(r)
                    gpu.synchronize()
                    calls = [record(lambda r=r: fn(r)) for r in range(reps)]
                    ms, _, _ = time_calls(lib, calls, steps, warmup, 0.0)
                    rows.append({
                        "model": model, "dtype": dt, "M": M, "form": form, "ms_per_layer": ms,
                        "tflops": flops / (ms * 1e-3) / 1e12, "frac_mfma": flops / (ms * 1e-3) / 1e12 / peak,
                        "gbs": nbytes / (ms * 1e-3) / 1e9, "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                    })
                    log(f"gemm {model} {dt} M={M} {form}: {ms * 1e3:.1f} us/layer, {rows[-1]['tflops']:.1f} TFLOP/s, "
                        f"{rows[-1]['gbs']:.0f} GB/s")
                if vs_rocblas and M == prompt:
                    rcalls = rocblas_calls(lib, shapes, x, W[0], out, M, dt)
                    ms, _, _ = time_calls(lib, [lambda: [c() for c in rcalls]], steps, warmup, 0.0)
                    rows.append({
                        "model": model, "dtype": dt, "M": M, "form": "rocBLAS, seven calls (reference point)",
                        "ms_per_layer": ms, "tflops": flops / (ms * 1e-3) / 1e12,
                        "frac_mfma": flops / (ms * 1e-3) / 1e12 / peak,
                        "gbs": nbytes / (ms * 1e-3) / 1e9, "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                    })
                    log(f"gemm {model} {dt} M={M} rocBLAS reference: {ms * 1e3:.1f} us/layer, "
                        f"{rows[-1]['tflops']:.1f} TFLOP/s")
                del W
    res = {"metric": "projection GEMMs per layer (tl_gemm)", "rows": rows}
    res["layers"] = bench_layers(steps, warmup)
    res["sample"] = bench_sample(steps, warmup, cpu=cpu)
    if cpu:
        cpu_rows = []
        for model in models:
            e, q, kv, inter = GEMM_MODELS[model]
            shapes = [(e, q), (e, kv), (e, kv), (q, e), (e, inter), (e, inter), (inter, e)]
            for M in (1, 128):
                t = 0.0
                flops = 0
                for K, N in shapes:
                    a = np.random.standard_normal((M, K)).astype(np.float32)
                    b = np.random.standard_normal((K, N)).astype(np.float32)
                    t0 = time.perf_counter()
                    a @ b
                    t += time.perf_counter() - t0
                    flops += 2 * M * K * N
                cpu_rows.append({"model": model, "dtype": "float32", "M": M, "ms_per_layer": t * 1e3, "tflops": flops / t / 1e12})
        res["cpu_baseline"] = {"rows": cpu_rows, "cores": cpu_threads(), "host": cpu_host(), "kind": "numpy",
                               "sample": "one pass per projection shape, M = 1 and 128"}
    return res


def bench_layers(steps, warmup, rows=2048, e=3072, inter=8192):
    """RMSNorm, fused add + RMSNorm, SwiGLU and add at a Llama-3.2-3B prompt's
    size (fp32): algorithmic bytes (every input read once, every output
    written once) per event-timed call, against 8 TB/s."""
    from triton_llm import gpu
    from triton_llm.kernels import add, add_rms_norm, rms_norm, swiglu

    lib = gpu.runtime()
    rng = np.random.default_rng(0)
    dev = lambda *shape: gpu.to_device(rng.standard_normal(shape, dtype=np.float32))  # noqa: E731
    a, b, w = dev(rows, e), dev(rows, e), dev(e)
    h, y = gpu.allocate((rows, e), np.float32), gpu.allocate((rows, e), np.float32)
    g, u, o = dev(rows, inter), dev(rows, inter), gpu.allocate((rows, inter), np.float32)
    n, ni = rows * e * 4, rows * inter * 4
    cases = [("rms_norm", lambda: rms_norm(a, w, y), 2 * n),
             ("add_rms_norm", lambda: add_rms_norm(a, b, h, w, y), 4 * n),
             ("swiglu", lambda: swiglu(g, u, o), 3 * ni),
             ("add", lambda: add(a, b, h), 3 * n)]
    out = []
    for name, fn, nbytes in cases:
        for _ in range(warmup):
            fn()
        ev = Events(lib, 2)
        ev.record(0)
        for _ in range(steps):
            fn()
        ev.record(1)
        ms = ev.ms(0, 1) / steps
        ev.close()
        out.append({"op": name, "shape": [rows, inter if name == "swiglu" else e], "us": ms * 1e3,
                    "gbs": nbytes / (ms * 1e-3) / 1e9, "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS})
        log(f"{name}: {ms * 1e3:.1f} us, {out[-1]['gbs']:.0f} GB/s")
    return out


def cpu_decode_baseline(cfg, data, oa, on, budget_s=10.0):
    """NumPy fp32 decode attention over every sequence of the workload,
    repeated until ``budget_s`` of CPU time; the median pass is reported."""
    dt = cfg.dtype
    lens = data["lens"] + 1
    B, Hkv, D = cfg.batch, cfg.n_kv_head, cfg.d_k
    # fp32 copies of each sequence's valid prefix (conversion not timed)
    seqs = []
    for b in range(B):
        L = int(lens[b])
        seqs.append((on.from_storage(data["q"][b:b + 1], dt),
                     on.from_storage(data["k_cache"][b:b + 1, :, :L], dt),
                     on.from_storage(data["v_cache"][b:b + 1, :, :L], dt), L))
    e = 4 if dt == "float32" else 2
    nbytes = int(np.sum(2 * Hkv * lens.astype(np.int64) * D * e)) + 2 * B * cfg.n_head * D * e
    passes, t_total = [], 0.0
    while t_total < budget_s or len(passes) < 3:
        t0 = time.perf_counter()
        for qf, kf, vf, L in seqs:
            oa.decode_ref(qf, kf, vf, np.array([L]), sm_scale=cfg.scale)
        passes.append(time.perf_counter() - t0)
        t_total += passes[-1]
    t = float(np.median(passes))
    return {
        "value": nbytes / t / 1e9,
        "unit": "GB/s",
        "cores": cpu_threads(),
        "host": cpu_host(),
        "kind": "port",
        "sample": f"the whole workload ({B} sequences, {int(np.sum(lens))} positions), NumPy fp32 "
                  f"oracle decode, median of {len(passes)} passes ({t_total:.1f}s); bytes counted as "
                  f"the GPU's {DT_SHORT[dt]} K/V/q/o traffic",
    }


# ---------------------------------------------------------------------------
# prefill
# ---------------------------------------------------------------------------

def prefill_kernel_name(cfg):
    """The kernels tl_attention_fwd runs for a prefill config: fp32 takes the
    key-split kernel when fewer than 64 blocks of 128 query rows would run;
    16-bit d_k 128 reads V through the vt_pack copy."""
    if cfg.dtype == "float32":
        blocks = -(-cfg.seq // 128) * cfg.n_head * cfg.batch
        return "flash_fwd_f32_ks" if blocks < 64 else "flash_fwd_f32"
    return "flash_fwd_16 + vt_pack_kernel" if cfg.d_k == 128 else "flash_fwd_16"


def bench_prefill(cfg, steps, warmup, replicas=1, cpu=True, cpu_budget_s=10.0, ramp_ms=0.0):
    from oracle import attention as oa
    from oracle import inputs as oi
    from oracle import numerics as on
    from triton_llm import gpu
    from triton_llm.kernels import apply_rope, flash_attention, precompute_cos_sin
    from triton_llm.kernels.flash import flash_workspace_bytes

    dt = cfg.dtype
    gdt = {"bfloat16": gpu.bfloat16, "float16": np.float16, "float32": np.float32}[dt]
    raw = oi.make_prefill_raw(cfg)
    B, Hq, Hkv, S, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.seq, cfg.d_k
    if cfg.rope_theta is not None:
        cos, sin = precompute_cos_sin(S, D, cfg.rope_theta)
        cd, sd = gpu.to_device(cos), gpu.to_device(sin)
    sets = []  # rotate replicas so a step's inputs are not served from MALL
    for _ in range(replicas):
        q = gpu.to_device(raw["q"], gdt)
        k = gpu.to_device(raw["k"], gdt)
        v = gpu.to_device(raw["v"], gdt)
        if cfg.rope_theta is not None:
            apply_rope(gpu.view(q, (B * Hq * S, D)), cd, sd, seq_len=S)
            apply_rope(gpu.view(k, (B * Hkv * S, D)), cd, sd, seq_len=S)
        sets.append((q, k, v, gpu.allocate(q.shape, gdt)))
    wsb = flash_workspace_bytes(B, Hkv, S, D, gdt, n_head=Hq, seq_q=S)
    ws = gpu.allocate((max(wsb, 1),), np.uint8)
    lib = gpu.runtime()

    def step(i):
        q, k, v, out = sets[i % replicas]
        flash_attention(q, k, v, causal=True, sm_scale=cfg.scale, out=out, workspace=ws)

    # one recorded launcher (V^T staging + flash kernel) per input replica
    from triton_llm.kernels._common import record

    for i in range(replicas):
        step(i)
    gpu.synchronize()
    calls = [record(lambda i=i: step(i)) for i in range(replicas)]
    ms, ramp, wall_ms = time_calls(lib, calls, steps, warmup, ramp_ms)
    flops = oi.prefill_flops(cfg)
    tf = flops / (ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[dt]
    res = {
        "value": tf,
        "unit": "TFLOP/s",
        "ms_per_step": ms,
        "wall_ms_per_step": wall_ms,
        "timing": f"{steps} calls enqueued back to back between two events (C-ABI launches recorded "
                  f"from the wrapper), cycling over {replicas} input replica(s)",
        "clock_ramp": {"calls": ramp[0], "ms": round(ramp[1], 1)},
        "roofline": {
            "bound": "mfma",
            "kernel": prefill_kernel_name(cfg) + " (tl_attention_fwd)",
            "achieved": tf,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": tf / peak,
            "traffic": profile_traffic(f"{'flash_fwd_f32' if dt == 'float32' else 'flash_fwd_16'}_{cfg.name}.md"),
            "algorithmic_flops": flops,
            "kernel_ms": ms,
        },
    }
    if cpu:
        res["cpu_baseline"] = cpu_prefill_baseline(cfg, raw, oa, on, oi, budget_s=cpu_budget_s)
    return res


def cpu_prefill_baseline(cfg, raw, oa, on, oi, budget_s=10.0):
    """NumPy fp32 causal attention of the whole workload (every KV group, all
    rows, blockwise over 512-row query tiles inside the oracle), repeated
    until ``budget_s``; the median pass is reported."""
    dt = cfg.dtype
    B, Hq, Hkv, S, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.seq, cfg.d_k
    g = Hq // Hkv
    groups = [(on.from_storage(raw["q"][b:b + 1, h * g:(h + 1) * g], dt),
               on.from_storage(raw["k"][b:b + 1, h:h + 1], dt),
               on.from_storage(raw["v"][b:b + 1, h:h + 1], dt))
              for b in range(B) for h in range(Hkv)]
    flops = oi.prefill_flops(cfg)
    passes, t_total = [], 0.0
    while t_total < budget_s or len(passes) < 3:
        t0 = time.perf_counter()
        for q, k, v in groups:
            oa.attention_bhsd(q, k, v, causal=True, sm_scale=cfg.scale, block_q=512)
        passes.append(time.perf_counter() - t0)
        t_total += passes[-1]
    t = float(np.median(passes))
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": cpu_threads(),
        "host": cpu_host(),
        "kind": "port",
        "sample": f"the whole workload ({B * Hkv} KV groups of {g} heads x {S} rows, 512-row "
                  f"query tiles), NumPy fp32 oracle, median of {len(passes)} passes ({t_total:.1f}s)",
    }


# ---------------------------------------------------------------------------
# prompt-size RoPE + KV append (what the GPU-resident cache runs before prefill)
# ---------------------------------------------------------------------------

APPEND_CASES = {
    # name: (prefill config whose prompt it appends, workload name)
    "append-5a": ("5a", "llama3.2-3b-prompt-rope-append-bf16"),
    "append-3": ("3", "smollm2-135m-prompt-rope-append-bf16"),
}


def append_bytes(cfg):
    """Algorithmic HBM bytes of one S-token append into an empty cache: q read
    and written (rotated in place), k_new read and written to the cache
    (rotated), v_new read and written to the cache, and the cos / sin table
    rows of the S positions read once (2 x d_k / 2 fp32 each)."""
    e = 4 if cfg.dtype == "float32" else 2
    B, S, Hq, Hkv, D = cfg.batch, cfg.seq, cfg.n_head, cfg.n_kv_head, cfg.d_k
    return 2 * B * S * (Hq + 2 * Hkv) * D * e + S * D * 4


# Extra prefill lines beside the six configs, shapes on which flash_fwd_16
# splits its longest tiles' keys over two workgroups: 5a's heads at a
# 2048-token prompt (192 query tiles for 256 CUs) and config 3's prompt at
# batch 1 (72 tiles).
PREFILL_EXTRA = {"5a-2048": ("5a", {"seq": 2048}, "llama3.2-3b-prefill-2048-bf16"),
                 "3-b1": ("3", {"batch": 1}, "smollm2-135m-prefill-b1-bf16")}


def prefill_extra(name):
    from oracle import inputs as oi

    base, fields, workload = PREFILL_EXTRA[name]
    return oi.scaled(oi.CONFIGS[base], name=workload, **fields)


def bench_append(name, steps, warmup, cpu=True, cpu_budget_s=4.0, ramp_ms=0.0):
    """tl_rope_kv_append at a prefill config's full prompt, as
    GpuKVCache.attention runs it (rows (B, S, H, D), an empty cache of
    capacity S, RoPE tables of S rows).  Input replicas rotate so that >= 1
    GB of other data passes between two uses of one set."""
    from oracle import inputs as oi
    from oracle import numerics as on
    from oracle import rope as orope
    from triton_llm import gpu
    from triton_llm.kernels import precompute_cos_sin, rope_kv_append
    from triton_llm.kernels._common import record

    base, workload = APPEND_CASES[name]
    cfg = oi.CONFIGS[base]
    dt = cfg.dtype
    gdt = {"bfloat16": gpu.bfloat16, "float16": np.float16, "float32": np.float32}[dt]
    B, S, Hq, Hkv, D = cfg.batch, cfg.seq, cfg.n_head, cfg.n_kv_head, cfg.d_k
    rng = np.random.default_rng(cfg.seed)
    q = on.to_storage(rng.standard_normal((B, S, Hq, D), dtype=np.float32), dt)
    kn = on.to_storage(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), dt)
    vn = on.to_storage(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), dt)
    cos, sin = precompute_cos_sin(S, D, cfg.rope_theta)
    cd, sd = gpu.to_device(cos), gpu.to_device(sin)
    lens = gpu.to_device(np.zeros(B, np.int32))
    nbytes = append_bytes(cfg)
    replicas = max(1, int(np.ceil(1024e6 / nbytes)))
    sets = []
    for _ in range(replicas):
        sets.append((gpu.to_device(q, gdt), gpu.to_device(kn, gdt), gpu.to_device(vn, gdt),
                     gpu.zeros((B, Hkv, S, D), gdt), gpu.zeros((B, Hkv, S, D), gdt)))
    lib = gpu.runtime()

    def step(i):
        qd, kd, vd, kc, vc = sets[i % replicas]
        rope_kv_append(qd, kd, vd, kc, vc, lens, cd, sd)

    calls = [record(lambda i=i: step(i)) for i in range(replicas)]
    ms, ramp, wall_ms = time_calls(lib, calls, steps, warmup, ramp_ms)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {
        "value": gbs,
        "unit": "GB/s",
        "ms_per_step": ms,
        "wall_ms_per_step": wall_ms,
        "timing": f"{steps} calls enqueued back to back between two events (C-ABI launch recorded from "
                  f"the wrapper), cycling over {replicas} input replica(s)",
        "clock_ramp": {"calls": ramp[0], "ms": round(ramp[1], 1)},
        "roofline": {
            "bound": "hbm",
            "kernel": "rope_kv_append_vec_kernel (tl_rope_kv_append)",
            "achieved": gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": gbs / HBM_PEAK_GBS,
            "traffic": profile_traffic(f"rope_kv_append_{workload}.md"),
            "algorithmic_bytes": nbytes,
            "kernel_ms": ms,
        },
    }
    if cpu:
        # The oracle's restatement of the same append on host storage: q and
        # k rotated in fp32 and rounded to the storage type, k and v written
        # into an empty cache; whole workload, repeated for cpu_budget_s.
        kc_h = np.zeros((B, Hkv, S, D), kn.dtype)
        vc_h = np.zeros((B, Hkv, S, D), vn.dtype)
        pos = np.arange(S)[:, None]
        passes, t_total = [], 0.0
        while t_total < cpu_budget_s or len(passes) < 3:
            t0 = time.perf_counter()
            for b in range(B):
                orope.apply_rope_storage(q[b], cos, sin, pos, dt)
                kc_h[b] = np.swapaxes(orope.apply_rope_storage(kn[b], cos, sin, pos, dt), 0, 1)
                vc_h[b] = np.swapaxes(vn[b], 0, 1)
            passes.append(time.perf_counter() - t0)
            t_total += passes[-1]
        t = float(np.median(passes))
        res["cpu_baseline"] = {
            "value": nbytes / t / 1e9, "unit": "GB/s", "cores": 1, "host": cpu_host(), "kind": "port",
            "sample": f"the whole workload ({B} x {S} tokens), the oracle's NumPy RoPE + cache write "
                      f"(oracle/rope.py apply_rope_storage; elementwise NumPy, one thread), median of "
                      f"{len(passes)} passes ({t_total:.1f}s); bytes counted as the GPU's",
        }
    return res


def copy_probe(mib):
    """Five plain device-to-device copies of ``mib`` MiB each (one blit kernel
    per copy): a dispatch of known HBM traffic -- mib MiB read, mib MiB
    written -- that scales the FETCH_SIZE / WRITE_SIZE counters."""
    from triton_llm import gpu

    n = mib << 20
    src = gpu.zeros((n,), np.uint8)
    dst = gpu.allocate((n,), np.uint8)
    lib = gpu.runtime()
    for _ in range(5):
        assert lib.tl_memcpy_dtod(dst.ptr, src.ptr, n) == 0
    gpu.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "copies": 5}))


SAMPLE_MODES = {"greedy": (0.0, 0), "t0.8": (0.8, 0), "t0.8_k50": (0.8, 50)}


def bench_gemm_case(model, dt, M, steps):
    """One GEMM layer case only, for rocprofv3: ``steps`` grouped one-layer
    projection passes (gemm_grouped q/k/v, gemm o, gemm_grouped gate/up, gemm
    down) of ``model`` in ``dt`` at M rows, weights rotated over >= 1 GB of
    copies for M <= 64 (decoded tokens) as in bench_gemm."""
    from triton_llm import gpu
    from triton_llm.kernels import gemm, gemm_grouped

    e, q, kv, inter = GEMM_MODELS[model]
    shapes = {"q": (e, q), "k": (e, kv), "v": (e, kv), "o": (q, e), "gate": (e, inter), "up": (e, inter),
              "down": (inter, e)}
    gdt, esz = (np.float32, 4) if dt == "float32" else (gpu.bfloat16, 2)
    rng = np.random.default_rng(0)

    def host(shape):
        x = rng.standard_normal(shape, dtype=np.float32)
        return (x.view(np.uint32) >> 16).astype(np.uint16) if dt == "bfloat16" else x

    layer_w = sum(K * N for K, N in shapes.values()) * esz
    reps = max(1, int(np.ceil(1e9 / layer_w))) if M <= 64 else 1
    W = [{name: gpu.to_device(host(shape), gdt) for name, shape in shapes.items()} for _ in range(reps)]
    x = {d: gpu.to_device(host((M, d)), gdt) for d in {e, q, inter}}
    out = {name: gpu.allocate((M, N), gdt) for name, (K, N) in shapes.items()}
    for i in range(steps):
        w = W[i % reps]
        gemm_grouped(x[e], [w["q"], w["k"], w["v"]], [out["q"], out["k"], out["v"]])
        gemm(x[q], w["o"], out_dev=out["o"])
        gemm_grouped(x[e], [w["gate"], w["up"]], [out["gate"], out["up"]])
        gemm(x[inter], w["down"], out_dev=out["down"])
    gpu.synchronize()
    log(f"gemm case {model} {dt} M={M}: {steps} grouped layers")


def bench_sample_case(vocab, rows, mode, steps):
    """One sampling case only, for rocprofv3: ``steps`` calls of
    sample_rows on fp32 logits (rows, vocab)."""
    from triton_llm import gpu
    from triton_llm.kernels import sample_rows

    rng = np.random.default_rng(0)
    T, k = SAMPLE_MODES[mode]
    x = gpu.to_device((3.0 * rng.standard_normal((rows, vocab))).astype(np.float32))
    u = gpu.to_device(rng.random(rows))
    tok = gpu.allocate((rows,), np.int32)
    for _ in range(steps):
        sample_rows(x, T, k, uniforms=u, out_dev=tok)
    gpu.synchronize()
    log(f"sample case vocab={vocab} rows={rows} {mode}: {steps} calls")


def bench_sample(steps, warmup, cpu=True, vocabs=(49152, 128256)):
    """Next-token sampling (tl_sample) on fp32 logits at SmolLM2's and
    Llama-3.2's vocabularies: event-timed kernel time per call for 1 and 64
    rows, greedy / temperature 0.8 / temperature 0.8 with top_k 50, and the
    wall time of one ``sample()`` per token from Python (draw upload, kernel,
    token download).  Algorithmic bytes: the logits read once.  The CPU
    baseline is the reference's host ``_sample`` (NumPy) on one row, without
    the logits download it also needs."""
    from oracle import sample as osm
    from triton_llm import gpu
    from triton_llm.kernels import sample, sample_rows

    lib = gpu.runtime()
    rng = np.random.default_rng(0)
    modes = tuple((name, T, k) for name, (T, k) in SAMPLE_MODES.items())
    out = []
    for V in vocabs:
        for rows in (1, 64):
            x = gpu.to_device((3.0 * rng.standard_normal((rows, V))).astype(np.float32))
            u = gpu.to_device(rng.random(rows))
            tok = gpu.allocate((rows,), np.int32)
            for name, T, k in modes:
                for _ in range(warmup):
                    sample_rows(x, T, k, uniforms=u, out_dev=tok)
                ev = Events(lib, 2)
                ev.record(0)
                for _ in range(steps):
                    sample_rows(x, T, k, uniforms=u, out_dev=tok)
                ev.record(1)
                ms = ev.ms(0, 1) / steps
                ev.close()
                nbytes = rows * V * 4
                out.append({"vocab": V, "rows": rows, "mode": name, "us": ms * 1e3,
                            "gbs": nbytes / (ms * 1e-3) / 1e9})
                log(f"sample V={V} rows={rows} {name}: {ms * 1e3:.1f} us")
        x1 = gpu.to_device((3.0 * rng.standard_normal((1, V))).astype(np.float32))
        for name, T, k in modes:
            for _ in range(5):
                sample(x1, T, k)
            t0 = time.perf_counter()
            for _ in range(steps):
                sample(x1, T, k)
            us = (time.perf_counter() - t0) / steps * 1e6
            out.append({"vocab": V, "rows": 1, "mode": name, "python_call_us": us})
            log(f"sample() V={V} {name}: {us:.1f} us per token from Python")
    res = {"metric": "next-token sampling (tl_sample)", "rows": out}
    if cpu:
        cpu_rows = []
        for V in vocabs:
            row = (3.0 * rng.standard_normal(V)).astype(np.float32)
            for name, T, k in modes:
                n = 50
                t0 = time.perf_counter()
                for _ in range(n):
                    if T > 0:
                        np.random.choice(V, p=osm.probs_ref(row, T, k))
                    else:
                        np.argmax(row)
                cpu_rows.append({"vocab": V, "mode": name, "us": (time.perf_counter() - t0) / n * 1e6})
        res["cpu_baseline"] = {"rows": cpu_rows, "cores": 1, "kind": "port",
                               "sample": "the reference's _sample on one host row, 50 calls per case"}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="all",
                    help="all (default: every BASELINE config, headline 5b, plus the prompt-size RoPE + "
                         "KV append of 5a and 3, 5a at 2048 tokens and 3 at batch 1), 5 (5a + 5b), append "
                         "(both appends), or one of 1 2 3 4 5a 5b append-5a append-3 5a-2048 3-b1")
    # The GPU's shader clock climbs over the first tens of milliseconds of
    # sustained load: each config first runs its own step untimed for this long
    # (measured: 5 warm-up steps alone left 5a ~10% slow).
    ap.add_argument("--clock-ramp-ms", type=float, default=200.0)
    ap.add_argument("--cpu-budget-s", type=float, default=4.0,
                    help="CPU time per config for the NumPy baseline (at least 3 passes)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gemm", action="store_true",
                    help="time the model's projection GEMMs (tl_gemm) instead of attention")
    ap.add_argument("--gemm-rocblas", action="store_true",
                    help="with --gemm: also time rocBLAS (rocblas_gemm_ex through its C API, the "
                         "seven calls back to back on the library stream) at the prompt size, as a "
                         "reference point; the library itself never calls rocBLAS")
    ap.add_argument("--sample", action="store_true",
                    help="time next-token sampling (tl_sample) instead of attention")
    ap.add_argument("--sample-case", default="",
                    help="VOCAB,ROWS,MODE (mode: greedy, t0.8, t0.8_k50): run only --steps calls "
                         "of that sampling case (for rocprofv3) and exit")
    ap.add_argument("--gemm-case", default="",
                    help="MODEL,DTYPE,M (e.g. llama3.2-3b,float32,1): run only --steps grouped "
                         "projection layers of that case (for rocprofv3) and exit")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="only run 5 device-to-device copies of this many MiB (the known-size "
                         "reference for calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--decode-split", type=int, default=0,
                    help="positions per decode split (multiple of 16); 0 = the library's choice")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only; the attention path does not "
                                   "shard across GPUs in this build",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    from oracle import inputs as oi
    from triton_llm import gpu

    gpu.synchronize()  # initialise
    if args.copy_probe_mb:
        copy_probe(args.copy_probe_mb)
        return
    cpu = not args.no_cpu
    if args.sample_case:
        vocab, rows, mode = args.sample_case.split(",")
        bench_sample_case(int(vocab), int(rows), mode, args.steps)
        return
    if args.gemm_case:
        model, dt, m = args.gemm_case.split(",")
        bench_gemm_case(model, dt, int(m), args.steps)
        return
    if args.sample:
        print(json.dumps(bench_sample(min(args.steps, 50), min(args.warmup, 5), cpu=cpu)))
        return
    if args.gemm:
        print(json.dumps(bench_gemm(min(args.steps, 20), min(args.warmup, 5), cpu=cpu,
                                    vs_rocblas=args.gemm_rocblas)))
        return
    sel = {"5": ["5a", "5b"], "all": ["1", "2", "3", "4", "5a", "5b", "append-5a", "append-3", "5a-2048", "3-b1"],
           "append": ["append-5a", "append-3"]}.get(args.config, [args.config])
    results = {}
    for name in sel:
        if name in APPEND_CASES:
            log(f"config {name}: {APPEND_CASES[name][1]}")
            results[name] = bench_append(name, args.steps, args.warmup, cpu=cpu,
                                         cpu_budget_s=args.cpu_budget_s, ramp_ms=args.clock_ramp_ms)
            results[name]["workload"] = APPEND_CASES[name][1]
            gpu.empty_cache()
            log(f"config {name}: {results[name]['value']:.1f} GB/s "
                f"({results[name]['roofline']['frac'] * 100:.1f}% of roofline)")
            continue
        cfg = prefill_extra(name) if name in PREFILL_EXTRA else oi.CONFIGS[name]
        log(f"config {name}: {cfg.name}")
        kw = dict(cpu=cpu, cpu_budget_s=args.cpu_budget_s, ramp_ms=args.clock_ramp_ms)
        if cfg.kind == "decode":
            cache_mb = 2 * cfg.batch * cfg.n_kv_head * cfg.max_ctx * cfg.d_k * (4 if cfg.dtype == "float32" else 2) / 1e6
            replicas = max(1, int(np.ceil(1024 / cache_mb))) if cache_mb < 1024 else 1
            results[name] = bench_decode(cfg, args.steps, args.warmup, replicas=replicas,
                                         split=args.decode_split, **kw)
        else:
            # Q, K, V and O of one step; replicas so that >= 1 GB of other
            # inputs passes between two uses of one set (MALL is 256 MB).
            set_mb = (2 * cfg.n_head + 2 * cfg.n_kv_head) * cfg.batch * cfg.seq * cfg.d_k * (4 if cfg.dtype == "float32" else 2) / 1e6
            replicas = max(1, int(np.ceil(1024 / set_mb))) if set_mb < 1024 else 1
            results[name] = bench_prefill(cfg, args.steps, args.warmup, replicas=replicas, **kw)
        results[name]["workload"] = cfg.name
        gpu.empty_cache()
        log(f"config {name}: {results[name]['value']:.1f} {results[name]['unit']} "
            f"({results[name]['roofline']['frac'] * 100:.1f}% of roofline)")

    head = "5b" if "5b" in results else sel[0]
    r = results[head]
    if head in PREFILL_EXTRA:
        cfg = prefill_extra(head)
    else:
        cfg = oi.CONFIGS[APPEND_CASES[head][0] if head in APPEND_CASES else head]
    line = {
        "metric": METRIC,
        "value": r["value"],
        "unit": r["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DT_SHORT[cfg.dtype],
        "data": "synthetic (seeded N(0,1) q/k/v per BASELINE config; decode lengths drawn U[lo, hi])",
        "config": {
            "workload": (r["workload"] if head in APPEND_CASES else f"{cfg.name} (config {head})")
                        + (" + llama3.2-3b-prefill-bf16 (config 5a)" if "5a" in results and head == "5b" else ""),
            "batch": cfg.batch, "n_head": cfg.n_head, "n_kv_head": cfg.n_kv_head, "d_k": cfg.d_k,
            "max_ctx": cfg.max_ctx or None, "seq": cfg.seq or None,
        },
        "roofline": r["roofline"],
    }
    if "cpu_baseline" in r:
        line["cpu_baseline"] = r["cpu_baseline"]
    line["clock_ramp"] = {"ms": args.clock_ramp_ms,
                          "note": "untimed steps of the same workload before the warm-up steps"}
    if "5a" in results and head != "5a":
        line["prefill"] = results["5a"]
    if len(results) > 1:
        line["configs"] = {k: v for k, v in results.items()}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
