"""HIP graph capture and replay (tl_graph_*, gpu.capture): a recorded decode
step and a recorded prefill call, replayed several times with eager work
and synchronisation between the replays, give exactly the eager result every
time (the kernels are deterministic, so bit-equal)."""

import ctypes

import numpy as np
import pytest

from oracle import inputs as oi
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import attention_decode, flash_attention, rope_kv_append
from triton_llm.kernels.decode import decode_workspace

pytestmark = pytest.mark.gpu


def _eager_noise():
    # unrelated eager work on the same stream between replays
    a = gpu.to_device(np.arange(4096, dtype=np.float32))
    b = gpu.allocate((4096,), np.float32)
    gpu.copy_(b, a)
    gpu.synchronize()


def test_graph_replays_decode_step():
    cfg = oi.scaled(oi.CONFIGS["4"], batch=6, max_ctx=640, lo=1, hi=600, seed=41)
    dt = cfg.dtype
    B, Hq, Hkv, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.d_k
    print(f"[case] graph decode B={B} Hq={Hq} Hkv={Hkv} D={D} {dt}", flush=True)
    d = oi.make_decode(cfg, fill="zero")
    cos, sin = oi.rope_tables(cfg)
    q0 = H.upload(d["q"], dt)
    q = H.upload(d["q"], dt)
    kn, vn = H.upload(d["k_new"], dt), H.upload(d["v_new"], dt)
    kc, vc = H.upload(d["k_cache"], dt), H.upload(d["v_cache"], dt)
    lens = gpu.to_device(d["lens"])
    cos_d, sin_d = gpu.to_device(cos), gpu.to_device(sin)
    out = gpu.allocate((B, Hq, D), q.dtype)
    ws = decode_workspace(B, Hq, Hkv, cfg.max_ctx, D)

    def step():
        gpu.copy_(q, q0)  # RoPE rotates q in place: start every step from the same q
        rope_kv_append(q, kn, vn, kc, vc, lens, cos_d, sin_d)
        attention_decode(q, kc, vc, lens, Hq, Hkv, sm_scale=cfg.scale, len_add=1, out=out, workspace=ws)

    step()
    want = H.download(out).copy()
    with gpu.capture() as g:
        step()
    for rep in range(4):
        gpu.copy_(out, gpu.zeros(out.shape, out.dtype))
        g.replay()
        got = H.download(out)
        np.testing.assert_array_equal(got, want, err_msg=f"replay {rep}")
        _eager_noise()


def test_graph_replays_prefill():
    dt = "bfloat16"
    cfg = oi.Config("graph-prefill", "prefill", dt, 1, 6, 2, 128, 43, 0.088, seq=700)
    raw = oi.make_prefill_raw(cfg)
    print(f"[case] graph prefill S={cfg.seq} {dt}", flush=True)
    q, k, v = H.upload(raw["q"], dt), H.upload(raw["k"], dt), H.upload(raw["v"], dt)
    out = gpu.allocate(q.shape, q.dtype)
    flash_attention(q, k, v, causal=True, sm_scale=cfg.scale, out=out)
    want = H.download(out).copy()
    with gpu.capture() as g:
        flash_attention(q, k, v, causal=True, sm_scale=cfg.scale, out=out)
    for rep in range(4):
        gpu.copy_(out, gpu.zeros(out.shape, out.dtype))
        g.replay()
        np.testing.assert_array_equal(H.download(out), want, err_msg=f"replay {rep}")
        _eager_noise()


def test_recorded_and_captured_launches_keep_their_workspace():
    """A recorded launcher and a captured graph hold raw pointers to the shared
    few-row GEMM workspace.  A later, larger product grows (replaces) that
    workspace; the old buffer must stay with the launcher / graph, so their
    replays still compute the right product and do not write into memory the
    larger product's call now uses."""
    from oracle.gemm import gemm_ref
    from triton_llm.kernels import _common, gemm
    from triton_llm.kernels._common import record, shared_workspace

    _common._shared.pop("gemm", None)  # start from the smallest workspace, whatever ran before
    rng = np.random.default_rng(8)
    print("[case] workspace keep-alive: launcher and graph, then a growing gemm", flush=True)
    a = rng.standard_normal((1, 3072), dtype=np.float32)
    b = (rng.standard_normal((3072, 1024), dtype=np.float32) / 64).astype(np.float32)
    a_d, b_d = gpu.to_device(a), gpu.to_device(b)
    out_l = gpu.allocate((1, 1024), np.float32)
    out_g = gpu.allocate((1, 1024), np.float32)
    gemm(a_d, b_d, out_dev=out_l)  # warm
    launcher = record(lambda: gemm(a_d, b_d, out_dev=out_l))
    with gpu.capture() as g:
        gemm(a_d, b_d, out_dev=out_g)
    before = shared_workspace("gemm", 1).ptr.value
    # a product whose split-K partials need far more workspace: the shared
    # buffer is replaced by a larger one
    big_a = rng.standard_normal((8, 8192), dtype=np.float32)
    big_b = (rng.standard_normal((8192, 16384), dtype=np.float32) / 90).astype(np.float32)
    big_a_d, big_b_d = gpu.to_device(big_a), gpu.to_device(big_b)
    big_out = gemm(big_a_d, big_b_d)
    assert shared_workspace("gemm", 1).ptr.value != before, "the workspace did not grow"
    exp = gemm_ref(a, b)
    for rep in range(3):
        launcher()
        g.replay()
        big_out2 = gemm(big_a_d, big_b_d)
        gpu.synchronize()
        for name, t in (("launcher", out_l), ("graph", out_g)):
            err = H.max_abs(t.to_numpy(), exp)
            H.report(f"keep-alive {name} rep {rep}", err, 2e-3)
            assert err <= 2e-3
        np.testing.assert_array_equal(big_out2.to_numpy(), big_out.to_numpy())


def test_memset_fills_bytes_at_any_alignment():
    """tl_memset is a fill kernel (16-byte stores over the aligned middle,
    single bytes for an unaligned head and tail): every offset and length
    sets exactly its bytes."""
    rt = gpu.runtime()
    base = gpu.allocate((4096,), np.uint8)
    print("[case] memset offsets/lengths", flush=True)
    for off in (0, 1, 3, 15, 16, 17):
        for n in (1, 7, 15, 16, 17, 100, 1000, 3000):
            base.from_numpy(np.zeros(4096, np.uint8))
            ptr = ctypes.c_void_p(base.ptr.value + off)
            assert rt.tl_memset(ptr, 0xAB, n) == 0
            got = base.to_numpy()
            exp = np.zeros(4096, np.uint8)
            exp[off:off + n] = 0xAB
            np.testing.assert_array_equal(got, exp, err_msg=f"offset {off} length {n}")


def test_graph_replays_fill():
    """A fill recorded in a graph is a kernel node: each replay zeroes the
    buffer again after eager work dirtied it."""
    rt = gpu.runtime()
    buf = gpu.allocate((1 << 16,), np.float32)
    ones = np.ones(1 << 16, np.float32)
    print("[case] graph fill", flush=True)
    buf.from_numpy(ones)
    with gpu.capture() as g:
        assert rt.tl_memset(buf.ptr, 0, buf.nbytes) == 0
    for rep in range(3):
        buf.from_numpy(ones)
        g.replay()
        assert not buf.to_numpy().any(), f"replay {rep}"
        _eager_noise()
