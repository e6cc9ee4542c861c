"""Decode over the resident KV cache (configs 2, 4, 5b and edge cases) against
the oracle.  Positions past each sequence's length hold NaN, so any read of
them would poison the output.  Tolerance: 2e-2 max-abs for 16-bit, 2e-3 fp32.
"""

import numpy as np
import pytest

from oracle import attention as oa
from oracle import inputs as oi
from oracle import numerics as on
from oracle import rope as orope
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import attention_decode, decode_step, precompute_cos_sin, rope_kv_append

pytestmark = pytest.mark.gpu

TOL = {"float32": 2e-3, "float16": 2e-2, "bfloat16": 2e-2}

# Small caches (max_ctx <= 2048, <= 64 MiB of K/V) run one workgroup per
# (sequence, KV head) that finishes its pair ("pair"); larger ones equal
# shares of all positions plus a combine ("shares").  This variable forces
# the shares path, so the edge cases below run on both.
SHARES_ENV = "TRITON_LLM_HIP_DECODE_SHARES"
MODES = ["pair", "shares"]


def set_mode(monkeypatch, mode):
    H.set_override(monkeypatch, SHARES_ENV, 1 if mode == "shares" else None)


def run_decode_step(cfg, data, batches=None, split=0):
    """GPU: append (+RoPE) then attend over len + 1.  Oracle on the same inputs.

    Returns (gpu_out_f32, oracle_out, appended caches from the GPU)."""
    dt = cfg.dtype
    B, Hq, Hkv, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.d_k
    lens = data["lens"]
    cos, sin = oi.rope_tables(cfg)
    q_d = H.upload(data["q"], dt)
    kc_d, vc_d = H.upload(data["k_cache"], dt), H.upload(data["v_cache"], dt)
    lens_d = gpu.to_device(lens)
    cos_d = gpu.to_device(cos) if cos is not None else None
    sin_d = gpu.to_device(sin) if sin is not None else None
    print(f"[case] {cfg.name} B={B} Hq={Hq} Hkv={Hkv} D={D} max_ctx={cfg.max_ctx} "
          f"lens=[{lens.min()},{lens.max()}] split={split}", flush=True)
    out_d = decode_step(q_d, H.upload(data["k_new"], dt), H.upload(data["v_new"], dt), kc_d, vc_d,
                        lens_d, Hq, Hkv, cos_d, sin_d, sm_scale=cfg.scale, split=split)
    got = on.from_storage(H.download(out_d), dt)

    # Oracle: the same append on host storage, then attention over len + 1.
    q = data["q"].copy()
    kc, vc = data["k_cache"], data["v_cache"]
    for b in range(B):
        p = int(lens[b])
        if cos is not None:
            q[b] = orope.apply_rope_storage(data["q"][b], cos, sin, p, dt)
            kc[b, :, p] = orope.apply_rope_storage(data["k_new"][b], cos, sin, p, dt)
        else:
            kc[b, :, p] = data["k_new"][b]
        vc[b, :, p] = data["v_new"][b]
    exp = oa.decode_ref(q, kc, vc, lens + 1, sm_scale=cfg.scale, dtype=dt, batches=batches)
    # q is rotated in place, bit for bit as the oracle rotates it
    np.testing.assert_array_equal(H.download(q_d).view(np.uint8), q.view(np.uint8))
    return got, exp, kc_d, vc_d


def compare(name, got, exp, tol, batches=None):
    sel = slice(None) if batches is None else list(batches)
    g, e = got[sel], exp[sel]
    assert np.all(np.isfinite(got)), f"{name}: non-finite output"
    err = H.max_abs(g, e)
    H.report(name, err, tol)
    assert err <= tol


def assert_caches_bitwise(kc_d, vc_d, data):
    """The GPU K and V caches after the append equal the oracle's bit for
    bit at every position: the appended rows (RoPE'd K, raw V), the cached
    prefix, and the NaN-filled tail, which must stay untouched."""
    for name, dev in (("k_cache", kc_d), ("v_cache", vc_d)):
        got = H.download(dev).view(np.uint16)
        exp = data[name].view(np.uint16)
        mismatch = int(np.count_nonzero(got != exp))
        print(f"[bits] {name}: {mismatch} of {exp.size} elements differ", flush=True)
        assert mismatch == 0, f"{name}: {mismatch} elements differ"
        del got


@pytest.mark.parametrize("name", ["2", "4"])
def test_decode_config_full(name):
    cfg = oi.CONFIGS[name]
    data = oi.make_decode(cfg, fill="nan")
    got, exp, kc_d, vc_d = run_decode_step(cfg, data)
    compare(f"config{name}", got, exp, TOL[cfg.dtype])
    assert_caches_bitwise(kc_d, vc_d, data)


def test_decode_config_5b_full():
    """Config 5b at full size: all 64 sequences against the oracle, and both
    2.1 GB caches bitwise after the RoPE + append."""
    cfg = oi.CONFIGS["5b"]
    data = oi.make_decode(cfg, fill="nan")
    got, exp, kc_d, vc_d = run_decode_step(cfg, data)
    compare("config5b", got, exp, TOL[cfg.dtype])
    assert_caches_bitwise(kc_d, vc_d, data)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("group,d_k", [(1, 64), (3, 128), (4, 64), (8, 128), (12, 64)])
def test_decode_shapes_and_dtypes(monkeypatch, mode, dtype, group, d_k):
    set_mode(monkeypatch, mode)
    Hkv = 2
    cfg = oi.Config("decode-edge", "decode", dtype, 5, Hkv * group, Hkv, d_k, 11, 0.3,
                    max_ctx=300, lo=0, hi=299, rope_theta=1e4)
    lens = oi.draw_lens(cfg)
    lens[:3] = [0, 299, 15]  # empty prefix, full cache, short
    data = oi.make_decode(cfg, fill="nan", lens=lens)
    got, exp, _, _ = run_decode_step(cfg, data, split=32)
    compare(f"edge {mode} {dtype} g{group} d{d_k}", got, exp, TOL[dtype])


@pytest.mark.parametrize("mode", MODES)
def test_decode_without_append_and_len_zero_gives_zeros(monkeypatch, mode):
    set_mode(monkeypatch, mode)
    dt = "bfloat16"
    cfg = oi.Config("decode-noappend", "decode", dt, 4, 6, 2, 64, 5, 0.125, max_ctx=128, lo=1, hi=127)
    lens = oi.draw_lens(cfg)
    lens[0] = 0
    data = oi.make_decode(cfg, fill="nan", lens=lens)
    lens_d = gpu.to_device(data["lens"])
    out = attention_decode(H.upload(data["q"], dt), H.upload(data["k_cache"], dt), H.upload(data["v_cache"], dt),
                           lens_d, 6, 2, sm_scale=0.125, len_add=0)
    got = on.from_storage(H.download(out), dt)
    exp = oa.decode_ref(data["q"], data["k_cache"], data["v_cache"], data["lens"], sm_scale=0.125, dtype=dt)
    assert np.all(got[0] == 0)
    compare("no-append", got, exp, TOL[dt])


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("n_head,n_kv,d_k", [(2, 2, 64), (6, 2, 64), (3, 1, 128)])
def test_decode_iteration_boundary_lengths(monkeypatch, mode, dtype, n_head, n_kv, d_k):
    """Lengths at and around the kernels' iteration sizes: a pair-mode
    workgroup takes 512 or 1024 keys per full iteration (8- or 16-lane rows),
    an equal-share workgroup 64; positions past each length hold NaN, and a
    zero length gives zeros."""
    set_mode(monkeypatch, mode)
    lens = np.array([0, 1, 63, 64, 65, 127, 128, 511, 512, 513, 1023, 1024, 1025, 2047, 2048], np.int32)
    print(f"[case] decode boundary lengths {mode} {dtype} Hq{n_head} Hkv{n_kv} d{d_k}", flush=True)
    cfg = oi.Config("decode-bounds", "decode", dtype, len(lens), n_head, n_kv, d_k, 41, 1 / np.sqrt(d_k),
                    max_ctx=2048, lo=1, hi=2047)
    data = oi.make_decode(cfg, fill="nan", lens=lens)
    out = attention_decode(H.upload(data["q"], dtype), H.upload(data["k_cache"], dtype),
                           H.upload(data["v_cache"], dtype), gpu.to_device(data["lens"]), n_head, n_kv,
                           sm_scale=cfg.scale, len_add=0)
    got = on.from_storage(H.download(out), dtype)
    exp = oa.decode_ref(data["q"], data["k_cache"], data["v_cache"], data["lens"], sm_scale=cfg.scale, dtype=dtype)
    assert np.all(got[0] == 0)
    compare(f"boundary-lens {mode} {dtype}", got[1:], exp[1:], TOL[dtype])


@pytest.mark.parametrize("split", [16, 64, 256, 2048])
def test_decode_split_sizes_agree(monkeypatch, split):
    H.set_override(monkeypatch, SHARES_ENV, 1)  # split sizes apply to the shares path
    cfg = oi.scaled(oi.CONFIGS["4"], batch=6, max_ctx=2048, lo=1, hi=2047)
    data = oi.make_decode(cfg, fill="nan")
    got, exp, _, _ = run_decode_step(cfg, data, split=split)
    compare(f"split{split}", got, exp, TOL[cfg.dtype])


@pytest.mark.parametrize("cus,batch", [(1, 70), (3, 9), (7, 66)])
def test_decode_few_workgroups_span_many_sequences(monkeypatch, cus, batch):
    """Capping the device at a few compute units leaves a handful of
    workgroups, so each share crosses many (sequence, head) pairs and most
    pairs are split between two shares; batches above 64 take the lengths
    scan in several chunks.  Some sequences hold only the appended token, one
    fills the cache."""
    H.set_override(monkeypatch, "TRITON_LLM_HIP_MAX_CUS", cus)
    H.set_override(monkeypatch, SHARES_ENV, 1)
    cfg = oi.scaled(oi.CONFIGS["4"], batch=batch, max_ctx=640, lo=0, hi=639)
    lens = oi.draw_lens(cfg)
    lens[: min(4, batch)] = [0, 639, 1, 0][: min(4, batch)]
    data = oi.make_decode(cfg, fill="nan", lens=lens)
    got, exp, _, _ = run_decode_step(cfg, data, split=16)
    compare(f"cus{cus} b{batch}", got, exp, TOL[cfg.dtype])


@pytest.mark.parametrize("mode", MODES)
def test_decode_all_sequences_empty_over_64(monkeypatch, mode):
    """Every length 0 (no append).  Shares: the split kernel finds no
    positions and exits, the combine writes zeros for all heads, and 70
    sequences take the lengths scan in two chunks.  Pair: each workgroup
    finds an empty pair and writes its zeros."""
    set_mode(monkeypatch, mode)
    dt = "bfloat16"
    cfg = oi.Config("decode-empty", "decode", dt, 70, 6, 2, 64, 5, 0.125, max_ctx=64, lo=0, hi=0)
    lens = np.zeros(70, np.int32)
    data = oi.make_decode(cfg, fill="nan", lens=lens)
    out = attention_decode(H.upload(data["q"], dt), H.upload(data["k_cache"], dt), H.upload(data["v_cache"], dt),
                           gpu.to_device(lens), 6, 2, sm_scale=0.125, len_add=0)
    got = on.from_storage(H.download(out), dt)
    assert np.all(got == 0)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("dtype,group,d_k,rope", [("float16", 1, 64, False), ("bfloat16", 3, 64, True),
                                                  ("bfloat16", 12, 128, True), ("float32", 2, 128, True)])
def test_decode_step_fused_equals_append_then_decode(monkeypatch, mode, dtype, group, d_k, rope):
    """decode_step (one tl_attention_decode_append call: in the small-cache
    mode the append runs inside the decode kernel) against rope_kv_append
    followed by attention_decode on copies of the same inputs: q, both
    caches and the output agree bit for bit.  Lengths include 0, max_ctx - 1
    (the token fills the cache), max_ctx (no room: nothing is written) and,
    with RoPE, positions past the table (not rotated, not written)."""
    set_mode(monkeypatch, mode)
    Hkv, max_ctx = 2, 300
    cfg = oi.Config("decode-fused", "decode", dtype, 7, Hkv * group, Hkv, d_k, 23, 0.2,
                    max_ctx=max_ctx, lo=0, hi=max_ctx - 1, rope_theta=1e4 if rope else None)
    lens = oi.draw_lens(cfg)
    lens[:4] = [0, max_ctx - 1, max_ctx, 250]
    data = oi.make_decode(cfg, fill="nan", lens=lens)
    cos, sin = oi.rope_tables(cfg)
    cos_d = sin_d = None
    if rope:
        rows = 200  # sequences at positions >= 200 are past the table
        cos_d, sin_d = gpu.to_device(np.ascontiguousarray(cos[:rows])), gpu.to_device(np.ascontiguousarray(sin[:rows]))
    lens_d = gpu.to_device(lens)
    outs = {}
    for path in ("fused", "separate"):
        q_d = H.upload(data["q"], dtype)
        kn_d, vn_d = H.upload(data["k_new"], dtype), H.upload(data["v_new"], dtype)
        kc_d, vc_d = H.upload(data["k_cache"], dtype), H.upload(data["v_cache"], dtype)
        print(f"[case] decode fused-vs-separate {mode} {dtype} g{group} d{d_k} rope={rope} {path}", flush=True)
        if path == "fused":
            o = decode_step(q_d, kn_d, vn_d, kc_d, vc_d, lens_d, cfg.n_head, Hkv, cos_d, sin_d, sm_scale=cfg.scale)
        else:
            rope_kv_append(q_d, kn_d, vn_d, kc_d, vc_d, lens_d, cos_d, sin_d)
            o = attention_decode(q_d, kc_d, vc_d, lens_d, cfg.n_head, Hkv, sm_scale=cfg.scale, len_add=1)
        outs[path] = [H.download(x).view(np.uint8) for x in (o, q_d, kc_d, vc_d)]
    for name, a, b in zip(("out", "q", "k_cache", "v_cache"), outs["fused"], outs["separate"]):
        np.testing.assert_array_equal(a, b, err_msg=name)
