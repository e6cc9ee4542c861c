"""Flash prefill (configs 1, 3, 5a and edge shapes) against the oracle.

Config 3 and 5a apply RoPE on the GPU (bit-exact, tested separately) to the
raw rounded inputs, exactly as the oracle's input recipe does on the host.
Tolerances: 2e-3 max-abs for fp32, 2e-2 for bf16/fp16.
"""

import numpy as np
import pytest

from oracle import attention as oa
from oracle import inputs as oi
from oracle import numerics as on
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import (apply_rope, attention_gqa, flash_attention, flash_attention_strided,
                                precompute_cos_sin)

pytestmark = pytest.mark.gpu

TOL = {"float32": 2e-3, "float16": 2e-2, "bfloat16": 2e-2}


@pytest.fixture(params=["w32", "w64"])
def d128_kernel(request, monkeypatch):
    """16-bit d_k 128 prefill has two kernels: 32 query rows per wave (the
    default) and 64 rows per wave (TRITON_LLM_HIP_PREFILL_W64); tests that
    take this fixture run on both.  Other d_k / dtypes have one kernel, so
    their second run is skipped."""
    H.set_override(monkeypatch, "TRITON_LLM_HIP_PREFILL_W64", 1 if request.param == "w64" else None)
    return request.param


def skip_w64_repeat(kernel, d_k, dtype="bfloat16"):
    if kernel == "w64" and (d_k != 128 or dtype == "float32"):
        pytest.skip("one prefill kernel for this d_k / dtype")


def gpu_prefill(cfg, raw, causal=True):
    dt = cfg.dtype
    B, Hq, Hkv, S, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.seq, cfg.d_k
    print(f"[case] {cfg.name} B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} {dt} causal={causal}", flush=True)
    q_d, k_d, v_d = H.upload(raw["q"], dt), H.upload(raw["k"], dt), H.upload(raw["v"], dt)
    if cfg.rope_theta is not None:
        cos, sin = precompute_cos_sin(S, D, cfg.rope_theta)
        cos_d, sin_d = gpu.to_device(cos), gpu.to_device(sin)
        apply_rope(gpu.view(q_d, (B * Hq * S, D)), cos_d, sin_d, seq_len=S)
        apply_rope(gpu.view(k_d, (B * Hkv * S, D)), cos_d, sin_d, seq_len=S)
    o_d = flash_attention(q_d, k_d, v_d, causal=causal, sm_scale=cfg.scale)
    return on.from_storage(H.download(o_d), dt)


def compare(name, got, exp, tol):
    err = H.max_abs(got, exp)
    H.report(name, err, tol)
    assert err <= tol


@pytest.mark.parametrize("name", ["1", "3"])
def test_prefill_config_full(name):
    cfg = oi.CONFIGS[name]
    got = gpu_prefill(cfg, oi.make_prefill_raw(cfg))
    ref = oi.make_prefill(cfg)
    exp = oa.attention_bhsd(ref["q"], ref["k"], ref["v"], causal=True, sm_scale=cfg.scale, dtype=cfg.dtype)
    assert np.all(np.isfinite(got))
    compare(f"config{name}", got, exp, TOL[cfg.dtype])


def test_prefill_config_5a_full_size_sampled_rows():
    cfg = oi.CONFIGS["5a"]
    got = gpu_prefill(cfg, oi.make_prefill_raw(cfg))
    assert np.all(np.isfinite(got))
    ref = oi.make_prefill(cfg)
    # Both rows either side of every 256-row query-tile boundary (255/256,
    # 511/512, ... 8191), the 128-key boundary, the first and last rows, and
    # an even spread in between.
    tile = np.arange(256, cfg.seq, 256)
    rows = np.unique(np.concatenate([np.arange(0, 8), np.arange(127, 136), tile - 1, tile,
                                     np.linspace(0, cfg.seq - 1, 48).astype(int),
                                     np.arange(cfg.seq - 8, cfg.seq)]))
    exp = oa.attention_bhsd(ref["q"], ref["k"], ref["v"], causal=True, sm_scale=cfg.scale,
                            rows=rows, dtype=cfg.dtype)
    compare("config5a(rows)", got[:, :, rows], exp[:, :, rows], TOL[cfg.dtype])


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("d_k", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ragged_shapes(d128_kernel, dtype, d_k, causal):
    # seq not a multiple of either tile size; GQA group 3; batch 2.
    skip_w64_repeat(d128_kernel, d_k, dtype)
    cfg = oi.Config("ragged", "prefill", dtype, 2, 6, 2, d_k, 21, 1 / np.sqrt(d_k), seq=200)
    raw = oi.make_prefill_raw(cfg)
    got = gpu_prefill(cfg, raw, causal=causal)
    exp = oa.attention_bhsd(raw["q"], raw["k"], raw["v"], causal=causal, sm_scale=cfg.scale, dtype=dtype)
    compare(f"ragged {dtype} d{d_k} causal={causal}", got, exp, TOL[dtype])


@pytest.mark.parametrize("d_k", [64, 128])
@pytest.mark.parametrize("sq,sk", [(1, 1), (1, 300), (37, 300), (130, 129), (64, 64), (5, 3), (300, 700)])
def test_prefill_seq_q_ne_seq_k(d128_kernel, sq, sk, d_k):
    """Bottom-right causal alignment; sq > sk leaves the first rows fully masked (NaN).
    d_k 64 reads V in place, d_k 128 through its V^T copy."""
    skip_w64_repeat(d128_kernel, d_k)
    dt = "bfloat16"
    rng = np.random.default_rng(sq * 1000 + sk + d_k)
    B, Hq, Hkv, D = 1, 4, 2, d_k
    q = on.to_storage(rng.standard_normal((B, Hq, sq, D), dtype=np.float32), dt)
    k = on.to_storage(rng.standard_normal((B, Hkv, sk, D), dtype=np.float32), dt)
    v = on.to_storage(rng.standard_normal((B, Hkv, sk, D), dtype=np.float32), dt)
    o = flash_attention(H.upload(q, dt), H.upload(k, dt), H.upload(v, dt), causal=True)
    got = on.from_storage(H.download(o), dt)
    exp = oa.attention_bhsd(q, k, v, causal=True, dtype=dt)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(exp))
    compare(f"sq{sq} sk{sk}", np.nan_to_num(got), np.nan_to_num(exp), TOL[dt])


@pytest.mark.parametrize("d_k", [64, 128])
@pytest.mark.parametrize("B,Hq,Hkv,sq,sk,causal", [
    (1, 12, 12, 128, 128, True),   # GPT-2 prompt: 12 query blocks (key-split kernel)
    (2, 6, 2, 37, 300, True),      # key-split, bottom-right causal, GQA
    (1, 4, 2, 300, 129, True),     # key-split, the first rows fully masked
    (1, 3, 3, 70, 70, False),      # key-split, non-causal, ragged
    (1, 16, 4, 600, 600, True),    # 80 blocks of 128 rows: the tiled kernel
    (1, 16, 16, 520, 520, False),  # tiled, non-causal
])
def test_prefill_fp32_paths(B, Hq, Hkv, sq, sk, causal, d_k):
    """fp32 runs the key-split kernel when fewer than 64 blocks of 128 query
    rows would run, the tiled kernel otherwise; both against the oracle."""
    dt = "float32"
    print(f"[case] fp32 B={B} Hq={Hq} Hkv={Hkv} sq={sq} sk={sk} D={d_k} causal={causal}", flush=True)
    rng = np.random.default_rng(sq * 1000 + sk + d_k + Hq)
    q = rng.standard_normal((B, Hq, sq, d_k), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, sk, d_k), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, sk, d_k), dtype=np.float32)
    o = flash_attention(H.upload(q, dt), H.upload(k, dt), H.upload(v, dt), causal=causal)
    got = H.download(o)
    exp = oa.attention_bhsd(q, k, v, causal=causal, dtype=dt)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(exp))
    compare(f"fp32 sq{sq} sk{sk} d{d_k}", np.nan_to_num(got), np.nan_to_num(exp), TOL[dt])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("d_k", [16, 32, 256, 512, 1024])
def test_prefill_generic_head_sizes(dtype, d_k):
    """Head sizes the MFMA kernels do not take run the generic kernel; the
    reference accepts any power-of-two d_k (attention_gqa.py:230-233), and
    this build computes up to 4096."""
    cfg = oi.Config("generic", "prefill", dtype, 1, 4, 2, d_k, 5, 1 / np.sqrt(d_k), seq=70)
    raw = oi.make_prefill_raw(cfg)
    got = gpu_prefill(cfg, raw)
    exp = oa.attention_bhsd(raw["q"], raw["k"], raw["v"], causal=True, sm_scale=cfg.scale, dtype=dtype)
    compare(f"generic {dtype} d{d_k}", got, exp, TOL[dtype])


def test_attention_gqa_head_size_512_and_beyond_the_limit():
    """The drop-in entry point computes d_k 512 (the reference's power-of-two
    rule) and refuses d_k above 4096 with the ValueError it documents."""
    rng = np.random.default_rng(512)
    q = rng.standard_normal((2 * 9, 512), dtype=np.float32)
    k = rng.standard_normal((1 * 9, 512), dtype=np.float32)
    v = rng.standard_normal((1 * 9, 512), dtype=np.float32)
    got = H.attention_gqa_cpu(q, k, v, 2, 1, causal=True)
    exp = oa.attention_gqa_ref(q, k, v, 2, 1, causal=True)
    compare("attention_gqa d512", got, exp, TOL["float32"])
    big = gpu.allocate((2, 8192), np.float32)
    with pytest.raises(ValueError, match="not supported"):
        attention_gqa(big, big, big, 1, 1)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d_k", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_scale_past_fp16_range(dtype, d_k, causal):
    """sm_scale 4 (4 log2 e = 5.8 in the log2 domain) with q[..., 0] = 60000
    and k[..., 0] = 0: q * sm_scale * log2 e exceeds the fp16 range (65504)
    while every score is moderate.  fp16 then scales the scores in fp32
    instead of pre-scaling Q (which would give inf * 0 = NaN); bf16 keeps
    fp32's range and pre-scales.  Both must match the oracle."""
    rng = np.random.default_rng(4000 + d_k + causal)
    B, Hq, Hkv, S = 1, 6, 2, 300
    q = 0.1 * rng.standard_normal((B, Hq, S, d_k), dtype=np.float32)
    k = 0.25 * rng.standard_normal((B, Hkv, S, d_k), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, S, d_k), dtype=np.float32)
    q[..., 0] = 60000.0
    k[..., 0] = 0.0
    q, k, v = (on.to_storage(x, dtype) for x in (q, k, v))
    print(f"[case] scale past fp16 range {dtype} d{d_k} causal={causal}", flush=True)
    o = flash_attention(H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype), causal=causal,
                        sm_scale=4.0)
    got = on.from_storage(H.download(o), dtype)
    exp = oa.attention_bhsd(q, k, v, causal=causal, sm_scale=4.0, dtype=dtype)
    assert np.all(np.isfinite(got))
    compare(f"scale 4 {dtype} d{d_k} causal={causal}", got, exp, TOL[dtype])


@pytest.mark.parametrize("d_k", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 3, 4, 8])
def test_prefill_gqa_groups(group, d_k):
    dt = "bfloat16"
    cfg = oi.Config("groups", "prefill", dt, 1, 2 * group, 2, d_k, 30 + group, 1 / np.sqrt(d_k), seq=256)
    raw = oi.make_prefill_raw(cfg)
    got = gpu_prefill(cfg, raw)
    exp = oa.attention_bhsd(raw["q"], raw["k"], raw["v"], causal=True, sm_scale=cfg.scale, dtype=dt)
    compare(f"group{group} d{d_k}", got, exp, TOL[dt])


def test_prefill_reads_cache_layout_and_seq_major_rows():
    """K/V straight from a (B, Hkv, max_ctx, D) cache; Q and O as (B, S, Hq*D) rows."""
    dt = "bfloat16"
    rng = np.random.default_rng(3)
    B, Hq, Hkv, S, D, C = 2, 6, 2, 150, 64, 512
    q_rows = on.to_storage(rng.standard_normal((B, S, Hq, D), dtype=np.float32), dt)
    kc = on.to_storage(rng.standard_normal((B, Hkv, C, D), dtype=np.float32), dt)
    vc = on.to_storage(rng.standard_normal((B, Hkv, C, D), dtype=np.float32), dt)
    q_d, kc_d, vc_d = H.upload(q_rows, dt), H.upload(kc, dt), H.upload(vc, dt)
    o_d = gpu.allocate((B, S, Hq, D), gpu.bfloat16)
    flash_attention_strided(
        q_d, kc_d, vc_d, o_d, batch=B, n_head=Hq, n_kv_head=Hkv, seq_q=S, seq_k=S, d_k=D,
        q_strides=(S * Hq * D, D, Hq * D), k_strides=(Hkv * C * D, C * D, D),
        v_strides=(Hkv * C * D, C * D, D), o_strides=(S * Hq * D, D, Hq * D), causal=True)
    got = on.from_storage(H.download(o_d), dt).transpose(0, 2, 1, 3)
    exp = oa.attention_bhsd(q_rows.transpose(0, 2, 1, 3), kc[:, :, :S], vc[:, :, :S], causal=True, dtype=dt)
    compare("cache-layout", got, exp, TOL[dt])


@pytest.mark.parametrize("cus,seq_q,seq_k,n_head,n_kv,causal", [
    (16, 1536, 1536, 8, 8, True),    # 2 workgroups per XCD list, 3 rounds: balanced-triple order
    (16, 1024, 1024, 8, 8, True),    # 2 rounds: alternating order
    (16, 1280, 1280, 8, 8, False),   # 5 tiles on 2 workgroups: partial last round
    (24, 1536, 256, 16, 8, True),    # bottom-right causal: tiles with no visible key between others
    (8, 768, 768, 6, 2, True),       # 2 (batch, kv) units: one list, 3 workgroups
    (16, 2048, 2048, 6, 2, True),    # 6 heads in 8 lists: 4 parts per head (qt % 4), 3 parts per list
    (16, 1024, 1024, 12, 4, True),   # 12 heads: 2 parts per head, lists cut inside a (batch, kv) unit
    (8, 2048, 2048, 9, 3, False),    # 9 heads, 8 parts per head of one tile each, one workgroup per list
])
@pytest.mark.parametrize("d_k", [64, 128])
def test_prefill_persistent_schedules(monkeypatch, d128_kernel, cus, seq_q, seq_k, n_head, n_kv, causal, d_k):
    """The persistent kernel walks several query tiles per workgroup (forced by capping the CU
    count), switching tiles with prefetched Q / K and, after a tile with no visible key, cold;
    d_k 64 and 128 (different LDS tile sizes and load slots)."""
    skip_w64_repeat(d128_kernel, d_k)
    H.set_override(monkeypatch, "TRITON_LLM_HIP_MAX_CUS", cus)
    dtype = "bfloat16"
    cfg = oi.Config("sched", "prefill", dtype, 1, n_head, n_kv, d_k, 77, 1 / np.sqrt(d_k), seq=seq_q)
    print(f"[case] persistent cus={cus} sq={seq_q} sk={seq_k} Hq={n_head} Hkv={n_kv} causal={causal} "
          f"d_k={d_k}", flush=True)
    rng = np.random.default_rng(cus + seq_q + seq_k)
    q = on.to_storage(rng.standard_normal((1, n_head, seq_q, d_k), dtype=np.float32), dtype)
    k = on.to_storage(rng.standard_normal((1, n_kv, seq_k, d_k), dtype=np.float32), dtype)
    v = on.to_storage(rng.standard_normal((1, n_kv, seq_k, d_k), dtype=np.float32), dtype)
    o_d = flash_attention(H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype), causal=causal,
                          sm_scale=cfg.scale)
    got = on.from_storage(H.download(o_d), dtype)
    exp = oa.attention_bhsd(q, k, v, causal=causal, sm_scale=cfg.scale, dtype=dtype)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(exp))
    compare(f"persistent cus={cus} sq={seq_q} sk={seq_k}", np.nan_to_num(got), np.nan_to_num(exp), TOL[dtype])


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("sq,sk,causal", [
    (64, 64, True),      # one key tile (the stream pads to two; the second reads zeros)
    (65, 65, True),      # a wave with one row; keys past seq_k in the first 64-key tile
    (200, 40, False),    # seq_k < 64, non-causal
    (130, 100, True),    # bottom-right causal with sq > sk: the first rows see no key (NaN)
    (257, 257, True),    # two query tiles, the second with one row (three waves without rows)
    (520, 2000, True),   # sq < sk: every row sees the first 1481 keys
    (1000, 1000, False),
])
def test_prefill_w64_edges(monkeypatch, dtype, sq, sk, causal):
    """The d_k 128 kernel with 64 rows per wave: 64-key tiles padded to two
    per query tile, waves whose rows end early or do not exist, keys past
    seq_k inside a tile, fully masked rows."""
    H.set_override(monkeypatch, "TRITON_LLM_HIP_PREFILL_W64", 1)
    rng = np.random.default_rng(7 * sq + sk + causal)
    B, Hq, Hkv, D = 2, 6, 2, 128
    print(f"[case] w64 edge {dtype} sq={sq} sk={sk} causal={causal}", flush=True)
    q = on.to_storage(rng.standard_normal((B, Hq, sq, D), dtype=np.float32), dtype)
    k = on.to_storage(rng.standard_normal((B, Hkv, sk, D), dtype=np.float32), dtype)
    v = on.to_storage(rng.standard_normal((B, Hkv, sk, D), dtype=np.float32), dtype)
    o = flash_attention(H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype), causal=causal)
    got = on.from_storage(H.download(o), dtype)
    exp = oa.attention_bhsd(q, k, v, causal=causal, dtype=dtype)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(exp))
    compare(f"w64 edge {dtype} sq{sq} sk{sk}", np.nan_to_num(got), np.nan_to_num(exp), TOL[dtype])


@pytest.mark.parametrize("kernel", ["w64", "w32"])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_growing_scores_rescale(monkeypatch, kernel, causal):
    """Scores that rise along the keys: q[..., 0] = 1 and k[j, 0] = 2.35 j
    add about 0.3 (log2 units) per key on top of moderate noise, so each
    row's running maximum passes the lazy-rescale threshold (8) about every
    27 keys and the accumulated output is rescaled some 25 times per row,
    while the softmax stays well conditioned (weights spread over the last
    few keys)."""
    H.set_override(monkeypatch, "TRITON_LLM_HIP_PREFILL_W64", 1 if kernel == "w64" else None)
    dtype = "bfloat16"
    rng = np.random.default_rng(99 + causal)
    B, Hq, Hkv, S, D = 1, 4, 2, 700, 128
    q = 0.5 * rng.standard_normal((B, Hq, S, D), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, S, D), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, S, D), dtype=np.float32)
    q[..., 0] = 1.0
    k[..., 0] = 2.35 * np.arange(S, dtype=np.float32)
    q, k, v = (on.to_storage(x, dtype) for x in (q, k, v))
    print(f"[case] growing scores {kernel} causal={causal}", flush=True)
    o = flash_attention(H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype), causal=causal)
    got = on.from_storage(H.download(o), dtype)
    exp = oa.attention_bhsd(q, k, v, causal=causal, dtype=dtype)
    compare(f"growing scores {kernel} causal={causal}", got, exp, TOL[dtype])


def test_prefill_w64_and_w32_agree_on_5a_rows(monkeypatch):
    """Config 5a's prompt through both d_k 128 kernels: the same rows within
    the bf16 tolerance of each other (and of the oracle, which the full-size
    5a test checks for the default kernel)."""
    cfg = oi.CONFIGS["5a"]
    raw = oi.make_prefill_raw(cfg)
    outs = {}
    for kernel in ("w64", "w32"):
        H.set_override(monkeypatch, "TRITON_LLM_HIP_PREFILL_W64", 1 if kernel == "w64" else None)
        outs[kernel] = gpu_prefill(cfg, raw)
    compare("5a w64 vs w32", outs["w64"], outs["w32"], TOL[cfg.dtype])
