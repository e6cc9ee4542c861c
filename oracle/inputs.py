"""Seeded synthetic inputs of the five benchmark configurations.

Recipe (fixed once, shared by GPU runs, parity tests and the CPU baseline):
  * generator ``np.random.default_rng(seed)``; values ``standard_normal`` in
    float32, times ``amp``, rounded (RNE) to the config dtype -- the rounded
    values ARE the inputs of both sides;
  * prefill: q, k, v drawn in that order with shapes (B, H, S, D); RoPE (if
    the config has a theta) is applied to q and k at positions 0..S-1 in
    float32 and rounded once more to the dtype;
  * decode: ``lens`` (tokens already cached) drawn first, inclusive from
    [lo, min(hi, max_ctx - 1)] -- the reference rejects len + 1 > max_ctx
    (smollm2_triton/model.py:262-268) -- then per sequence b a generator
    ``default_rng([seed, b])`` yields K_b, V_b (Hkv, len_b, D), q_b (Hq, D),
    k_new_b, v_new_b (Hkv, D), in that order.  The new token is written at
    position len_b (after RoPE when the config has a theta) and attention
    covers len_b + 1 positions.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .numerics import f32_to_bf16_bits, nan_storage, round_to, storage_dtype, to_storage
from .rope import precompute_cos_sin, rotate


@dataclass(frozen=True)
class Config:
    name: str
    kind: str  # "prefill" | "decode"
    dtype: str
    batch: int
    n_head: int
    n_kv_head: int
    d_k: int
    seed: int
    scale: float
    seq: int = 0  # prefill length
    max_ctx: int = 0  # decode cache capacity
    lo: int = 0
    hi: int = 0
    amp: float = 1.0
    rope_theta: float | None = None
    causal: bool = True


CONFIGS: dict[str, Config] = {
    "1": Config("gpt2-prefill-fp32", "prefill", "float32", 1, 12, 12, 64, 0, 1 / 8, seq=128),
    "2": Config("gpt2-decode-fp16", "decode", "float16", 8, 12, 12, 64, 1, 1 / 8,
                max_ctx=1024, lo=1, hi=1024, amp=0.5),
    "3": Config("smollm2-135m-prefill-bf16", "prefill", "bfloat16", 4, 9, 3, 64, 2, 1 / 8,
                seq=2048, rope_theta=1e4),
    "4": Config("smollm2-360m-decode-bf16", "decode", "bfloat16", 32, 15, 5, 64, 3, 1 / 8,
                max_ctx=8192, lo=512, hi=8192, rope_theta=1e4),
    "5a": Config("llama3.2-3b-prefill-bf16", "prefill", "bfloat16", 1, 24, 8, 128, 4,
                 1 / math.sqrt(128), seq=8192, rope_theta=5e5),
    "5b": Config("llama3.2-3b-decode-bf16", "decode", "bfloat16", 64, 24, 8, 128, 4,
                 1 / math.sqrt(128), max_ctx=16384, lo=4096, hi=16384, rope_theta=5e5),
}


def scaled(cfg: Config, **overrides) -> Config:
    """A copy of ``cfg`` with some fields replaced (smaller parity variants)."""
    d = cfg.__dict__.copy()
    d.update(overrides)
    return Config(**d)


def draw_lens(cfg: Config) -> np.ndarray:
    rng = np.random.default_rng(cfg.seed)
    hi = min(cfg.hi, cfg.max_ctx - 1)
    return rng.integers(cfg.lo, hi, size=cfg.batch, endpoint=True).astype(np.int32)


def _normal(rng, shape, amp):
    x = rng.standard_normal(shape, dtype=np.float32)
    if amp != 1.0:
        x *= np.float32(amp)
    return x


def make_prefill(cfg: Config):
    """Storage arrays q (B,Hq,S,D), k/v (B,Hkv,S,D) after rounding and RoPE."""
    rng = np.random.default_rng(cfg.seed)
    B, Hq, Hkv, S, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.seq, cfg.d_k
    q = round_to(_normal(rng, (B, Hq, S, D), cfg.amp), cfg.dtype)
    k = round_to(_normal(rng, (B, Hkv, S, D), cfg.amp), cfg.dtype)
    v = round_to(_normal(rng, (B, Hkv, S, D), cfg.amp), cfg.dtype)
    if cfg.rope_theta is not None:
        cos, sin = precompute_cos_sin(S, D, cfg.rope_theta)
        q = round_to(rotate(q, cos[None, None], sin[None, None]), cfg.dtype)
        k = round_to(rotate(k, cos[None, None], sin[None, None]), cfg.dtype)
    return {
        "q": to_storage(q, cfg.dtype),
        "k": to_storage(k, cfg.dtype),
        "v": to_storage(v, cfg.dtype),
    }


def make_prefill_raw(cfg: Config):
    """Rounded q/k/v BEFORE RoPE (storage arrays), for GPU-side RoPE tests."""
    rng = np.random.default_rng(cfg.seed)
    B, Hq, Hkv, S, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.seq, cfg.d_k
    q = _normal(rng, (B, Hq, S, D), cfg.amp)
    k = _normal(rng, (B, Hkv, S, D), cfg.amp)
    v = _normal(rng, (B, Hkv, S, D), cfg.amp)
    return {n: to_storage(x, cfg.dtype) for n, x in (("q", q), ("k", k), ("v", v))}


def make_decode(cfg: Config, fill: str = "nan", lens=None):
    """Decode inputs as storage arrays.

    Returns dict with lens (B,) int32, caches k/v (B, Hkv, max_ctx, D) holding
    the cached prefix (positions >= len filled with NaN or zeros per ``fill``),
    q (B, Hq, D), k_new / v_new (B, Hkv, D) -- all BEFORE RoPE of the new token.
    ``lens`` overrides the drawn lengths (edge-case tests).
    """
    B, Hq, Hkv, D, C = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.d_k, cfg.max_ctx
    lens = draw_lens(cfg) if lens is None else np.asarray(lens, dtype=np.int32)
    sd = storage_dtype(cfg.dtype)
    fill_val = nan_storage(cfg.dtype) if fill == "nan" else sd(0)
    kc = np.empty((B, Hkv, C, D), dtype=sd)
    vc = np.empty((B, Hkv, C, D), dtype=sd)
    q = np.empty((B, Hq, D), dtype=sd)
    kn = np.empty((B, Hkv, D), dtype=sd)
    vn = np.empty((B, Hkv, D), dtype=sd)
    for b in range(B):
        rng = np.random.default_rng([cfg.seed, b])
        L = int(lens[b])
        kc[b, :, :L] = to_storage(_normal(rng, (Hkv, L, D), cfg.amp), cfg.dtype)
        vc[b, :, :L] = to_storage(_normal(rng, (Hkv, L, D), cfg.amp), cfg.dtype)
        kc[b, :, L:] = fill_val
        vc[b, :, L:] = fill_val
        q[b] = to_storage(_normal(rng, (Hq, D), cfg.amp), cfg.dtype)
        kn[b] = to_storage(_normal(rng, (Hkv, D), cfg.amp), cfg.dtype)
        vn[b] = to_storage(_normal(rng, (Hkv, D), cfg.amp), cfg.dtype)
    return {"lens": lens, "k_cache": kc, "v_cache": vc, "q": q, "k_new": kn, "v_new": vn}


def rope_tables(cfg: Config):
    if cfg.rope_theta is None:
        return None, None
    rows = cfg.max_ctx if cfg.kind == "decode" else cfg.seq
    return precompute_cos_sin(rows, cfg.d_k, cfg.rope_theta)


def decode_bytes(cfg: Config, lens) -> int:
    """Algorithmic HBM bytes of one decode step (append + attention):
    every valid K/V element read once (len + 1 positions), q read, o written,
    the new K/V written."""
    e = 4 if cfg.dtype == "float32" else 2
    B, Hq, Hkv, D = cfg.batch, cfg.n_head, cfg.n_kv_head, cfg.d_k
    kv_read = int(np.sum(2 * Hkv * (np.asarray(lens, dtype=np.int64) + 1) * D * e))
    return kv_read + B * Hq * D * (e + e) + 2 * B * Hkv * D * e


def prefill_flops(cfg: Config) -> int:
    """Algorithmic FLOPs: unmasked QK^T and PV multiply-adds times two."""
    B, Hq, D, S = cfg.batch, cfg.n_head, cfg.d_k, cfg.seq
    if cfg.causal:
        return 2 * B * Hq * D * S * (S + 1)
    return 4 * B * Hq * D * S * S


__all__ = [
    "Config", "CONFIGS", "scaled", "draw_lens", "make_prefill", "make_prefill_raw",
    "make_decode", "rope_tables", "decode_bytes", "prefill_flops", "f32_to_bf16_bits",
]
