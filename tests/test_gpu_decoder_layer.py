"""One SmolLM2/Llama decoder layer, the whole step on this library --
RMSNorm, q/k/v projections (gemm), the GPU-resident cached attention block
(RoPE + append + attention), o projection, fused residual add + RMSNorm,
gate/up projections, SwiGLU, down projection, residual add -- against the
oracle's restatement of smollm2_triton/model.py:276-365 (oracle/layers.py
decoder_layer_ref).  A 17-token prompt then 3 decoded tokens over 2 layers,
fp32 (the reference model's type); tolerance 2e-3 max-abs on the layer
output.
"""

import numpy as np
import pytest

from oracle import layers as ol
from oracle import rope as orope
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import add, add_rms_norm, gemm, rms_norm, swiglu
from triton_llm.kv_cache import GpuKVCache

pytestmark = pytest.mark.gpu


def test_decoder_layers_prefill_then_decode():
    E, Hq, Hkv, D, I, n_layer, max_seq = 384, 6, 2, 64, 1024, 2, 64
    rng = np.random.default_rng(21)
    mk = lambda *s, scale=1.0: (scale * rng.standard_normal(s)).astype(np.float32)  # noqa: E731
    weights = []
    for _ in range(n_layer):
        weights.append({"ln1": 1.0 + mk(E, scale=0.1), "ln2": 1.0 + mk(E, scale=0.1),
                        "q": mk(E, Hq * D, scale=E ** -0.5), "k": mk(E, Hkv * D, scale=E ** -0.5),
                        "v": mk(E, Hkv * D, scale=E ** -0.5), "o": mk(Hq * D, E, scale=(Hq * D) ** -0.5),
                        "gate": mk(E, I, scale=E ** -0.5), "up": mk(E, I, scale=E ** -0.5),
                        "down": mk(I, E, scale=I ** -0.5)})
    wd = [{k: gpu.to_device(v) for k, v in w.items()} for w in weights]
    cos, sin = orope.precompute_cos_sin(max_seq, D, 1e4)
    cos_d, sin_d = gpu.to_device(cos), gpu.to_device(sin)
    cache = GpuKVCache(n_layer, Hq, Hkv, D, max_seq=max_seq)
    host_cache = [{"k": np.zeros((Hkv, max_seq, D), np.float32), "v": np.zeros((Hkv, max_seq, D), np.float32)}
                  for _ in range(n_layer)]
    for seq in (17, 1, 1, 1):
        prev = cache.cache_len
        print(f"[case] decoder layer prev={prev} seq={seq}", flush=True)
        h_host = mk(seq, E)
        h = gpu.to_device(h_host)
        for i in range(n_layer):
            w = wd[i]
            x = rms_norm(h, w["ln1"], gpu.allocate((seq, E), np.float32))
            att = cache.attention(i, gemm(x, w["q"]), gemm(x, w["k"]), gemm(x, w["v"]), cos_d, sin_d)
            h1, x2 = add_rms_norm(gemm(att, w["o"]), h, gpu.allocate((seq, E), np.float32), w["ln2"],
                                  gpu.allocate((seq, E), np.float32))
            a = swiglu(gemm(x2, w["gate"]), gemm(x2, w["up"]))
            h = add(gemm(a, w["down"]), h1)
            h_host = ol.decoder_layer_ref(h_host, weights[i], host_cache[i], prev, cos, sin, Hq, Hkv)
            err = H.max_abs(H.download(h), h_host)
            H.report(f"layer {i} prev {prev} seq {seq}", err, 2e-3)
            assert err <= 2e-3
        cache.advance(seq)


def test_gpu_full_prompt_equals_prefill_then_decode():
    """The reference's cached == full-recompute invariant
    (tests/test_smollm2_model.py:95-165) on the GPU stack: a 12-token prompt
    through GpuKVCache and two layers gives, row for row, what a 9-token
    prefill followed by 3 one-token decode steps gives, and both match the
    oracle's full recompute."""
    E, Hq, Hkv, D, I, n_layer, max_seq, S, k = 256, 4, 2, 64, 512, 2, 32, 12, 3
    tol = 2e-3  # fp32, the reference model's type
    rng = np.random.default_rng(33)
    mk = lambda *s, scale=1.0: (scale * rng.standard_normal(s)).astype(np.float32)  # noqa: E731
    weights = [{"ln1": 1.0 + mk(E, scale=0.1), "ln2": 1.0 + mk(E, scale=0.1),
                "q": mk(E, Hq * D, scale=E ** -0.5), "k": mk(E, Hkv * D, scale=E ** -0.5),
                "v": mk(E, Hkv * D, scale=E ** -0.5), "o": mk(Hq * D, E, scale=(Hq * D) ** -0.5),
                "gate": mk(E, I, scale=E ** -0.5), "up": mk(E, I, scale=E ** -0.5),
                "down": mk(I, E, scale=I ** -0.5)} for _ in range(n_layer)]
    wd = [{name: gpu.to_device(v) for name, v in w.items()} for w in weights]
    cos, sin = orope.precompute_cos_sin(max_seq, D, 1e4)
    cos_d, sin_d = gpu.to_device(cos), gpu.to_device(sin)
    h_all = mk(S, E)

    def run(cache, rows):
        seq = rows.shape[0]
        h = gpu.to_device(rows)
        for i in range(n_layer):
            w = wd[i]
            x = rms_norm(h, w["ln1"], gpu.allocate((seq, E), np.float32))
            att = cache.attention(i, gemm(x, w["q"]), gemm(x, w["k"]), gemm(x, w["v"]), cos_d, sin_d)
            h1, x2 = add_rms_norm(gemm(att, w["o"]), h, gpu.allocate((seq, E), np.float32), w["ln2"],
                                  gpu.allocate((seq, E), np.float32))
            h = add(gemm(swiglu(gemm(x2, w["gate"]), gemm(x2, w["up"])), w["down"]), h1)
        cache.advance(seq)
        return H.download(h)

    print(f"[case] full-vs-cached S={S} k={k} float32", flush=True)
    full = run(GpuKVCache(n_layer, Hq, Hkv, D, max_seq=max_seq), h_all)
    cache = GpuKVCache(n_layer, Hq, Hkv, D, max_seq=max_seq)
    cached = np.concatenate([run(cache, h_all[:S - k])] + [run(cache, h_all[t:t + 1]) for t in range(S - k, S)])
    host = h_all
    host_cache = [{"k": np.zeros((Hkv, max_seq, D), np.float32), "v": np.zeros((Hkv, max_seq, D), np.float32)}
                  for _ in range(n_layer)]
    for i in range(n_layer):
        host = ol.decoder_layer_ref(host, weights[i], host_cache[i], 0, cos, sin, Hq, Hkv)
    for name, got in (("full", full), ("cached", cached)):
        err = H.max_abs(got, host)
        H.report(f"{name} vs oracle full recompute", err, tol)
        assert err <= tol
    err = H.max_abs(cached, full)
    H.report("cached vs full (GPU)", err, tol)
    assert err <= tol
