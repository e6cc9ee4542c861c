"""The GPU-resident KV cache and cached attention sub-block against the
reference model's host flow (smollm2_triton/model.py:286-347): RoPE of q/k at
the step's positions, the cache written row by row, causal attention_gqa for
the prompt and non-causal attention_gqa over the cache prefix for each
decoded token.  The oracle runs that flow on the host with the oracle's RoPE
and GQA attention, on the same storage-rounded inputs.
Tolerance: 2e-3 max-abs fp32, 2e-2 bf16; cache rows and rotated q bit-exact.
"""

import numpy as np
import pytest

from oracle import attention as oa
from oracle import numerics as on
from oracle import rope as orope
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kv_cache import GpuKVCache

pytestmark = pytest.mark.gpu

TOL = {"float32": 2e-3, "bfloat16": 2e-2}


@pytest.mark.parametrize("dtype,d_k,n_head,n_kv", [("float32", 64, 9, 3), ("bfloat16", 64, 9, 3),
                                                   ("bfloat16", 128, 24, 8), ("float32", 128, 8, 8)])
def test_cached_attention_block_prefill_then_decode(dtype, d_k, n_head, n_kv):
    run_block(dtype, d_k, n_head, n_kv, n_layer=2, max_seq=96, prompt=41, steps=5)


def test_cached_attention_long_prompt_splits_its_tiles():
    """A 1536-token prompt with Llama-3.2-3B heads: the flash call splits
    its longest tiles' keys over two workgroups (the cache's workspace has
    room for a full-length prompt's split), then two decoded tokens."""
    from triton_llm.kernels.flash import flash_workspace_bytes
    assert (flash_workspace_bytes(1, 8, 1536, 128, gpu.bfloat16, n_head=24, seq_q=1536)
            > flash_workspace_bytes(1, 8, 1536, 128, gpu.bfloat16))
    run_block("bfloat16", 128, 24, 8, n_layer=1, max_seq=2048, prompt=1536, steps=2)


def run_block(dtype, d_k, n_head, n_kv, n_layer, max_seq, prompt, steps):
    D = d_k
    cos, sin = orope.precompute_cos_sin(max_seq, D, 1e4)
    cos_d, sin_d = gpu.to_device(cos), gpu.to_device(sin)
    cache = GpuKVCache(n_layer, n_head, n_kv, D, max_seq=max_seq, max_position_embeddings=max_seq,
                       dtype=H.GPU_DTYPES[dtype])
    host = [{"k": np.zeros((n_kv, max_seq, D), np.float32), "v": np.zeros((n_kv, max_seq, D), np.float32)}
            for _ in range(n_layer)]
    rng = np.random.default_rng(11)
    for seq in [prompt] + [1] * steps:
        prev = cache.cache_len
        pos = np.arange(prev, prev + seq)
        print(f"[case] {dtype} d{D} H{n_head}/{n_kv} prev={prev} seq={seq}", flush=True)
        for layer in range(n_layer):
            qs = on.to_storage(rng.standard_normal((seq, n_head * D), dtype=np.float32), dtype)
            ks = on.to_storage(rng.standard_normal((seq, n_kv * D), dtype=np.float32), dtype)
            vs = on.to_storage(rng.standard_normal((seq, n_kv * D), dtype=np.float32), dtype)
            q_d, k_d, v_d = H.upload(qs, dtype), H.upload(ks, dtype), H.upload(vs, dtype)
            out = cache.attention(layer, q_d, k_d, v_d, cos_d, sin_d)
            got = on.from_storage(H.download(out), dtype)

            # Host flow of the reference model on the same values.
            q_rot = orope.apply_rope_storage(qs.reshape(seq, n_head, D), cos, sin, pos[:, None], dtype)
            k_rot = orope.apply_rope_storage(ks.reshape(seq, n_kv, D), cos, sin, pos[:, None], dtype)
            host[layer]["k"][:, prev:prev + seq] = on.from_storage(k_rot, dtype).transpose(1, 0, 2)
            host[layer]["v"][:, prev:prev + seq] = on.from_storage(vs.reshape(seq, n_kv, D), dtype).transpose(1, 0, 2)
            qf = on.from_storage(q_rot, dtype).transpose(1, 0, 2).reshape(-1, D)
            kf = host[layer]["k"][:, :prev + seq].reshape(-1, D)
            vf = host[layer]["v"][:, :prev + seq].reshape(-1, D)
            exp = oa.attention_gqa_ref(qf, kf, vf, n_head, n_kv, causal=(prev == 0))
            exp = exp.reshape(n_head, seq, D).transpose(1, 0, 2).reshape(seq, n_head * D)
            err = H.max_abs(got, exp)
            H.report(f"layer{layer} prev{prev} seq{seq}", err, TOL[dtype])
            assert np.all(np.isfinite(got)) and err <= TOL[dtype]

            # q rotated in place, cache rows bitwise.
            np.testing.assert_array_equal(H.download(q_d).reshape(seq, n_head, D), q_rot)
            kc = H.download(cache.kv_cache_dev[layer]["k"])[0, :, :prev + seq]
            vc = H.download(cache.kv_cache_dev[layer]["v"])[0, :, :prev + seq]
            np.testing.assert_array_equal(kc, on.to_storage(host[layer]["k"][:, :prev + seq], dtype))
            np.testing.assert_array_equal(vc, on.to_storage(host[layer]["v"][:, :prev + seq], dtype))
        cache.advance(seq)
    assert cache.cache_len == prompt + steps


def test_cached_attention_block_limits():
    cache = GpuKVCache(1, 4, 2, 64, max_seq=8, dtype=np.float32)
    z = lambda rows, w: gpu.zeros((rows, w), np.float32)
    with pytest.raises(ValueError, match="exceeds pre-allocated cache size"):
        cache.attention(0, z(9, 256), z(9, 128), z(9, 128))
    cache.attention(0, z(6, 256), z(6, 128), z(6, 128))
    cache.advance(6)
    with pytest.raises(ValueError, match="Decode mode requires seq=1"):
        cache.attention(0, z(2, 256), z(2, 128), z(2, 128))
    cache.attention(0, z(1, 256), z(1, 128), z(1, 128))
    cache.advance(1)
    cache.advance(1)
    with pytest.raises(ValueError, match="exceeds pre-allocated cache size"):
        cache.attention(0, z(1, 256), z(1, 128), z(1, 128))
    cache.reset()
    assert cache.cache_len == 0
