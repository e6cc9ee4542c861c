"""Key-split prefill: causal 16-bit calls with few query tiles split the key
range of their costliest tiles over two workgroups, which merge in
the kernel (tl_attention_fwd_workspace_bytes_split sizes the workspace that
allows it).  Each case first checks that the call does split (the size query
asks for more than the minimum), then compares with the oracle (2e-2
max-abs, as every 16-bit prefill test) and with the same call run unsplit
(given only the minimum workspace).
"""

import numpy as np
import pytest

from oracle import attention as oa
from oracle import numerics as on
from tests import _helpers as H
from triton_llm import gpu
from triton_llm.kernels import flash_attention

pytestmark = pytest.mark.gpu

TOL = 2e-2


def split_bytes(B, Hq, Hkv, sq, sk, d_k, dtype, causal=True):
    lib = gpu.runtime()
    code = gpu.dtype_code(H.GPU_DTYPES[dtype])
    base = lib.tl_attention_fwd_workspace_bytes(B, Hkv, sk, d_k, code)
    full = lib.tl_attention_fwd_workspace_bytes_split(B, Hq, Hkv, sq, sk, d_k, 1 if causal else 0, code)
    return base, full


def inputs(B, Hq, Hkv, sq, sk, d_k, dtype, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    q = on.to_storage(scale * rng.standard_normal((B, Hq, sq, d_k), dtype=np.float32), dtype)
    k = on.to_storage(rng.standard_normal((B, Hkv, sk, d_k), dtype=np.float32), dtype)
    v = on.to_storage(rng.standard_normal((B, Hkv, sk, d_k), dtype=np.float32), dtype)
    return q, k, v


def run(q_d, k_d, v_d, sm_scale, ws, dtype):
    o_d = flash_attention(q_d, k_d, v_d, causal=True, sm_scale=sm_scale, workspace=ws)
    return on.from_storage(H.download(o_d), dtype), H.download(o_d).copy()


@pytest.mark.parametrize("cus", [None, 16])
@pytest.mark.parametrize("dtype,sm_scale", [("bfloat16", None), ("float16", None), ("float16", 3.0)])
@pytest.mark.parametrize("B,Hq,Hkv,sq,sk,d_k", [
    (1, 8, 8, 1024, 1024, 128),    # 8 heads: one per XCD list, 4 levels
    (1, 24, 8, 2048, 2048, 128),   # Llama-3.2-3B heads, a 2048-token prompt
    (2, 6, 2, 1000, 1000, 128),    # ragged last query tile, one list
    (1, 8, 4, 700, 1500, 128),     # seq_k > seq_q: bottom-right causal offset
    (1, 12, 4, 1536, 1536, 128),   # GQA group 3, 6 levels
    (2, 9, 3, 2048, 2048, 64),     # SmolLM2-135M heads at batch 2: d_k 64, V read in place
    (1, 16, 4, 2048, 2048, 64),
    (4, 9, 3, 1000, 1000, 64),     # ragged, d_k 64
    (1, 9, 3, 2048, 2048, 64),     # SmolLM2-135M at batch 1: one list of whole heads, then split
    (1, 15, 5, 1536, 1536, 64),    # SmolLM2-360M heads at batch 1
])
def test_split_matches_oracle_and_unsplit(monkeypatch, cus, dtype, sm_scale, B, Hq, Hkv, sq, sk, d_k):
    H.set_override(monkeypatch, "TRITON_LLM_HIP_MAX_CUS", cus)
    base, full = split_bytes(B, Hq, Hkv, sq, sk, d_k, dtype)
    if full <= base:
        pytest.skip("the planner does not split this shape on this CU count")
    # fp16 with |sm_scale * log2 e| > 1 (3.0) scales the scores in fp32
    # instead of pre-scaling Q: the other kernel instance
    scale = (1 / np.sqrt(d_k)) if sm_scale is None else sm_scale
    print(f"[case] split cus={cus} {dtype} scale={scale:.3f} B={B} Hq={Hq} Hkv={Hkv} sq={sq} sk={sk} d_k={d_k} "
          f"split_ws={full} min_ws={base}", flush=True)
    q, k, v = inputs(B, Hq, Hkv, sq, sk, d_k, dtype, seed=sq + sk + d_k)
    q_d, k_d, v_d = H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype)
    ws_split = gpu.allocate((full,), np.uint8)
    ws_min = gpu.allocate((max(base, 16),), np.uint8)
    got, raw1 = run(q_d, k_d, v_d, scale, ws_split, dtype)
    unsplit, _ = run(q_d, k_d, v_d, scale, ws_min, dtype)
    exp = oa.attention_bhsd(q, k, v, causal=True, sm_scale=scale, dtype=dtype)
    assert np.all(np.isfinite(got))
    err = H.max_abs(got, exp)
    H.report("split vs oracle", err, TOL)
    assert err <= TOL
    err_u = H.max_abs(got, unsplit)
    H.report("split vs unsplit", err_u, TOL)
    assert err_u <= TOL
    # deterministic: the merge order is fixed, whichever part arrives last
    _, raw2 = run(q_d, k_d, v_d, scale, ws_split, dtype)
    np.testing.assert_array_equal(raw1, raw2)


def test_split_needs_no_workspace_initialisation():
    """Random bytes in the workspace (arrival words included) do not matter:
    each call tags its arrivals with a fresh value, and a merge clears them."""
    dtype, B, Hq, Hkv, S, d_k = "bfloat16", 1, 8, 8, 1024, 128
    base, full = split_bytes(B, Hq, Hkv, S, S, d_k, dtype)
    assert full > base
    print(f"[case] split random workspace S={S} d_k={d_k}", flush=True)
    q, k, v = inputs(B, Hq, Hkv, S, S, d_k, dtype, seed=5)
    q_d, k_d, v_d = H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype)
    rng = np.random.default_rng(11)
    ws = gpu.to_device(rng.integers(0, 256, size=full, dtype=np.uint8))
    got, raw = run(q_d, k_d, v_d, 0.125, ws, dtype)
    exp = oa.attention_bhsd(q, k, v, causal=True, sm_scale=0.125, dtype=dtype)
    err = H.max_abs(got, exp)
    H.report("split random ws", err, TOL)
    assert err <= TOL
    # the same workspace, refilled with all-one bits, gives the same output
    gpu.copy_(ws, gpu.to_device(np.full(full, 255, np.uint8)))
    _, raw2 = run(q_d, k_d, v_d, 0.125, ws, dtype)
    np.testing.assert_array_equal(raw, raw2)


def test_split_workspace_reused_across_shapes():
    """One workspace serves calls of different shapes in turn (each merge
    leaves its words cleared for the next call)."""
    dtype = "bfloat16"
    shapes = [(1, 8, 8, 1024, 1024, 128), (2, 6, 2, 1000, 1000, 128), (1, 8, 4, 700, 1500, 128)]
    need = max(split_bytes(*s, dtype)[1] for s in shapes)
    ws = gpu.allocate((need,), np.uint8)
    first = {}
    for rnd in range(2):
        for i, (B, Hq, Hkv, sq, sk, d_k) in enumerate(shapes):
            print(f"[case] split reuse round {rnd} shape {i}", flush=True)
            q, k, v = inputs(B, Hq, Hkv, sq, sk, d_k, dtype, seed=100 + i)
            got, raw = run(H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype), 0.1, ws, dtype)
            if rnd == 0:
                exp = oa.attention_bhsd(q, k, v, causal=True, sm_scale=0.1, dtype=dtype)
                assert H.max_abs(got, exp) <= TOL
                first[i] = raw
            else:
                np.testing.assert_array_equal(raw, first[i])


def test_split_graph_replays():
    """A captured split call replays correctly: its tag is fixed in the graph,
    and every merge clears the words it used, so each replay starts clean."""
    dtype, B, Hq, Hkv, S, d_k = "bfloat16", 1, 24, 8, 2048, 128
    base, full = split_bytes(B, Hq, Hkv, S, S, d_k, dtype)
    assert full > base
    print(f"[case] split graph replays S={S}", flush=True)
    q, k, v = inputs(B, Hq, Hkv, S, S, d_k, dtype, seed=21)
    q_d, k_d, v_d = H.upload(q, dtype), H.upload(k, dtype), H.upload(v, dtype)
    ws = gpu.allocate((full,), np.uint8)
    out = gpu.allocate(q_d.shape, q_d.dtype)
    flash_attention(q_d, k_d, v_d, causal=True, sm_scale=0.125, out=out, workspace=ws)
    want = H.download(out).copy()
    with gpu.capture() as g:
        flash_attention(q_d, k_d, v_d, causal=True, sm_scale=0.125, out=out, workspace=ws)
    for rep in range(4):
        gpu.copy_(out, gpu.zeros(out.shape, out.dtype))
        g.replay()
        np.testing.assert_array_equal(H.download(out), want, err_msg=f"replay {rep}")
        # an eager split call with its own tag between replays
        flash_attention(q_d, k_d, v_d, causal=True, sm_scale=0.125, workspace=ws)
    gpu.synchronize()
