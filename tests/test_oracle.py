"""Pin the CPU oracle against facts fixed independently of its code.

Each check is chosen so a plausible slip in the restatement -- dropped scale,
wrong mask direction or alignment, ``h % n_kv`` instead of ``h // group``,
(2i, 2i+1) RoPE pairing, wrong sign, bad bf16 tie rounding, a shifted
position -- fails at least one of them.  CPU only.
"""

import math

import numpy as np
import pytest

from oracle import attention as oa
from oracle import inputs as oi
from oracle import numerics as on
from oracle import rope as orope


# --------------------------------------------------------------------------
# brute force (pure Python, float64, direct softmax definition)
# --------------------------------------------------------------------------

def brute_attention(q, k, v, scale, visible):
    sq, d = len(q), len(q[0])
    out = []
    for i in range(sq):
        w = []
        for j in range(len(k)):
            if visible(i, j):
                w.append(math.exp(scale * sum(float(q[i][e]) * float(k[j][e]) for e in range(d))))
            else:
                w.append(0.0)
        z = sum(w)
        out.append([sum(w[j] * float(v[j][e]) for j in range(len(k))) / z for e in range(d)])
    return np.array(out)


@pytest.mark.parametrize("sq,sk,d,causal", [(5, 5, 8, True), (3, 7, 4, True), (4, 6, 8, False), (1, 9, 4, False)])
def test_gqa_ref_matches_bruteforce(sq, sk, d, causal):
    rng = np.random.default_rng(10 + sq * 7 + sk)
    nh, nkv = 4, 2
    q = rng.standard_normal((nh * sq, d)).astype(np.float32)
    k = rng.standard_normal((nkv * sk, d)).astype(np.float32)
    v = rng.standard_normal((nkv * sk, d)).astype(np.float32)
    got = oa.attention_gqa_ref(q, k, v, nh, nkv, causal=causal, sm_scale=0.37)
    for h in range(nh):
        kv = h // 2
        exp = brute_attention(q[h * sq:(h + 1) * sq], k[kv * sk:(kv + 1) * sk], v[kv * sk:(kv + 1) * sk],
                              0.37, (lambda i, j: j <= i + sk - sq) if causal else (lambda i, j: True))
        np.testing.assert_allclose(got[h * sq:(h + 1) * sq], exp, atol=2e-6)


def test_mha_ref_matches_bruteforce():
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((6, 8)).astype(np.float32) for _ in range(3))
    exp = brute_attention(q, k, v, 1 / math.sqrt(8), lambda i, j: j <= i)
    np.testing.assert_allclose(oa.attention_ref(q, k, v, causal=True), exp, atol=2e-6)
    exp_nc = brute_attention(q[:1], k, v, 1 / math.sqrt(8), lambda i, j: True)
    np.testing.assert_allclose(oa.attention_ref(q[:1], k, v, causal=False), exp_nc, atol=2e-6)


# --------------------------------------------------------------------------
# closed forms and invariants
# --------------------------------------------------------------------------

def test_single_token_returns_v():
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_array_equal(oa.attention_ref(q, k, v), v)


def test_identity_closed_form():
    # Q=K=V=I (8 x 64): row i sees s_ij = c * [i == j] for j <= i, c = 1/8, so
    # O[i] = (e^c e_i + sum_{j<i} e_j) / (e^c + i).
    n, d = 8, 64
    eye = np.eye(n, d, dtype=np.float32)
    c = 1 / math.sqrt(d)
    exp = np.zeros((n, d))
    for i in range(n):
        exp[i, :i] = 1.0
        exp[i, i] = math.exp(c)
        exp[i] /= math.exp(c) + i
    np.testing.assert_allclose(oa.attention_ref(eye, eye, eye), exp, atol=1e-6)


def test_uniform_scores_give_prefix_means_bottom_right():
    # q = 0 -> all visible scores equal -> output = mean of visible V rows.
    sq, sk, d = 3, 7, 4
    rng = np.random.default_rng(5)
    v = rng.standard_normal((sk, d)).astype(np.float32)
    q = np.zeros((sq, d), np.float32)
    k = rng.standard_normal((sk, d)).astype(np.float32)
    out = oa.attention_gqa_ref(q, k, v, 1, 1, causal=True)
    for i in range(sq):
        last = sk - sq + i  # bottom-right alignment
        np.testing.assert_allclose(out[i], v[: last + 1].mean(axis=0), atol=1e-6)


def test_gqa_head_map_is_floor_division():
    # V of KV head j is the constant j + 1; with q = 0 every query head returns
    # the constant of the KV head it reads: h // (n_head // n_kv_head).
    nh, nkv, s, d = 6, 3, 4, 8
    q = np.zeros((nh * s, d), np.float32)
    k = np.random.default_rng(1).standard_normal((nkv * s, d)).astype(np.float32)
    v = np.repeat(np.arange(1, nkv + 1, dtype=np.float32), s)[:, None] * np.ones((1, d), np.float32)
    out = oa.attention_gqa_ref(q, k, v, nh, nkv, causal=False).reshape(nh, s, d)
    for h in range(nh):
        assert np.allclose(out[h], h // (nh // nkv) + 1)


def test_gqa_equals_per_head_mha_when_groups_are_one():
    rng = np.random.default_rng(2)
    h, s, d = 3, 5, 8
    q, k, v = (rng.standard_normal((h * s, d)).astype(np.float32) for _ in range(3))
    g = oa.attention_gqa_ref(q, k, v, h, h, causal=True)
    for i in range(h):
        np.testing.assert_allclose(g[i * s:(i + 1) * s],
                                   oa.attention_ref(q[i * s:(i + 1) * s], k[i * s:(i + 1) * s], v[i * s:(i + 1) * s]),
                                   atol=1e-6)


def test_causal_perturbation_invariance():
    rng = np.random.default_rng(4)
    n, d = 12, 16
    q, k, v = (rng.standard_normal((n, d)).astype(np.float32) for _ in range(3))
    a = oa.attention_ref(q, k, v)
    k2, v2 = k.copy(), v.copy()
    k2[-1] += 5
    v2[-1] -= 3
    b = oa.attention_ref(q, k2, v2)
    np.testing.assert_array_equal(a[:-1], b[:-1])
    assert not np.allclose(a[-1], b[-1])


def test_scale_placement():
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((4 * 3, 8)).astype(np.float32) for _ in range(3))
    a = oa.attention_gqa_ref(q, k, v, 4, 4, causal=False, sm_scale=0.5)
    b = oa.attention_gqa_ref(q * 2, k, v, 4, 4, causal=False, sm_scale=0.25)
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_empty_kv_gives_zeros_and_fully_masked_rows_nan():
    q = np.ones((2 * 3, 8), np.float32)
    k = np.empty((0, 8), np.float32)
    assert np.all(oa.attention_gqa_ref(q, k, k, 2, 1) == 0)
    # seq_q = 3 > seq_k = 2, causal: query 0 sees no key (j <= i - 1).
    k2 = np.ones((2, 8), np.float32)
    out = oa.attention_gqa_ref(np.ones((3, 8), np.float32), k2, k2, 1, 1, causal=True)
    assert np.all(np.isnan(out[0])) and np.all(np.isfinite(out[1:]))


def test_batched_blockwise_matches_flat_reference():
    rng = np.random.default_rng(7)
    B, Hq, Hkv, S, D = 2, 6, 2, 70, 16
    q = rng.standard_normal((B, Hq, S, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    got = oa.attention_bhsd(q, k, v, causal=True, block_q=16)
    for b in range(B):
        exp = oa.attention_gqa_ref(q[b].reshape(-1, D), k[b].reshape(-1, D), v[b].reshape(-1, D), Hq, Hkv)
        np.testing.assert_allclose(got[b].reshape(-1, D), exp, atol=2e-6)
    rows = np.array([0, 5, 69])
    part = oa.attention_bhsd(q, k, v, causal=True, rows=rows)
    np.testing.assert_allclose(part[:, :, rows], got[:, :, rows], atol=1e-6)


def test_decode_ref_is_gqa_noncausal_on_prefix_and_ignores_tail():
    rng = np.random.default_rng(8)
    B, Hq, Hkv, C, D = 3, 4, 2, 20, 8
    kc = rng.standard_normal((B, Hkv, C, D)).astype(np.float32)
    vc = rng.standard_normal((B, Hkv, C, D)).astype(np.float32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    lens = np.array([1, 7, 20])
    out = oa.decode_ref(q, kc, vc, lens)
    for b in range(B):
        L = lens[b]
        exp = oa.attention_gqa_ref(q[b], kc[b, :, :L].reshape(-1, D), vc[b, :, :L].reshape(-1, D), Hq, Hkv, causal=False)
        np.testing.assert_allclose(out[b], exp, atol=1e-6)
    kc2, vc2 = kc.copy(), vc.copy()
    for b in range(B):
        kc2[b, :, lens[b]:] = np.nan
        vc2[b, :, lens[b]:] = np.nan
    np.testing.assert_array_equal(oa.decode_ref(q, kc2, vc2, lens), out)


def test_kv_append_writes_only_position_len():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, C, D = 2, 4, 2, 10, 8
    kc = rng.standard_normal((B, Hkv, C, D)).astype(np.float32)
    vc = rng.standard_normal((B, Hkv, C, D)).astype(np.float32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    kn = rng.standard_normal((B, Hkv, D)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, D)).astype(np.float32)
    lens = np.array([3, 9])
    cos, sin = orope.precompute_cos_sin(C, D, 1e4)
    q2, kc2, vc2 = oa.kv_append_ref(q, kn, vn, kc, vc, lens, cos, sin)
    for b in range(B):
        mask = np.ones(C, bool)
        mask[lens[b]] = False
        np.testing.assert_array_equal(kc2[b][:, mask], kc[b][:, mask])
        np.testing.assert_array_equal(vc2[b][:, lens[b]], vn[b])
        # rotation preserves the norm of every (i, i + D/2) pair
        h = D // 2
        n_in = kn[b][:, :h] ** 2 + kn[b][:, h:] ** 2
        n_out = kc2[b][:, lens[b], :h] ** 2 + kc2[b][:, lens[b], h:] ** 2
        np.testing.assert_allclose(n_out, n_in, rtol=1e-5)
        np.testing.assert_allclose(q2[b], orope.rotate(q[b], cos[lens[b]], sin[lens[b]]))


# --------------------------------------------------------------------------
# RoPE
# --------------------------------------------------------------------------

def test_rope_tables_against_float64():
    for theta in (1e4, 1e5, 5e5):
        cos, sin = orope.precompute_cos_sin(300, 64, theta)
        assert cos.dtype == np.float32 and cos.shape == (300, 32)
        p = np.arange(300)[:, None]
        inv = theta ** (-2.0 * np.arange(32) / 64)
        # float32 angle rounding grows with the angle; 2e-5 bounds it at p < 300.
        np.testing.assert_allclose(cos, np.cos(p * inv), atol=2e-5)
        np.testing.assert_allclose(sin, np.sin(p * inv), atol=2e-5)
        assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
        np.testing.assert_allclose(cos[:, 0], np.cos(np.arange(300, dtype=np.float32)), atol=1e-6)


def test_rope_pairing_is_half_split():
    d = 8
    cos, sin = orope.precompute_cos_sin(4, d, 1e4)
    x = np.zeros((1, d), np.float32)
    x[0, 1] = 1.0  # only element 1 set
    out = orope.apply_rope(x, cos, sin, seq_len=1, position_offset=3)
    nz = set(np.flatnonzero(out[0]).tolist())
    assert nz == {1, 1 + d // 2}, nz  # pairs with i + d/2, not i ^ 1
    assert out[0, 1] == np.float32(cos[3, 1]) and out[0, 5] == np.float32(sin[3, 1])


def test_rope_matches_complex_rotation_and_position_rule():
    rng = np.random.default_rng(11)
    n_rows, seq, d, off = 12, 4, 16, 5
    cos, sin = orope.precompute_cos_sin(16, d, 1e5)
    x = rng.standard_normal((n_rows, d)).astype(np.float32)
    out = orope.apply_rope(x, cos, sin, seq, off)
    for r in range(n_rows):
        p = r % seq + off
        z = (x[r, : d // 2] + 1j * x[r, d // 2:]) * (cos[p].astype(np.float64) + 1j * sin[p])
        np.testing.assert_allclose(out[r, : d // 2], z.real, atol=1e-6)
        np.testing.assert_allclose(out[r, d // 2:], z.imag, atol=1e-6)
    np.testing.assert_array_equal(orope.apply_rope(x, cos, sin, 1, 0), x)  # position 0 = identity


# --------------------------------------------------------------------------
# bf16 rounding (exhaustive on a slice of float32 space)
# --------------------------------------------------------------------------

def _bf16_nearest_even_brute(x):
    """Pick the nearer of the two bf16 neighbours in float64; ties to even."""
    u = np.float32(x).view(np.uint32)
    lo = np.uint32(u & 0xFFFF0000)
    hi = np.uint32(lo + 0x10000)
    flo = float(np.uint32(lo).view(np.float32))
    # Above the largest finite bf16 the upper neighbour is 2**128 (which
    # rounds to infinity), not the float32 infinity bit pattern.
    fhi = 2.0 ** 128 if hi == 0x7F800000 else float(np.uint32(hi).view(np.float32))
    dl, dh = abs(float(x) - flo), abs(fhi - float(x))
    if dl < dh:
        return int(lo >> 16)
    if dh < dl:
        return int(hi >> 16)
    return int(lo >> 16) if ((lo >> 16) & 1) == 0 else int(hi >> 16)


def test_bf16_rne_exhaustive_slice_and_specials():
    rng = np.random.default_rng(12)
    bits = np.concatenate([
        np.arange(0x3F800000, 0x3F800000 + 0x30000, 7, dtype=np.uint32),  # around 1.0, incl. ties
        rng.integers(0, 0x7F7FFFFF, 20000, dtype=np.uint32),
        (0x3F808000 + 0x10000 * np.arange(16)).astype(np.uint32),  # exact ties
    ])
    xs = bits.view(np.float32)
    got = on.f32_to_bf16_bits(xs)
    exp = np.array([_bf16_nearest_even_brute(x) for x in xs], dtype=np.uint16)
    np.testing.assert_array_equal(got, exp)
    assert on.f32_to_bf16_bits(np.float32(1.0)) == 0x3F80
    assert on.f32_to_bf16_bits(np.float32(1.0 + 2 ** -8)) == 0x3F80  # tie to even
    assert on.f32_to_bf16_bits(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F82  # tie to even (up)
    assert on.f32_to_bf16_bits(np.float32(np.inf)) == 0x7F80
    assert on.f32_to_bf16_bits(np.float32(-np.nan)) in (0xFFC0,)
    assert on.f32_to_bf16_bits(np.float32(3.3895314e38)) == 0x7F7F  # max finite stays finite
    np.testing.assert_array_equal(on.bf16_bits_to_f32(np.array([0x3F80, 0xC000], np.uint16)), [1.0, -2.0])


# --------------------------------------------------------------------------
# input recipe: the length draws quoted for the benchmark configurations
# --------------------------------------------------------------------------

def test_decode_length_draws_match_published_recipe():
    # lens + 1 summed (positions attended), and the first draws of config 2.
    assert list(oi.draw_lens(oi.CONFIGS["2"])[:4]) == [485, 524, 773, 973]
    for name, total in (("2", 4760), ("4", 129443), ("5b", 708012)):
        lens = oi.draw_lens(oi.CONFIGS[name])
        assert int(lens.sum()) + len(lens) == total, name
        cfg = oi.CONFIGS[name]
        assert lens.min() >= cfg.lo and lens.max() <= cfg.max_ctx - 1


def test_work_formulas():
    assert oi.prefill_flops(oi.CONFIGS["5a"]) == 2 * 24 * 128 * 8192 * 8193
    assert abs(oi.prefill_flops(oi.CONFIGS["3"]) / 1e9 - 19.34) < 0.01
    b = oi.decode_bytes(oi.CONFIGS["5b"], oi.draw_lens(oi.CONFIGS["5b"]))
    assert abs(b / 1e9 - 2.901) < 0.002


def test_small_decode_inputs_shapes_and_poison():
    cfg = oi.scaled(oi.CONFIGS["4"], batch=3, max_ctx=64, lo=1, hi=64)
    d = oi.make_decode(cfg)
    assert d["k_cache"].dtype == np.uint16 and d["k_cache"].shape == (3, 5, 64, 64)
    for b in range(3):
        L = d["lens"][b]
        assert np.all(d["k_cache"][b, :, L:] == 0x7FC0)
        assert not np.any(d["k_cache"][b, :, :L] == 0x7FC0)


def test_gemm_ref_pins():
    """gemm_ref against facts a transposed operand or dropped term would break."""
    from oracle.gemm import gemm_ref

    rng = np.random.default_rng(3)
    a = rng.standard_normal((7, 5)).astype(np.float32)
    b = rng.standard_normal((5, 9)).astype(np.float32)
    np.testing.assert_array_equal(gemm_ref(np.eye(7, dtype=np.float32), a), a)
    np.testing.assert_array_equal(gemm_ref(a, np.eye(5, dtype=np.float32)), a)
    u, v = rng.standard_normal((6, 1)), rng.standard_normal((1, 4))
    np.testing.assert_allclose(gemm_ref(u, v), u * v, rtol=1e-6)  # rank one: outer product
    x = rng.standard_normal(9)
    np.testing.assert_allclose(gemm_ref(a, b) @ x, a.astype(np.float64) @ (b.astype(np.float64) @ x), rtol=1e-5, atol=1e-5)
    assert gemm_ref(np.zeros((3, 0)), np.zeros((0, 4))).shape == (3, 4)
    assert not gemm_ref(np.zeros((3, 0)), np.zeros((0, 4))).any()


def test_layers_ref_pins():
    """rms_norm_ref / swiglu_ref / decoder_layer_ref against invariants a wrong
    axis, a dropped term or a sign slip would break."""
    from oracle import layers as ol

    rng = np.random.default_rng(9)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    y1 = ol.rms_norm_ref(x, w, eps=0.0)
    np.testing.assert_allclose(ol.rms_norm_ref(7.5 * x, w, eps=0.0), y1, rtol=1e-5, atol=1e-6)  # scale invariant
    unit = ol.rms_norm_ref(x, np.ones(96), eps=0.0).astype(np.float64)
    np.testing.assert_allclose(np.sqrt(np.mean(unit * unit, axis=-1)), 1.0, rtol=1e-6)  # unit RMS per row
    assert not ol.rms_norm_ref(np.zeros((2, 8)), np.ones(8)).any()  # zeros stay zero (eps > 0)
    g = np.array([0.0, 40.0, -40.0, 1.0], np.float32)
    u = np.array([3.0, 2.0, 5.0, 1.0], np.float32)
    s = ol.swiglu_ref(g, u)
    assert s[0] == 0.0 and abs(s[1] - 80.0) < 1e-4 and abs(s[2]) < 1e-12
    np.testing.assert_allclose(s[3], 1.0 / (1.0 + np.exp(-1.0)), rtol=1e-6)  # silu(1) = sigmoid(1)
    # Zero weights: attention and MLP add nothing, the layer returns its input.
    E, H, Hkv, D, I, S = 32, 4, 2, 8, 48, 6
    zw = {"ln1": np.ones(E, np.float32), "ln2": np.ones(E, np.float32), "q": np.zeros((E, H * D)), "k": np.zeros((E, Hkv * D)),
          "v": np.zeros((E, Hkv * D)), "o": np.zeros((H * D, E)), "gate": np.zeros((E, I)), "up": np.zeros((E, I)),
          "down": np.zeros((I, E))}
    cache = {"k": np.zeros((Hkv, 16, D), np.float32), "v": np.zeros((Hkv, 16, D), np.float32)}
    cos, sin = orope.precompute_cos_sin(16, D, 1e4)
    h = rng.standard_normal((S, E)).astype(np.float32)
    np.testing.assert_array_equal(ol.decoder_layer_ref(h, zw, cache, 0, cos, sin, H, Hkv), h)


def test_sample_ref_pins():
    """sample_ref against np.random.choice / np.argmax themselves, plus the
    softmax closed form and the empirical distribution of many draws."""
    from scipy.special import softmax

    from oracle import sample as osm

    rng = np.random.default_rng(11)
    for V in (1, 2, 100, 5000):
        x = (3.0 * rng.standard_normal(V)).astype(np.float32)
        for T in (0.5, 1.0, 1.7):
            # probabilities: softmax(x / T) from the library
            np.testing.assert_allclose(osm.probs_ref(x, T, 0), softmax(x.astype(np.float64) / np.float32(T)),
                                       rtol=1e-5, atol=1e-12)
            for k in (0, 1, 3, 50, V, 999999):
                p = osm.probs_ref(x, T, k)
                for seed in range(6):
                    np.random.seed(seed)
                    want = int(np.random.choice(V, p=p))  # the reference's call
                    np.random.seed(seed)
                    assert osm.sample_ref(x, T, k, np.random.random_sample()) == want
                if 0 < k < V:  # the k largest logits survive, renormalised
                    top = np.argsort(x)[::-1][:k]
                    assert set(np.nonzero(p)[0]) == set(top)
                    np.testing.assert_allclose(p[top], softmax(x[top].astype(np.float64) / np.float32(T)), rtol=1e-5)
                    assert osm.kept_mask(x, k).sum() == k
    # greedy: first maximum, NaN first, exactly np.argmax
    y = np.array([1.0, 5.0, 5.0, -2.0], np.float32)
    assert osm.sample_ref(y, 0.0, 0, 0.3) == 1 == np.argmax(y)
    assert osm.sample_ref(y, 1e-6, 3, 0.9) == 1  # the cut-off itself is greedy
    assert osm.sample_ref(np.array([1.0, np.nan, 3.0, np.nan], np.float32), 0.0, 0, 0.5) == 1
    # ties at the k-th: the device keeps all of them; without ties its rule
    # is the reference's
    z = np.array([0.0, 2.0, 1.0, 2.0, 1.0, 1.0], np.float32)
    assert osm.kept_mask(z, 3).tolist() == [False, True, True, True, True, True]
    # p = [0, e^2, e, e^2, e, e] / (2 e^2 + 3 e): steps at .322 .441 .763 .882 1
    assert [osm.sample_kept_ref(z, 1.0, 3, u) for u in (0.1, 0.4, 0.7, 0.9, 0.99)] == [1, 2, 3, 5, 5]
    x = (2.0 * rng.standard_normal(3000)).astype(np.float32)
    for k in (0, 1, 7, 64, 2999, 5000):
        for u in rng.random(50):
            assert osm.sample_kept_ref(x, 0.9, k, u) == osm.sample_ref(x, 0.9, k, u)
    # u = 0 picks the first entry with mass; u -> 1 the last
    w = np.array([-np.inf, 0.0, 0.0, -np.inf], np.float32)
    assert osm.sample_ref(w, 1.0, 0, 0.0) == 1 and osm.sample_ref(w, 1.0, 0, 1 - 2.0 ** -53) == 2
    # many draws follow p
    x = rng.standard_normal(8).astype(np.float32)
    p = osm.probs_ref(x, 0.8, 5)
    u = rng.random(40000)
    counts = np.bincount([osm.sample_ref(x, 0.8, 5, ui) for ui in u], minlength=8) / u.size
    np.testing.assert_allclose(counts, p, atol=0.012)
