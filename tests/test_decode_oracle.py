"""CPU pins of the decode-step oracle (oracle/decode_ref.py) by closed forms
and invariants, so that the GPU decode test compares against a checked
reference: RoPE sign and frequency convention (layers/mha/rope.go:6-21),
RMSNorm (layers/rmsnorm/cpu.go:70-85), softmax attention and its GQA head
mapping (layers/mha/attn.go:40-118), SiLU*up (layers/swiglu/cpu.go:41-53)."""
import math

import numpy as np

from oracle import decode_ref as dr


def test_rope_identity_at_pos0():
    rng = np.random.default_rng(0)
    v = rng.standard_normal(2 * 8)
    w = v.copy()
    dr.rope(w, 0, 2, 8, 5e5)
    assert np.array_equal(v, w)


def test_rope_closed_form_and_sign():
    # hd = 4: pairs (0, 2) with angle pos, (1, 3) with angle pos / theta^(1/2)
    theta, pos = 10000.0, 1
    v = np.array([1.0, 2.0, 3.0, 4.0])
    dr.rope(v, pos, 1, 4, theta)
    a0, a1 = 1.0, 1.0 / math.sqrt(theta)
    want = [1 * math.cos(a0) - 3 * math.sin(a0), 2 * math.cos(a1) - 4 * math.sin(a1),
            1 * math.sin(a0) + 3 * math.cos(a0), 2 * math.sin(a1) + 4 * math.cos(a1)]
    assert np.allclose(v, want, rtol=0, atol=1e-15)


def test_rope_composes_and_preserves_pair_norms():
    rng = np.random.default_rng(1)
    v = rng.standard_normal(3 * 16)
    a, b = v.copy(), v.copy()
    dr.rope(a, 5, 3, 16, 5e5)
    dr.rope(a, 7, 3, 16, 5e5)
    dr.rope(b, 12, 3, 16, 5e5)
    assert np.allclose(a, b, atol=1e-12)
    r = v.reshape(3, 16)
    ra = b.reshape(3, 16)
    assert np.allclose(r[:, :8] ** 2 + r[:, 8:] ** 2, ra[:, :8] ** 2 + ra[:, 8:] ** 2, atol=1e-12)


def test_rmsnorm_closed_form():
    x = np.full(64, 3.0, np.float32)
    g = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y = dr.rmsnorm(x, g, 1e-5)
    want = (3.0 / math.sqrt(9.0 + 1e-5)) * g.astype(np.float64)
    assert np.allclose(y, want.astype(np.float32), rtol=1e-7, atol=0)
    rng = np.random.default_rng(2)
    z = rng.standard_normal(256).astype(np.float32)
    yz = dr.rmsnorm(z, None, 0.0).astype(np.float64)
    assert abs(np.mean(yz ** 2) - 1.0) < 1e-6  # unit RMS with eps = 0


def test_attention_single_and_uniform_keys_and_gqa_mapping():
    hd, nh, nkv = 4, 4, 2
    q = np.ones(nh * hd)
    kc = np.zeros((8, nkv * hd))
    vc = np.zeros((8, nkv * hd))
    vc[0, :hd] = [1, 2, 3, 4]
    vc[0, hd:] = [5, 6, 7, 8]
    out = dr.attention(q, kc, vc, 1, nh, nkv, hd)  # one key: output is v of the head's KV group
    assert np.allclose(out, [1, 2, 3, 4, 1, 2, 3, 4, 5, 6, 7, 8, 5, 6, 7, 8])
    vc[1, :hd] = [3, 2, 1, 0]
    out = dr.attention(q, kc, vc, 2, nh, nkv, hd)  # equal scores: the mean
    assert np.allclose(out[:hd], [2, 2, 2, 2])
    kc[1, :hd] = 10.0  # key 1 dominates head 0-1 (scores 0 vs 40/2 = 20)
    out = dr.attention(q, kc, vc, 2, nh, nkv, hd)
    p1 = 1.0 / (1.0 + math.exp(-20.0))
    assert np.allclose(out[:hd], (1 - p1) * np.array([1, 2, 3, 4]) + p1 * np.array([3, 2, 1, 0]))


def test_silu_mul_closed_form():
    g = np.array([0.0, 1.0, -2.0, 30.0], np.float32)
    u = np.array([5.0, 2.0, 3.0, 0.5], np.float32)
    want = [0.0, 2.0 / (1 + math.exp(-1.0)), 3.0 * -2.0 / (1 + math.exp(2.0)), 0.5 * 30.0 / (1 + math.exp(-30.0))]
    assert np.allclose(dr.silu_mul(g, u), np.array(want, np.float32), rtol=1e-7)
