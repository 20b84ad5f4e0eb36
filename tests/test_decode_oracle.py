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


class _Dense:
    """A projection with an exact f64 weight matrix (stands in for DenseW)."""

    def __init__(self, w):
        self.w = w

    def __call__(self, x32):
        return (self.w @ x32.astype(np.float64)).astype(np.float32)


def _block_forward(cfg, layers, lm, fnorm, emb, tokens):
    """ForwardTokens over a token block written independently of DecodeRef:
    every row at once, attention under an explicit causal mask over the
    block's own K/V rows (layers/mha/attn.go:40-118)."""
    n, hd = len(tokens), cfg.head_dim
    g = cfg.n_heads // cfg.n_kv_heads
    h = emb[np.asarray(tokens)].astype(np.float32)
    f32 = np.float32
    for w, an, fn in layers:
        def norm(x, gm):
            x64 = x.astype(np.float64)
            inv = 1.0 / np.sqrt((x64 * x64).sum(1, keepdims=True) / x.shape[1] + cfg.rms_eps)
            return (x64 * inv * gm.astype(np.float64)).astype(f32)

        n1 = norm(h, an)
        q = (n1.astype(np.float64) @ w["q"].w.T).astype(f32).astype(np.float64)
        k = (n1.astype(np.float64) @ w["k"].w.T).astype(f32).astype(np.float64)
        v = (n1.astype(np.float64) @ w["v"].w.T).astype(f32).astype(np.float64)
        for s in range(n):
            dr.rope(q[s], s, cfg.n_heads, hd, cfg.rope_theta)
            dr.rope(k[s], s, cfg.n_kv_heads, hd, cfg.rope_theta)
        att = np.zeros((n, cfg.n_heads * hd))
        mask = np.tril(np.ones((n, n), bool))
        for hh in range(cfg.n_heads):
            kv = hh // g
            Q = q[:, hh * hd:(hh + 1) * hd]
            K = k[:, kv * hd:(kv + 1) * hd]
            V = v[:, kv * hd:(kv + 1) * hd]
            sc = np.where(mask, Q @ K.T / math.sqrt(hd), -np.inf)
            p = np.exp(sc - sc.max(1, keepdims=True))
            att[:, hh * hd:(hh + 1) * hd] = (p / p.sum(1, keepdims=True)) @ V
        att = att.astype(f32)
        h = (h + (att.astype(np.float64) @ w["o"].w.T).astype(f32)).astype(f32)
        n2 = norm(h, fn)
        gt = (n2.astype(np.float64) @ w["gate"].w.T).astype(f32).astype(np.float64)
        up = (n2.astype(np.float64) @ w["up"].w.T).astype(f32).astype(np.float64)
        hm = (gt / (1.0 + np.exp(-gt)) * up).astype(f32)
        h = (h + (hm.astype(np.float64) @ w["down"].w.T).astype(f32)).astype(f32)
    last = dr.rmsnorm(h[-1], fnorm, cfg.rms_eps)
    return (lm.w @ last.astype(np.float64)).astype(f32)


def test_prefill_equals_block_forward():
    """DecodeRef.prefill (per-position steps) against the whole-block forward."""
    from welvet_amd.decode import Config

    cfg = Config(n_layers=2, hidden=32, n_heads=4, n_kv_heads=2, head_dim=8, ffn=48, vocab=50, max_seq=40)
    rng = np.random.default_rng(3)
    shapes = {"q": (cfg.q_dim, cfg.hidden), "k": (cfg.kv_dim, cfg.hidden), "v": (cfg.kv_dim, cfg.hidden),
              "o": (cfg.hidden, cfg.q_dim), "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden),
              "down": (cfg.hidden, cfg.ffn)}
    layers = []
    for _ in range(cfg.n_layers):
        w = {k: _Dense(rng.standard_normal(s) * 0.2) for k, s in shapes.items()}
        layers.append((w, (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
                       (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)))
    lm = _Dense(rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.2)
    fnorm = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    emb = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    tokens = rng.integers(0, cfg.vocab, 13)
    ref = dr.DecodeRef(cfg, layers, lm, fnorm, emb)
    logits, tok = ref.prefill(tokens)
    want = _block_forward(cfg, layers, lm, fnorm, emb, tokens)
    assert np.abs(logits.astype(np.float64) - want).max() <= 1e-5 * np.abs(want).max()
    assert tok == int(np.argmax(want))
    # the caches hold the rotated K of every prompt position afterwards
    assert np.count_nonzero(np.abs(ref.kc[0][:13]).sum(1)) == 13 and not ref.kc[0][13:].any()
