"""The device prompt forward (wv_decoder_prefill) and the decode steps that
follow it, against the f64 oracle (oracle/decode_ref.py DecodeRef.prefill,
pinned against a whole-block forward in tests/test_decode_oracle.py).

Bars: the last prompt row's logits, and the logits of the decode steps that
continue from the device caches, within 2e-3 normwise where the projections
run on the fp16-MFMA prefill GEMM (its K and V rows feed every later step),
and within 1e-5 where the block is short enough for the batched f32 GEMVs
(Q8_0, 8 tokens). Tokens are compared where the oracle's top-2 logit gap
exceeds the bar."""
import numpy as np
import pytest

import welvet_amd as wv
from oracle import decode_ref as dr
from welvet_amd.decode import Config, Decoder

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / np.abs(ref).max())


def build(cfg: Config, fmt: str, seed: int, tweak=None):
    """tweak(name, w) may rescale rows of a projection's (rows, cols) f32
    weights before packing."""
    rng = np.random.default_rng(seed)
    shapes = {"q": (cfg.q_dim, cfg.hidden), "k": (cfg.kv_dim, cfg.hidden), "v": (cfg.kv_dim, cfg.hidden),
              "o": (cfg.hidden, cfg.q_dim), "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden),
              "down": (cfg.hidden, cfg.ffn)}
    dec = Decoder(cfg)
    ref_layers = []
    for L in range(cfg.n_layers):
        blobs, dense = [], {}
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            r, c = shapes[name]
            w = (rng.standard_normal(r * c) * 0.02).astype(np.float32)
            if tweak is not None:
                w = np.ascontiguousarray(tweak(name, w.reshape(r, c)), np.float32).ravel()
            p = wv.pack(fmt, w, r, c)
            blobs.append(wv.upload(p))
            dense[name] = dr.DenseW(p)
        an = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        fn = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        dec.set_layer(L, blobs, an, fn)
        ref_layers.append((dense, an, fn))
    pl = wv.pack(fmt, (rng.standard_normal(cfg.vocab * cfg.hidden) * 0.02).astype(np.float32), cfg.vocab, cfg.hidden)
    fnorm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    emb = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    dec.set_output(wv.upload(pl), fnorm, emb)
    return dec, dr.DecodeRef(cfg, ref_layers, dr.DenseW(pl), fnorm, emb)


def check_token(tok, rl, tol):
    top2 = np.sort(rl)[-2:]
    if top2[1] - top2[0] > tol * np.abs(rl).max():
        assert tok == int(np.argmax(rl))


# Token counts by GEMM plan: 33 (A-fragment operands, 32-token tiles plus a
# padded one), 100 (A fragments, 64-token blocks on the few row groups of
# these widths), 300 (row-major operands, 128-token tiles).
CASES = [("Q4_K", 33, 2e-3), ("Q4_K", 100, 2e-3), ("Q4_K", 300, 2e-3), ("Q6_K", 33, 2e-3), ("Q8_0", 8, 1e-5)]


# Head dims and heads: G = nh / nkv query heads per KV head. The MFMA
# attention (head dims 64 and 128, G = 1, 2, 4, 8) maps G heads of 128 / G
# positions to a block's rows; G = 3 takes the scalar kernel.
HEADS = [(64, 8, 2), (128, 4, 1), (64, 8, 8), (128, 8, 4), (64, 8, 1), (64, 6, 2)]


@pytest.mark.parametrize("fmt,n,tol", CASES)
@pytest.mark.parametrize("hd,nh,nkv", HEADS)
def test_prefill_then_decode(fmt, n, tol, hd, nh, nkv):
    print(f"[gpu] prefill {fmt} n={n} hd={hd} heads {nh}/{nkv}", flush=True)
    cfg = Config(n_layers=2, hidden=512, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=1024, vocab=500, max_seq=320)
    dec, ref = build(cfg, fmt, 7 + n + hd)
    toks = np.random.default_rng(n).integers(0, cfg.vocab, n)
    nxt, logits = dec.prefill(toks, 0, want_logits=True)
    rl, _ = ref.prefill(toks)
    err = normwise(logits, rl)
    print(f"[gpu]   prompt logits normwise {err:.2e}", flush=True)
    assert err <= tol
    check_token(nxt, rl, tol)
    steps = 3
    t_dev, l_dev = dec.generate(nxt, n, steps, advance_pos=True, want_logits=True)
    t = nxt
    for i in range(steps):
        rl, _ = ref.step(t, n + i)
        check_token(int(t_dev[i]), rl, tol)
        t = int(t_dev[i])
    err = normwise(l_dev, rl)
    print(f"[gpu]   decode logits after the prompt normwise {err:.2e}", flush=True)
    assert err <= tol
    dec.free()


@pytest.mark.parametrize("hd,nh,nkv", [(64, 32, 4), (128, 32, 8)])
def test_prefill_long_prompt(hd, nh, nkv):
    """A 1030-token prompt whose MFMA attention blocks (128 rows each) number
    256 or more, launched longest key range first; then one decode step from
    its caches."""
    n = 1030
    G = nh // nkv
    assert nkv * -(-n // (128 // G)) >= 256
    print(f"[gpu] long prefill n={n} hd={hd} heads {nh}/{nkv}", flush=True)
    cfg = Config(n_layers=1, hidden=256, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=512, vocab=300, max_seq=1040)
    dec, ref = build(cfg, "Q4_K", 11 + hd)
    toks = np.random.default_rng(hd).integers(0, cfg.vocab, n)
    nxt, logits = dec.prefill(toks, 0, want_logits=True)
    rl, _ = ref.prefill(toks)
    err = normwise(logits, rl)
    print(f"[gpu]   prompt logits normwise {err:.2e}", flush=True)
    assert err <= 2e-3
    check_token(nxt, rl, 2e-3)
    t_dev, l_dev = dec.generate(nxt, n, 1, advance_pos=True, want_logits=True)
    rl, _ = ref.step(nxt, n)
    assert normwise(l_dev, rl) <= 2e-3
    check_token(int(t_dev[0]), rl, 2e-3)
    dec.free()


def test_prefill_qkv_stack_row_factors():
    """Q, K and V blobs with a few rows scaled by 1e-6: their prefill-GEMM row
    factors (powers of two putting a row's largest fp16 operand in [2^12,
    2^13)) pass 2^20, so the GEMM applies every row's factor. The prompt's one
    GEMM on the decoder's Q|K|V stack must take the three blobs' factors in
    stack order; a factor on the wrong row would scale that row's outputs by
    the ratio of two factors."""
    print("[gpu] prefill Q|K|V stack with row factors", flush=True)
    cfg = Config(n_layers=2, hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=500, max_seq=320)

    def tweak(name, w):
        if name in ("q", "k", "v"):
            w = w.copy()
            w[[3, 40, w.shape[0] - 1]] *= np.float32(1e-6)
        return w

    dec, ref = build(cfg, "Q4_K", 61, tweak)
    toks = np.random.default_rng(9).integers(0, cfg.vocab, 300)
    nxt, logits = dec.prefill(toks, 0, want_logits=True)
    rl, _ = ref.prefill(toks)
    err = normwise(logits, rl)
    print(f"[gpu]   prompt logits normwise {err:.2e}", flush=True)
    assert np.isfinite(logits).all()
    assert err <= 2e-3
    check_token(nxt, rl, 2e-3)
    t_dev, l_dev = dec.generate(nxt, 300, 1, advance_pos=True, want_logits=True)
    rl, _ = ref.step(nxt, 300)
    assert normwise(l_dev, rl) <= 2e-3
    dec.free()


@pytest.mark.parametrize("n", [33, 100, 200])
def test_prefill_split_projections(n):
    """One layer at hidden 4096 and SwiGLU 8192 (Q|K|V 6144 x 4096, O 4096 x
    4096, down 4096 x 8192), where the prompt GEMMs split K over blocks: at 33
    and 100 tokens O splits 2 ways and down 4 and 2 ways, their slices left
    unsummed for the norm after them to add; at 200 tokens (128-token tiles)
    O and down split 8 ways and are summed before it. The Q|K|V stack splits
    2, 1 and 4 ways, its slices added by RoPE."""
    print(f"[gpu] prefill with split projections n={n}", flush=True)
    cfg = Config(n_layers=1, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=8192, vocab=300, max_seq=208)
    dec, ref = build(cfg, "Q4_K", 71 + n)
    toks = np.random.default_rng(n + 3).integers(0, cfg.vocab, n)
    nxt, logits = dec.prefill(toks, 0, want_logits=True)
    rl, _ = ref.prefill(toks)
    err = normwise(logits, rl)
    print(f"[gpu]   prompt logits normwise {err:.2e}", flush=True)
    assert err <= 2e-3
    check_token(nxt, rl, 2e-3)
    t_dev, l_dev = dec.generate(nxt, n, 1, advance_pos=True, want_logits=True)
    rl, _ = ref.step(nxt, n)
    assert normwise(l_dev, rl) <= 2e-3
    dec.free()


def test_prefill_in_two_blocks():
    """A prompt in two calls (20 rows at position 0, then 13 at 20): the second
    block attends to the cache rows the first one wrote."""
    print("[gpu] prefill in two blocks", flush=True)
    cfg = Config(n_layers=2, hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=500, max_seq=64)
    dec, ref = build(cfg, "Q4_K", 41)
    toks = np.random.default_rng(5).integers(0, cfg.vocab, 33)
    dec.prefill(toks[:20], 0)
    nxt, logits = dec.prefill(toks[20:], 20, want_logits=True)
    rl, _ = ref.prefill(toks)
    assert normwise(logits, rl) <= 2e-3
    check_token(nxt, rl, 2e-3)
    dec.free()


def test_prefill_errors():
    cfg = Config(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, max_seq=16)
    dec, _ = build(cfg, "Q4_K", 3)
    with pytest.raises(wv.WelvetError, match="empty ids"):
        dec.prefill(np.zeros(0, np.int32))
    with pytest.raises(wv.WelvetError, match="SHAPE"):
        dec.prefill(np.zeros(10, np.int32), 8)
    dec.free()
