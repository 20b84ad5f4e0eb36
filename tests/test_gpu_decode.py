"""GPU parity of the device decode step (wv_decoder_*) against the f64 oracle
(oracle/decode_ref.py), through the C ABI.

Bar: the last step's logits within 1e-5 normwise (max|dl| / max|l|, the
north star's f32 bar) of the oracle after several greedy steps, and every
generated token equal to the oracle's where the oracle's top-2 logit gap
exceeds that tolerance (a nearer tie may legitimately flip under f32
rounding). Measured errors are 1e-7 to 2e-6 although attention and norms run
in f32 where the reference uses f64. Graph replays must equal eager launches
bit for bit (the kernels are deterministic).
"""
import numpy as np
import pytest

import welvet_amd as wv
from oracle import decode_ref as dr
from welvet_amd.decode import Config, Decoder

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def build(cfg: Config, fmt: str, seed: int, kv_fill: int):
    rng = np.random.default_rng(seed)
    shapes = {"q": (cfg.q_dim, cfg.hidden), "k": (cfg.kv_dim, cfg.hidden), "v": (cfg.kv_dim, cfg.hidden),
              "o": (cfg.hidden, cfg.q_dim), "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden),
              "down": (cfg.hidden, cfg.ffn)}
    dec = Decoder(cfg)
    keep, ref_layers = [], []
    for L in range(cfg.n_layers):
        blobs, dense = [], {}
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            r, c = shapes[name]
            w = (rng.standard_normal(r * c) * 0.02).astype(np.float32)
            p = wv.pack(fmt, w, r, c)
            blobs.append(wv.upload(p))
            dense[name] = dr.DenseW(p)
        an = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        fn = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        dec.set_layer(L, blobs, an, fn)
        keep += blobs
        ref_layers.append((dense, an, fn))
    wl = (rng.standard_normal(cfg.vocab * cfg.hidden) * 0.02).astype(np.float32)
    pl = wv.pack(fmt, wl, cfg.vocab, cfg.hidden)
    lm = wv.upload(pl)
    keep.append(lm)
    fnorm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    emb = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    dec.set_output(lm, fnorm, emb)
    ref = dr.DecodeRef(cfg, ref_layers, dr.DenseW(pl), fnorm, emb)
    for L in range(cfg.n_layers):
        k = rng.standard_normal((kv_fill, cfg.kv_dim)).astype(np.float32)
        v = rng.standard_normal((kv_fill, cfg.kv_dim)).astype(np.float32)
        dec.set_kv(L, 0, k, v)
        ref.set_kv(L, 0, k, v)
    return dec, ref, keep


def check_against_oracle(dec, ref, token, pos, steps):
    toks, logits = dec.generate(token, pos, steps, advance_pos=True, want_logits=True)
    t = token
    for i in range(steps):
        rl, rt = ref.step(t, pos + i)
        top2 = np.sort(rl)[-2:]
        if top2[1] - top2[0] > TOL * np.abs(rl).max():
            assert toks[i] == rt, f"step {i}: token {toks[i]} vs oracle {rt}"
        t = int(toks[i])  # follow the device's choice so both decode the same sequence
    err = float(np.abs(logits.astype(np.float64) - rl).max() / np.abs(rl).max())
    print(f"[gpu]   logits normwise err {err:.3e}", flush=True)
    assert err <= TOL
    return toks


@pytest.mark.parametrize("fmt", ["Q4_K", "Q5_K", "Q8_0", "Q3_K"])
def test_decode_small_hd64(fmt):
    """2 layers, GQA 4/2, head_dim 64; the steps cross a 32-position chunk boundary (positions 62-65)."""
    print(f"[gpu] decode small hd64 {fmt}", flush=True)
    cfg = Config(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, max_seq=96)
    dec, ref, keep = build(cfg, fmt, 7, kv_fill=62)
    check_against_oracle(dec, ref, token=11, pos=62, steps=4)
    dec.free()


def test_decode_padded_pairs_and_raw_down():
    """ffn 480: fused gate/up over a padded 64-row group; down (480 columns) stays on the raw layout."""
    print("[gpu] decode ffn 480", flush=True)
    cfg = Config(n_layers=2, hidden=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn=480, vocab=257, max_seq=80)
    dec, ref, keep = build(cfg, "Q4_K", 5, kv_fill=40)
    check_against_oracle(dec, ref, token=200, pos=40, steps=3)
    dec.free()


def test_decode_hd128_gqa4():
    print("[gpu] decode hd128 gqa4", flush=True)
    cfg = Config(n_layers=2, hidden=512, n_heads=4, n_kv_heads=1, head_dim=128, ffn=768, vocab=500, max_seq=200)
    dec, ref, keep = build(cfg, "Q4_K", 9, kv_fill=150)
    check_against_oracle(dec, ref, token=3, pos=150, steps=3)
    dec.free()


@pytest.mark.parametrize("hd", [64, 128])
def test_decode_gqa8(hd):
    """Eight query heads per KV head (the register attention kernel's widest
    case); the cache ends inside a chunk and the steps append into it."""
    print(f"[gpu] decode gqa8 hd {hd}", flush=True)
    cfg = Config(n_layers=2, hidden=512, n_heads=8, n_kv_heads=1, head_dim=hd, ffn=768, vocab=400, max_seq=128)
    dec, ref, keep = build(cfg, "Q4_K", 17, kv_fill=70)
    check_against_oracle(dec, ref, token=5, pos=70, steps=3)
    dec.free()


@pytest.mark.parametrize("hd", [64, 128])
def test_decode_gqa3_tile_kernel(hd):
    """Three query heads per KV head: the attention falls back to the LDS-tile kernel."""
    print(f"[gpu] decode gqa3 hd {hd}", flush=True)
    cfg = Config(n_layers=2, hidden=384, n_heads=6, n_kv_heads=2, head_dim=hd, ffn=512, vocab=300, max_seq=100)
    dec, ref, keep = build(cfg, "Q4_K", 23, kv_fill=45)
    check_against_oracle(dec, ref, token=8, pos=45, steps=3)
    dec.free()


@pytest.mark.parametrize("max_seq,kv_fill,hd", [(3000, 2900, 128), (6000, 5600, 64)])
def test_decode_long_cache(max_seq, kv_fill, hd):
    """Caches of 94 and 188 chunks of 32 positions: the combine variants past one wave of chunks."""
    print(f"[gpu] decode long cache max_seq {max_seq} hd {hd}", flush=True)
    cfg = Config(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=hd, ffn=512, vocab=300, max_seq=max_seq)
    dec, ref, keep = build(cfg, "Q4_K", 31, kv_fill=kv_fill)
    check_against_oracle(dec, ref, token=9, pos=kv_fill, steps=2)
    dec.free()


def test_decode_graph_equals_eager():
    print("[gpu] decode graph vs eager", flush=True)
    cfg = Config(n_layers=2, hidden=256, n_heads=8, n_kv_heads=2, head_dim=64, ffn=768, vocab=400, max_seq=160)
    dec, ref, keep = build(cfg, "Q4_K", 13, kv_fill=100)
    t_e, l_e = dec.generate(5, 100, 6, advance_pos=True, want_logits=True)
    dec.use_graph(True)
    for _ in range(3):  # replays after the first must match too
        t_g, l_g = dec.generate(5, 100, 6, advance_pos=True, want_logits=True)
        assert np.array_equal(t_e, t_g)
        assert np.array_equal(l_e, l_g)
    # fixed-position mode recomputes the same position each step
    t_f = dec.generate(5, 100, 3, advance_pos=False)
    dec.use_graph(False)
    t_f2 = dec.generate(5, 100, 3, advance_pos=False)
    assert np.array_equal(t_f, t_f2)
    dec.free()


def test_decode_full_width_one_layer():
    """BASELINE config 5 widths (hidden 4096, 32/8 heads, head_dim 128, SwiGLU 14336) on one layer, KV 2047 + 1."""
    print("[gpu] decode full-width layer", flush=True)
    cfg = Config(n_layers=1, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=2048,
                 max_seq=2048)
    dec, ref, keep = build(cfg, "Q4_K", 21, kv_fill=2047)
    check_against_oracle(dec, ref, token=17, pos=2047, steps=1)
    dec.free()


@pytest.mark.timeout(900)
def test_decode_config5_full():
    """BASELINE config 5 as bench.py runs it: 32 layers (4 distinct Q4_K layers
    cycled), hidden 4096, 32/8 heads x 128, SwiGLU 14336, vocab 32000, RoPE
    5e5, RMSNorm 1e-5, 2047 cached positions + this step. One greedy step
    against the f64 oracle (token, and logits within 1e-5 normwise), then two
    fixed-position steps eager and as graph replays: finite, bit-identical,
    and each against the oracle."""
    print("[gpu] decode config 5 (32 layers, vocab 32000)", flush=True)
    cfg = Config(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=32000,
                 max_seq=2048, rope_theta=5e5, rms_eps=1e-5)
    rng = np.random.default_rng(55)
    names = ("q", "k", "v", "o", "gate", "up", "down")
    shapes = {"q": (cfg.q_dim, cfg.hidden), "k": (cfg.kv_dim, cfg.hidden), "v": (cfg.kv_dim, cfg.hidden),
              "o": (cfg.hidden, cfg.q_dim), "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden),
              "down": (cfg.hidden, cfg.ffn)}
    distinct = []
    for i in range(4):
        ps = [wv.pack("Q4_K", rng.standard_normal(shapes[n][0] * shapes[n][1], dtype=np.float32) * np.float32(0.02),
                      *shapes[n]) for n in names]
        dense = {n: dr.DenseW(p) for n, p in zip(names, ps)}
        an = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        fn = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        distinct.append((ps, dense, an, fn))
        print(f"[gpu]   distinct layer {i} packed", flush=True)
    dec = Decoder(cfg)
    ref_layers = []
    for L in range(cfg.n_layers):
        ps, dense, an, fn = distinct[L % 4]
        dec.set_layer(L, [wv.upload(p) for p in ps], an, fn)
        ref_layers.append((dense, an, fn))
    pl = wv.pack("Q4_K", rng.standard_normal(cfg.vocab * cfg.hidden, dtype=np.float32) * np.float32(0.02),
                 cfg.vocab, cfg.hidden)
    fnorm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    emb = rng.standard_normal((cfg.vocab, cfg.hidden), dtype=np.float32)
    dec.set_output(wv.upload(pl), fnorm, emb)
    ref = dr.DecodeRef(cfg, ref_layers, dr.DenseW(pl), fnorm, emb)
    for L in range(cfg.n_layers):
        k = rng.standard_normal((cfg.max_seq - 1, cfg.kv_dim), dtype=np.float32)
        v = rng.standard_normal((cfg.max_seq - 1, cfg.kv_dim), dtype=np.float32)
        dec.set_kv(L, 0, k, v)
        ref.set_kv(L, 0, k, v)
    print("[gpu]   model resident", flush=True)
    pos = cfg.max_seq - 1
    tok = int(check_against_oracle(dec, ref, token=17, pos=pos, steps=1)[0])
    # fixed position: each step recomputes position `pos` from the previous step's token
    t_e, l_e = dec.generate(tok, pos, 2, advance_pos=False, want_logits=True)
    assert np.isfinite(l_e).all()
    dec.use_graph(True)
    for _ in range(2):
        t_g, l_g = dec.generate(tok, pos, 2, advance_pos=False, want_logits=True)
        assert np.array_equal(t_e, t_g) and np.array_equal(l_e, l_g)
    t = tok
    for i in range(2):
        rl, rt = ref.step(t, pos)
        top2 = np.sort(rl)[-2:]
        if top2[1] - top2[0] > TOL * np.abs(rl).max():
            assert t_e[i] == rt
        t = int(t_e[i])
    err = float(np.abs(l_e.astype(np.float64) - rl).max() / np.abs(rl).max())
    print(f"[gpu]   fixed-position logits normwise err {err:.3e}", flush=True)
    assert err <= TOL
    dec.free()
