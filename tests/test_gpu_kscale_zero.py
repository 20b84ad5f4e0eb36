"""k-quant blobs whose u8 group scales are 0, on every device path.

welvet decodes a k-quant group scale as sc = d*u/255 and, when that is 0,
as d/255 instead (quant/kquant.go:178-188). The packer writes u = 0 whenever
a group's range is below 1/510 of its super-block's largest
(kquant.go:149), which happens where near-zero channels share a
super-block with an outlier. The device layouts store u' = max(u, 1), which
gives d*u'/255 = d/255 for u = 0; this file checks that against the oracle on
the row-interleaved forward (an L > 1 plan, a K-split plan and the wide
no-split plan), the reference layout, MatVecT on both layouts, the prefill
GEMM and a decoder layer.

Weights: N(0, 0.02) with a sixth of the 16-column groups scaled by 1e-4 (so
their u rounds to 0). The "tiny" blobs also have the d of every seventh
super-block patched to 1e-44 or 1e-42 and some of its scale bytes to 1..17,
so that d*u/255 underflows to 0 and the fallback d/255 is itself 0 or
subnormal (those super-blocks then contribute their min term only). Bars:
the GEMV bar 1e-5 and the fp16-MFMA bar 2e-3, normwise against the f64
product over the reference's dequantized weights.
"""
import struct

import numpy as np
import pytest

import oracle
import welvet_amd as wv
from oracle import decode_ref as dr
from welvet_amd.decode import Config, Decoder

pytestmark = pytest.mark.gpu

TOL = 1e-5
TOL_MFMA = 2e-3
KFMT = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
BITS = {"Q2_K": 2, "Q3_K": 3, "Q4_K": 4, "Q5_K": 5, "Q6_K": 6}


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def sb_bytes(fmt):
    """kSuperBytes (kquant.go:53-60): d, dmin, 16 scales, 16 mins (not Q6_K), codes."""
    return 8 + 16 + (0 if fmt == "Q6_K" else 16) + 256 * BITS[fmt] // 8


def zero_scale_weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols // 16, 16)) * 0.02).astype(np.float32)
    quiet = rng.random((rows, cols // 16)) < 1 / 6
    w[quiet] *= np.float32(1e-4)
    return w.reshape(-1), rng


def zero_scale_blob(fmt, rows, cols, seed, tiny=False):
    w, rng = zero_scale_weights(rows, cols, seed)
    p = wv.pack(fmt, w, rows, cols)
    raw = p.raw.copy()
    nb = sb_bytes(fmt)
    nsb = raw.size // nb
    scales = raw.reshape(nsb, nb)[:, 8:24]
    if tiny:
        for si in range(0, nsb, 7):
            off = si * nb
            raw[off:off + 4] = np.frombuffer(struct.pack("<f", 1e-44 if si % 2 else 1e-42), np.uint8)
            raw[off + 8:off + 12] = [1, 5, 17, 0]
        scales = raw.reshape(nsb, nb)[:, 8:24]
    zeros = int((scales == 0).sum())
    assert zeros >= scales.size // 10, f"{fmt}: only {zeros} of {scales.size} group scales are 0"
    p.raw = raw
    return p, rng


def packed_of(p):
    return oracle.Packed(p.fmt, p.rows, p.cols, p.raw, p.scales, p.meta, p.block_weights, p.mins)


# (rows, cols): L = 4 / S = 2 plan (K <= 4096), K split over blocks, and the
# wide L = 4 / S = 4 plan without a split (the decoder's down shape).
FWD_SHAPES = [(256, 4096), (130, 8192), (4096, 14336)]


@pytest.mark.parametrize("fmt", KFMT)
@pytest.mark.parametrize("shape", FWD_SHAPES)
@pytest.mark.parametrize("tiny", [False, True])
def test_forward_zero_group_scales(fmt, shape, tiny):
    rows, cols = shape
    print(f"[gpu] kscale0 forward {fmt} {rows}x{cols} tiny={tiny}", flush=True)
    p, rng = zero_scale_blob(fmt, rows, cols, rows + cols, tiny)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    ref = oracle.reference_y(packed_of(p), x)
    for reference_layout in (False, True):
        d = wv.upload(p, reference_layout=reference_layout)
        assert d.info()["layout"] == ("raw" if reference_layout else "row-interleaved")
        y = d.matvec(x)
        assert np.isfinite(y).all()
        err = normwise(y, ref)
        print(f"[gpu]   layout {d.info()['layout']}: normwise {err:.2e}", flush=True)
        assert err <= TOL
        d.free()


@pytest.mark.parametrize("fmt", KFMT)
@pytest.mark.parametrize("shape", [(300, 2048), (130, 8192)])
def test_matvec_t_zero_group_scales(fmt, shape):
    rows, cols = shape
    print(f"[gpu] kscale0 matvec_t {fmt} {rows}x{cols}", flush=True)
    p, rng = zero_scale_blob(fmt, rows, cols, 3 * rows + cols, tiny=True)
    wd = oracle.unpack(packed_of(p)).reshape(rows, cols).astype(np.float64)
    gy = rng.standard_normal((2, rows)).astype(np.float32)
    gx0 = rng.standard_normal((2, cols)).astype(np.float32)
    want = gx0 + gy.astype(np.float64) @ wd
    for reference_layout in (False, True):
        d = wv.upload(p, reference_layout=reference_layout)
        assert normwise(d.matvec_t(gy, gx0), want) <= TOL
        d.free()


@pytest.mark.parametrize("fmt", KFMT)
@pytest.mark.parametrize("m", [32, 300])
def test_prefill_zero_group_scales(fmt, m):
    rows, cols = 448, 2048
    print(f"[gpu] kscale0 prefill {fmt} {cols}->{rows} M={m}", flush=True)
    p, rng = zero_scale_blob(fmt, rows, cols, 5 * m + rows, tiny=True)
    wd = oracle.unpack(packed_of(p)).reshape(rows, cols).astype(np.float64)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    d = wv.upload(p)
    assert d.info()["layout"] == "row-interleaved"
    y = d.matmul(x)
    assert np.isfinite(y).all()
    assert normwise(y, x.astype(np.float64) @ wd.T) <= TOL_MFMA
    d.free()


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K"])
def test_decoder_layer_zero_group_scales(fmt):
    """One decoder layer (Q||K||V, O, gate||up, down fused copies and the LM
    head built from such blobs), three greedy steps against the f64 oracle."""
    print(f"[gpu] kscale0 decoder {fmt}", flush=True)
    cfg = Config(n_layers=1, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1024, vocab=600, max_seq=96)
    shapes = {"q": (cfg.q_dim, cfg.hidden), "k": (cfg.kv_dim, cfg.hidden), "v": (cfg.kv_dim, cfg.hidden),
              "o": (cfg.hidden, cfg.q_dim), "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden),
              "down": (cfg.hidden, cfg.ffn)}
    rng = np.random.default_rng(99)
    dec = Decoder(cfg)
    blobs, dense = [], {}
    for i, name in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
        p, _ = zero_scale_blob(fmt, *shapes[name], seed=200 + i, tiny=(i % 2 == 0))
        blobs.append(wv.upload(p))
        dense[name] = dr.DenseW(p)
    an = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    fn = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    dec.set_layer(0, blobs, an, fn)
    pl, _ = zero_scale_blob(fmt, cfg.vocab, cfg.hidden, seed=300)
    lm = wv.upload(pl)
    fnorm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    emb = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    dec.set_output(lm, fnorm, emb)
    ref = dr.DecodeRef(cfg, [(dense, an, fn)], dr.DenseW(pl), fnorm, emb)
    k = rng.standard_normal((40, cfg.kv_dim)).astype(np.float32)
    v = rng.standard_normal((40, cfg.kv_dim)).astype(np.float32)
    dec.set_kv(0, 0, k, v)
    ref.set_kv(0, 0, k, v)
    toks, logits = dec.generate(7, 40, 3, advance_pos=True, want_logits=True)
    t = 7
    for i in range(3):
        rl, rt = ref.step(t, 40 + i)
        top2 = np.sort(rl)[-2:]
        if top2[1] - top2[0] > TOL * np.abs(rl).max():
            assert toks[i] == rt
        t = int(toks[i])
    err = float(np.abs(logits.astype(np.float64) - rl).max() / np.abs(rl).max())
    print(f"[gpu]   logits normwise {err:.2e}", flush=True)
    assert err <= TOL
    dec.free()
    for b in blobs + [lm]:
        b.free()
