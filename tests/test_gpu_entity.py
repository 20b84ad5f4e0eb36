"""ENTITY wire uploads and the decoder built from a checkpoint, on the GPU.

A blob uploaded from its packed wire (wv_blob_upload_wire) must give the same
outputs bit for bit as the same blob uploaded from its fields (wv_blob_upload):
same layout, same kernels. The wire carries no Meta / BlockWeights, so IQ
formats take their default spec and BinaryPacked g128 / AffinePacked groups
are inferred from the scale counts (quant/binary_g128.go:79-94,
quant/affine_g64.go:99-122). The decoder loaded from a written checkpoint must
equal the decoder assembled from the same blobs, and the f64 oracle within
1e-5.
"""
import numpy as np
import pytest

import oracle
import welvet_amd as wv
from oracle import decode_ref as dr
from welvet_amd import entity
from welvet_amd.decode import Config, Decoder

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def _g128_blob(rows, cols, rng):
    words = rng.integers(0, 2**32, size=rows * cols // 32, dtype=np.uint64).astype(np.uint32)
    scales = (np.abs(rng.standard_normal(rows * cols // 128)) * 0.02 + 1e-3).astype(np.float32)
    return wv.PackedBlob("BinaryPacked", rows, cols, words.view(np.uint8), scales, None, 128)


def _affine32_blob(rows, cols, rng):
    words = rng.integers(0, 2**32, size=rows * cols // 8, dtype=np.uint64).astype(np.uint32)
    ng = rows * cols // 32
    return wv.PackedBlob("AffinePacked", rows, cols, words.view(np.uint8),
                         (np.abs(rng.standard_normal(ng)) * 0.01).astype(np.float32), np.array([4], np.uint8), 32,
                         mins=(rng.standard_normal(ng) * 0.05).astype(np.float32))


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K", "Q8_0", "Q5_K", "IQ4_XS", "IQ2_XXS", "TernaryPacked",
                                 "BinaryPacked", "AffinePacked", "g128", "affine32"])
def test_wire_upload_equals_field_upload(fmt):
    print(f"[gpu] wire upload {fmt}", flush=True)
    rng = np.random.default_rng(5)
    rows, cols = 96, 512
    if fmt == "g128":
        p = _g128_blob(rows, cols, rng)
    elif fmt == "affine32":
        p = _affine32_blob(rows, cols, rng)
    else:
        p = wv.pack(fmt, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32), rows, cols)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    gy = rng.standard_normal(rows).astype(np.float32)
    gx0 = rng.standard_normal(cols).astype(np.float32)
    a = wv.upload(p)
    b = wv.DeviceBlob.from_wire(p.fmt, rows, cols, entity.encode_packed_blob(p))
    assert a.info()["layout"] == b.info()["layout"]
    assert np.array_equal(a.matvec(x), b.matvec(x))
    assert np.array_equal(a.matvec_t(gy, gx0), b.matvec_t(gy, gx0))
    ref = oracle.reference_y(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins), x)
    assert np.abs(b.matvec(x) - ref).max() / np.abs(ref).max() <= 1e-5
    a.free()
    b.free()


def test_decoder_from_entity(tmp_path):
    """A 2-layer Q4_K checkpoint (GQA 4/2, head_dim 64, tied LM head packed,
    final norm): the loaded decoder equals the assembled one and the oracle."""
    print("[gpu] decoder from entity", flush=True)
    cfg = Config(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, max_seq=96,
                 rope_theta=1e4, rms_eps=1e-6)
    rng = np.random.default_rng(17)
    shapes = {"q": (cfg.q_dim, cfg.hidden), "k": (cfg.kv_dim, cfg.hidden), "v": (cfg.kv_dim, cfg.hidden),
              "o": (cfg.hidden, cfg.q_dim), "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden),
              "down": (cfg.hidden, cfg.ffn)}
    items, layers, ref_layers = [], [], []
    for L in range(cfg.n_layers):
        packed = {}
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            r, c = shapes[name]
            packed[name] = wv.pack("Q4_K", (rng.standard_normal(r * c) * 0.02).astype(np.float32), r, c)
            items.append((f"blocks.{L}.{name}", packed[name]))
        an = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        fn = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        items += [(f"blocks.{L}.attn_norm", an), (f"blocks.{L}.ffn_norm", fn)]
        layers.append((packed, an, fn))
        ref_layers.append(({k: dr.DenseW(v) for k, v in packed.items()}, an, fn))
    lm = wv.pack("Q4_K", (rng.standard_normal(cfg.vocab * cfg.hidden) * 0.02).astype(np.float32), cfg.vocab, cfg.hidden)
    fnorm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    emb = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    items += [("transformer.lm_head.packed", lm), ("transformer.final_norm", fnorm), ("transformer.embeddings", emb)]
    spec = {"architecture": "llama", "hidden_size": cfg.hidden, "vocab_size": cfg.vocab, "max_seq_len": cfg.max_seq,
            "lm_head_tied": True, "has_final_norm": True, "pack_format": "Q4_K",
            "dims": {"num_layers": cfg.n_layers, "num_heads": cfg.n_heads, "num_kv_heads": cfg.n_kv_heads,
                     "head_dim": cfg.head_dim, "intermediate_size": cfg.ffn}}
    path = tmp_path / "tiny.entity"
    entity.write_transformer_file(str(path), spec, items)

    dec_f = entity.decoder_from_entity(str(path))
    assert dec_f.cfg == cfg
    dec_a = Decoder(cfg)
    keep = []
    for L, (packed, an, fn) in enumerate(layers):
        blobs = [wv.upload(packed[n]) for n in ("q", "k", "v", "o", "gate", "up", "down")]
        keep += blobs
        dec_a.set_layer(L, blobs, an, fn)
    lm_d = wv.upload(lm)
    keep.append(lm_d)
    dec_a.set_output(lm_d, fnorm, emb)
    ref = dr.DecodeRef(cfg, ref_layers, dr.DenseW(lm), fnorm, emb)
    for L in range(cfg.n_layers):
        k = rng.standard_normal((40, cfg.kv_dim)).astype(np.float32)
        v = rng.standard_normal((40, cfg.kv_dim)).astype(np.float32)
        for d in (dec_f, dec_a):
            d.set_kv(L, 0, k, v)
        ref.set_kv(L, 0, k, v)
    t_f, l_f = dec_f.generate(7, 40, 3, advance_pos=True, want_logits=True)
    t_a, l_a = dec_a.generate(7, 40, 3, advance_pos=True, want_logits=True)
    assert np.array_equal(t_f, t_a) and np.array_equal(l_f, l_a)
    t = 7
    for i in range(3):
        rl, _ = ref.step(t, 40 + i)
        t = int(t_f[i])
    assert np.abs(l_f.astype(np.float64) - rl).max() / np.abs(rl).max() <= 1e-5
    dec_f.free()
    dec_a.free()
