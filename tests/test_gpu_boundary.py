"""The drop-in boundary on the GPU, through the C ABI:

* quant.MatVec / MatVecT's single-vector contract (quant/matvec.go:3-8,
  matvec_t.go:3-8, checkBlobYX / checkBlobGYGX quant/helpers.go:94-114):
  longer x / y are allowed and ignored, y past Rows and gx past Cols are not
  touched, short buffers fail with the reference's wording;
* dense.Forward's bias + activation epilogue (applyBiasAct,
  layers/dense/dense.go:145-167) on every layout, against the oracle;
* concurrent calls, as layers/dense/cpu.go:53-83 enters Forward from
  goroutines: host threads on one K-split blob and on distinct blobs, host
  and device-pointer entry points, each result checked against the oracle;
* a decoder whose LM head and final norm are replaced after a graph capture.
"""
import threading

import numpy as np
import pytest

import oracle
import welvet_amd as wv
from oracle import decode_ref as dr
from oracle import dense_ref
from welvet_amd.decode import Config, Decoder

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-300))


def packed_ref(p):
    return oracle.Packed(p.fmt, p.rows, p.cols, p.raw, p.scales, p.meta, p.block_weights, p.mins)


def make(fmt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    return p, wv.upload(p), rng


def test_quant_matvec_contract():
    p, d, rng = make("Q4_K", 256, 1024, 1)
    x = rng.standard_normal(1024 + 5).astype(np.float32)  # len(x) > Cols: the tail is not read
    y = np.full(256 + 3, -9.0, np.float32)  # len(y) > Rows: the tail is not written
    d.quant_matvec(x, y)
    ref = oracle.reference_y(packed_ref(p), x[:1024])[0]
    assert normwise(y[:256], ref) <= TOL and list(y[256:]) == [-9.0, -9.0, -9.0]
    with pytest.raises(wv.WelvetError, match=r"^SHAPE: MatVec: size mismatch rows=256 cols=1024 len\(x\)=1023 len\(y\)=259$"):
        d.quant_matvec(x[:1023], y)
    with pytest.raises(wv.WelvetError, match=r"MatVec: size mismatch rows=256 cols=1024 len\(x\)=1029 len\(y\)=255$"):
        d.quant_matvec(x, y[:255])
    # MatVecT: gx[:Cols] += W^T gy[:Rows]; a longer gy is ignored, a short gx rejected
    gy = rng.standard_normal(256 + 7).astype(np.float32)
    gx = np.concatenate([rng.standard_normal(1024), [4.0, 5.0]]).astype(np.float32)
    want = gx[:1024] + gy[:256].astype(np.float64) @ oracle.unpack(packed_ref(p)).reshape(256, 1024).astype(np.float64)
    d.quant_matvec_t(gy, gx)
    assert normwise(gx[:1024], want) <= TOL and list(gx[1024:]) == [4.0, 5.0]
    with pytest.raises(wv.WelvetError, match=r"MatVecT: size mismatch rows=256 cols=1024 len\(gy\)=263 len\(gx\)=1023$"):
        d.quant_matvec_t(gy, gx[:1023])
    with pytest.raises(wv.WelvetError, match=r"MatVecT: size mismatch rows=256 cols=1024 len\(gy\)=255 len\(gx\)=1026$"):
        d.quant_matvec_t(gy[:255], gx)
    d.free()
    pn = wv.pack("NativeTernary", np.ones(64 * 64, np.float32), 64, 64)
    dn = wv.upload(pn)
    with pytest.raises(wv.WelvetError, match="quant: MatVec not implemented for ternary"):
        dn.quant_matvec(np.zeros(64, np.float32), np.zeros(64, np.float32))
    dn.free()


def test_matvec_packed_blob_contract():
    """dense.MatVecPackedBlob (layers/dense/simd.go:570-614): packed formats
    as quant.MatVec; its shape error; FormatNone (and a Store's narrow DType)
    falls to the format switch's default error."""
    p, d, rng = make("Q6_K", 300, 512, 4)
    x = rng.standard_normal(512 + 3).astype(np.float32)
    y = np.full(300 + 2, -9.0, np.float32)
    d.matvec_packed_blob(x, y)
    ref = oracle.reference_y(packed_ref(p), x[:512])[0]
    assert normwise(y[:300], ref) <= TOL and list(y[300:]) == [-9.0, -9.0]
    with pytest.raises(wv.WelvetError, match=r"^SHAPE: dense: packed matvec shape$"):
        d.matvec_packed_blob(x[:511], y)
    with pytest.raises(wv.WelvetError, match=r"^SHAPE: dense: packed matvec shape$"):
        d.matvec_packed_blob(x, y[:299])
    d.free()
    for fmt in ("none", "NativeInt8"):
        pn = wv.pack(fmt, np.ones(64 * 128, np.float32), 64, 128)
        dn = wv.upload(pn)
        yn = np.full(64, -9.0, np.float32)
        with pytest.raises(wv.WelvetError, match=r"^FORMAT: dense: MatVecPackedBlob unsupported none$"):
            dn.matvec_packed_blob(np.ones(128, np.float32), yn)
        assert (yn == -9.0).all()
        dn.free()


def test_weight_budget_full_is_oom():
    """The resident-weight cap (the reference's soft cap on its weight caches,
    webgpu/affine_cache.go:111-123): an upload past it is WV_E_OOM with a
    message that IsAffineVRAMFull (affine_cache.go:73-83) classifies as VRAM
    full, reserves nothing, and fits again once a blob is freed."""
    p, a, rng = make("Q4_K", 256, 4096, 11)
    r1, cap0 = wv.weight_bytes()
    size = a.info()["device_bytes"]
    assert size >= p.nbytes
    wv.set_weight_budget(r1 + size // 2)
    try:
        with pytest.raises(wv.WelvetError) as e:
            wv.upload(p)
        assert e.value.code == -4
        msg = str(e.value)
        assert "weight VRAM budget full" in msg and "vram" in msg.lower() and "budget full" in msg
        assert wv.weight_bytes()[0] == r1  # the failed upload holds nothing
        a.free()
        assert wv.weight_bytes()[0] == r1 - size
        b = wv.upload(p)  # fits again
        x = rng.standard_normal(4096).astype(np.float32)
        ref = oracle.reference_y(packed_ref(p), x)[0]
        assert normwise(b.matvec(x), ref) <= TOL
        assert wv.weight_bytes()[0] == r1
        b.free()
    finally:
        wv.set_weight_budget(cap0)
    assert wv.weight_bytes()[0] == r1 - size


EPI = [("Q4_K", (512, 1024), "row-interleaved"), ("IQ4_NL", (300, 544), "raw"),
       ("Q6_K", (100, 700), "raw"), ("NativeInt4", (300, 512), "narrow"), ("none", (200, 300), "f32")]


@pytest.mark.parametrize("fmt,shape,layout", EPI)
@pytest.mark.parametrize("act", ["linear", "relu", "silu", "gelu", "tanh", "sigmoid", "leaky_relu", "relu2"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_dense_forward_bias_act(fmt, shape, layout, act, with_bias):
    rows, cols = shape
    p, d, rng = make(fmt, rows, cols, rows + len(act))
    assert d.info()["layout"] == layout
    x = rng.standard_normal((3, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1 if with_bias else None
    y = d.matvec(x)  # the product the epilogue starts from (checked against the oracle elsewhere)
    want_pre, want_post = dense_ref.apply_bias_act(y, bias, act)
    pre, post = d.dense_forward(x, bias, act)
    # pre and post come from the same GEMV sums: bit-equal up to the f64
    # activation math, which may differ from numpy's libm by 1 f64 ulp
    assert np.array_equal(pre, want_pre)
    assert np.abs(post.astype(np.float64) - want_post).max() <= 1e-6 * max(1.0, np.abs(want_post).max())
    d.free()


@pytest.mark.parametrize("fmt,rows,cols,batch,layout",
                         [("Q4_K", 512, 1024, 40, "row-interleaved"), ("Q8_0", 300, 1024, 20, "row-interleaved"),
                          ("IQ4_NL", 256, 512, 33, "row-interleaved"), ("Q4_K", 512, 1024, 5, "row-interleaved"),
                          ("Q8_0", 300, 1024, 6, "row-interleaved"), ("Q6_K", 100, 700, 20, "raw")])
@pytest.mark.parametrize("act", ["linear", "silu", "gelu"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_dense_forward_block(fmt, rows, cols, batch, layout, act, with_bias):
    """wv_dense_forward_block: a token block's pre = W x is the prefill GEMM's
    (bit-equal to wv_matmul, within 2e-3 of the f64 product) wherever
    wv_matmul takes the GEMM, wv_dense_forward's GEMV otherwise (Q8_0 at 6
    rows, the reference-layout Q6_K); bias and act as in wv_dense_forward."""
    print(f"[gpu] dense_forward_block {fmt} {cols}->{rows} batch {batch} {act} bias={with_bias}", flush=True)
    p, d, rng = make(fmt, rows, cols, rows + batch)
    assert d.info()["layout"] == layout
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1 if with_bias else None
    gemm = layout == "row-interleaved" and (fmt == "Q4_K" or batch > 8)
    y = d.matmul(x) if gemm else d.matvec(x)
    want_pre, want_post = dense_ref.apply_bias_act(y, bias, act)
    pre, post = d.dense_forward(x, bias, act, block=True)
    assert np.array_equal(pre, want_pre)
    assert np.abs(post.astype(np.float64) - want_post).max() <= 1e-6 * max(1.0, np.abs(want_post).max())
    wd = oracle.unpack(packed_ref(p)).reshape(rows, cols).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    assert normwise(y, ref) <= (2e-3 if gemm else TOL)
    d.free()


def test_dense_forward_needs_post_for_epilogue():
    p, d, rng = make("Q4_K", 64, 256, 2)
    L = wv.lib()
    x = np.zeros(256, np.float32)
    y = np.zeros(64, np.float32)
    rc = L.wv_dense_forward(d.handle, x.ctypes.data, y.ctypes.data, None, 1, None, 1)
    assert rc == -1 and "post buffer" in L.wv_last_error().decode()
    rc = L.wv_dense_forward(d.handle, x.ctypes.data, y.ctypes.data, None, 1, None, 99)
    assert rc == -1 and "ActivationType" in L.wv_last_error().decode()
    assert L.wv_dense_forward(d.handle, x.ctypes.data, y.ctypes.data, None, 1, None, -1) == 0
    d.free()


def test_concurrent_calls_on_shared_and_distinct_blobs():
    """8 host threads: wv_matvec and wv_matvec_t on one K-split Q4_K blob (512 x
    16384 splits K four ways; its MatVecT takes 8 slices), wv_matvec_dev on
    per-thread torch streams, and private blobs of other formats; 10 rounds
    each, every result checked against the oracle."""
    import torch
    shared_p, shared, rng = make("Q4_K", 512, 16384, 3)
    wd = oracle.unpack(packed_ref(shared_p)).reshape(512, 16384).astype(np.float64)
    errors = []

    def worker(tid):
        try:
            r = np.random.default_rng(100 + tid)
            fmt = ["Q6_K", "Q8_0", "IQ4_NL", "NativeTernary"][tid % 4]
            own_p = wv.pack(fmt, (r.standard_normal(300 * 1024) * 0.02).astype(np.float32), 300, 1024)
            own = wv.upload(own_p)
            stream = torch.cuda.Stream()
            for it in range(10):
                x = r.standard_normal(16384).astype(np.float32)
                y = shared.matvec(x)
                if normwise(y, wd @ x.astype(np.float64)) > TOL:
                    errors.append(f"thread {tid} round {it}: shared matvec")
                gy = r.standard_normal(512).astype(np.float32)
                gx = shared.matvec_t(gy)
                if normwise(gx, gy.astype(np.float64) @ wd) > TOL:
                    errors.append(f"thread {tid} round {it}: shared matvec_t")
                tx = torch.from_numpy(x).cuda()
                ty = torch.empty(512, device="cuda")
                torch.cuda.synchronize()
                shared.matvec_dev(tx.data_ptr(), ty.data_ptr(), 1, stream.cuda_stream)
                stream.synchronize()
                if normwise(ty.cpu().numpy(), wd @ x.astype(np.float64)) > TOL:
                    errors.append(f"thread {tid} round {it}: shared matvec_dev")
                xo = r.standard_normal(1024).astype(np.float32)
                yo = own.matvec(xo)
                if fmt == "NativeTernary":
                    ok = np.array_equal(yo, oracle.narrow_i8_forward(fmt, own_p.raw, own_p.tensor_scale, 300, 1024, xo)[0])
                else:
                    ok = normwise(yo, oracle.reference_y(packed_ref(own_p), xo)[0]) <= TOL
                if not ok:
                    errors.append(f"thread {tid} round {it}: own {fmt}")
            own.free()
        except Exception as e:  # noqa: BLE001
            errors.append(f"thread {tid}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors[:5]
    shared.free()


def test_decoder_output_replaced_after_capture():
    """Capture the step in a graph, then replace the LM head (and drop the
    final norm): the next steps must use the new head, and the old head may be
    freed (the decoder no longer reads it)."""
    cfg = Config(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, max_seq=64)
    rng = np.random.default_rng(21)
    dec = Decoder(cfg)
    shapes = [(cfg.q_dim, cfg.hidden), (cfg.kv_dim, cfg.hidden), (cfg.kv_dim, cfg.hidden), (cfg.hidden, cfg.q_dim),
              (cfg.ffn, cfg.hidden), (cfg.ffn, cfg.hidden), (cfg.hidden, cfg.ffn)]
    dense = {}
    blobs = []
    for name, (r, c) in zip(("q", "k", "v", "o", "gate", "up", "down"), shapes):
        p = wv.pack("Q4_K", (rng.standard_normal(r * c) * 0.02).astype(np.float32), r, c)
        dense[name] = dr.DenseW(p)
        blobs.append(wv.upload(p))
    an = np.ones(cfg.hidden, np.float32)
    fn = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    dec.set_layer(0, blobs, an, an)
    del blobs  # the Decoder keeps the layer's blobs alive
    emb = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    heads = [wv.pack("Q4_K", (rng.standard_normal(cfg.vocab * cfg.hidden) * 0.02).astype(np.float32), cfg.vocab,
                     cfg.hidden) for _ in range(2)]
    k = rng.standard_normal((20, cfg.kv_dim)).astype(np.float32)
    v = rng.standard_normal((20, cfg.kv_dim)).astype(np.float32)
    dec.set_kv(0, 0, k, v)
    dec.use_graph(True)
    dec.set_output(wv.upload(heads[0]), fn, emb)
    _, l0 = dec.generate(7, 20, 1, advance_pos=False, want_logits=True)
    dec.set_output(wv.upload(heads[1]), None, emb)  # the first head's only reference is dropped here
    import gc
    gc.collect()
    _, l1 = dec.generate(7, 20, 1, advance_pos=False, want_logits=True)
    for head, norm, got in ((heads[0], fn, l0), (heads[1], None, l1)):
        ref = dr.DecodeRef(cfg, [(dense, an, an)], dr.DenseW(head), norm, emb)
        ref.set_kv(0, 0, k, v)
        rl, _ = ref.step(7, 20)
        assert normwise(got, rl) <= TOL
    dec.free()
