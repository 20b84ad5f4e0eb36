"""GPU parity of the batched prefill (wv_matmul*) through the C ABI.

Row-interleaved Q4_K blobs run the fp16-MFMA GEMM (each token row scaled by
a power of two into fp16's range); the bar there is the
north-star's bf16/fp16-MFMA tolerance: max|Y - Y_ref| / max|Y_ref| <= 2e-3
against the f64 textbook product over the reference's dequantized weights
(which is what welvet's M independent f64-accumulated GEMVs compute, up to
one f32 rounding). Blobs without an MFMA kernel run the batched GEMV kernels
and keep the GEMV bar of 1e-5.
"""

import numpy as np
import pytest

import oracle
import welvet_amd as wv

pytestmark = pytest.mark.gpu

TOL_MFMA = 2e-3
TOL_F32 = 1e-5


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def rowwise(y, ref):
    ref = np.asarray(ref, np.float64)
    err = np.abs(np.asarray(y, np.float64) - ref).max(axis=1)
    return float((err / np.maximum(np.abs(ref).max(axis=1), 1e-30)).max())


def packed_q4k(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    p = wv.pack("Q4_K", w, rows, cols)
    wd = oracle.unpack(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights))
    return p, wd.reshape(rows, cols).astype(np.float64), rng


@pytest.mark.parametrize("shape", [(256, 1024), (200, 512), (64, 256), (448, 2048)])
@pytest.mark.parametrize("m", [1, 7, 32, 33, 64, 65, 128, 130])
def test_prefill_q4k_small(shape, m):
    rows, cols = shape
    print(f"[gpu] prefill q4k {cols}->{rows} M={m}", flush=True)
    p, wd, rng = packed_q4k(rows, cols, rows + m)
    d = wv.upload(p)
    assert d.info()["layout"] == "row-interleaved"
    x = rng.standard_normal((m, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ wd.T
    ys = []
    for _ in range(2):  # split-K scratch is per call; results must not depend on the previous call
        y = d.matmul(x)
        assert normwise(y, ref) <= TOL_MFMA
        assert rowwise(y, ref) <= 4 * TOL_MFMA
        ys.append(y)
    assert np.array_equal(ys[0], ys[1])  # fixed-order sums: the same bits every call
    d.free()


@pytest.mark.parametrize("shape", [(256, 1024), (200, 512), (448, 2048), (1000, 4096)])
@pytest.mark.parametrize("m", [256, 300])
def test_prefill_q4k_wide(shape, m):
    """Token blocks of 256 and more (several 128-token tiles): padded rows, a
    ragged last token tile, and K split over blocks (every shape here leaves
    CUs idle)."""
    rows, cols = shape
    print(f"[gpu] prefill wide q4k {cols}->{rows} M={m}", flush=True)
    p, wd, rng = packed_q4k(rows, cols, rows + m)
    d = wv.upload(p)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ wd.T
    ys = []
    for _ in range(2):
        y = d.matmul(x)
        assert normwise(y, ref) <= TOL_MFMA
        assert rowwise(y, ref) <= 4 * TOL_MFMA
        ys.append(y)
    assert np.array_equal(ys[0], ys[1])
    d.free()


@pytest.mark.parametrize("fmt", ["Q2_K", "Q3_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q4_1", "Q5_0", "Q5_1",
                                 "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S", "IQ4_XS", "IQ4_NL",
                                 "TernaryPacked", "BinaryPacked", "AffinePacked"])
@pytest.mark.parametrize("shape,m", [((256, 1024), 128), ((448, 2048), 300), ((1000, 4096), 130), ((300, 1024), 9),
                                     ((520, 2048), 33), ((256, 1024), 64)])
def test_prefill_other_formats_mfma(fmt, shape, m):
    """Token blocks over 8 of every other row-interleaved format take the
    packed-W MFMA GEMM (32-, 64- and 128-token tiles), each with its own
    B-operand builder (IQ4_NL's looks its float grid up as fp16)."""
    rows, cols = shape
    print(f"[gpu] prefill {fmt} {cols}->{rows} M={m}", flush=True)
    rng = np.random.default_rng(rows + m)
    w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    wd = oracle.unpack(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins))
    wd = wd.reshape(rows, cols).astype(np.float64)
    d = wv.upload(p)
    assert d.info()["layout"] == "row-interleaved"
    x = rng.standard_normal((m, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ wd.T
    for _ in range(2):
        y = d.matmul(x)
        assert normwise(y, ref) <= TOL_MFMA
        assert rowwise(y, ref) <= 4 * TOL_MFMA
    d.free()


@pytest.mark.parametrize("fmt", ["Q4_K", "Q8_0", "Q4_0", "IQ2_XS", "IQ4_NL"])
@pytest.mark.parametrize("m", [65, 100, 128])
def test_prefill_four_tile_blocks(fmt, m):
    """65 to 128 tokens on 200 row groups or more take the K-split-free
    small-M kernel with four 32-token tiles per wave (a ragged last tile)."""
    rows, cols = 12800, 512
    print(f"[gpu] prefill four-tile {fmt} {cols}->{rows} M={m}", flush=True)
    rng = np.random.default_rng(7 + m)
    w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    wd = oracle.unpack(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins))
    wd = wd.reshape(rows, cols).astype(np.float64)
    d = wv.upload(p)
    assert d.info()["layout"] == "row-interleaved"
    x = rng.standard_normal((m, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ wd.T
    for _ in range(2):
        y = d.matmul(x)
        assert normwise(y, ref) <= TOL_MFMA
        assert rowwise(y, ref) <= 4 * TOL_MFMA
    d.free()


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("m", [32, 64, 128, 300])
def test_prefill_outlier_and_tiny_activations(fmt, m):
    """Token rows the fp16 operand cannot hold unscaled: a few columns at
    +-1e3 and at +-1e5 (past fp16's 65504), a row of activations around 1e-9
    (fp16-subnormal), an all-zero row. Each row is scaled by a power of two
    before the fp16 cast and back in the epilogue, so every row meets the
    2e-3 bar on its own and nothing turns inf or NaN."""
    rows, cols = 448, 2048
    print(f"[gpu] prefill outliers {fmt} M={m}", flush=True)
    rng = np.random.default_rng(11 + m)
    w = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    wd = oracle.unpack(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins))
    wd = wd.reshape(rows, cols).astype(np.float64)
    d = wv.upload(p)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    for r in range(4):
        cs = rng.choice(cols, 5, replace=False)
        x[r, cs] = rng.choice([-1.0, 1.0], 5) * 1e3
        x[r + 4, cs] = rng.choice([-1.0, 1.0], 5) * 1e5
    x[8] *= np.float32(1e-9)
    x[9] = 0.0
    x[m - 1, :3] = [7e4, -9e4, 3.3e5]  # the last (possibly ragged) token tile too
    ref = x.astype(np.float64) @ wd.T
    y = d.matmul(x)
    assert np.isfinite(y).all()
    assert np.array_equal(y[9], np.zeros(rows, np.float32))
    err = rowwise(y, ref)
    print(f"[gpu]   rowwise err {err:.3e}", flush=True)
    assert err <= TOL_MFMA
    d.free()


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K", "Q3_K", "Q8_0", "Q4_0", "Q5_1", "IQ2_XS", "IQ4_NL",
                                 "TernaryPacked", "AffinePacked"])
@pytest.mark.parametrize("m", [16, 64, 300])
def test_prefill_tiny_and_huge_weight_rows(fmt, m):
    """Weight rows the fp16 B operand cannot hold unscaled: rows scaled by
    1e-9 (scales and weights fp16-subnormal or zero) up to 1e6 (weights past
    65504), and an all-zero row. Each row's scales and mins are multiplied by
    a power-of-two row factor before the fp16 cast and its outputs divided by
    it, so the rows of every scale meet the 2e-3 normwise bar on their own
    (and each row the 4x looser row-wise bar the other prefill tests use),
    with nothing inf or NaN, in both GEMM kernels (16 and 64 tokens: one block
    per row group; 300: 256-row tiles)."""
    rows, cols = 448, 2048
    print(f"[gpu] prefill weight rows 1e-9..1e6 {fmt} M={m}", flush=True)
    rng = np.random.default_rng(23 + m)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    decade = rng.choice([-9, -7, -5, -3, 0, 2, 4, 6], rows)
    w *= (10.0 ** decade).astype(np.float32)[:, None]
    w[5] = 0.0
    w = np.ascontiguousarray(w, np.float32).ravel()
    p = wv.pack(fmt, w, rows, cols)
    wd = oracle.unpack(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins))
    wd = wd.reshape(rows, cols).astype(np.float64)
    d = wv.upload(p)
    assert d.info()["layout"] == "row-interleaved"
    x = rng.standard_normal((m, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ wd.T
    y = d.matmul(x)
    assert np.isfinite(y).all()
    zero = ~wd.any(axis=1)  # the zero row, unless the format decodes zeros off zero (IQ2_XS: +-scale/2)
    assert np.array_equal(y[:, zero], np.zeros((m, int(zero.sum())), np.float32))
    live = ~zero
    for e in np.unique(decade):
        sel = live & (decade == e)
        err = normwise(y[:, sel], ref[:, sel])
        print(f"[gpu]   rows x 1e{e}: normwise err {err:.3e}", flush=True)
        assert err <= TOL_MFMA
    assert rowwise(y.T[live], ref.T[live]) <= 4 * TOL_MFMA  # per weight row
    d.free()


_BASE = {}


@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [32, 128, 512])
def test_prefill_q4k_baseline(shape, m):
    """Q4_K 4096->14336 and 14336->4096 at M = 32, 128, 512."""
    import torch
    rows, cols = shape
    print(f"[gpu] prefill baseline q4k {cols}->{rows} M={m}", flush=True)
    if shape not in _BASE:
        _BASE.clear()
        p, wd, _ = packed_q4k(rows, cols, 4242)
        _BASE[shape] = (p, wd.T.copy(), wv.upload(p))
    p, wdt, d = _BASE[shape]
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ wdt
    tx = torch.from_numpy(x).cuda()
    ty = torch.empty((m, rows), device="cuda")
    torch.cuda.synchronize()
    d.matmul_dev(tx.data_ptr(), ty.data_ptr(), m)
    wv.sync()
    y = ty.cpu().numpy()
    err = normwise(y, ref)
    print(f"[gpu]   normwise err {err:.3e}", flush=True)
    assert err <= TOL_MFMA


@pytest.mark.parametrize("fmt,m", [("Q8_0", 8), ("Q6_K", 8), ("Q5_K", 3), ("IQ4_NL", 8)])
def test_prefill_other_formats_use_batched_gemv(fmt, m):
    """Up to 8 token rows run the batched GEMVs, with the GEMV bar."""
    rows, cols = 300, 1024
    print(f"[gpu] prefill {fmt} M={m} via batched gemv", flush=True)
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    d = wv.upload(p)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    op = oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights)
    ref = oracle.reference_y(op, x)
    assert normwise(d.matmul(x), ref) <= TOL_F32
    d.free()


@pytest.mark.parametrize("fmt,cols,force_raw", [("Q4_K", 1024, True), ("IQ4_NL", 1024, True), ("Q8_0", 96, False),
                                                ("Q4_0", 160, False)])
def test_prefill_reference_layout_uses_batched_gemv(fmt, cols, force_raw):
    """Blobs on the reference layout (forced, or cols not a multiple of 256)
    take the batched GEMVs at any M, with the GEMV bar; token rows go 8 per
    launch, so M = 20 ends on a ragged launch."""
    rows, m = 200, 20
    print(f"[gpu] prefill {fmt} {cols}->{rows} M={m} on the reference layout", flush=True)
    rng = np.random.default_rng(31)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    d = wv.upload(p, reference_layout=force_raw)
    assert d.info()["layout"] == "raw"
    x = rng.standard_normal((m, cols)).astype(np.float32)
    op = oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins)
    ref = oracle.reference_y(op, x)
    assert normwise(d.matmul(x), ref) <= TOL_F32
    d.free()
