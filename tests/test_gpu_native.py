"""GPU parity of the weights.Store DTypes through the C ABI.

* Dense's int8 path for Int8 / Int4 / Int2 / Ternary / Binary
  (layers/dense/simd.go:130-195, 303-326): int32 accumulators, activation
  scales and y bit-exact against the C oracle.
* FormatNone f32 weights (quant/none.go, forwardSIMDMasterF32): within 1e-5
  normwise of the f64 product.
* weights.Store.MatVec / MatVecT on FormatNone stores (weights/store.go:133-206,
  matVecNativeF64): f64 results within 1e-12 normwise of exact sums.
* MatVecT on the native layouts (BackwardSIMD's input gradient): 1e-5.
"""
import numpy as np
import pytest

import oracle
import welvet_amd as wv
from oracle import dense_ref, np_ref

pytestmark = pytest.mark.gpu

NARROW = ["NativeInt8", "NativeInt4", "NativeInt2", "NativeTernary", "NativeBinary"]
TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-300))


def native_blob(dt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    if dt == "NativeTernary":  # t in {-1, 0, +1}, P(0) = 0.33, absmean scale
        t = rng.choice([-1, 0, 1], size=rows * cols, p=[0.335, 0.33, 0.335]).astype(np.float32)
        w = (t * np.float32(0.013)).astype(np.float32)
    else:
        w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack(dt, w, rows, cols)
    return p, wv.upload(p), rng


@pytest.mark.parametrize("dt", NARROW)
@pytest.mark.parametrize("shape", [(6912, 2560), (2560, 6912), (300, 1024), (4500, 1024), (9001, 768), (4200, 8192),
                                   (1000, 14336), (300, 32768), (37, 100), (5, 4104)])
def test_narrow_int8_path_bit_exact(dt, shape):
    """(6912, 2560) and (2560, 6912) are BASELINE config 3's shapes; 4500 and
    9001 rows give each wave 4 rows (9001 leaves a ragged last block);
    4200 x 8192 holds 4 code vectors per lane and row for Int4 and 8 for
    Int8; 14336 and 32768 columns (the longest narrow row) take the kernel
    that walks each row's code vectors;
    37x100 and 5x4104 leave the vector kernel (rows not whole code vectors, or
    a row of Binary codes that is not 16-byte aligned) for the per-element one."""
    import torch
    rows, cols = shape
    print(f"[gpu] narrow {dt} {cols}->{rows}", flush=True)
    p, d, rng = native_blob(dt, rows, cols, rows + cols)
    assert d.info()["layout"] == "narrow"
    x = rng.standard_normal((2, cols)).astype(np.float32)
    x[1, :7] = [0.0, 5.0, -5.0, 2.5, -2.5, 1e-3, -0.0]  # ties of the act quantization around the absmax
    y_ref, acc_ref, as_ref = oracle.narrow_i8_forward(dt, p.raw, p.tensor_scale, rows, cols, x)
    tx = torch.from_numpy(x).cuda()
    acc = torch.zeros(2 * rows, dtype=torch.int32, device="cuda")
    act = torch.zeros(2, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    d.native_acc_dev(tx.data_ptr(), acc.data_ptr(), act.data_ptr(), 2)
    wv.sync()
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    assert np.array_equal(act.cpu().numpy(), as_ref)
    assert np.array_equal(d.matvec(x).reshape(-1), y_ref)
    d.free()


@pytest.mark.parametrize("dt", ["NativeInt4", "NativeTernary"])
@pytest.mark.parametrize("shape", [(2560, 6912), (37, 100)])
@pytest.mark.parametrize("mag", [1e-38, 1e-42])
def test_narrow_tiny_activations(dt, shape, mag):
    """max|x| below 127 * 2^-128 makes 1/act overflow (and 1e-42 is all
    subnormal): quantizeActsI8 still divides exactly, element by element."""
    rows, cols = shape
    p, d, rng = native_blob(dt, rows, cols, 7)
    x = (rng.standard_normal((1, cols)) * mag).astype(np.float32)
    y_ref, acc_ref, as_ref = oracle.narrow_i8_forward(dt, p.raw, p.tensor_scale, rows, cols, x)
    assert as_ref[0] != 1.0 and np.count_nonzero(x) > cols // 2
    assert np.array_equal(d.matvec(x).reshape(-1), y_ref)
    d.free()


def test_narrow_zero_activations():
    """quantizeActsI8 of an all-zero x: scale 1, every accumulator 0."""
    p, d, _ = native_blob("NativeInt4", 64, 256, 1)
    y = d.matvec(np.zeros(256, np.float32))
    assert np.array_equal(y, np.zeros(64, np.float32))
    d.free()


@pytest.mark.parametrize("shape", [(4096, 4096), (300, 1000), (7, 77)])
def test_f32_formatnone_forward(shape):
    rows, cols = shape
    print(f"[gpu] f32 {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    d = wv.upload(wv.pack("none", w, rows, cols))
    assert d.info()["layout"] == "f32"
    ref = x.astype(np.float64) @ w.reshape(rows, cols).astype(np.float64).T
    assert normwise(d.matvec(x), ref) <= TOL
    y = np.full(rows + 3, 7.0, np.float32)
    d.quant_matvec(np.concatenate([x[0], [1.0, 2.0]]).astype(np.float32), y)  # quant.MatVec FormatNone
    assert normwise(y[:rows], ref[0]) <= TOL and list(y[rows:]) == [7.0, 7.0, 7.0]
    d.free()


@pytest.mark.parametrize("fmt", ["none"] + NARROW)
def test_store_matvec_f64(fmt):
    """weights.Store.MatVec / MatVecT on a FormatNone store: f64 over the
    decoded weights (weightAt), y past rows zeroed, gx accumulated."""
    rows, cols = 300, 520
    print(f"[gpu] store f64 {fmt}", flush=True)
    rng = np.random.default_rng(31)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    d = wv.upload(p)
    wd = w if fmt == "none" else np_ref.native_decode(oracle.DTYPES[fmt], p.raw, p.tensor_scale, rows * cols)
    x = rng.standard_normal(cols + 2)
    y = np.full(rows + 4, 3.0)
    d.store_matvec(x, y)
    ref = dense_ref.store_matvec_f64(wd, rows, cols, x)
    assert normwise(y[:rows], ref) <= 1e-12 and list(y[rows:]) == [0.0] * 4
    gy = rng.standard_normal(rows)
    gy[::3] = 0.0
    gx = rng.standard_normal(cols)
    want = dense_ref.store_matvec_t_f64(wd, rows, cols, gy, gx)
    d.store_matvec_t(gy, gx)
    assert normwise(gx, want) <= 1e-12
    with pytest.raises(wv.WelvetError, match="weights: matvecF64 shape"):
        d.store_matvec(x[: cols - 1], y)
    with pytest.raises(wv.WelvetError, match="weights: matvecTF64 shape"):
        d.store_matvec_t(gy[: rows - 1], gx)
    d.free()


def test_store_matvec_packed_goes_through_f32():
    """Packed stores run quant.MatVec on f32(x) and widen y (weights/store.go:162-180)."""
    rows, cols = 256, 512
    rng = np.random.default_rng(4)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack("Q4_K", w, rows, cols)
    d = wv.upload(p)
    x = rng.standard_normal(cols)
    y = np.full(rows + 2, 5.0)
    d.store_matvec(x, y)
    yf = np.zeros(rows, np.float32)
    d.quant_matvec(x.astype(np.float32), yf)
    assert np.array_equal(y[:rows], yf.astype(np.float64)) and list(y[rows:]) == [0.0, 0.0]
    with pytest.raises(wv.WelvetError, match=r"MatVec: size mismatch rows=256 cols=512 len\(x\)=511 len\(y\)=258"):
        d.store_matvec(x[:511], y)
    d.free()


@pytest.mark.parametrize("fmt", ["none", "NativeInt4", "NativeTernary", "NativeBinary"])
def test_matvec_t_native_layouts(fmt):
    """gx += W^T gy over the decoded weights (BackwardSIMD's input gradient)."""
    rows, cols = 520, 1000
    rng = np.random.default_rng(8)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = wv.pack(fmt, w, rows, cols)
    d = wv.upload(p)
    wd = w if fmt == "none" else np_ref.native_decode(oracle.DTYPES[fmt], p.raw, p.tensor_scale, rows * cols)
    gy = rng.standard_normal((2, rows)).astype(np.float32)
    gx0 = rng.standard_normal((2, cols)).astype(np.float32)
    want = gx0 + gy.astype(np.float64) @ wd.reshape(rows, cols).astype(np.float64)
    assert normwise(d.matvec_t(gy, gx0), want) <= TOL
    d.free()
