"""GPU parity through the C ABI: libwelvet_hip on an MI355X vs the CPU oracle.

Tolerances: f32 outputs within 1e-5 normwise relative
error of the f64 textbook GEMV over the reference's dequantized weights
(max|y_gpu - y_ref| / max|y_ref|); DTypeTernary int32 accumulators bit-exact.
"""

import numpy as np
import pytest

import oracle
import welvet_amd as wv

pytestmark = pytest.mark.gpu

TOL = 1e-5
ALL = ["Q4_0", "Q8_0", "Q4_1", "Q5_0", "Q5_1", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K",
       "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S", "IQ4_NL", "IQ4_XS",
       "TernaryPacked", "BinaryPacked"]
PLANAR = {f: "row-interleaved" for f in ("Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q4_1", "Q5_0", "Q5_1",
                                          "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S", "IQ4_XS", "IQ4_NL",
                                          "TernaryPacked", "BinaryPacked", "AffinePacked")}


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(rows * cols) * 0.02).astype(np.float32), rng


def upload(fmt, w, rows, cols, force_raw=False):
    p = wv.pack(fmt, w, rows, cols)
    return p, wv.upload(p, reference_layout=force_raw)


def oracle_packed(p):
    return oracle.Packed(p.fmt, p.rows, p.cols, p.raw, p.scales, p.meta, p.block_weights, p.mins)


@pytest.mark.parametrize("fmt", ALL)
@pytest.mark.parametrize("shape", [(96, 512), (7, 77), (33, 1000)])
def test_matvec_small(fmt, shape):
    rows, cols = shape
    print(f"[gpu] matvec {fmt} {rows}x{cols}", flush=True)
    w, rng = weights(rows, cols, 100 + rows)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    p, d = upload(fmt, w, rows, cols)
    ref = oracle.reference_y(oracle_packed(p), x)
    y = d.matvec(x)
    assert normwise(y, ref) <= TOL
    y1 = d.matvec(x[1])
    assert normwise(y1, ref[1]) <= TOL
    d.free()


@pytest.mark.parametrize("fmt", sorted(PLANAR))
def test_planar_and_raw_layouts_agree(fmt):
    rows, cols = 300, 2048
    print(f"[gpu] layouts {fmt}", flush=True)
    w, rng = weights(rows, cols, 5)
    x = rng.standard_normal(cols).astype(np.float32)
    p, dp = upload(fmt, w, rows, cols)
    _, dr = upload(fmt, w, rows, cols, force_raw=True)
    assert dp.info()["layout"] == PLANAR[fmt]
    assert dr.info()["layout"] == "raw"
    # same bytes as the reference blob, for rows padded to the 64-row group (+ section alignment),
    # plus (row-interleaved) the prefill GEMM's f32 row factor per padded row
    padded_rows = -(-rows // 64) * 64
    assert p.nbytes <= dp.info()["device_bytes"] <= p.nbytes * padded_rows // rows + 4 * padded_rows + 5 * 256
    ref = oracle.reference_y(oracle_packed(p), x)[0]
    assert normwise(dp.matvec(x), ref) <= TOL
    assert normwise(dr.matvec(x), ref) <= TOL


@pytest.mark.parametrize("fmt", ["Q4_K", "Q8_0", "Q6_K", "Q5_K", "Q3_K", "Q2_K", "Q4_1", "Q5_0", "Q5_1"])
@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_baseline_shapes(fmt, shape):
    rows, cols = shape
    print(f"[gpu] baseline {fmt} {cols}->{rows}", flush=True)
    w, rng = weights(rows, cols, 42)
    x = rng.standard_normal(cols).astype(np.float32)
    p, d = upload(fmt, w, rows, cols)
    ref = oracle.reference_y(oracle_packed(p), x)[0]
    assert normwise(d.matvec(x), ref) <= TOL
    d.free()


@pytest.mark.parametrize("fmt", sorted(PLANAR))
@pytest.mark.parametrize("shape,batch", [((1000, 2048), 11), ((130, 4096), 2), ((64, 256), 1)])
def test_row_interleaved_split_and_batch(fmt, shape, batch):
    """K split across blocks (partials added by a second launch), batch beyond one split launch."""
    rows, cols = shape
    print(f"[gpu] rpl split {fmt} {cols}->{rows} batch {batch}", flush=True)
    w, rng = weights(rows, cols, 17)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    p, d = upload(fmt, w, rows, cols)
    assert d.info()["layout"] == "row-interleaved"
    ref = oracle.reference_y(oracle_packed(p), x)
    for _ in range(2):  # the blob's split scratch is reused by the next launch
        assert normwise(d.matvec(x), ref) <= TOL


# Shapes that select each launch plan of the row-interleaved forward kernel:
# lanes per row L (1, 2, 4) with one or two super-blocks per wave S for
# K <= 4096; for wider matrices L = S = 4 with no K split when those blocks
# fill the GPU in one pass, else a K split across blocks.
PLAN_SHAPES = [
    ((12800, 1024), ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0"]),  # L=1 S=1
    ((8192, 1024), ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q4_1", "Q5_1", "IQ1_S", "IQ3_S"]),   # L=2 S=1
    ((1000, 2048), ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q4_1", "Q5_0", "Q5_1"]),   # L=4 S=2
    ((8192, 8192), ["Q4_K", "Q8_0"]),                           # L=4 S=4, 8-wave blocks, no split
    ((3000, 13312), ["Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q5_0"]),  # L=4 S=4, 13 waves, padded last row group
    ((3000, 13312), ["Q4_1", "Q5_1", "IQ2_XS", "IQ3_S", "IQ4_XS"]),  # two metadata words per chunk: at most 2 super-blocks per wave, K split
    ((3000, 13312), ["IQ1_S", "IQ2_XXS", "IQ3_XXS"]),  # L=4 S=4
    ((4096, 11008), ["Q4_K", "Q5_K", "Q6_K"]),                  # L=4 S=4, 43 super-blocks: last wave has 3
    ((2048, 16640), ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0"]),  # K split 5 over 13-wave blocks
    ((6400, 16640), ["Q4_K"]),                          # K split 2, 65 super-blocks
]


@pytest.mark.parametrize("shape,fmt", [(sh, f) for sh, fs in PLAN_SHAPES for f in fs])
def test_row_interleaved_plans(shape, fmt):
    rows, cols = shape
    print(f"[gpu] rpl plan {fmt} {cols}->{rows}", flush=True)
    w, rng = weights(rows, cols, 3)
    batch = 10 if rows * cols <= 40_000_000 else 2  # > 8 batch rows: two launches when K is split
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    p, d = upload(fmt, w, rows, cols)
    assert d.info()["layout"] == "row-interleaved"
    ref = oracle.reference_y(oracle_packed(p), x)
    for _ in range(2):
        assert normwise(d.matvec(x), ref) <= TOL
    d.free()


def test_q4_0_baseline_4096():
    w, rng = weights(4096, 4096, 1)
    x = rng.standard_normal(4096).astype(np.float32)
    p, d = upload("Q4_0", w, 4096, 4096)
    ref = oracle.reference_y(oracle_packed(p), x)[0]
    assert normwise(d.matvec(x), ref) <= TOL


def ternary_weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    t = rng.choice([-1, 0, 1], size=rows * cols, p=[0.335, 0.33, 0.335]).astype(np.int8)
    s = np.float32(np.abs(rng.standard_normal(1 << 16) * 0.02).astype(np.float32).mean())
    return t, s, (t * s).astype(np.float32), rng


@pytest.mark.parametrize("shape", [(6912, 2560), (2560, 6912), (37, 100), (64, 64)])
def test_native_ternary_bit_exact(shape):
    import torch
    rows, cols = shape
    print(f"[gpu] native ternary {cols}->{rows}", flush=True)
    t, s, w, rng = ternary_weights(rows, cols, rows)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    p = wv.pack_native_ternary(w, rows, cols)
    d = wv.upload(p)
    assert d.info()["layout"] == "narrow"
    y_ref, acc_ref, as_ref = oracle.ternary_i8_forward(p.raw, np.float32(p.tensor_scale), rows, cols, x)
    tx = torch.from_numpy(x).cuda()
    acc = torch.zeros(2 * rows, dtype=torch.int32, device="cuda")
    act = torch.zeros(2, dtype=torch.float32, device="cuda")
    y = torch.zeros(2 * rows, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()  # the library's stream does not wait for torch's
    d.native_acc_dev(tx.data_ptr(), acc.data_ptr(), act.data_ptr(), 2)
    d.matvec_dev(tx.data_ptr(), y.data_ptr(), 2)
    wv.sync()
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    assert np.array_equal(act.cpu().numpy(), as_ref)
    assert np.array_equal(y.cpu().numpy(), y_ref)
    assert np.array_equal(d.matvec(x).reshape(-1), y_ref)


@pytest.mark.parametrize("fmt", ALL + ["AffinePacked"])
@pytest.mark.parametrize("shape,batch", [((300, 512), 2), ((100, 1280), 1), ((33, 1000), 2), ((520, 2304), 3)])
def test_matvec_t_accumulates(fmt, shape, batch):
    """gx += W^T gy on the reference layout. cols % 256 == 0 takes the run kernel:
    300x512 in 4 row slices + reduce, 100x1280 in one slice added directly (two
    column tiles, the second partly past the row), 520x2304 in 8 slices over 3
    tiles with batch 3; 33x1000 takes the per-weight kernel."""
    rows, cols = shape
    if fmt == "AffinePacked" and cols % 64:
        pytest.skip("AffinePacked packs whole 64-groups per row")
    print(f"[gpu] matvec_t {fmt} {rows}x{cols} batch {batch}", flush=True)
    w, rng = weights(rows, cols, 9 + rows)
    gy = rng.standard_normal((batch, rows)).astype(np.float32)
    gx0 = rng.standard_normal((batch, cols)).astype(np.float32)
    p, d = upload(fmt, w, rows, cols, force_raw=True)
    assert d.info()["layout"] == "raw"
    wd = oracle.unpack(oracle_packed(p)).reshape(rows, cols).astype(np.float64)
    want = gx0 + gy.astype(np.float64) @ wd
    for _ in range(2):
        assert normwise(d.matvec_t(gy, gx0), want) <= TOL
    d.free()


@pytest.mark.parametrize("fmt", sorted(PLANAR))
@pytest.mark.parametrize("shape,batch", [((64, 512), 2), ((300, 2048), 2), ((1000, 2048), 3), ((130, 256), 1), ((300, 1024), 18)])
def test_matvec_t_row_interleaved(fmt, shape, batch):
    """gx += W^T gy on the resident row-interleaved layout: one slice (direct) and sliced + reduce."""
    rows, cols = shape
    print(f"[gpu] matvec_t rpl {fmt} {rows}x{cols} batch {batch}", flush=True)
    w, rng = weights(rows, cols, 23 + rows)
    gy = rng.standard_normal((batch, rows)).astype(np.float32)
    gx0 = rng.standard_normal((batch, cols)).astype(np.float32)
    p, d = upload(fmt, w, rows, cols)
    assert d.info()["layout"] == "row-interleaved"
    wd = oracle.unpack(oracle_packed(p)).reshape(rows, cols).astype(np.float64)
    want = gx0 + gy.astype(np.float64) @ wd
    for _ in range(2):
        assert normwise(d.matvec_t(gy, gx0), want) <= TOL
    d.free()


@pytest.mark.parametrize("fmt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_matvec_t_row_interleaved_baseline(fmt):
    import torch
    rows, cols = 14336, 4096
    print(f"[gpu] matvec_t rpl baseline {fmt} {rows}x{cols}", flush=True)
    w, rng = weights(rows, cols, 31)
    gy = rng.standard_normal(rows).astype(np.float32)
    p, d = upload(fmt, w, rows, cols)
    wd = oracle.unpack(oracle_packed(p)).reshape(rows, cols)
    want = gy.astype(np.float64) @ wd.astype(np.float64)
    del wd
    tg = torch.from_numpy(gy).cuda()
    tx = torch.zeros(cols, device="cuda")
    torch.cuda.synchronize()  # the library's stream does not wait for torch's
    d.matvec_t_dev(tg.data_ptr(), tx.data_ptr(), 1)
    wv.sync()
    assert normwise(tx.cpu().numpy(), want) <= TOL
    d.free()


def test_device_pointer_path_on_torch_stream():
    import torch
    rows, cols = 1024, 4096
    w, rng = weights(rows, cols, 77)
    x = rng.standard_normal(cols).astype(np.float32)
    p, d = upload("Q4_K", w, rows, cols)
    s = torch.cuda.Stream()
    tx = torch.from_numpy(x).cuda()
    ty = torch.empty(rows, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        d.matvec_dev(tx.data_ptr(), ty.data_ptr(), 1, s.cuda_stream)
    s.synchronize()
    ref = oracle.reference_y(oracle_packed(p), x)[0]
    assert normwise(ty.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("rows,cols", [(70, 512), (130, 2048)])
def test_ternary_code3_and_missing_scales(rows, cols):
    """TernaryPacked words holding code 3 (which decodes as 0, ternary.go:53-62)
    and fewer scales than groups (missing ones read as 1, ternary.go:69-72),
    on the row-interleaved layout and the reference one."""
    rng = np.random.default_rng(rows)
    words = rng.integers(0, 2**32, size=rows * cols // 16, dtype=np.uint64).astype(np.uint32)
    scales = (np.abs(rng.standard_normal(rows * cols // 16 - 37)) * 0.02 + 1e-3).astype(np.float32)
    p = wv.PackedBlob("TernaryPacked", rows, cols, words.view(np.uint8), scales, None, 16)
    x = rng.standard_normal(cols).astype(np.float32)
    op = oracle.Packed(p.fmt, rows, cols, p.raw, scales, None, 16)
    ref = oracle.reference_y(op, x)[0]
    for force_raw in (False, True):
        d = wv.upload(p, reference_layout=force_raw)
        assert d.info()["layout"] == ("raw" if force_raw else "row-interleaved")
        assert normwise(d.matvec(x), ref) <= TOL
        d.free()


def test_binary_g128_layout():
    rows, cols = 64, 512
    rng = np.random.default_rng(128)
    words = rng.integers(0, 2**32, size=rows * cols // 32, dtype=np.uint64).astype(np.uint32)
    scales = (np.abs(rng.standard_normal(rows * cols // 128)) * 0.02 + 1e-3).astype(np.float32)
    p = wv.PackedBlob("BinaryPacked", rows, cols, words.view(np.uint8), scales, None, 128)
    d = wv.upload(p)
    x = rng.standard_normal(cols).astype(np.float32)
    op = oracle.Packed(p.fmt, rows, cols, p.raw, scales, None, 128)
    ref = oracle.reference_y(op, x)[0]
    assert normwise(d.matvec(x), ref) <= TOL
    assert normwise(oracle.matvec_scalar(op, x), ref) <= TOL


# ---------------------------------------------------------------- AffinePacked (quant/affine_*.go)

@pytest.mark.parametrize("shape", [(96, 512), (33, 320), (16, 4096), (3, 64)])
def test_affine_matvec(shape):
    """Packed by PackAffine4 (group 64): the run-vectorised kernel when cols % 256 == 0, else the per-weight one."""
    rows, cols = shape
    print(f"[gpu] affine matvec {rows}x{cols}", flush=True)
    w, rng = weights(rows, cols, 300 + rows)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    p, d = upload("AffinePacked", w, rows, cols)
    ref = oracle.reference_y(oracle_packed(p), x)
    assert normwise(d.matvec(x), ref) <= TOL
    assert normwise(d.matvec(x[1]), ref[1]) <= TOL
    d.free()


@pytest.mark.parametrize("group,cols", [(32, 512), (128, 1024), (8, 256)])
def test_affine_mlx_groups(group, cols):
    """BlobFromMLXAffine4-style blobs (affine_g64.go:22-78) with other group widths: random
    4-bit words, per-group scales and biases; group 8 takes the per-weight kernel."""
    rows = 40
    print(f"[gpu] affine group {group} cols {cols}", flush=True)
    rng = np.random.default_rng(group)
    words = rng.integers(0, 2**32, size=rows * cols // 8, dtype=np.uint64).astype(np.uint32)
    ng = rows * cols // group
    scales = (np.abs(rng.standard_normal(ng)) * 0.01 + 1e-3).astype(np.float32)
    mins = (rng.standard_normal(ng) * 0.05).astype(np.float32)
    p = wv.PackedBlob("AffinePacked", rows, cols, words.view(np.uint8), scales, np.array([4], np.uint8), group,
                      mins=mins)
    d = wv.upload(p)
    x = rng.standard_normal(cols).astype(np.float32)
    op = oracle_packed(p)
    ref = oracle.reference_y(op, x)[0]
    assert normwise(d.matvec(x), ref) <= TOL
    assert normwise(oracle.matvec_scalar(op, x), ref) <= TOL
    gy = rng.standard_normal(rows).astype(np.float32)
    gx0 = rng.standard_normal(cols).astype(np.float32)
    wd = oracle.unpack(op).reshape(rows, cols).astype(np.float64)
    assert normwise(d.matvec_t(gy, gx0), gx0 + gy.astype(np.float64) @ wd) <= TOL
    d.free()


def test_affine_matvec_t_accumulates():
    rows, cols = 300, 512
    print("[gpu] affine matvec_t", flush=True)
    w, rng = weights(rows, cols, 19)
    gy = rng.standard_normal((2, rows)).astype(np.float32)
    gy[0, 5] = 0.0  # matVecTAffine skips such rows; with finite weights the sum is the same
    gx0 = rng.standard_normal((2, cols)).astype(np.float32)
    p, d = upload("AffinePacked", w, rows, cols)
    wd = oracle.unpack(oracle_packed(p)).reshape(rows, cols).astype(np.float64)
    want = gx0 + gy.astype(np.float64) @ wd
    assert normwise(d.matvec_t(gy, gx0), want) <= TOL
    assert normwise(oracle.matvec_t_scalar(oracle_packed(p), gy[0], gx0[0]), want[0]) <= TOL
    d.free()


@pytest.mark.parametrize("fmt", ["Q4_K", "Q6_K", "Q8_0", "Q4_0", "Q5_K", "IQ4_NL", "Q4_1"])
@pytest.mark.parametrize("shape", [(300, 2048), (130, 8192)])
def test_nonfinite_x_propagates(fmt, shape):
    """A NaN in x makes every output NaN, as in the reference's float
    accumulation (w * NaN is NaN for every w). An infinite x leaves no output
    finite (the reference gives +-inf, or NaN where w = 0 or infinities cancel).
    The int-x Q4_K path relies on its float group sums for this: the
    fixed-point x planes alone would drop the non-finite value. 130x8192
    splits K over blocks."""
    rows, cols = shape
    print(f"[gpu] nonfinite x {fmt} {cols}->{rows}", flush=True)
    w, rng = weights(rows, cols, 77)
    p, d = upload(fmt, w, rows, cols)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    x[0, cols // 3] = np.nan
    x[1, cols - 5] = np.inf
    y = d.matvec(x)
    assert np.isnan(y[0]).all()
    assert not np.isfinite(y[1]).any()
    ref = oracle.reference_y(oracle_packed(p), x[2:])[0]
    assert normwise(y[2], ref) <= TOL  # the finite batch row is unaffected
    d.free()


@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336)])
def test_q4k_outlier_activations(shape):
    """x ~ N(0, 1) with 8 channels at +-1e3 and 4 at +-1e5 (LLM-style
    outliers) through the row-interleaved Q4_K kernel, whose x planes are 24-bit
    fixed point with one exponent per 32-column chunk. Bars: the 1e-5
    normwise one, and per row the kernel's error model, |y - y_ref| <=
    sum_k |w_k| * 2^-23 * max|x| over k's chunk (the fixed-point step) +
    2^-20 * sum_k |w_k x_k| (f32 accumulation), with every row's error
    printed relative to that row's sum_k |w_k x_k|."""
    rows, cols = shape
    print(f"[gpu] outliers Q4_K {cols}->{rows}", flush=True)
    w, rng = weights(rows, cols, 77)
    x = rng.standard_normal(cols).astype(np.float32)
    cs = rng.choice(cols, 12, replace=False)
    x[cs[:8]] = rng.choice([-1.0, 1.0], 8) * 1e3
    x[cs[8:]] = rng.choice([-1.0, 1.0], 4) * 1e5
    p, d = upload("Q4_K", w, rows, cols)
    assert d.info()["layout"] == "row-interleaved"
    op = oracle_packed(p)
    ref = oracle.reference_y(op, x)[0]
    y = d.matvec(x).astype(np.float64)
    assert normwise(y, ref) <= TOL
    wa = np.abs(oracle.unpack(op).reshape(rows, cols).astype(np.float64))
    cmax = np.repeat(np.abs(x.astype(np.float64)).reshape(-1, 32).max(axis=1), 32)
    scale = wa @ np.abs(x.astype(np.float64))
    bound = wa @ (cmax * 2.0 ** -23) + 2.0 ** -20 * scale
    err = np.abs(y - ref)
    rel = err / scale
    print(f"[gpu]   err/sum|w x|: max {rel.max():.2e} median {np.median(rel):.2e}; "
          f"err/bound max {(err / bound).max():.3f}", flush=True)
    assert (err <= bound).all()
    d.free()


def shared_scale_blob(kind, rows, cols, seed):
    """AffinePacked with 32/128/256-column groups (BlobFromMLXAffine4-style:
    random 4-bit words, per-group scale and bias) or BinaryPacked g128 (random
    sign words, one scale per 128 weights)."""
    rng = np.random.default_rng(seed)
    if kind == "binary128":
        words = rng.integers(0, 2**32, size=rows * cols // 32, dtype=np.uint64).astype(np.uint32)
        scales = (np.abs(rng.standard_normal(rows * cols // 128)) * 0.02 + 1e-3).astype(np.float32)
        return wv.PackedBlob("BinaryPacked", rows, cols, words.view(np.uint8), scales, None, 128), rng
    group = int(kind[len("affine"):])
    words = rng.integers(0, 2**32, size=rows * cols // 8, dtype=np.uint64).astype(np.uint32)
    ng = rows * cols // group
    scales = (np.abs(rng.standard_normal(ng)) * 0.01 + 1e-3).astype(np.float32)
    mins = (rng.standard_normal(ng) * 0.05).astype(np.float32)
    return wv.PackedBlob("AffinePacked", rows, cols, words.view(np.uint8), scales, np.array([4], np.uint8), group,
                         mins=mins), rng


def upload_blob(p, force_raw):
    return wv.upload(p, reference_layout=force_raw)


@pytest.mark.parametrize("kind", ["affine32", "affine128", "affine256", "binary128"])
@pytest.mark.parametrize("shape,batch", [((300, 2048), 3), ((130, 8192), 2), ((64, 256), 1), ((1000, 4096), 11)])
def test_shared_scale_groups_row_interleaved(kind, shape, batch):
    """AffinePacked groups of 32, 128 and 256 columns and BinaryPacked g128 on
    the row-interleaved layout (one scale, and min, per 2^GSH chunks): the
    forward (batch rows, K split at 130x8192, batch 11 past the split's 8),
    MatVecT, the reference layout's result, and the prefill GEMM at M = 40."""
    rows, cols = shape
    print(f"[gpu] shared-scale {kind} {cols}->{rows} batch {batch}", flush=True)
    p, rng = shared_scale_blob(kind, rows, cols, rows + batch)
    op = oracle_packed(p)
    d = upload_blob(p, False)
    assert d.info()["layout"] == "row-interleaved"
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    ref = oracle.reference_y(op, x)
    y = d.matvec(x)
    assert normwise(y, ref) <= TOL
    dr_ = upload_blob(p, True)
    assert dr_.info()["layout"] == "raw"
    assert normwise(dr_.matvec(x), ref) <= TOL
    dr_.free()
    wd = oracle.unpack(op).reshape(rows, cols).astype(np.float64)
    gy = rng.standard_normal((2, rows)).astype(np.float32)
    gx0 = rng.standard_normal((2, cols)).astype(np.float32)
    assert normwise(d.matvec_t(gy, gx0), gx0 + gy.astype(np.float64) @ wd) <= TOL
    xm = rng.standard_normal((40, cols)).astype(np.float32)
    assert normwise(d.matmul(xm), xm.astype(np.float64) @ wd.T) <= 2e-3
    d.free()
