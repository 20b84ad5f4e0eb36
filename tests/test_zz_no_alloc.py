"""wv_matvec_dev_noalloc (no device allocation, a fixed per-GPU scratch array)
against wv_matvec_dev through the C ABI: calls in a row on K-split shapes,
each smaller than the last, and batches past 8 rows (the K-split forward
runs 8 rows per launch, so those launches reuse the array in stream order),
each bit-identical to the allocating entry point (same kernels and launch
plan) and within 1e-5 normwise of the f64 oracle. Also: a shape whose
partials exceed the array is refused before anything is enqueued, and a call
on a second stream while the first stream's call is still queued is refused
with WV_E_BUSY."""
import numpy as np
import pytest

import oracle
import welvet_amd as wv

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    print(f"[gpu] {__name__}: init device 0", flush=True)
    wv.init(0)
    yield


def normwise(y, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-300))


def run_pair(fmt, rows, cols, batch, seed):
    import torch
    rng = np.random.default_rng(seed)
    p = wv.pack(fmt, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32), rows, cols)
    d = wv.upload(p)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    tx = torch.from_numpy(x).cuda()
    y_alloc = torch.full((batch, rows), float("nan"), device="cuda")
    y_static = torch.full((batch, rows), float("nan"), device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    L = wv.lib()
    wv.check(L.wv_matvec_dev(d.handle, tx.data_ptr(), y_alloc.data_ptr(), batch, s.cuda_stream))
    wv.check(L.wv_matvec_dev_noalloc(d.handle, tx.data_ptr(), y_static.data_ptr(), batch, s.cuda_stream))
    s.synchronize()
    a, b = y_alloc.cpu().numpy(), y_static.cpu().numpy()
    ref = oracle.reference_y(oracle.Packed(p.fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins), x)
    d.free()
    return a, b, ref


def test_noalloc_matches_allocating_entry_point():
    # 512 x 16384 Q4_K splits K four ways; then a smaller 256 x 8192 Q4_K (split
    # two ways) and a small unsplit Q6_K reuse the same array.
    for fmt, rows, cols, batch in (("Q4_K", 512, 16384, 3), ("Q4_K", 256, 8192, 1), ("Q6_K", 64, 512, 2)):
        print(f"[gpu] no-alloc {fmt} {rows}x{cols} batch {batch}", flush=True)
        a, b, ref = run_pair(fmt, rows, cols, batch, rows + cols)
        assert np.array_equal(a, b), f"{fmt} {rows}x{cols}: no-alloc result differs from wv_matvec_dev"
        assert normwise(b, ref) <= 1e-5


@pytest.mark.parametrize("batch", [9, 17])
def test_noalloc_batches_past_one_split_launch(batch):
    # 9 rows run as launches of 8 + 1, 17 as 8 + 8 + 1, all through the same
    # partials in the array.
    print(f"[gpu] no-alloc Q4_K 512x16384 batch {batch}", flush=True)
    a, b, ref = run_pair("Q4_K", 512, 16384, batch, 77 + batch)
    assert np.array_equal(a, b)
    assert normwise(b, ref) <= 1e-5


def test_noalloc_rejects_partials_past_the_array():
    """8256 x 65536 Q4_K splits K 16 ways over 129 row groups: 8 batch rows
    need 8 * 16 * 8256 floats of partials, past the 2^20 the array holds; 7 rows
    fit. The blob is all zero bytes (d = dmin = 0), so the accepted call gives 0."""
    import torch
    rows, cols = 8256, 65536
    print(f"[gpu] no-alloc oversized Q4_K {rows}x{cols}", flush=True)
    raw = np.zeros(rows * (cols // 256) * 168, np.uint8)
    d = wv.upload(wv.PackedBlob("Q4_K", rows, cols, raw, block_weights=256))
    L = wv.lib()
    x = torch.ones((8, cols), device="cuda")
    y = torch.full((8, rows), float("nan"), device="cuda")
    torch.cuda.synchronize()
    rc = L.wv_matvec_dev_noalloc(d.handle, x.data_ptr(), y.data_ptr(), 8, None)
    assert rc == -2
    assert "needs 1056768 floats of scratch" in L.wv_last_error().decode()
    torch.cuda.synchronize()
    assert torch.isnan(y).all()
    wv.check(L.wv_matvec_dev_noalloc(d.handle, x.data_ptr(), y.data_ptr(), 7, None))
    torch.cuda.synchronize()
    assert (y[:7] == 0).all() and torch.isnan(y[7]).all()
    d.free()


def test_noalloc_refuses_a_second_stream_while_the_first_runs():
    import torch
    rows, cols = 512, 16384
    print("[gpu] no-alloc two streams", flush=True)
    rng = np.random.default_rng(5)
    p = wv.pack("Q4_K", (rng.standard_normal(rows * cols) * 0.02).astype(np.float32), rows, cols)
    d = wv.upload(p)
    L = wv.lib()
    x = torch.from_numpy(rng.standard_normal((1, cols)).astype(np.float32)).cuda()
    y_ref = torch.full((1, rows), float("nan"), device="cuda")
    y_a = torch.full((1, rows), float("nan"), device="cuda")
    y_b = torch.full((1, rows), float("nan"), device="cuda")
    m = torch.randn(8192, 8192, device="cuda")
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    wv.check(L.wv_matvec_dev(d.handle, x.data_ptr(), y_ref.data_ptr(), 1, sa.cuda_stream))
    with torch.cuda.stream(sa):
        for _ in range(4):  # tens of ms of work queued ahead of the no-alloc call
            torch.mm(m, m)
    wv.check(L.wv_matvec_dev_noalloc(d.handle, x.data_ptr(), y_a.data_ptr(), 1, sa.cuda_stream))
    rc = L.wv_matvec_dev_noalloc(d.handle, x.data_ptr(), y_b.data_ptr(), 1, sb.cuda_stream)
    assert rc == -8, rc
    assert "still running" in L.wv_last_error().decode()
    # the same stream is ordered, so a second call there is accepted
    wv.check(L.wv_matvec_dev_noalloc(d.handle, x.data_ptr(), y_a.data_ptr(), 1, sa.cuda_stream))
    sa.synchronize()
    wv.check(L.wv_matvec_dev_noalloc(d.handle, x.data_ptr(), y_b.data_ptr(), 1, sb.cuda_stream))
    sb.synchronize()
    assert torch.equal(y_a, y_ref) and torch.equal(y_b, y_ref)
    d.free()
