"""wv_matvec_dev_noalloc (no device allocation, a fixed per-GPU scratch array)
against wv_matvec_dev through the C ABI: two calls in a row on K-split
shapes, the second smaller, each bit-identical to the allocating entry point
(same kernels and launch plan) and within 1e-5 normwise of the f64 oracle."""
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
