"""C-ABI library checks that need no GPU: symbols, host packers, error paths."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
import welvet_amd as wv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKABLE = ["Q4_0", "Q8_0", "Q4_1", "Q5_0", "Q5_1", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K",
            "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S", "IQ4_NL", "IQ4_XS",
            "TernaryPacked", "BinaryPacked"]


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(wv_\w+)\s*\(", src, re.M))
    return names


def test_library_exports_every_declared_symbol():
    L = wv.lib()
    decl = declared_symbols()
    assert decl, "no declarations parsed"
    assert decl == set(wv.EXPORTS)
    for name in decl:
        assert hasattr(L, name), name
    assert b"gfx950" in L.wv_version()


@pytest.mark.parametrize("shape", [(16, 256), (5, 77), (64, 512), (3, 1000)])
@pytest.mark.parametrize("fmt", PACKABLE)
def test_host_packer_bit_exact_vs_oracle(fmt, shape):
    rows, cols = shape
    rng = np.random.default_rng(7 + rows)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    a = wv.pack(fmt, w, rows, cols)
    b = oracle.pack(fmt, w, rows, cols)
    assert np.array_equal(a.raw, b.raw)
    if b.scales is not None:
        assert np.array_equal(a.scales, b.scales)
    if b.meta is not None:
        assert np.array_equal(a.meta, b.meta)
    assert a.block_weights == b.block_weights


def test_host_packer_large_parallel_matches_oracle():
    # exercises the multi-threaded block split (> 4096 blocks)
    rng = np.random.default_rng(3)
    rows, cols = 512, 4096
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    for fmt in ("Q4_K", "Q6_K", "Q8_0", "Q4_0", "IQ4_NL"):
        assert np.array_equal(wv.pack(fmt, w, rows, cols).raw, oracle.pack(fmt, w, rows, cols).raw), fmt


def test_native_ternary_pack_matches_oracle():
    rng = np.random.default_rng(5)
    t = rng.choice([-1, 0, 1], size=2560 * 64, p=[0.335, 0.33, 0.335])
    s = np.abs(rng.standard_normal(4096) * 0.02).mean().astype(np.float32)
    w = (t * s).astype(np.float32)
    p = wv.pack_native_ternary(w, 64, 2560)
    codes, scale = oracle.pack_native_ternary(w)
    assert np.array_equal(p.raw, codes)
    assert np.float32(p.tensor_scale) == scale == np.float32(s)


def test_error_paths_without_device():
    with pytest.raises(wv.WelvetError) as e:
        wv.pack_sizes("Q4_K", 0, 256)
    assert e.value.code == -2
    with pytest.raises(wv.WelvetError) as e:
        wv.pack_sizes(0, 4, 64)  # FormatNone has no quant.Pack
    assert e.value.code == -3 and "not implemented" in str(e.value)
    short = wv.PackedBlob("Q4_K", 4, 256, np.zeros(10, np.uint8), block_weights=256)
    with pytest.raises(wv.WelvetError) as e:
        wv.upload(short)
    assert e.value.code == -2 and "raw short" in str(e.value)
    bad = wv.PackedBlob(99, 4, 256, np.zeros(1024, np.uint8))
    with pytest.raises(wv.WelvetError) as e:
        wv.upload(bad)
    assert e.value.code == -3
    with pytest.raises(wv.WelvetError) as e:
        wv.check(wv.lib().wv_blob_free(123456789))
    assert e.value.code == -7
    raw = np.zeros(144 * 4, np.uint8)
    h = ctypes.c_uint64()
    rc = wv.lib().wv_blob_upload_flags(8, 4, 256, 256, raw.ctypes.data, raw.size, None, 0, None, 0, None, 0,
                                       ctypes.c_float(0), 6, ctypes.byref(h))
    assert rc == -1 and "unknown flags 0x6" in wv.lib().wv_last_error().decode()


@pytest.mark.parametrize("shape", [(16, 256), (64, 512), (3, 64), (7, 1088)])
def test_host_packer_affine_bit_exact_vs_oracle(shape):
    rows, cols = shape
    rng = np.random.default_rng(11 + rows)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    a = wv.pack("AffinePacked", w, rows, cols)
    b = oracle.pack("AffinePacked", w, rows, cols)
    assert np.array_equal(a.raw, b.raw) and np.array_equal(a.scales, b.scales) and np.array_equal(a.mins, b.mins)
    assert list(a.meta) == [4] and a.block_weights == 64
    assert a.nbytes == rows * cols // 2 + 2 * 4 * (rows * cols // 64) + 1


def test_affine_pack_and_upload_errors():
    """PackAffine4 rejects cols % 64 != 0 (affine_pack.go:29-31); uploads need 4-bit
    codes and a bias per group (the fused path's cache checks, k_iq_simd.go:201-215)."""
    with pytest.raises(wv.WelvetError):
        wv.pack("AffinePacked", np.zeros(5 * 77, np.float32), 5, 77)
    rows, cols = 4, 128
    words = np.zeros(rows * cols // 2, np.uint8)
    scales = np.ones(rows * cols // 64, np.float32)
    p = wv.PackedBlob("AffinePacked", rows, cols, words, scales, np.array([3], np.uint8), 64, mins=scales)
    with pytest.raises(wv.WelvetError, match="bits=3"):
        wv.upload(p)
    p = wv.PackedBlob("AffinePacked", rows, cols, words, scales, np.array([4], np.uint8), 64)
    with pytest.raises(wv.WelvetError, match="mins"):
        wv.upload(p)


@pytest.mark.parametrize("dt", ["NativeInt8", "NativeInt4", "NativeInt2", "NativeTernary", "NativeBinary"])
def test_native_packers_match_oracle(dt):
    """The library's weights.Store packers (C++) against the C oracle's, byte for
    byte, on weights with exact ties and clamp edges mixed in."""
    rng = np.random.default_rng(11)
    n = 4096 * 3 + 5
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    amax = np.float32(0.05)
    w[:8] = [amax, -amax, 0, amax / 2, -amax / 2, amax * 0.25, -0.0, amax * 0.75]
    p = wv.pack_native(dt, w, 1, n)
    codes, scale = oracle.pack_native(dt, w)
    assert np.array_equal(p.raw, codes)
    assert np.float32(p.tensor_scale) == scale


def test_quant_contract_errors_without_device():
    """quant.MatVec / MatVecT and weights.Store entry points on an unknown
    handle fail with the reference's nil-blob wording before touching a device."""
    L = wv.lib()
    x = np.zeros(4, np.float32)
    rc = L.wv_quant_matvec(987654321, x.ctypes.data, 4, x.ctypes.data, 4)
    assert rc == -7 and L.wv_last_error().decode() == "MatVec: nil blob"
    rc = L.wv_quant_matvec_t(987654321, x.ctypes.data, 4, x.ctypes.data, 4)
    assert rc == -7 and L.wv_last_error().decode() == "MatVecT: nil blob"
    rc = L.wv_matvec_packed_blob(987654321, x.ctypes.data, 4, x.ctypes.data, 4)
    assert rc == -7 and L.wv_last_error().decode() == "dense: nil packed blob"
    xd = np.zeros(4, np.float64)
    assert L.wv_store_matvec(987654321, xd.ctypes.data, 4, xd.ctypes.data, 4) == -7
    assert L.wv_last_error().decode() == "weights: nil"
    assert L.wv_dense_forward(987654321, x.ctypes.data, x.ctypes.data, None, 1, None, -1) == -7
    with pytest.raises(wv.WelvetError) as e:
        wv.pack_native("Q4_K", np.zeros(8, np.float32), 1, 8)
    assert e.value.code != 0


def test_weight_budget_setting_needs_no_device():
    """wv_set_weight_budget / wv_weight_bytes only touch host state."""
    _, before = wv.weight_bytes()
    wv.set_weight_budget(12345)
    try:
        assert wv.weight_bytes()[1] == 12345
    finally:
        wv.set_weight_budget(before)
    assert wv.weight_bytes()[1] == before
