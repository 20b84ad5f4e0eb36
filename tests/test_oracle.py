"""Pins the CPU oracle (oracle/oracle.c) — CPU only.

The reference tree holds no tests, golden vectors or fixtures for this path
(its suites live in the absent openfluke/w2a repo), so the oracle is pinned by:
  * grid-exact round trips: weights placed exactly on a format's quantization
    grid must come back bit-identical from Pack → Unpack, with the packed
    bytes written out by hand from the chosen codes (catches nibble / bit
    order, sign offsets, scale placement, min handling);
  * closed-form special cases the reference code fixes (all-zero blocks,
    clamp edges, the u8 scale 0 → d/255 fallback);
  * brute force on tiny inputs (scalar MatVec / MatVecT / the fused SIMD
    path against a textbook f64 GEMV over Unpack(W));
  * an independent vectorised numpy restatement (oracle/np_ref.py),
    bit-exact on random and ragged inputs for every format.
"""
import struct

import numpy as np
import pytest

import oracle
from oracle import np_ref

ALL = ["Q4_0", "Q8_0", "Q4_1", "Q5_0", "Q5_1", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K",
       "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S", "IQ4_NL", "IQ4_XS",
       "TernaryPacked", "BinaryPacked"]


def f32b(v):
    return list(struct.pack("<f", v))


def lsb_bits(codes, bits):
    out = bytearray((len(codes) * bits + 7) // 8)
    pos = 0
    for c in codes:
        for i in range(bits):
            if (c >> i) & 1:
                out[pos >> 3] |= 1 << (pos & 7)
            pos += 1
    return list(out)


# ---------------------------------------------------------------- numpy cross-check

@pytest.mark.parametrize("shape", [(8, 256), (7, 77), (3, 1000), (32, 512), (1, 33)])
@pytest.mark.parametrize("fmt", ALL)
def test_c_oracle_matches_numpy_restatement(fmt, shape):
    rows, cols = shape
    rng = np.random.default_rng(rows * 1000 + cols)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = oracle.pack(fmt, w, rows, cols)
    r = np_ref.pack(fmt, w, rows, cols)
    assert np.array_equal(p.raw, r["raw"])
    if r["scales"] is not None:
        assert np.array_equal(p.scales, r["scales"])
    wc = oracle.unpack(p)
    wn = np_ref.unpack(fmt, rows, cols, p.raw, p.scales, p.meta, p.block_weights)
    assert np.array_equal(wc, wn)


# ---------------------------------------------------------------- grid-exact round trips

def test_q4_0_grid_roundtrip_and_bytes():
    q = np.array([(j % 15) - 7 for j in range(32)])  # -7..7, contains ±7
    w = (q * 0.5).astype(np.float32)                  # maxAbs 3.5 → scale 0.5 exactly
    p = oracle.pack("Q4_0", w, 1, 32)
    want = f32b(0.5) + [((q[2 * j] & 15) | ((q[2 * j + 1] & 15) << 4)) for j in range(16)]
    assert list(p.raw) == want
    assert np.array_equal(oracle.unpack(p), w)


def test_q8_0_grid_roundtrip_and_bytes():
    q = np.array([127 - 8 * j for j in range(32)])
    q[5] = -127
    w = (q * 0.25).astype(np.float32)
    p = oracle.pack("Q8_0", w, 1, 32)
    assert list(p.raw) == f32b(0.25) + [int(v) & 255 for v in q]
    assert np.array_equal(oracle.unpack(p), w)


@pytest.mark.parametrize("fmt,qmax,off", [("Q4_1", 15, 8), ("Q5_1", 31, 8)])
def test_asym32_grid_roundtrip(fmt, qmax, off):
    q = np.array([(7 * j) % (qmax + 1) for j in range(32)])
    q[0], q[1] = 0, qmax
    w = (-1.0 + q * 0.125).astype(np.float32)
    p = oracle.pack(fmt, w, 1, 32)
    body = [int(q[2 * j] | (q[2 * j + 1] << 4)) for j in range(16)] if qmax == 15 else lsb_bits(list(q), 5)
    assert list(p.raw) == f32b(0.125) + f32b(-1.0) + body
    assert np.array_equal(oracle.unpack(p), w)


def test_q5_0_grid_roundtrip():
    q = np.array([(j % 31) - 15 for j in range(32)])  # -15..15
    w = (q * 0.5).astype(np.float32)                   # maxAbs 7.5 → scale 0.5
    p = oracle.pack("Q5_0", w, 1, 32)
    assert list(p.raw) == f32b(0.5) + lsb_bits([int(v) + 16 for v in q], 5)
    assert np.array_equal(oracle.unpack(p), w)


@pytest.mark.parametrize("fmt,bits,qmax", [("Q2_K", 2, 3), ("Q3_K", 3, 7), ("Q4_K", 4, 15), ("Q5_K", 5, 31)])
def test_kquant_asym_grid_roundtrip_and_bytes(fmt, bits, qmax):
    # every group: min -1, step 1/8 (a power of two), both code ends present →
    # d = 1/8 and every u8 scale 255; dmin = 1 and every int8 min -127.
    rng = np.random.default_rng(bits)
    q = rng.integers(0, qmax + 1, size=512)
    q[0::16], q[1::16] = 0, qmax
    w = (-1.0 + q * 0.125).astype(np.float32)
    p = oracle.pack(fmt, w, 2, 256)
    for sb in range(2):
        want = f32b(0.125) + f32b(1.0) + [255] * 16 + [0x81] * 16 + lsb_bits(list(q[sb * 256:(sb + 1) * 256]), bits)
        sbb = len(want)
        assert list(p.raw[sb * sbb:(sb + 1) * sbb]) == want
    assert np.array_equal(oracle.unpack(p), w)


def test_q6_k_grid_roundtrip_and_bytes():
    rng = np.random.default_rng(6)
    q = rng.integers(1, 64, size=256)       # q in [1,63] → w = (q-32)*2^-4
    q[0::16] = 0                             # q = 0 is -32: amax = 32*step exactly
    w = ((q - 32) * 0.0625).astype(np.float32)
    p = oracle.pack("Q6_K", w, 1, 256)
    want = f32b(0.0625) + f32b(0.0) + [255] * 16 + lsb_bits(list(q), 6)
    assert list(p.raw) == want
    assert np.array_equal(oracle.unpack(p), w)


@pytest.mark.parametrize("fmt,bits,sg,mid", [("IQ2_XXS", 2, 32, 1.5), ("IQ2_XS", 2, 16, 1.5),
                                              ("IQ3_XXS", 3, 32, 3.5), ("IQ3_S", 3, 16, 3.5), ("IQ4_XS", 4, 16, 7.5)])
def test_iq_linear_grid_roundtrip(fmt, bits, sg, mid):
    qmax = (1 << bits) - 1
    q = np.array([(5 * j) % (qmax + 1) for j in range(64)])
    q[0::sg] = 0  # |0 - mid| = mid is the largest magnitude → amax = mid*step
    q[1::sg] = qmax
    w = ((q - mid) * 0.25).astype(np.float32)
    p = oracle.pack(fmt, w, 2, 32)
    assert list(p.raw) == lsb_bits(list(q), bits)
    assert np.array_equal(p.scales, np.full(64 // sg, 0.25, np.float32))
    assert list(p.meta) == [bits, sg]
    assert np.array_equal(oracle.unpack(p), w)


def test_iq4_nl_and_iq1_roundtrip():
    c = np.array([(3 * j) % 16 for j in range(32)])
    c[0] = 15
    w = (0.5 * np_ref.IQ4NL_GRID[c]).astype(np.float32)
    p = oracle.pack("IQ4_NL", w, 1, 32)
    assert list(p.raw) == lsb_bits(list(c), 4)
    assert np.array_equal(oracle.unpack(p), w)
    s = np.where(np.arange(32) % 3 == 0, -0.5, 0.5).astype(np.float32)
    p1 = oracle.pack("IQ1_S", s, 1, 32)
    assert list(p1.raw) == lsb_bits([int(v >= 0) for v in s], 1)
    assert np.array_equal(oracle.unpack(p1), s)


def test_ternary_binary_grid_roundtrip():
    t = np.where(np.arange(64) % 2 == 0, 1.0, -1.0) * 0.25
    w = t.astype(np.float32)
    p = oracle.pack("TernaryPacked", w, 1, 64)
    codes = [2 if v > 0 else 0 for v in w]
    words = [sum(codes[g * 16 + j] << (2 * j) for j in range(16)) for g in range(4)]
    assert list(p.raw) == list(struct.pack("<4I", *words))
    assert np.array_equal(oracle.unpack(p), w)
    pb = oracle.pack("BinaryPacked", w, 1, 64)
    assert np.array_equal(oracle.unpack(pb), w)


# ---------------------------------------------------------------- special cases

def test_all_zero_blocks():
    z = np.zeros(256, np.float32)
    p = oracle.pack("Q4_0", z, 1, 32)
    assert list(p.raw) == f32b(1.0) + [0] * 16                 # q4_0.go:25-27
    p = oracle.pack("Q5_0", z, 1, 32)
    assert list(p.raw) == f32b(1.0) + lsb_bits([16] * 32, 5)   # q5_0.go:33-35, code q+16
    p = oracle.pack("Q4_K", z, 1, 256)                         # kquant.go:96-98, 139-144
    assert list(p.raw) == f32b(1.0) + f32b(1.0) + [255] * 16 + [0] * 16 + [0] * 128
    p = oracle.pack("Q6_K", z, 1, 256)
    assert list(p.raw) == f32b(1.0) + f32b(0.0) + [255] * 16 + lsb_bits([32] * 256, 6)
    # Zero is off the grid of the half-integer-mid IQ formats: scale 1 and
    # q = round(0 + mid) (half away) decode to +0.5; sign-only formats map 0 to +scale.
    off_grid = {"IQ2_XXS": 0.5, "IQ2_XS": 0.5, "IQ3_XXS": 0.5, "IQ3_S": 0.5, "IQ4_XS": 0.5,
                "IQ1_S": 1.0, "BinaryPacked": 1.0}
    for fmt in ALL:
        assert np.all(oracle.unpack(oracle.pack(fmt, z, 1, 256)) == off_grid.get(fmt, 0.0)), fmt


def test_clamp_edges():
    w = np.zeros(32, np.float32)
    w[0], w[1] = -0.7, 0.7
    p = oracle.pack("Q4_0", w, 1, 32)  # -maxAbs maps to -7, never -8
    assert p.raw[4] == ((-7 & 15) | (7 << 4))
    w = np.zeros(256, np.float32)
    w[0], w[1] = 0.32, -0.32           # Q6_K: +amax → 64 → clamped to 63; -amax → 0
    p = oracle.pack("Q6_K", w, 1, 256)
    codes = p.raw[24:24 + 192]
    assert codes[0] & 63 == 63
    assert (codes[0] >> 6 | (codes[1] & 15) << 2) == 0


def test_k_scale_zero_falls_back_to_d_over_255():
    # group 1 spans 1e-4 while group 0 spans 15 → d = 1, group 1's u8 scale
    # rounds to 0 and decodes with d/255 (kquant.go:179-182) instead of 0, so
    # its 16 codes 0..15 decode to a ramp of 15 steps of 1/255.
    w = np.zeros(256, np.float32)
    w[:16] = np.linspace(0, 15, 16)
    w[16:32] = np.linspace(0, 1e-4, 16)
    p = oracle.pack("Q4_K", w, 1, 256)
    assert struct.unpack("<f", bytes(p.raw[:4]))[0] == 1.0
    assert p.raw[9] == 0
    g1 = oracle.unpack(p)[16:32].astype(np.float64)
    assert np.isclose(g1.max() - g1.min(), 15 / 255, rtol=1e-6)


def test_round_half_away_from_zero():
    x = np.array([127.0, -127.0, 63.5, -0.5, 0.5, 2.5, -2.5, 0.0], np.float32)
    q, s = oracle.quantize_acts_i8(x)
    assert s == 1.0
    assert list(q) == [127, -127, 64, -1, 1, 3, -3, 0]
    q, s = oracle.quantize_acts_i8(np.zeros(8, np.float32))
    assert s == 1.0 and not q.any()


# ---------------------------------------------------------------- brute force

@pytest.mark.parametrize("fmt", ALL)
def test_scalar_and_simd_matvec_vs_f64(fmt):
    rng = np.random.default_rng(11)
    rows, cols = 67, 512
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    p = oracle.pack(fmt, w, rows, cols)
    ref = oracle.reference_y(p, x)[0]
    wd = oracle.unpack(p).reshape(rows, cols)
    brute = np.array([sum(float(a) * float(b) for a, b in zip(wd[r], x)) for r in range(3)])
    assert np.allclose(ref[:3], brute, rtol=0, atol=1e-12)
    scale = np.abs(ref).max()
    y_scalar = oracle.matvec_scalar(p, x)
    assert np.abs(y_scalar - ref).max() / scale < 1e-5
    simd = oracle.SimdPath(p)
    y1 = simd.matvec(x, nthreads=1)
    y4 = simd.matvec(x, nthreads=4)
    assert np.array_equal(y1, y4)
    assert np.abs(y1 - ref).max() / scale < 1e-6


@pytest.mark.parametrize("fmt", ["Q4_0", "Q4_K", "Q6_K", "IQ3_S", "TernaryPacked"])
def test_scalar_matvec_t_vs_f64(fmt):
    rng = np.random.default_rng(12)
    rows, cols = 40, 96
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    gy = rng.standard_normal(rows).astype(np.float32)
    gx0 = rng.standard_normal(cols).astype(np.float32)
    p = oracle.pack(fmt, w, rows, cols)
    wd = oracle.unpack(p).reshape(rows, cols).astype(np.float64)
    want = gx0 + wd.T @ gy
    got = oracle.matvec_t_scalar(p, gy, gx0)  # accumulates, does not zero
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


def test_native_ternary_pack_and_int8_path():
    rng = np.random.default_rng(13)
    rows, cols = 48, 160
    t = rng.choice([-1, 0, 1], size=rows * cols, p=[0.335, 0.33, 0.335])
    s = np.float32(0.0137)
    w = (t * s).astype(np.float32)
    codes, scale = oracle.pack_native_ternary(w)
    assert scale == s
    nc, ns = np_ref.pack_native_ternary(w)
    assert np.array_equal(codes, nc) and ns == scale
    x = rng.standard_normal(cols).astype(np.float32)
    y, acc, asc = oracle.ternary_i8_forward(codes, scale, rows, cols, x)
    xq, xs = np_ref.quantize_acts_i8(x)
    assert asc[0] == xs
    brute = t.reshape(rows, cols).astype(np.int64) @ xq.astype(np.int64)
    assert np.array_equal(acc, brute.astype(np.int32))
    assert np.array_equal(y, (acc.astype(np.float32) * xs).astype(np.float32) * scale)


# ---------------------------------------------------------------- AffinePacked (quant/affine_*.go)

@pytest.mark.parametrize("shape", [(8, 256), (3, 64), (5, 576)])
def test_affine_c_oracle_matches_numpy_restatement(shape):
    rows, cols = shape
    rng = np.random.default_rng(rows * 7 + cols)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    p = oracle.pack("AffinePacked", w, rows, cols)
    r = np_ref.pack("AffinePacked", w, rows, cols)
    assert np.array_equal(p.raw, r["raw"])
    assert np.array_equal(p.scales, r["scales"]) and np.array_equal(p.mins, r["mins"])
    assert list(p.meta) == [4] and p.block_weights == 64
    wc = oracle.unpack(p)
    wn = np_ref.unpack("AffinePacked", rows, cols, p.raw, p.scales, p.meta, p.block_weights, p.mins)
    assert np.array_equal(wc, wn)


def test_affine_grid_roundtrip_and_bytes():
    """A group on the grid min + k*s (min -0.5, s 1/16, k = 0..15 each used) packs to codes k
    (nibble j of little-endian word = element j), scale 1/16, min -0.5, and decodes exactly."""
    k = np.array([(5 * j + 3) % 16 for j in range(64)], np.int64)
    k[:2] = (0, 15)  # min and max present
    w = (np.float32(-0.5) + k.astype(np.float32) * np.float32(0.0625)).astype(np.float32)
    p = oracle.pack("AffinePacked", w, 1, 64)
    assert p.scales.tolist() == [0.0625] and p.mins.tolist() == [-0.5]
    want = bytes((int(k[2 * b]) | (int(k[2 * b + 1]) << 4)) for b in range(32))
    assert bytes(p.raw) == want
    assert np.array_equal(oracle.unpack(p), w)


def test_affine_special_groups():
    """affine_pack.go:49-56: a group with max == min gets s = 1 and min = 0, so
    the codes are round-half-away(v) clamped to [0, 15]; ties round away."""
    zero = np.zeros(64, np.float32)
    half = np.full(64, 0.5, np.float32)
    big = np.full(64, 20.0, np.float32)
    ties = np.zeros(64, np.float32)
    ties[1] = 15.0  # s = 1, min = 0
    ties[2:6] = (2.5, 3.5, 0.5, 14.5)
    w = np.concatenate([zero, half, big, ties])
    p = oracle.pack("AffinePacked", w, 1, 256)
    assert p.scales.tolist() == [1.0, 1.0, 1.0, 1.0] and p.mins.tolist() == [0.0, 0.0, 0.0, 0.0]
    codes = np.stack([p.raw & 15, p.raw >> 4], axis=1).reshape(-1)
    assert not codes[:64].any()
    assert (codes[64:128] == 1).all()  # 0.5 -> 1 (half away), decodes to 1.0
    assert (codes[128:192] == 15).all()  # clamp
    assert codes[192:198].tolist() == [0, 15, 3, 4, 1, 15]
    assert oracle.unpack(p)[64] == 1.0


def test_affine_matvec_closed_form_and_f64():
    """Groups on exact binary grids (s = 1/16, min -0.5; s = 1/8, min 0.25) and
    x = 1: every product and sum is exact, so y is the plain sum of the weights
    (s*sum(code) + beta*64 per group); random blobs: scalar MatVec and the
    fused SIMD path against the f64 GEMV."""
    rows, cols = 3, 128
    rng = np.random.default_rng(20)
    w = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        k1, k2 = rng.integers(0, 16, 64), rng.integers(0, 16, 64)
        k1[:2], k2[:2] = (0, 15), (15, 0)
        w[r, :64] = -0.5 + k1 * 0.0625
        w[r, 64:] = 0.25 + k2 * 0.125
    p = oracle.pack("AffinePacked", w.reshape(-1), rows, cols)
    assert p.scales.tolist() == [0.0625, 0.125] * rows and p.mins.tolist() == [-0.5, 0.25] * rows
    x = np.ones(cols, np.float32)
    want = w.astype(np.float64).sum(axis=1)
    assert np.array_equal(oracle.matvec_scalar(p, x).astype(np.float64), want)
    assert np.array_equal(oracle.SimdPath(p).matvec(x, nthreads=1).astype(np.float64).reshape(-1), want)
    rng = np.random.default_rng(21)
    rows, cols = 67, 512
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    p = oracle.pack("AffinePacked", w, rows, cols)
    ref = oracle.reference_y(p, x)[0]
    scale = np.abs(ref).max()
    assert np.abs(oracle.matvec_scalar(p, x) - ref).max() / scale < 1e-5
    simd = oracle.SimdPath(p)
    y1 = simd.matvec(x, nthreads=1)
    assert np.array_equal(y1, simd.matvec(x, nthreads=4))
    assert np.abs(y1 - ref).max() / scale < 1e-6


def test_affine_matvec_t_skips_zero_rows():
    """matVecTAffine (affine_g64.go:269-286) accumulates into gx and skips rows whose gy is 0."""
    rng = np.random.default_rng(22)
    rows, cols = 9, 192
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    gy = rng.standard_normal(rows).astype(np.float32)
    gy[[1, 4]] = 0
    gx0 = rng.standard_normal(cols).astype(np.float32)
    p = oracle.pack("AffinePacked", w, rows, cols)
    wd = oracle.unpack(p).reshape(rows, cols).astype(np.float64)
    got = oracle.matvec_t_scalar(p, gy, gx0)
    want = gx0 + wd.T @ gy
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5
    neg = np.full(cols, -0.0, np.float32)  # a skipped row leaves -0.0 untouched
    gz = np.zeros(rows, np.float32)
    assert np.signbit(oracle.matvec_t_scalar(p, gz, neg)).all()


# ---- narrow weights.Store DTypes, Dense's bias/activation epilogue, Store f64 products ----

from oracle import dense_ref  # noqa: E402

NARROW = {"NativeInt8": 9, "NativeInt4": 14, "NativeInt2": 17, "NativeTernary": 19, "NativeBinary": 20}


def test_native_pack_known_answers():
    """Hand-computed packs (weights/native.go): Int4 scale = absMax/7, half-away
    ties and clamps; Int2 clamps to [-2, 1]; Binary sign bit (0 -> +1)."""
    w = np.array([0.7, -0.7, 0.05, -0.15, 0.35, 0.0, -0.0, 0.1], np.float32)
    codes, scale = oracle.pack_native("NativeInt4", w)
    assert scale == np.float32(np.float32(0.7) / np.float32(7))
    # q = round(w/s): 7, -7, 0.5 -> 1 (half away), -1.5 -> -2, 3.5 -> 4, 0, 0, 1
    q = [7, -7, 1, -2, 4, 0, 0, 1]
    assert list(codes) == [(q[0] & 15) | ((q[1] & 15) << 4), (q[2] & 15) | ((q[3] & 15) << 4),
                           (q[4] & 15) | ((q[5] & 15) << 4), (q[6] & 15) | ((q[7] & 15) << 4)]
    codes, scale = oracle.pack_native("NativeInt2", np.array([1.0, -1.0, 0.4, -0.6], np.float32))
    # scale = absMax, so q = round(w/s) is 1, -1, 0, -1 (-2 is never reached) -> codes q + 2
    assert scale == 1.0 and codes[0] == (3 | (1 << 2) | (2 << 4) | (1 << 6))
    codes, scale = oracle.pack_native("NativeBinary", np.array([0.5, -0.25, 0.0, -0.0, 1, -1, 2, -2, 3], np.float32))
    assert scale == 3.0 and list(codes) == [0b01011101, 0b1]  # -0.0 >= 0 holds: bit set
    codes, scale = oracle.pack_native("NativeInt8", np.array([127.0, -127.0, 0.5, -63.5], np.float32))
    assert scale == 1.0 and list(codes.view(np.int8)) == [127, -127, 1, -64]
    codes, scale = oracle.pack_native("NativeTernary", np.zeros(5, np.float32))
    assert scale == 1.0 and list(codes) == [0b01010101, 0b01]  # all-zero tensor: scale 1, codes "0"


@pytest.mark.parametrize("dt", sorted(NARROW))
def test_native_oracle_two_restatements(dt):
    """C oracle vs the numpy restatement: packs, int8 expansion and decode."""
    rng = np.random.default_rng(NARROW[dt])
    n = 1237
    w = (rng.standard_normal(n) * 0.03).astype(np.float32)
    codes, scale = oracle.pack_native(dt, w)
    nc, ns = np_ref.pack_native(NARROW[dt], w)
    assert np.array_equal(codes, nc) and scale == ns
    assert np.array_equal(oracle.expand_narrow_i8(dt, codes, n), np_ref.expand_narrow_i8(NARROW[dt], codes, n))
    assert np.array_equal(oracle.native_decode(dt, codes, scale, n), np_ref.native_decode(NARROW[dt], codes, scale, n))


def test_native_expand_closed_forms():
    """Every code of every DType maps as expandNarrowToI8 / weightAt state,
    including Ternary code 3 (+2 on the int8 path, 0 when decoded)."""
    allc = np.array([0b11100100], np.uint8)  # 2-bit codes 0, 1, 2, 3
    assert list(oracle.expand_narrow_i8("NativeTernary", allc, 4)) == [-1, 0, 1, 2]
    assert list(oracle.expand_narrow_i8("NativeInt2", allc, 4)) == [-2, -1, 0, 1]
    assert list(oracle.native_decode("NativeTernary", allc, 0.5, 4)) == [-0.5, 0, 0.5, 0]
    nib = np.array([0x87, 0xF0], np.uint8)  # nibbles 7, 8, 0, 15
    assert list(oracle.expand_narrow_i8("NativeInt4", nib, 4)) == [7, -8, 0, -1]
    assert list(oracle.expand_narrow_i8("NativeBinary", np.array([0b10100101], np.uint8), 8)) == [1, -1, 1, -1, -1, 1, -1, 1]
    assert list(oracle.expand_narrow_i8("NativeInt8", np.array([0x80, 0x7F, 0xFF], np.uint8), 3)) == [-128, 127, -1]
    assert list(oracle.native_decode("NativeInt4", nib, 0, 4)) == [7, -8, 0, -1]  # scale 0 reads as 1


@pytest.mark.parametrize("dt", sorted(NARROW))
def test_narrow_forward_brute_force(dt):
    """The C oracle's int8 path equals an exact int64 brute force over the numpy
    expansion and quantization (int32 accumulators bit for bit, y as f32)."""
    rng = np.random.default_rng(3 + NARROW[dt])
    rows, cols = 23, 200
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    codes, scale = oracle.pack_native(dt, w)
    y, acc, asc = oracle.narrow_i8_forward(dt, codes, scale, rows, cols, x)
    y2, acc2, asc2 = np_ref.narrow_i8_forward(NARROW[dt], codes, scale, rows, cols, x)
    assert np.array_equal(acc, acc2) and np.array_equal(asc, asc2) and np.array_equal(y, y2)


def test_activation_closed_forms():
    """core.Activate (core/activate.go:6-37) at points with known values."""
    x = np.array([-2.0, 0.0, 3.0])
    assert list(dense_ref.activate(x, "relu")) == [0.0, 0.0, 3.0]
    assert list(dense_ref.activate(x, "relu2")) == [0.0, 0.0, 9.0]
    assert list(dense_ref.activate(x, "leaky_relu")) == [-0.02, 0.0, 3.0]
    assert list(dense_ref.activate(x, "linear")) == [-2.0, 0.0, 3.0]
    assert dense_ref.activate(np.array([0.0]), "sigmoid")[0] == 0.5
    assert dense_ref.activate(np.array([0.0]), "tanh")[0] == 0.0
    assert dense_ref.activate(np.array([0.0]), "silu")[0] == 0.0
    # silu(x) = x * sigmoid(x); sigmoid(ln 3) = 3/4
    assert abs(dense_ref.activate(np.array([np.log(3.0)]), "silu")[0] - 0.75 * np.log(3.0)) < 1e-15
    # GELU tanh form at 1: 0.5 * (1 + tanh(sqrt(2/pi) * 1.044715))
    g = 0.5 * (1 + np.tanh(np.sqrt(2 / np.pi) * 1.044715))
    assert abs(dense_ref.activate(np.array([1.0]), "gelu")[0] - g) < 1e-15
    assert abs(g - 0.8411919906082768) < 1e-15


def test_apply_bias_act_rules():
    """applyBiasAct (layers/dense/dense.go:145-167): the bias is added in f64 and
    rounded into pre; without a bias pre stays; post = act(f32 pre); linear with
    no bias copies pre; a bias shorter than the row leaves the tail unbiased."""
    pre = np.array([[1.0, -2.0, 0.5]], np.float32)
    p, q = dense_ref.apply_bias_act(pre, None, "linear")
    assert np.array_equal(p, pre) and np.array_equal(q, pre)
    p, q = dense_ref.apply_bias_act(pre, np.array([0.25, 1.0]), "relu")
    assert list(p[0]) == [1.25, -1.0, 0.5] and list(q[0]) == [1.25, 0.0, 0.5]
    b = np.array([1e-9, 0, 0])  # below f32 resolution at 1.0: pre unchanged after rounding
    p, _ = dense_ref.apply_bias_act(pre, b, "linear")
    assert p[0, 0] == np.float32(1.0)
    p, q = dense_ref.apply_bias_act(pre, None, "sigmoid")
    assert np.array_equal(p, pre) and q[0, 0] == np.float32(1 / (1 + np.exp(-1.0)))


def test_store_f64_closed_forms():
    """matVecNativeF64 / matVecTNativeF64 on matrices whose products are exact."""
    w = np.array([1, 2, 3, 4, 5, 6], np.float32)  # 2 x 3
    y = dense_ref.store_matvec_f64(w, 2, 3, np.array([1.0, 0.5, 0.25, 99.0]))  # x longer than cols
    assert list(y) == [1 + 1 + 0.75, 4 + 2.5 + 1.5]
    gx = dense_ref.store_matvec_t_f64(w, 2, 3, np.array([1.0, 0.0]), np.array([0.5, 0.5, 0.5]))
    assert list(gx) == [1.5, 2.5, 3.5]
    wi = np.array([np.inf, 1, 1, 1, 1, 1], np.float32)  # a zero gy row is skipped, so inf never meets 0
    assert np.isfinite(dense_ref.store_matvec_t_f64(wi, 2, 3, np.array([0.0, 1.0]), np.zeros(3))).all()
