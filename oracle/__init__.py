"""TEST INFRASTRUCTURE ONLY: ctypes access to the C oracle (oracle/oracle.c).

Importable from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg. The product package welvet_amd never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import np_ref  # noqa: F401  (re-export)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

FMT = dict(np_ref.FORMATS)
FMT_NAME = {v: k for k, v in FMT.items()}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_pack_sizes.argtypes = [ctypes.c_int, _I64, _I64, _P]
        L.or_pack.argtypes = [ctypes.c_int, _P, _I64, _I64, _P, _P, _P, _P]
        blob_args = [ctypes.c_int, _I64, _I64, ctypes.c_int32, _P, _I64, _P, _I64, _P, _I64, _P, _I64]
        L.or_unpack.argtypes = blob_args + [_P]
        L.or_matvec_scalar.argtypes = blob_args + [_P, _P]
        L.or_matvec_t_scalar.argtypes = blob_args + [_P, _P]
        L.or_gemv_f64.argtypes = [_P, _I64, _I64, _P, _P]
        L.or_gemv_f64.restype = None
        L.or_simd_prepare.argtypes = blob_args
        L.or_simd_prepare.restype = _P
        L.or_simd_free.argtypes = [_P]
        L.or_simd_free.restype = None
        L.or_simd_matvec.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_int]
        L.or_pack_native_ternary.argtypes = [_P, _I64, _P, _P]
        L.or_pack_native_ternary.restype = None
        L.or_pack_native.argtypes = [ctypes.c_int, _P, _I64, _P, _P]
        L.or_expand_narrow_i8.argtypes = [ctypes.c_int, _P, _I64, _P]
        L.or_narrow_i8_forward.argtypes = [ctypes.c_int, _P, ctypes.c_float, _I64, _I64, _P, _P, _P, _P, ctypes.c_int]
        L.or_native_decode.argtypes = [ctypes.c_int, _P, ctypes.c_float, _I64, _P]
        L.or_quantize_acts_i8.argtypes = [_P, _I64, _P]
        L.or_quantize_acts_i8.restype = ctypes.c_float
        L.or_ternary_i8_forward.argtypes = [_P, ctypes.c_float, _I64, _I64, _P, _P, _P, _P, ctypes.c_int]
        L.or_num_cpus.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


class Packed:
    """The quant.Blob fields (format.go:110-131) as numpy arrays."""

    def __init__(self, fmt, rows, cols, raw, scales, meta, block_weights, mins=None):
        self.fmt = fmt if isinstance(fmt, int) else FMT[fmt]
        self.rows, self.cols = int(rows), int(cols)
        self.raw = np.ascontiguousarray(raw, dtype=np.uint8)
        self.scales = None if scales is None or len(scales) == 0 else np.ascontiguousarray(scales, dtype=np.float32)
        self.mins = None if mins is None or len(mins) == 0 else np.ascontiguousarray(mins, dtype=np.float32)
        self.meta = None if meta is None or len(meta) == 0 else np.ascontiguousarray(meta, dtype=np.uint8)
        self.block_weights = int(block_weights)

    @property
    def name(self):
        return FMT_NAME[self.fmt]

    def args(self):
        return (self.fmt, self.rows, self.cols, self.block_weights,
                _ptr(self.raw), self.raw.size,
                _ptr(self.scales), 0 if self.scales is None else self.scales.size,
                _ptr(self.mins), 0 if self.mins is None else self.mins.size,
                _ptr(self.meta), 0 if self.meta is None else self.meta.size)


def pack(fmt, w, rows, cols) -> Packed:
    f = fmt if isinstance(fmt, int) else FMT[fmt]
    sz = np.zeros(5, np.int64)
    if lib().or_pack_sizes(f, rows, cols, sz.ctypes.data) != 0:
        raise ValueError(f"oracle: no packer for {fmt}")
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    raw = np.zeros(int(sz[0]), np.uint8)
    scales = np.zeros(int(sz[1]), np.float32)
    mins = np.zeros(int(sz[2]), np.float32)
    meta = np.zeros(int(sz[3]), np.uint8)
    rc = lib().or_pack(f, w.ctypes.data, rows, cols, raw.ctypes.data,
                       scales.ctypes.data if sz[1] else None, mins.ctypes.data if sz[2] else None,
                       meta.ctypes.data if sz[3] else None)
    if rc != 0:
        raise ValueError("oracle: pack failed")
    return Packed(f, rows, cols, raw, scales, meta, int(sz[4]), mins)


def unpack(p: Packed) -> np.ndarray:
    out = np.zeros(p.rows * p.cols, np.float32)
    if lib().or_unpack(*p.args(), out.ctypes.data) != 0:
        raise ValueError("oracle: unpack failed")
    return out


def matvec_scalar(p: Packed, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(p.rows, np.float32)
    if lib().or_matvec_scalar(*p.args(), x.ctypes.data, y.ctypes.data) != 0:
        raise ValueError("oracle: matvec failed")
    return y


def matvec_t_scalar(p: Packed, gy: np.ndarray, gx: np.ndarray | None = None) -> np.ndarray:
    gy = np.ascontiguousarray(gy, np.float32)
    gx = np.zeros(p.cols, np.float32) if gx is None else np.array(gx, np.float32, copy=True)
    if lib().or_matvec_t_scalar(*p.args(), gy.ctypes.data, gx.ctypes.data) != 0:
        raise ValueError("oracle: matvec_t failed")
    return gx


def gemv_f64(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """Textbook GEMV over a dequantized f32 matrix, accumulated in long double."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(rows, np.float64)
    lib().or_gemv_f64(w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data)
    return y


def reference_y(p: Packed, x: np.ndarray) -> np.ndarray:
    """f64 y = Unpack(W) @ x for each row of x (batch, cols) → (batch, rows)."""
    w = unpack(p).reshape(p.rows, p.cols).astype(np.float64)
    x2 = np.asarray(x, np.float64).reshape(-1, p.cols)
    return x2 @ w.T


class SimdPath:
    """The fused SIMD path (Ensure*SIMDCache + Dot*Row + row-sharded threads)."""

    def __init__(self, p: Packed):
        self._keep = p
        self.h = lib().or_simd_prepare(*p.args())
        if not self.h:
            raise ValueError("oracle: simd prepare failed")
        self.rows, self.cols = p.rows, p.cols

    def matvec(self, x: np.ndarray, nthreads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        batch = x.size // self.cols
        y = np.zeros(batch * self.rows, np.float32)
        lib().or_simd_matvec(self.h, x.ctypes.data, y.ctypes.data, batch, nthreads)
        return y.reshape(batch, self.rows) if batch > 1 else y

    def close(self):
        if self.h:
            lib().or_simd_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pack_native_ternary(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    codes = np.zeros((w.size + 3) // 4, np.uint8)
    scale = np.zeros(1, np.float32)
    lib().or_pack_native_ternary(w.ctypes.data, w.size, codes.ctypes.data, scale.ctypes.data)
    return codes, np.float32(scale[0])


def quantize_acts_i8(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    q = np.zeros(x.size, np.int8)
    s = lib().or_quantize_acts_i8(x.ctypes.data, x.size, q.ctypes.data)
    return q, np.float32(s)


def ternary_i8_forward(codes, scale, rows, cols, x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    batch = x.size // cols
    y = np.zeros(batch * rows, np.float32)
    acc = np.zeros(batch * rows, np.int32)
    asc = np.zeros(batch, np.float32)
    codes = np.ascontiguousarray(codes, np.uint8)
    lib().or_ternary_i8_forward(codes.ctypes.data, ctypes.c_float(scale), rows, cols, x.ctypes.data,
                                y.ctypes.data, acc.ctypes.data, asc.ctypes.data, batch)
    return y, acc, asc


# core.DType values of the narrow weights.Store DTypes (core/dtype.go:23-34).
DTYPES = {"NativeInt8": 9, "NativeInt4": 14, "NativeInt2": 17, "NativeTernary": 19, "NativeBinary": 20}


def _dt(dt) -> int:
    return DTYPES[dt] if isinstance(dt, str) else int(dt)


def pack_native(dt, w: np.ndarray):
    """weights.Store packNative of a narrow DType -> (codes, scale)."""
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    bits = {9: 8, 14: 4, 17: 2, 19: 2, 20: 1}[_dt(dt)]
    codes = np.zeros((w.size * bits + 7) // 8, np.uint8)
    scale = np.zeros(1, np.float32)
    if lib().or_pack_native(_dt(dt), w.ctypes.data, w.size, codes.ctypes.data, scale.ctypes.data) != bits:
        raise ValueError(f"oracle: no native pack for {dt}")
    return codes, np.float32(scale[0])


def expand_narrow_i8(dt, codes, n: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint8)
    out = np.zeros(n, np.int8)
    if lib().or_expand_narrow_i8(_dt(dt), codes.ctypes.data, n, out.ctypes.data):
        raise ValueError(f"oracle: no int8 expansion for {dt}")
    return out


def narrow_i8_forward(dt, codes, scale, rows, cols, x):
    """Dense's int8 path for a narrow DType -> (y, acc, act_scale)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    batch = x.size // cols
    y = np.zeros(batch * rows, np.float32)
    acc = np.zeros(batch * rows, np.int32)
    asc = np.zeros(batch, np.float32)
    codes = np.ascontiguousarray(codes, np.uint8)
    if lib().or_narrow_i8_forward(_dt(dt), codes.ctypes.data, ctypes.c_float(scale), rows, cols, x.ctypes.data,
                                  y.ctypes.data, acc.ctypes.data, asc.ctypes.data, batch):
        raise ValueError(f"oracle: no int8 path for {dt}")
    return y, acc, asc


def native_decode(dt, codes, scale, n: int) -> np.ndarray:
    """weightAt: the f32 weights a narrow-DType weights.Store decodes to."""
    codes = np.ascontiguousarray(codes, np.uint8)
    out = np.zeros(n, np.float32)
    if lib().or_native_decode(_dt(dt), codes.ctypes.data, ctypes.c_float(scale), n, out.ctypes.data):
        raise ValueError(f"oracle: no decode for {dt}")
    return out


def num_cpus() -> int:
    return int(lib().or_num_cpus())
