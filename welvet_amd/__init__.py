"""welvet_amd — Python plumbing over libwelvet_hip.so (the C ABI in include/welvet_hip.h).

The library is the MI355X (gfx950) backend of welvet's Dense MatVec path; this
module only loads it with ctypes and moves numpy / torch buffers across the
boundary, for the tests and the benchmark. Importing it fails loudly when the
built library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwelvet_hip.so")

# quant.Format numbering (quant/format.go:9-39; "none" = f32 weights) and the
# FormatNone weights.Store DTypes (1000 + core.DType, core/dtype.go:11-52).
FORMATS = {
    "none": 0, "Q8_0": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 4, "Q5_1": 5,
    "Q2_K": 6, "Q3_K": 7, "Q4_K": 8, "Q5_K": 9, "Q6_K": 10,
    "IQ1_S": 11, "IQ2_XXS": 12, "IQ2_XS": 13, "IQ3_XXS": 14, "IQ3_S": 15,
    "IQ4_NL": 16, "IQ4_XS": 17, "TernaryPacked": 18, "BinaryPacked": 19, "AffinePacked": 20,
    "NativeInt8": 1009, "NativeInt4": 1014, "NativeInt2": 1017, "NativeTernary": 1019, "NativeBinary": 1020,
}
NATIVE = ("NativeInt8", "NativeInt4", "NativeInt2", "NativeTernary", "NativeBinary")
NATIVE_BITS = {"NativeInt8": 8, "NativeInt4": 4, "NativeInt2": 2, "NativeTernary": 2, "NativeBinary": 1}
# core.ActivationType (core/layer.go:88-99)
ACT = {"linear": -1, "relu": 0, "silu": 1, "gelu": 2, "tanh": 3, "sigmoid": 4, "leaky_relu": 5, "relu2": 6}
FORMAT_NAMES = {v: k for k, v in FORMATS.items()}
LAYOUTS = {0: "raw", 1: "row-interleaved", 4: "narrow", 5: "f32"}

REFERENCE_LAYOUT = 1  # WV_UPLOAD_REFERENCE_LAYOUT
WV_E = {-1: "ARG", -2: "SHAPE", -3: "FORMAT", -4: "OOM", -5: "HIP", -6: "NODEV", -7: "HANDLE", -8: "BUSY"}

# Every symbol include/welvet_hip.h declares.
EXPORTS = (
    "wv_init", "wv_last_error", "wv_version", "wv_pack_sizes", "wv_pack",
    "wv_pack_native", "wv_blob_upload", "wv_blob_upload_flags", "wv_blob_upload_wire", "wv_blob_free", "wv_blob_info",
    "wv_set_weight_budget", "wv_weight_bytes",
    "wv_matvec", "wv_matvec_dev", "wv_matvec_dev_noalloc", "wv_quant_matvec", "wv_matvec_packed_blob", "wv_dense_forward", "wv_dense_forward_dev",
    "wv_dense_forward_block", "wv_dense_forward_block_dev",
    "wv_native_acc_dev", "wv_store_matvec", "wv_matvec_t", "wv_matvec_t_dev", "wv_quant_matvec_t",
    "wv_store_matvec_t", "wv_matmul", "wv_matmul_dev", "wv_sync",
    "wv_decoder_create", "wv_decoder_set_layer", "wv_decoder_set_output", "wv_decoder_set_kv",
    "wv_decoder_use_graph", "wv_decoder_generate", "wv_decoder_prefill", "wv_decoder_free",
)


class WelvetError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{WV_E.get(code, code)}: {msg}")
        self.code = code


_lib = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t


def lib():
    """The loaded library; raises if libwelvet_hip.so has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run `python -m welvet_amd.build` (no CPU fallback exists)")
    L = ctypes.CDLL(LIB_PATH)
    L.wv_init.argtypes = [ctypes.c_int]
    L.wv_last_error.restype = ctypes.c_char_p
    L.wv_version.restype = ctypes.c_char_p
    L.wv_pack_sizes.argtypes = [ctypes.c_int, _I64, _I64, _P, _P, _P, _P, _P]
    L.wv_pack.argtypes = [ctypes.c_int, _P, _I64, _I64, _P, _P, _P, _P]
    L.wv_pack_native.argtypes = [ctypes.c_int, _P, _I64, _P, _P]
    L.wv_blob_upload.argtypes = [ctypes.c_int, _I64, _I64, ctypes.c_int32, _P, _SZ, _P, _SZ, _P, _SZ, _P, _SZ,
                                 ctypes.c_float, _P]
    L.wv_blob_upload_flags.argtypes = [ctypes.c_int, _I64, _I64, ctypes.c_int32, _P, _SZ, _P, _SZ, _P, _SZ, _P, _SZ,
                                       ctypes.c_float, ctypes.c_uint32, _P]
    L.wv_blob_upload_wire.argtypes = [ctypes.c_int, _I64, _I64, _P, _SZ, _P]
    L.wv_blob_free.argtypes = [ctypes.c_uint64]
    L.wv_blob_info.argtypes = [ctypes.c_uint64, _P, _P, _P, _P, _P]
    L.wv_set_weight_budget.argtypes = [ctypes.c_uint64]
    L.wv_weight_bytes.argtypes = [_P, _P]
    L.wv_matvec.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32]
    L.wv_matvec_dev.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32, _P]
    L.wv_matvec_dev_noalloc.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32, _P]
    L.wv_native_acc_dev.argtypes = [ctypes.c_uint64, _P, _P, _P, ctypes.c_int32, _P]
    L.wv_quant_matvec.argtypes = [ctypes.c_uint64, _P, _SZ, _P, _SZ]
    L.wv_matvec_packed_blob.argtypes = [ctypes.c_uint64, _P, _SZ, _P, _SZ]
    L.wv_quant_matvec_t.argtypes = [ctypes.c_uint64, _P, _SZ, _P, _SZ]
    L.wv_dense_forward.argtypes = [ctypes.c_uint64, _P, _P, _P, ctypes.c_int32, _P, ctypes.c_int32]
    L.wv_dense_forward_dev.argtypes = [ctypes.c_uint64, _P, _P, _P, ctypes.c_int32, _P, ctypes.c_int32, _P]
    L.wv_dense_forward_block.argtypes = [ctypes.c_uint64, _P, _P, _P, ctypes.c_int32, _P, ctypes.c_int32]
    L.wv_dense_forward_block_dev.argtypes = [ctypes.c_uint64, _P, _P, _P, ctypes.c_int32, _P, ctypes.c_int32, _P]
    L.wv_store_matvec.argtypes = [ctypes.c_uint64, _P, _SZ, _P, _SZ]
    L.wv_store_matvec_t.argtypes = [ctypes.c_uint64, _P, _SZ, _P, _SZ]
    L.wv_matvec_t.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32]
    L.wv_matvec_t_dev.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32, _P]
    L.wv_matmul.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32]
    L.wv_matmul_dev.argtypes = [ctypes.c_uint64, _P, _P, ctypes.c_int32, _P]
    L.wv_sync.argtypes = [_P]
    L.wv_decoder_create.argtypes = [_P, _P]
    L.wv_decoder_set_layer.argtypes = [ctypes.c_uint64, ctypes.c_int32, _P, _P, _P]
    L.wv_decoder_set_output.argtypes = [ctypes.c_uint64, ctypes.c_uint64, _P, _P]
    L.wv_decoder_set_kv.argtypes = [ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, _P]
    L.wv_decoder_use_graph.argtypes = [ctypes.c_uint64, ctypes.c_int32]
    L.wv_decoder_generate.argtypes = [ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                      _P, _P]
    L.wv_decoder_prefill.argtypes = [ctypes.c_uint64, _P, ctypes.c_int32, ctypes.c_int32, _P, _P]
    L.wv_decoder_free.argtypes = [ctypes.c_uint64]
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        raise WelvetError(rc, lib().wv_last_error().decode())


def _fmt(fmt) -> int:
    return fmt if isinstance(fmt, int) else FORMATS[fmt]


def init(device: int = 0) -> None:
    check(lib().wv_init(device))


class PackedBlob:
    """Host-side quant.Blob fields (quant/format.go:110-131)."""

    def __init__(self, fmt, rows, cols, raw, scales=None, meta=None, block_weights=0, tensor_scale=0.0, mins=None):
        self.fmt = _fmt(fmt)
        self.rows, self.cols = int(rows), int(cols)
        self.raw = np.ascontiguousarray(raw, np.uint8)
        self.scales = None if scales is None or len(scales) == 0 else np.ascontiguousarray(scales, np.float32)
        self.mins = None if mins is None or len(mins) == 0 else np.ascontiguousarray(mins, np.float32)
        self.meta = None if meta is None or len(meta) == 0 else np.ascontiguousarray(meta, np.uint8)
        self.block_weights = int(block_weights)
        self.tensor_scale = float(tensor_scale)

    @property
    def name(self) -> str:
        return FORMAT_NAMES.get(self.fmt, str(self.fmt))

    @property
    def nbytes(self) -> int:
        """Packed bytes in the reference layout (Raw + Scales + Mins + Meta)."""
        return (self.raw.nbytes + (0 if self.scales is None else self.scales.nbytes)
                + (0 if self.mins is None else self.mins.nbytes) + (0 if self.meta is None else self.meta.nbytes))


def pack_sizes(fmt, rows: int, cols: int):
    raw, ns, nm, nmeta = _SZ(), _SZ(), _SZ(), _SZ()
    bw = ctypes.c_int32()
    check(lib().wv_pack_sizes(_fmt(fmt), rows, cols, ctypes.byref(raw), ctypes.byref(ns), ctypes.byref(nm),
                              ctypes.byref(nmeta), ctypes.byref(bw)))
    return raw.value, ns.value, nm.value, nmeta.value, bw.value


def pack(fmt, w: np.ndarray, rows: int, cols: int) -> PackedBlob:
    """quant.Pack (quant/pack.go:4) through the library's host packer; the
    WV_NATIVE_* DTypes through the weights.Store packers; "none" keeps f32."""
    if _fmt(fmt) in (FORMATS[n] for n in NATIVE):
        return pack_native(fmt, w, rows, cols)
    if _fmt(fmt) == 0:
        w = np.ascontiguousarray(w, np.float32).reshape(-1)[: rows * cols]
        return PackedBlob(0, rows, cols, w.view(np.uint8).copy())
    raw_n, ns, nmins, nmeta, bw = pack_sizes(fmt, rows, cols)
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    if w.size < rows * cols:
        raise WelvetError(-2, f"Pack: bad shape rows={rows} cols={cols} len={w.size}")
    raw = np.zeros(raw_n, np.uint8)
    scales = np.zeros(ns, np.float32) if ns else None
    mins = np.zeros(nmins, np.float32) if nmins else None
    meta = np.zeros(nmeta, np.uint8) if nmeta else None
    check(lib().wv_pack(_fmt(fmt), w.ctypes.data, rows, cols, raw.ctypes.data, _p(scales), _p(mins), _p(meta)))
    return PackedBlob(fmt, rows, cols, raw, scales, meta, bw, mins=mins)


def pack_native(fmt, w: np.ndarray, rows: int, cols: int) -> PackedBlob:
    """weights.Store pack of a narrow DType (weights/native.go:88-283): codes + Store.Scale."""
    f = _fmt(fmt)
    w = np.ascontiguousarray(w, np.float32).reshape(-1)[: rows * cols]
    codes = np.zeros((w.size * NATIVE_BITS.get(FORMAT_NAMES.get(f), 8) + 7) // 8, np.uint8)
    scale = ctypes.c_float()
    check(lib().wv_pack_native(f, w.ctypes.data, w.size, codes.ctypes.data, ctypes.byref(scale)))
    return PackedBlob(f, rows, cols, codes, None, None, 0, scale.value)


def pack_native_ternary(w: np.ndarray, rows: int, cols: int) -> PackedBlob:
    """weights.Store DTypeTernary pack (weights/native.go:249-269)."""
    return pack_native("NativeTernary", w, rows, cols)


def _p(a):
    return None if a is None else a.ctypes.data


class DeviceBlob:
    """A blob resident in HBM (wv_blob_upload); freed with free() or on GC."""

    def __init__(self, packed: PackedBlob, reference_layout: bool = False):
        h = ctypes.c_uint64()
        p = packed
        check(lib().wv_blob_upload_flags(p.fmt, p.rows, p.cols, p.block_weights, _p(p.raw), p.raw.size,
                                         _p(p.scales), 0 if p.scales is None else p.scales.size,
                                         _p(p.mins), 0 if p.mins is None else p.mins.size,
                                         _p(p.meta), 0 if p.meta is None else p.meta.size,
                                         ctypes.c_float(p.tensor_scale),
                                         REFERENCE_LAYOUT if reference_layout else 0, ctypes.byref(h)))
        self.handle = h.value
        self.fmt, self.rows, self.cols = p.fmt, p.rows, p.cols
        self.packed_bytes = p.nbytes

    @classmethod
    def from_wire(cls, fmt, rows: int, cols: int, wire) -> "DeviceBlob":
        """Uploads an ENTITY packed-blob wire (ns, nm, nr, scales, mins, raw) with
        wv_blob_upload_wire; `wire` is any buffer (bytes, numpy, a memoryview of
        an mmap), read in place."""
        buf = np.frombuffer(wire, np.uint8)
        h = ctypes.c_uint64()
        check(lib().wv_blob_upload_wire(_fmt(fmt), int(rows), int(cols), buf.ctypes.data if buf.size else None,
                                        buf.size, ctypes.byref(h)))
        self = cls.__new__(cls)
        self.handle = h.value
        self.fmt, self.rows, self.cols = _fmt(fmt), int(rows), int(cols)
        if buf.size >= 12:
            ns, nm, nr = (int(v) for v in buf[:12].view("<u4"))
            self.packed_bytes = nr + 4 * (ns + nm)
        else:
            self.packed_bytes = 0
        return self

    def info(self):
        fmt, layout = ctypes.c_int(), ctypes.c_int()
        rows, cols = ctypes.c_int64(), ctypes.c_int64()
        nb = _SZ()
        check(lib().wv_blob_info(self.handle, ctypes.byref(fmt), ctypes.byref(rows), ctypes.byref(cols),
                                 ctypes.byref(nb), ctypes.byref(layout)))
        return dict(format=FORMAT_NAMES.get(fmt.value, fmt.value), rows=rows.value, cols=cols.value,
                    device_bytes=nb.value, layout=LAYOUTS.get(layout.value, layout.value))

    def matvec(self, x: np.ndarray) -> np.ndarray:
        """Host path: y = W x for x of shape (cols,) or (batch, cols)."""
        x = np.ascontiguousarray(x, np.float32)
        batch = x.size // self.cols
        y = np.zeros((batch, self.rows), np.float32)
        check(lib().wv_matvec(self.handle, x.ctypes.data, y.ctypes.data, batch))
        return y.reshape(self.rows) if x.ndim == 1 else y

    def matvec_t(self, gy: np.ndarray, gx: np.ndarray | None = None) -> np.ndarray:
        """Host path: gx += W^T gy (gx starts at 0 when not given)."""
        gy = np.ascontiguousarray(gy, np.float32)
        batch = gy.size // self.rows
        out = np.zeros((batch, self.cols), np.float32) if gx is None else np.array(gx, np.float32, copy=True).reshape(batch, self.cols)
        check(lib().wv_matvec_t(self.handle, gy.ctypes.data, out.ctypes.data, batch))
        return out.reshape(self.cols) if gy.ndim == 1 else out

    def matmul(self, x: np.ndarray) -> np.ndarray:
        """Host path of the batched prefill: Y = X W^T for X of shape (M, cols)."""
        x = np.ascontiguousarray(x, np.float32)
        m = x.size // self.cols
        y = np.zeros((m, self.rows), np.float32)
        check(lib().wv_matmul(self.handle, x.ctypes.data, y.ctypes.data, m))
        return y

    def matmul_dev(self, x_ptr: int, y_ptr: int, m: int, stream: int | None = None) -> None:
        check(lib().wv_matmul_dev(self.handle, x_ptr, y_ptr, m, stream))

    def matvec_dev(self, x_ptr: int, y_ptr: int, batch: int = 1, stream: int | None = None) -> None:
        check(lib().wv_matvec_dev(self.handle, x_ptr, y_ptr, batch, stream))

    def matvec_t_dev(self, gy_ptr: int, gx_ptr: int, batch: int = 1, stream: int | None = None) -> None:
        check(lib().wv_matvec_t_dev(self.handle, gy_ptr, gx_ptr, batch, stream))

    def native_acc_dev(self, x_ptr: int, acc_ptr: int, act_ptr: int, batch: int = 1, stream: int | None = None) -> None:
        check(lib().wv_native_acc_dev(self.handle, x_ptr, acc_ptr, act_ptr, batch, stream))

    ternary_acc_dev = native_acc_dev

    def quant_matvec(self, x: np.ndarray, y: np.ndarray) -> None:
        """quant.MatVec(b, x, y) (quant/matvec.go:5): one vector, checkBlobYX, y[:rows] overwritten."""
        x = np.ascontiguousarray(x, np.float32)
        assert y.dtype == np.float32 and y.flags.c_contiguous
        check(lib().wv_quant_matvec(self.handle, x.ctypes.data if x.size else None, x.size,
                                    y.ctypes.data if y.size else None, y.size))

    def matvec_packed_blob(self, x: np.ndarray, y: np.ndarray) -> None:
        """dense.MatVecPackedBlob(b, x, y) (layers/dense/simd.go:570-614): one vector,
        y[:rows] overwritten; FormatNone blobs are rejected as the reference does."""
        x = np.ascontiguousarray(x, np.float32)
        assert y.dtype == np.float32 and y.flags.c_contiguous
        check(lib().wv_matvec_packed_blob(self.handle, x.ctypes.data if x.size else None, x.size,
                                          y.ctypes.data if y.size else None, y.size))

    def quant_matvec_t(self, gy: np.ndarray, gx: np.ndarray) -> None:
        """quant.MatVecT(b, gy, gx) (quant/matvec_t.go:5): gx[:cols] += W^T gy[:rows], checkBlobGYGX."""
        gy = np.ascontiguousarray(gy, np.float32)
        assert gx.dtype == np.float32 and gx.flags.c_contiguous
        check(lib().wv_quant_matvec_t(self.handle, gy.ctypes.data if gy.size else None, gy.size,
                                      gx.ctypes.data if gx.size else None, gx.size))

    def dense_forward(self, x: np.ndarray, bias: np.ndarray | None = None, act="linear", block=False):
        """dense.Forward (layers/dense/dense.go:100): (pre, post) with applyBiasAct (dense.go:145-167).
        block=True: a token block through the prefill GEMM (wv_dense_forward_block, 2e-3 tolerance)."""
        x = np.ascontiguousarray(x, np.float32)
        batch = x.size // self.cols
        pre = np.zeros((batch, self.rows), np.float32)
        post = np.zeros((batch, self.rows), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        a = ACT[act] if isinstance(act, str) else int(act)
        fn = lib().wv_dense_forward_block if block else lib().wv_dense_forward
        check(fn(self.handle, x.ctypes.data, pre.ctypes.data, post.ctypes.data, batch, _p(b), a))
        if x.ndim == 1:
            return pre.reshape(self.rows), post.reshape(self.rows)
        return pre, post

    def dense_forward_dev(self, x_ptr: int, pre_ptr: int, post_ptr: int | None, batch: int = 1,
                          bias_ptr: int | None = None, act=-1, stream: int | None = None) -> None:
        a = ACT[act] if isinstance(act, str) else int(act)
        check(lib().wv_dense_forward_dev(self.handle, x_ptr, pre_ptr, post_ptr, batch, bias_ptr, a, stream))

    def store_matvec(self, x: np.ndarray, y: np.ndarray) -> None:
        """weights.Store.MatVec with f64 x / y (weights/store.go:133-145)."""
        x = np.ascontiguousarray(x, np.float64)
        assert y.dtype == np.float64 and y.flags.c_contiguous
        check(lib().wv_store_matvec(self.handle, x.ctypes.data if x.size else None, x.size,
                                    y.ctypes.data if y.size else None, y.size))

    def store_matvec_t(self, gy: np.ndarray, gx: np.ndarray) -> None:
        """weights.Store.MatVecT with f64 gy / gx (weights/store.go:147-160): gx += W^T gy."""
        gy = np.ascontiguousarray(gy, np.float64)
        assert gx.dtype == np.float64 and gx.flags.c_contiguous
        check(lib().wv_store_matvec_t(self.handle, gy.ctypes.data if gy.size else None, gy.size,
                                      gx.ctypes.data if gx.size else None, gx.size))

    def free(self) -> None:
        if self.handle:
            check(lib().wv_blob_free(self.handle))
            self.handle = 0

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.wv_blob_free(self.handle)
                self.handle = 0
        except Exception:
            pass


def set_weight_budget(nbytes: int) -> None:
    """Cap the device bytes uploaded blobs may hold per GPU (0: no cap); an
    upload past it raises WelvetError OOM "weight VRAM budget full"."""
    check(lib().wv_set_weight_budget(int(nbytes)))


def weight_bytes():
    """(resident blob bytes on the current device, the cap or 0)."""
    r, b = ctypes.c_uint64(), ctypes.c_uint64()
    check(lib().wv_weight_bytes(ctypes.byref(r), ctypes.byref(b)))
    return r.value, b.value


def upload(packed: PackedBlob, reference_layout: bool = False) -> DeviceBlob:
    """wv_blob_upload; reference_layout=True keeps the reference's byte order on
    the device (WV_UPLOAD_REFERENCE_LAYOUT) instead of the row-interleaved layout."""
    return DeviceBlob(packed, reference_layout)


def sync(stream: int | None = None) -> None:
    check(lib().wv_sync(stream))
