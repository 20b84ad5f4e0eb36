"""ENTITY checkpoints on the device path (model/entity/*.go, model/transformer/load*.go).

File layout (model/entity/doc.go:15-22, file.go:145-185, write.go:45-80):
  b"ENTITY\\0\\0" | u16 format_version (1) | u16 flags | u64 header_len |
  header JSON {format_version, engine, status, transformer{...}, blobs[...]} |
  payload, each blob at `offset` bytes from the payload start, `length` long.
A blob with format "none" holds numbers (dtype FLOAT32 / FLOAT64 / FLOAT16 /
BFLOAT16, file.go:296-320). A packed blob (dtype "PACKED", format "Q4_K", ...)
holds the EncodePackedBlob wire (model/entity/packed.go:11-35):
u32 ns | u32 nm | u32 nr | f32 scales[ns] | f32 mins[nm] | raw[nr].

EntityFile maps the file read-only and passes each packed wire to
wv_blob_upload_wire where it lies in the mapping: no host decode and no
Int8QS / F32 cache inflation (the reference's DecodePackedBlob + Ensure*SIMDCache),
one host-to-device copy per blob. decoder_from_entity builds the device decode
step from a dense transformer checkpoint as model/transformer/load.go:19-240 does.
"""
from __future__ import annotations

import json
import mmap
import struct
from dataclasses import dataclass

import numpy as np

from . import FORMATS, DeviceBlob, PackedBlob

MAGIC = b"ENTITY\x00\x00"
FORMAT_VERSION = 1
FIXED_HEADER = 20
HEADER_MAX = 256 << 20
DEFAULT_MAX_SEQ = 2048  # fusedgpu/limits.go:19
HOST_MAX_SEQ_CAP = 8192  # fusedgpu/limits.go:22


class EntityError(ValueError):
    pass


@dataclass
class WeightBlob:
    """One payload index entry (model/entity/file.go:16-27)."""
    path: str
    offset: int
    length: int
    dtype: str = ""
    format: str = ""
    rows: int = 0
    cols: int = 0
    scale: float = 0.0
    native: bool = False

    @classmethod
    def from_json(cls, d: dict) -> "WeightBlob":
        return cls(d.get("path", ""), int(d.get("offset", 0)), int(d.get("length", 0)), d.get("dtype", ""),
                   d.get("format", ""), int(d.get("rows", 0) or 0), int(d.get("cols", 0) or 0),
                   float(d.get("scale", 0.0) or 0.0), bool(d.get("native", False)))

    def to_json(self) -> dict:
        d = {"path": self.path, "offset": self.offset, "length": self.length, "dtype": self.dtype,
             "format": self.format, "native": self.native}
        if self.rows:
            d["rows"] = self.rows
        if self.cols:
            d["cols"] = self.cols
        if self.scale:
            d["scale"] = self.scale
        return d


def parse_format_name(s: str) -> int:
    """quant.ParseFormatName (quant/format.go:134-144): exact names, else FormatNone (0)."""
    if s in ("", "none"):
        return 0
    f = FORMATS.get(s, 0)
    return 0 if f == FORMATS["NativeTernary"] else f


class EntityFile:
    """Random-access reader of a .entity checkpoint (entity.Open, file.go:110-185)."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        try:
            self._map = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as e:  # empty file
            self._f.close()
            raise EntityError(f"entity fixed header: {e}") from None
        try:
            self._read_header()
        except Exception:
            self.close()
            raise

    def _read_header(self) -> None:
        m = self._map
        if len(m) < FIXED_HEADER:
            raise EntityError("entity fixed header: short file")
        if m[:8] != MAGIC:
            raise EntityError(f"invalid entity magic: {bytes(m[:8])!r} (want ENTITY)")
        version, flags, header_len = struct.unpack_from("<HHQ", m, 8)
        if version != FORMAT_VERSION:
            raise EntityError(f"unsupported entity version: {version}")
        if header_len > HEADER_MAX:
            raise EntityError(f"entity header size unreasonable: {header_len}")
        if FIXED_HEADER + header_len > len(m):
            raise EntityError("entity header JSON: unexpected EOF")
        try:
            doc = json.loads(bytes(m[FIXED_HEADER:FIXED_HEADER + header_len]))
        except json.JSONDecodeError as e:
            raise EntityError(f"entity header JSON: {e}") from None
        self.version, self.flags = version, flags
        self.doc = doc
        self.data_offset = FIXED_HEADER + header_len
        self.blobs = [WeightBlob.from_json(b) for b in doc.get("blobs") or []]

    @property
    def transformer(self) -> dict | None:
        return self.doc.get("transformer")

    def find(self, path: str) -> WeightBlob:
        for b in self.blobs:  # first match, as findBlob (file.go:251-262)
            if b.path == path:
                return b
        raise EntityError(f"entity blob {path!r} not found")

    def blob_bytes(self, path: str) -> memoryview:
        """The payload bytes of one blob, in place in the mapping (LoadBlobBytes, file.go:216-229)."""
        b = self.find(path)
        lo = self.data_offset + b.offset
        if lo + b.length > len(self._map):
            raise EntityError(f"entity blob {path!r}: unexpected EOF")
        return memoryview(self._map)[lo:lo + b.length]

    def load_blob(self, path: str) -> np.ndarray:
        """A numeric (format "none") blob as float32 (LoadBlob, file.go:191-214; decodeNumericBlob :296-320)."""
        b = self.find(path)
        if b.format.strip().lower() not in ("", "none"):
            raise EntityError(f"entity blob {path!r}: packed format {b.format!r} — use upload_quant")
        dtype = b.dtype.strip().upper() or "FLOAT32"
        if dtype == "PACKED":
            raise EntityError(f"entity blob {path!r}: packed payload — use upload_quant")
        if dtype == "JSON":
            raise EntityError(f"entity blob {path!r}: JSON payload — use blob_bytes")
        raw = self.blob_bytes(path)
        width = {"FLOAT32": 4, "F32": 4, "FLOAT64": 8, "F64": 8, "DOUBLE": 8, "FLOAT16": 2, "F16": 2, "FP16": 2,
                 "BFLOAT16": 2, "BF16": 2}.get(dtype)
        if width is None:
            raise EntityError(f"entity blob {path!r}: dtype {dtype!r} is not a float payload")
        if len(raw) % width:
            raise EntityError(f"entity blob {path!r}: cannot derive element count for dtype {dtype!r} (len={len(raw)})")
        if width == 4:
            return np.frombuffer(raw, "<f4").astype(np.float32)
        if width == 8:
            return np.frombuffer(raw, "<f8").astype(np.float32)
        if dtype in ("BFLOAT16", "BF16"):
            return (np.frombuffer(raw, "<u2").astype(np.uint32) << 16).view(np.float32)
        return np.frombuffer(raw, "<f2").astype(np.float32)

    def upload_quant(self, path: str) -> DeviceBlob:
        """A packed blob straight to HBM (LoadQuantBlob, file.go:231-249, via wv_blob_upload_wire)."""
        b = self.find(path)
        fmt = parse_format_name(b.format)
        if fmt == 0:
            raise EntityError(f"entity blob {path!r}: not a packed quant blob (format={b.format!r})")
        if b.rows <= 0 or b.cols <= 0:
            raise EntityError(f"entity blob {path!r}: missing rows/cols")
        return DeviceBlob.from_wire(fmt, b.rows, b.cols, self.blob_bytes(path))

    def close(self) -> None:
        if getattr(self, "_map", None) is not None:
            try:
                self._map.close()
            except BufferError:  # a caller still holds a view: the mapping closes with the last one
                pass
            self._map = None
        if getattr(self, "_f", None) is not None:
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def encode_packed_blob(p: PackedBlob) -> bytes:
    """EncodePackedBlob (model/entity/packed.go:11-35)."""
    sc = np.zeros(0, "<f4") if p.scales is None else np.asarray(p.scales, "<f4")
    mn = np.zeros(0, "<f4") if p.mins is None else np.asarray(p.mins, "<f4")
    return struct.pack("<III", sc.size, mn.size, p.raw.size) + sc.tobytes() + mn.tobytes() + p.raw.tobytes()


def write_transformer_file(path: str, spec: dict, items: list) -> None:
    """WriteTransformerFile (model/entity/write.go:11-80). `items` are
    (blob path, value): a PackedBlob is stored as its packed wire (dtype
    PACKED), anything else as FLOAT32 numbers (format "none")."""
    blobs, payload, off = [], [], 0
    for bpath, value in items:
        if isinstance(value, PackedBlob):
            name = next(k for k, v in FORMATS.items() if v == value.fmt)
            data = encode_packed_blob(value)
            blobs.append(WeightBlob(bpath, off, len(data), "PACKED", name, value.rows, value.cols, native=True))
        else:
            data = np.ascontiguousarray(value, "<f4").tobytes()
            blobs.append(WeightBlob(bpath, off, len(data), "FLOAT32", "none"))
        payload.append(data)
        off += len(data)
    doc = {"format_version": FORMAT_VERSION, "engine": spec.get("engine") or "welvet", "status": "packed",
           "transformer": spec, "blobs": [b.to_json() for b in blobs]}
    hj = json.dumps(doc, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<HHQ", FORMAT_VERSION, 0, len(hj)) + hj)
        for data in payload:
            f.write(data)


def resolve_max_seq(spec: dict) -> int:
    """resolveMaxSeqLen without the HF snapshot lookup (load.go:243-256, ClampHostMaxSeq)."""
    n = int(spec.get("max_seq_len") or 0)
    n = n if n > 0 else DEFAULT_MAX_SEQ
    return min(n, HOST_MAX_SEQ_CAP)


def decoder_from_entity(path: str, max_seq: int | None = None):
    """A device Decoder over a dense packed transformer checkpoint, loaded as
    model/transformer/load.go:19-240 loads it: embeddings
    "transformer.embeddings", optional "transformer.final_norm", per block
    "blocks.{i}.attn_norm" / "ffn_norm" and packed q, k, v, o, gate, up, down in
    the spec's pack_format, the LM head "transformer.lm_head" (or
    "transformer.lm_head.packed" when tied); RMSNorm eps defaults to 1e-6 and
    the RoPE base to 10000. The decoder owns its blobs."""
    from .decode import Config, Decoder

    with EntityFile(path) as ef:
        spec = ef.transformer
        if not spec or not spec.get("dims"):
            raise EntityError("entity: not a transformer checkpoint (missing transformer.dims)")
        d = spec["dims"]
        if spec.get("architecture") in ("qwen35_hybrid", "qwen3_dense") or d.get("layer_types"):
            raise EntityError(f"entity: architecture {spec.get('architecture')!r} (hybrid loader) is not on the device path")
        if parse_format_name(spec.get("pack_format", "")) == 0:
            raise EntityError("entity: FormatNone (f32) projections are not on the device path; repack the checkpoint")
        n_layers, n_heads, hd = int(d["num_layers"]), int(d["num_heads"]), int(d["head_dim"])
        n_kv = int(d.get("num_kv_heads") or n_heads)
        if int(d.get("query_dim") or n_heads * hd) != n_heads * hd or int(d.get("kv_dim") or n_kv * hd) != n_kv * hd:
            raise EntityError("entity: query_dim / kv_dim must equal heads * head_dim on the device path")
        hidden, vocab = int(spec["hidden_size"]), int(spec["vocab_size"])
        eps = float(d.get("rms_norm_eps") or 0) or 1e-6
        rope = float(d.get("rope_freq_base") or 0) or 10000.0
        cfg = Config(n_layers=n_layers, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=hd,
                     ffn=int(d["intermediate_size"]), vocab=vocab, max_seq=max_seq or resolve_max_seq(spec),
                     rope_theta=rope, rms_eps=eps)
        dec = Decoder(cfg)
        owned = []
        try:
            for i in range(n_layers):
                p = f"blocks.{i}"
                blobs = [ef.upload_quant(f"{p}.{n}") for n in ("q", "k", "v", "o", "gate", "up", "down")]
                owned += blobs
                dec.set_layer(i, blobs, ef.load_blob(f"{p}.attn_norm"), ef.load_blob(f"{p}.ffn_norm"))
            lm = ef.upload_quant("transformer.lm_head.packed" if spec.get("lm_head_tied") else "transformer.lm_head")
            owned.append(lm)
            fnorm = ef.load_blob("transformer.final_norm") if spec.get("has_final_norm") else None
            dec.set_output(lm, fnorm, ef.load_blob("transformer.embeddings").reshape(vocab, hidden))
        except Exception:
            dec.free()
            for b in owned:
                b.free()
            raise
        dec.blobs = owned
        return dec
