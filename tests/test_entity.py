"""ENTITY checkpoint reader / writer (model/entity/*.go) — CPU only.

Pinned by hand-built bytes: the fixed header (magic, version, flags, JSON
length), the EncodePackedBlob wire layout (ns, nm, nr, scales, mins, raw),
payload offsets relative to the data section, and the numeric dtypes
(FLOAT32 / FLOAT64 / FLOAT16 / BFLOAT16). Wire parsing errors come from the
C ABI before any device call, with the reference's wording.
"""
import json
import struct

import numpy as np
import pytest

import welvet_amd as wv
from welvet_amd import entity


def test_packed_wire_layout_by_hand():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal(2 * 128) * 0.02).astype(np.float32)
    p = wv.pack("AffinePacked", w, 2, 128)
    wire = entity.encode_packed_blob(p)
    ns, nm, nr = struct.unpack_from("<III", wire, 0)
    assert (ns, nm, nr) == (4, 4, 128)
    assert wire[12:28] == p.scales.astype("<f4").tobytes()
    assert wire[28:44] == p.mins.astype("<f4").tobytes()
    assert wire[44:] == p.raw.tobytes() and len(wire) == 12 + 16 + 16 + 128
    q = wv.pack("Q4_K", np.zeros(256, np.float32), 1, 256)
    assert entity.encode_packed_blob(q)[:12] == struct.pack("<III", 0, 0, q.raw.size)


def test_write_read_round_trip(tmp_path):
    rng = np.random.default_rng(2)
    emb = rng.standard_normal((10, 64)).astype(np.float32)
    p = wv.pack("Q4_K", (rng.standard_normal(32 * 256) * 0.02).astype(np.float32), 32, 256)
    spec = {"architecture": "llama", "hidden_size": 64, "vocab_size": 10, "pack_format": "Q4_K",
            "dims": {"num_layers": 1, "num_heads": 1, "num_kv_heads": 1, "head_dim": 64, "intermediate_size": 128}}
    f = tmp_path / "m.entity"
    entity.write_transformer_file(str(f), spec, [("transformer.embeddings", emb), ("blocks.0.q", p)])
    raw = f.read_bytes()
    assert raw[:8] == b"ENTITY\x00\x00"
    ver, flags, hlen = struct.unpack_from("<HHQ", raw, 8)
    assert (ver, flags) == (1, 0)
    doc = json.loads(raw[20:20 + hlen])
    assert doc["format_version"] == 1 and doc["status"] == "packed" and doc["transformer"]["pack_format"] == "Q4_K"
    b0, b1 = doc["blobs"]
    assert b0 == {"path": "transformer.embeddings", "offset": 0, "length": emb.nbytes, "dtype": "FLOAT32",
                  "format": "none", "native": False}
    assert b1["offset"] == emb.nbytes and b1["dtype"] == "PACKED" and b1["format"] == "Q4_K"
    assert (b1["rows"], b1["cols"]) == (32, 256)
    data = 20 + hlen
    assert raw[data:data + emb.nbytes] == emb.tobytes()
    with entity.EntityFile(str(f)) as ef:
        assert ef.data_offset == data and ef.transformer["hidden_size"] == 64
        assert np.array_equal(ef.load_blob("transformer.embeddings").reshape(10, 64), emb)
        assert bytes(ef.blob_bytes("blocks.0.q")) == entity.encode_packed_blob(p)
        with pytest.raises(entity.EntityError, match="packed format"):
            ef.load_blob("blocks.0.q")
        with pytest.raises(entity.EntityError, match="not a packed quant blob"):
            ef.upload_quant("transformer.embeddings")
        with pytest.raises(entity.EntityError, match="not found"):
            ef.find("blocks.9.q")


def test_numeric_dtypes(tmp_path):
    """decodeNumericBlob (file.go:296-320): F64 / F16 / BF16 payloads widen (or round) to f32."""
    v = np.array([1.5, -2.25, 3.0e-3, 65504.0], np.float64)
    payload = [v.astype("<f8").tobytes(), v.astype("<f2").tobytes(),
               (v.astype(np.float32).view(np.uint32) >> 16).astype("<u2").tobytes()]
    blobs, off = [], 0
    for name, dt, data in zip(("a", "b", "c"), ("FLOAT64", "FLOAT16", "BF16"), payload):
        blobs.append({"path": name, "offset": off, "length": len(data), "dtype": dt, "format": "none", "native": False})
        off += len(data)
    hj = json.dumps({"format_version": 1, "engine": "welvet", "status": "packed", "blobs": blobs}).encode()
    f = tmp_path / "n.entity"
    f.write_bytes(b"ENTITY\x00\x00" + struct.pack("<HHQ", 1, 0, len(hj)) + hj + b"".join(payload))
    with entity.EntityFile(str(f)) as ef:
        assert np.array_equal(ef.load_blob("a"), v.astype(np.float32))
        assert np.array_equal(ef.load_blob("b"), v.astype(np.float16).astype(np.float32))
        bf = ((v.astype(np.float32).view(np.uint32) >> 16) << 16).view(np.float32)
        assert np.array_equal(ef.load_blob("c"), bf)


def test_header_errors(tmp_path):
    f = tmp_path / "bad.entity"
    f.write_bytes(b"NOTENTIT" + bytes(40))
    with pytest.raises(entity.EntityError, match="invalid entity magic"):
        entity.EntityFile(str(f))
    f.write_bytes(b"ENTITY\x00\x00" + struct.pack("<HHQ", 2, 0, 2) + b"{}")
    with pytest.raises(entity.EntityError, match="unsupported entity version: 2"):
        entity.EntityFile(str(f))
    f.write_bytes(b"ENTITY\x00\x00" + struct.pack("<HHQ", 1, 0, 300 << 20))
    with pytest.raises(entity.EntityError, match="unreasonable"):
        entity.EntityFile(str(f))


def test_wire_errors_without_device():
    with pytest.raises(wv.WelvetError, match="packed wire too short"):
        wv.DeviceBlob.from_wire("Q4_K", 1, 256, b"\x00" * 8)
    wire = struct.pack("<III", 1, 0, 144) + b"\x00" * 4 + b"\x00" * 100
    with pytest.raises(wv.WelvetError, match=r"packed wire truncated \(need 160, have 116\)"):
        wv.DeviceBlob.from_wire("Q4_K", 1, 256, wire)
    with pytest.raises(wv.WelvetError, match="not a packed quant blob"):
        wv.DeviceBlob.from_wire(0, 1, 256, struct.pack("<III", 0, 0, 0))


def test_decoder_from_entity_rejects_unsupported(tmp_path):
    f = tmp_path / "h.entity"
    spec = {"architecture": "qwen35_hybrid", "hidden_size": 64, "vocab_size": 10,
            "dims": {"num_layers": 1, "num_heads": 1, "head_dim": 64, "intermediate_size": 64, "layer_types": ["x"]}}
    entity.write_transformer_file(str(f), spec, [])
    with pytest.raises(entity.EntityError, match="hybrid"):
        entity.decoder_from_entity(str(f))
    spec = {"architecture": "llama", "hidden_size": 64, "vocab_size": 10, "pack_format": "",
            "dims": {"num_layers": 1, "num_heads": 1, "head_dim": 64, "intermediate_size": 64}}
    entity.write_transformer_file(str(f), spec, [])
    with pytest.raises(entity.EntityError, match="FormatNone"):
        entity.decoder_from_entity(str(f))
