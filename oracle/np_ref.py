"""TEST INFRASTRUCTURE ONLY: an independent numpy restatement of welvet's packers
and decoders, written vectorised (per block) rather than as the reference's
scalar loops, so that a slip in either restatement shows up as a mismatch
against oracle/oracle.c.

Rules restated (reference github.com/openfluke/welvet at /root/reference):
  PackQ4_0 quant/q4_0.go:10-45, PackQ8_0 quant/q8_0.go:8-44,
  packQ4_1 quant/q4_1.go:8-49, packQ5_0 quant/q5_0.go:8-45,
  packQ5_1 quant/q5_1.go:8-47, packK quant/kquant.go:62-176,
  packIQ quant/iq.go:70-167, packTernary quant/ternary.go:11-51,
  packBinary quant/binary.go:11-47, DTypeTernary weights/native.go:249-267,
  decoders quant/*.go (forEach*, unpack*), quantizeActsI8
  layers/dense/simd.go:526-549.

float32 numpy operations round after every operation, like Go float32.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

FORMATS = {
    "none": 0, "Q8_0": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 4, "Q5_1": 5,
    "Q2_K": 6, "Q3_K": 7, "Q4_K": 8, "Q5_K": 9, "Q6_K": 10,
    "IQ1_S": 11, "IQ2_XXS": 12, "IQ2_XS": 13, "IQ3_XXS": 14, "IQ3_S": 15,
    "IQ4_NL": 16, "IQ4_XS": 17, "TernaryPacked": 18, "BinaryPacked": 19,
    "AffinePacked": 20,
}

KSPEC = {  # bits, hasDmin, qMax, mid  (kquant.go:36-51)
    "Q2_K": (2, True, 3, 0), "Q3_K": (3, True, 7, 0), "Q4_K": (4, True, 15, 0),
    "Q5_K": (5, True, 31, 0), "Q6_K": (6, False, 63, 32),
}
IQSPEC = {  # bits, scaleGroup, nonlinear, mid  (iq.go:49-68)
    "IQ1_S": (1, 32, False, 0.5), "IQ2_XXS": (2, 32, False, 1.5),
    "IQ2_XS": (2, 16, False, 1.5), "IQ3_XXS": (3, 32, False, 3.5),
    "IQ3_S": (3, 16, False, 3.5), "IQ4_NL": (4, 32, True, 0.0),
    "IQ4_XS": (4, 16, False, 7.5),
}
IQ4NL_GRID = np.array([
    -1.0, -0.6961928, -0.52507305, -0.3949175, -0.28444138, -0.18477343,
    -0.091050036, 0.0, 0.0795803, 0.1609302, 0.2461123, 0.33791524,
    0.44070983, 0.562617, 0.72295684, 1.0], dtype=F32)


def round_half_away(v: np.ndarray) -> np.ndarray:
    """math.Round for float64 arrays, exact (no +0.5 double rounding)."""
    v = np.asarray(v, dtype=np.float64)
    t = np.trunc(v)
    frac = np.abs(v - t)
    return (t + np.where(frac >= 0.5, np.sign(v), 0.0)).astype(np.int64)


def _blocks(w: np.ndarray, bs: int):
    """(nblocks, bs) float32 view padded with 0 plus a validity mask."""
    n = w.size
    nb = -(-n // bs)
    pad = np.zeros(nb * bs, dtype=F32)
    pad[:n] = w
    mask = np.zeros(nb * bs, dtype=bool)
    mask[:n] = True
    return pad.reshape(nb, bs), mask.reshape(nb, bs)


def _maxabs(b, m):
    return np.where(m, np.abs(b), F32(0)).max(axis=1).astype(F32)


def _minmax(b, m):
    mn = np.where(m, b, F32(np.inf)).min(axis=1)
    mx = np.where(m, b, F32(-np.inf)).max(axis=1)
    empty = ~m.any(axis=1)
    mn[empty] = 0
    mx[empty] = 0
    return mn.astype(F32), mx.astype(F32)


def _absmean(b, m):
    # sequential float32 sum (helpers.go:49-58), column by column
    s = np.zeros(b.shape[0], dtype=F32)
    for j in range(b.shape[1]):
        s = np.where(m[:, j], (s + np.abs(b[:, j])).astype(F32), s)
    cnt = m.sum(axis=1).astype(F32)
    out = np.zeros_like(s)
    nz = cnt > 0
    out[nz] = (s[nz] / cnt[nz]).astype(F32)
    return out


def _bits_lsb(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack unsigned codes (flat) into an LSB-first bit stream (bytes)."""
    codes = np.asarray(codes, dtype=np.uint32)
    bitarr = ((codes[:, None] >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8).reshape(-1)
    return np.packbits(bitarr, bitorder="little")


def _unbits_lsb(raw: np.ndarray, bits: int, count: int) -> np.ndarray:
    allbits = np.unpackbits(np.asarray(raw, dtype=np.uint8), bitorder="little")
    need = count * bits
    if allbits.size < need:
        allbits = np.concatenate([allbits, np.zeros(need - allbits.size, dtype=np.uint8)])
    b = allbits[:need].reshape(count, bits).astype(np.uint32)
    return (b << np.arange(bits, dtype=np.uint32)).sum(axis=1).astype(np.uint32)


def _f32bytes(a) -> np.ndarray:
    return np.asarray(a, dtype="<f4").view(np.uint8).reshape(-1, 4)


def pack(fmt: str, w: np.ndarray, rows: int, cols: int):
    """Returns dict(raw, scales, meta, block_weights)."""
    w = np.asarray(w, dtype=F32).reshape(-1)[: rows * cols]
    n = rows * cols
    if fmt == "Q4_0":
        b, m = _blocks(w, 32)
        scale = (_maxabs(b, m) / F32(7)).astype(F32)
        scale[scale == 0] = 1
        q = round_half_away((b / scale[:, None]).astype(F32).astype(np.float64))
        q = np.clip(q, -8, 7)
        q[~m] = 0
        nib = (q & 0xF).astype(np.uint8)
        body = nib[:, 0::2] | (nib[:, 1::2] << 4)
        raw = np.concatenate([_f32bytes(scale), body], axis=1).reshape(-1)
        return dict(raw=raw, scales=None, meta=None, block_weights=32)
    if fmt == "Q8_0":
        b, m = _blocks(w, 32)
        scale = (_maxabs(b, m) / F32(127)).astype(F32)
        scale[scale == 0] = 1
        q = np.clip(round_half_away(b.astype(np.float64) / scale[:, None].astype(np.float64)), -127, 127)
        q[~m] = 0
        raw = np.concatenate([_f32bytes(scale), q.astype(np.int8).view(np.uint8)], axis=1).reshape(-1)
        return dict(raw=raw, scales=None, meta=None, block_weights=32)
    if fmt in ("Q4_1", "Q5_1"):
        qmax = 15 if fmt == "Q4_1" else 31
        b, m = _blocks(w, 32)
        mn, mx = _minmax(b, m)
        scale = ((mx - mn) / F32(qmax)).astype(F32)
        scale[scale == 0] = 1
        t = ((b - mn[:, None]).astype(F32) / scale[:, None]).astype(F32)
        q = np.clip(round_half_away(t.astype(np.float64)), 0, qmax)
        q[~m] = 0
        if fmt == "Q4_1":
            body = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
        else:
            body = _bits_lsb(q.reshape(-1), 5).reshape(-1, 20)
        raw = np.concatenate([_f32bytes(scale), _f32bytes(mn), body], axis=1).reshape(-1)
        return dict(raw=raw, scales=None, meta=None, block_weights=32)
    if fmt == "Q5_0":
        b, m = _blocks(w, 32)
        scale = (_maxabs(b, m) / F32(15)).astype(F32)
        scale[scale == 0] = 1
        q = np.clip(round_half_away(b.astype(np.float64) / scale[:, None].astype(np.float64)) + 16, 0, 31)
        q[~m] = 16
        body = _bits_lsb(q.reshape(-1), 5).reshape(-1, 20)
        raw = np.concatenate([_f32bytes(scale), body], axis=1).reshape(-1)
        return dict(raw=raw, scales=None, meta=None, block_weights=32)
    if fmt in KSPEC:
        bits, has_dmin, qmax, mid = KSPEC[fmt]
        b, m = _blocks(w, 16)  # groups of 16
        ng = b.shape[0]
        nsb = -(-n // 256)
        gpad = nsb * 16
        if gpad > ng:
            b = np.concatenate([b, np.zeros((gpad - ng, 16), F32)])
            m = np.concatenate([m, np.zeros((gpad - ng, 16), bool)])
        present = m.any(axis=1)
        if has_dmin:
            gmin, gmx = _minmax(b, m)
            gscale = ((gmx - gmin) / F32(qmax)).astype(F32)
            gscale[gscale == 0] = 1
            t = ((b - gmin[:, None]).astype(F32) / gscale[:, None]).astype(F32)
            q = np.clip(round_half_away(t.astype(np.float64)), 0, qmax)
            q[~m] = 0
        else:
            gmin = np.zeros(gpad, F32)
            amax = _maxabs(b, m)
            gscale = (amax / F32(mid)).astype(F32)
            gscale[gscale == 0] = 1
            q = np.clip(round_half_away(b.astype(np.float64) / gscale[:, None].astype(np.float64)) + mid, 0, qmax)
            q[~m] = mid
        gscale[~present] = 1
        gmin[~present] = 0
        q[~present] = 0
        gs = gscale.reshape(nsb, 16)
        gm = gmin.reshape(nsb, 16)
        d = gs.max(axis=1).astype(F32)
        d[d == 0] = 1
        if has_dmin:
            dmin = np.abs(gm).max(axis=1).astype(F32)
            dmin[dmin == 0] = 1
        else:
            dmin = np.zeros(nsb, F32)
        su = np.clip(round_half_away(gs.astype(np.float64) / d[:, None].astype(np.float64) * 255), 0, 255).astype(np.uint8)
        parts = [_f32bytes(d), _f32bytes(dmin), su]
        if has_dmin:
            mu = np.clip(round_half_away(gm.astype(np.float64) / dmin[:, None].astype(np.float64) * 127), -127, 127)
            parts.append(mu.astype(np.int8).view(np.uint8))
        codes = _bits_lsb(q.reshape(-1), bits).reshape(nsb, 256 * bits // 8)
        parts.append(codes)
        raw = np.concatenate(parts, axis=1).reshape(-1)
        return dict(raw=raw, scales=None, meta=None, block_weights=256)
    if fmt in IQSPEC:
        bits, sg, nonlinear, mid = IQSPEC[fmt]
        b, m = _blocks(w, sg)
        qmax = (1 << bits) - 1
        amax = _maxabs(b, m)
        present = m.any(axis=1)
        if nonlinear:
            scale = amax.copy()
            scale[scale == 0] = 1
            target = (b / scale[:, None]).astype(F32)
            err = np.abs((IQ4NL_GRID[None, None, :] - target[:, :, None]).astype(F32))
            q = np.argmin(err, axis=2).astype(np.int64)  # first minimum wins
            q[~m] = 0
        else:
            if bits == 1:
                scale = amax.copy()
            else:
                denom = max(F32(qmax) - F32(mid), F32(1))
                scale = (amax / F32(denom)).astype(F32)
            scale[scale == 0] = 1
            if bits == 1:
                q = (b >= 0).astype(np.int64)
            else:
                q = np.clip(round_half_away(b.astype(np.float64) / scale[:, None].astype(np.float64) + float(np.float32(mid))), 0, qmax)
            q[~m] = 0
        scale[~present] = 1
        raw = _bits_lsb(q.reshape(-1), bits)
        return dict(raw=raw, scales=scale.astype(F32), meta=np.array([bits, sg], np.uint8), block_weights=32)
    if fmt == "TernaryPacked":
        b, m = _blocks(w, 16)
        scale = _absmean(b, m)
        scale[scale == 0] = 1
        q = np.clip(round_half_away((b / scale[:, None]).astype(F32).astype(np.float64)), -1, 1) + 1
        q[~m] = 1
        words = (q.astype(np.uint32) << (2 * np.arange(16, dtype=np.uint32))).sum(axis=1).astype("<u4")
        return dict(raw=words.view(np.uint8), scales=scale, meta=None, block_weights=16)
    if fmt == "BinaryPacked":
        b, m = _blocks(w, 32)
        scale = _absmean(b, m)
        scale[scale == 0] = 1
        bitsv = ((b >= 0) & m).astype(np.uint32)
        words = (bitsv << np.arange(32, dtype=np.uint32)).sum(axis=1).astype("<u4")
        return dict(raw=words.view(np.uint8), scales=scale, meta=None, block_weights=32)
    if fmt == "AffinePacked":  # PackAffine4, group 64 along cols (affine_pack.go:15-86)
        if cols % 64:
            raise ValueError("AffinePacked: cols must be a multiple of 64")
        g = w.reshape(rows, cols // 64, 64)
        mn = g.min(axis=2)
        mx = g.max(axis=2)
        s = ((mx - mn) / F32(15)).astype(F32)
        bad = (s == 0) | ~np.isfinite(s)
        s[bad] = 1
        mn[bad] = 0
        inv = (F32(1) / s).astype(F32)
        t = ((g - mn[:, :, None]).astype(F32) * inv[:, :, None]).astype(F32)
        code = np.clip(round_half_away(t.astype(np.float64)), 0, 15).astype(np.uint32).reshape(-1, 8)
        words = (code << (4 * np.arange(8, dtype=np.uint32))).sum(axis=1).astype("<u4")
        return dict(raw=words.view(np.uint8), scales=s.reshape(-1), mins=mn.reshape(-1).astype(F32),
                    meta=np.array([4], np.uint8), block_weights=64)
    raise ValueError(f"unsupported format {fmt}")


def unpack(fmt: str, rows: int, cols: int, raw, scales=None, meta=None, block_weights=0, mins=None):
    """Dequantize to float32[rows*cols] with the reference's f32 formulas."""
    raw = np.asarray(raw, dtype=np.uint8)
    n = rows * cols
    if fmt in ("Q4_0", "Q8_0", "Q4_1", "Q5_0", "Q5_1"):
        bb = {"Q4_0": 20, "Q8_0": 36, "Q4_1": 24, "Q5_0": 24, "Q5_1": 28}[fmt]
        blk = raw.reshape(-1, bb)
        scale = blk[:, 0:4].copy().view("<f4").reshape(-1)
        if fmt == "Q4_0":
            body = blk[:, 4:]
            q = np.stack([body & 0xF, body >> 4], axis=2).reshape(-1, 32).astype(np.int32)
            q = np.where(q > 7, q - 16, q)
            w = (q.astype(F32) * scale[:, None]).astype(F32)
        elif fmt == "Q8_0":
            q = blk[:, 4:].view(np.int8).astype(F32)
            w = (q * scale[:, None]).astype(F32)
        elif fmt == "Q5_0":
            q = _unbits_lsb(blk[:, 4:].reshape(-1), 5, blk.shape[0] * 32).reshape(-1, 32).astype(np.int32) - 16
            w = (q.astype(F32) * scale[:, None]).astype(F32)
        else:
            mn = blk[:, 4:8].copy().view("<f4").reshape(-1)
            if fmt == "Q4_1":
                body = blk[:, 8:]
                q = np.stack([body & 0xF, body >> 4], axis=2).reshape(-1, 32)
            else:
                q = _unbits_lsb(blk[:, 8:].reshape(-1), 5, blk.shape[0] * 32).reshape(-1, 32)
            w = (mn[:, None] + (q.astype(F32) * scale[:, None]).astype(F32)).astype(F32)
        return w.reshape(-1)[:n]
    if fmt in KSPEC:
        bits, has_dmin, qmax, mid = KSPEC[fmt]
        sbb = 8 + 16 + (16 if has_dmin else 0) + 256 * bits // 8
        sb = raw.reshape(-1, sbb)
        d = sb[:, 0:4].copy().view("<f4").reshape(-1)
        dmin = sb[:, 4:8].copy().view("<f4").reshape(-1)
        su = sb[:, 8:24].astype(F32)
        sc = ((d[:, None] * su).astype(F32) / F32(255)).astype(F32)
        fallback = (d / F32(255)).astype(F32)
        sc = np.where(sc == 0, fallback[:, None], sc)
        qoff = 40 if has_dmin else 24
        q = _unbits_lsb(sb[:, qoff:].reshape(-1), bits, sb.shape[0] * 256).reshape(-1, 16, 16)
        if has_dmin:
            mu = sb[:, 24:40].view(np.int8).astype(F32)
            mn = ((dmin[:, None] * mu).astype(F32) / F32(127)).astype(F32)
            w = (mn[:, :, None] + (q.astype(F32) * sc[:, :, None]).astype(F32)).astype(F32)
        else:
            w = (sc[:, :, None] * (q.astype(np.int32) - mid).astype(F32)).astype(F32)
        return w.reshape(-1)[:n]
    if fmt in IQSPEC:
        bits, sg, nonlinear, mid = IQSPEC[fmt]
        if meta is not None and len(meta) >= 2:
            bits, sg = int(meta[0]), int(meta[1])
        scales = np.asarray(scales, F32)
        q = _unbits_lsb(raw, bits, scales.size * sg).reshape(-1, sg)
        if nonlinear:
            w = (scales[:, None] * IQ4NL_GRID[q & 15]).astype(F32)
        elif bits == 1:
            w = np.where(q & 1, scales[:, None], -scales[:, None]).astype(F32)
        else:
            w = (scales[:, None] * (q.astype(F32) - F32(mid)).astype(F32)).astype(F32)
        return w.reshape(-1)[:n]
    if fmt == "TernaryPacked":
        words = raw.view("<u4")
        c = (words[:, None] >> (2 * np.arange(16, dtype=np.uint32))) & 3
        s = np.asarray(scales, F32)[:, None]
        w = np.where(c == 0, -s, np.where(c == 2, s, F32(0))).astype(F32)
        return w.reshape(-1)[:n]
    if fmt == "BinaryPacked":
        words = raw.view("<u4")
        if block_weights == 128:
            wpr = cols // 32
            bitsv = ((words.reshape(rows, wpr)[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(rows, cols)
            s = np.asarray(scales, F32).reshape(rows, cols // 128)
            s = np.repeat(s, 128, axis=1)
            return np.where(bitsv == 1, s, -s).astype(F32).reshape(-1)
        bitsv = (words[:, None] >> np.arange(32, dtype=np.uint32)) & 1
        s = np.asarray(scales, F32)[:, None]
        return np.where(bitsv == 1, s, -s).astype(F32).reshape(-1)[:n]
    if fmt == "AffinePacked":  # decodeRowAffine (affine_g64.go:124-161): f32(s*code) + beta
        g = block_weights or 64
        code = np.stack([raw & 0xF, raw >> 4], axis=1).reshape(rows, cols // g, g).astype(F32)
        s = np.asarray(scales, F32).reshape(rows, cols // g, 1)
        beta = np.asarray(mins, F32).reshape(rows, cols // g, 1)
        return ((s * code).astype(F32) + beta).astype(F32).reshape(-1)
    raise ValueError(f"unsupported format {fmt}")


def pack_native_ternary(w: np.ndarray):
    """weights/native.go:249-267 (absMax scale, thresholds ±0.5)."""
    w = np.asarray(w, F32).reshape(-1)
    scale = F32(np.abs(w).max()) if w.size else F32(0)
    if scale == 0:
        scale = F32(1)
    r = (w / scale).astype(F32)
    code = np.where(r > F32(0.5), 2, np.where(r < F32(-0.5), 0, 1)).astype(np.uint8)
    padn = -(-w.size // 4) * 4
    c = np.ones(padn, np.uint8) * 0
    c[: w.size] = code
    c = c.reshape(-1, 4)
    packed = (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)
    return packed, scale


def quantize_acts_i8(x: np.ndarray):
    """layers/dense/simd.go:526-549."""
    x = np.asarray(x, F32)
    maxabs = F32(np.abs(x).max()) if x.size else F32(0)
    scale = F32(maxabs / F32(127))
    if scale == 0:
        scale = F32(1)
    q = np.clip(round_half_away((x / scale).astype(F32).astype(np.float64)), -128, 127).astype(np.int8)
    return q, scale


# ---- narrow weights.Store DTypes (core.DType: 9 Int8, 14 Int4, 17 Int2, 19 Ternary, 20 Binary) ----

NATIVE_BITS = {9: 8, 14: 4, 17: 2, 19: 2, 20: 1}


def _pack_bits(codes: np.ndarray, bits: int) -> np.ndarray:
    """LSB-first packing of `bits`-bit codes, element i at bit i*bits."""
    per = 8 // bits
    padn = -(-codes.size // per) * per
    c = np.zeros(padn, np.uint16)
    c[: codes.size] = codes
    c = c.reshape(-1, per)
    out = np.zeros(c.shape[0], np.uint16)
    for k in range(per):
        out |= c[:, k] << (bits * k)
    return out.astype(np.uint8)


def pack_native(dt: int, w: np.ndarray):
    """packNative for the narrow DTypes (weights/native.go:88-97, 180-283)."""
    w = np.asarray(w, F32).reshape(-1)
    amax = F32(np.abs(w).max()) if w.size else F32(0)
    scale = {9: F32(amax / F32(127)), 14: F32(amax / F32(7))}.get(dt, amax)
    if scale == 0:
        scale = F32(1)
    r = (w / scale).astype(F32)
    q = round_half_away(r.astype(np.float64))
    if dt == 9:
        codes = np.clip(q, -128, 127).astype(np.int64) & 0xFF
    elif dt == 14:
        codes = np.clip(q, -8, 7).astype(np.int64) & 0xF
    elif dt == 17:
        codes = (np.clip(q, -2, 1).astype(np.int64) + 2) & 3
    elif dt == 19:
        codes = np.where(r > F32(0.5), 2, np.where(r < F32(-0.5), 0, 1))
    else:
        codes = (w >= 0).astype(np.int64)
    return _pack_bits(codes.astype(np.uint16), NATIVE_BITS[dt]), scale


def unpack_codes(dt: int, codes: np.ndarray, n: int) -> np.ndarray:
    """The unsigned codes of elements 0..n-1 (LSB-first)."""
    bits = NATIVE_BITS[dt]
    b = np.asarray(codes, np.uint8)
    idx = np.arange(n, dtype=np.int64) * bits
    return ((b[idx >> 3].astype(np.uint16) >> (idx & 7)) & ((1 << bits) - 1)).astype(np.int64)


def expand_narrow_i8(dt: int, codes: np.ndarray, n: int) -> np.ndarray:
    """expandNarrowToI8 (layers/dense/simd.go:149-195); Int8 bytes as signed."""
    u = unpack_codes(dt, codes, n)
    if dt == 9:
        return u.astype(np.uint8).view(np.int8).astype(np.int8)
    if dt == 14:
        return np.where(u > 7, u - 16, u).astype(np.int8)
    if dt == 17:
        return (u - 2).astype(np.int8)
    if dt == 19:
        return (u - 1).astype(np.int8)
    return (2 * u - 1).astype(np.int8)


def native_decode(dt: int, codes: np.ndarray, scale, n: int) -> np.ndarray:
    """weightAt (weights/decode.go:50-215): f32(q) * scale; Ternary 0/2 -> -s/+s, 1/3 -> 0."""
    scale = F32(scale) if F32(scale) != 0 else F32(1)
    u = unpack_codes(dt, codes, n)
    if dt == 19:
        return np.where(u == 0, -scale, np.where(u == 2, scale, F32(0))).astype(F32)
    if dt == 20:
        return np.where(u == 1, scale, -scale).astype(F32)
    return (expand_narrow_i8(dt, codes, n).astype(F32) * scale).astype(F32)


def narrow_i8_forward(dt: int, codes: np.ndarray, scale, rows: int, cols: int, x: np.ndarray):
    """Dense's int8 path (simd.go:130-147, 303-326) with exact int64 sums."""
    scale = F32(scale) if F32(scale) != 0 else F32(1)
    wi8 = expand_narrow_i8(dt, codes, rows * cols).reshape(rows, cols).astype(np.int64)
    x = np.asarray(x, F32).reshape(-1, cols)
    ys, accs, acts = [], [], []
    for xb in x:
        q, a = quantize_acts_i8(xb)
        acc = wi8 @ q.astype(np.int64)
        ys.append(((acc.astype(np.int32).astype(F32) * a).astype(F32) * scale).astype(F32))
        accs.append(acc.astype(np.int32))
        acts.append(a)
    return np.concatenate(ys), np.concatenate(accs), np.array(acts, F32)
