"""Independent numpy decoder of the ggml block formats (test infrastructure).

Written from the block layouts (field offsets and bit packing), vectorised
over whole blocks, without reference to the oracle's loops. It pins the
oracle's dequantisation: both must agree bit for bit.

Arithmetic follows the formats' defining expressions with one f32 rounding
per operation, as the reference evaluates them (src/quant.rs:191-385):
  Q4_0  (q - 8) * d              Q4_1  q * d + m
  Q5_0  (q - 16) * d             Q5_1  q * d + m
  Q8_0  q * d
  Q4_K  (d*sc) * q - (dmin*m)    Q5_K  same with a 5th bit
  Q6_K  (d*sc) * (q - 32)
"""
import numpy as np

F32 = np.float32


def f16(lo, hi):
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(F32)


def _blocks(data, ts):
    data = np.ascontiguousarray(data, dtype=np.uint8)
    return data.reshape(-1, ts)


def unpack_scale_min_k4(s12):
    """(sc, m) of the 8 sub-blocks of a K super-block from its 12 scale bytes
    (columns 0..11). Sub-blocks 0-3: low 6 bits of bytes 0-3 / 4-7.
    Sub-blocks 4-7: low nibble / high nibble of bytes 8-11, with the two top
    bits taken from bytes 0-3 (scales) and 4-7 (mins)."""
    s = s12.astype(np.uint32)
    sc = np.empty((s.shape[0], 8), np.uint32)
    m = np.empty((s.shape[0], 8), np.uint32)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def dequant(ty, data, n):
    if ty == 0:
        return np.ascontiguousarray(data, np.uint8)[: 4 * n].view(F32).copy()
    if ty == 1:
        return np.ascontiguousarray(data, np.uint8)[: 2 * n].view(np.float16).astype(F32)
    if ty == 30:
        h = np.ascontiguousarray(data, np.uint8)[: 2 * n].view(np.uint16).astype(np.uint32) << 16
        return h.view(F32)
    if ty == 2:  # Q4_0: d, 16 bytes; value j<16 low nibble of byte j, j>=16 high nibble of byte j-16
        b = _blocks(data, 18)
        d = f16(b[:, 0], b[:, 1])[:, None]
        q = b[:, 2:18]
        vals = np.concatenate([q & 0xF, q >> 4], axis=1).astype(np.int32) - 8
        return (vals.astype(F32) * d).reshape(-1)[:n]
    if ty == 3:  # Q4_1: d, m, 16 bytes
        b = _blocks(data, 20)
        d = f16(b[:, 0], b[:, 1])[:, None]
        m = f16(b[:, 2], b[:, 3])[:, None]
        q = b[:, 4:20]
        vals = np.concatenate([q & 0xF, q >> 4], axis=1).astype(F32)
        return (vals * d + m).reshape(-1)[:n]
    if ty in (6, 7):  # Q5_0 / Q5_1: 5th bit of value j is bit j of the u32 qh
        ts = 22 if ty == 6 else 24
        b = _blocks(data, ts)
        d = f16(b[:, 0], b[:, 1])[:, None]
        off = 2 if ty == 6 else 4
        qh = b[:, off:off + 4].copy().view(np.uint32).reshape(-1).astype(np.uint64)
        q = b[:, off + 4:off + 20]
        j = np.arange(32, dtype=np.uint64)
        hbit = ((qh[:, None] >> j[None, :]) & 1).astype(np.uint32) << 4
        vals = np.concatenate([q & 0xF, q >> 4], axis=1).astype(np.uint32) | hbit
        if ty == 6:
            return ((vals.astype(np.int32) - 16).astype(F32) * d).reshape(-1)[:n]
        m = f16(b[:, 2], b[:, 3])[:, None]
        return (vals.astype(F32) * d + m).reshape(-1)[:n]
    if ty == 8:  # Q8_0
        b = _blocks(data, 34)
        d = f16(b[:, 0], b[:, 1])[:, None]
        return (b[:, 2:34].view(np.int8).astype(F32) * d).reshape(-1)[:n]
    if ty in (12, 13):  # Q4_K / Q5_K
        ts = 144 if ty == 12 else 176
        b = _blocks(data, ts)
        d = f16(b[:, 0], b[:, 1])
        dmin = f16(b[:, 2], b[:, 3])
        sc, m = unpack_scale_min_k4(b[:, 4:16])
        qs = b[:, 16:144] if ty == 12 else b[:, 48:176]
        # sub-block 2g = low nibbles of qs[32g:32g+32], 2g+1 = high nibbles
        q = np.empty((b.shape[0], 8, 32), np.uint32)
        for g in range(4):
            q[:, 2 * g] = qs[:, 32 * g:32 * g + 32] & 0xF
            q[:, 2 * g + 1] = qs[:, 32 * g:32 * g + 32] >> 4
        if ty == 13:  # 5th bit of sub-block j is bit j of qh[l]
            qh = b[:, 16:48].astype(np.uint32)
            for j in range(8):
                q[:, j] |= ((qh >> j) & 1) << 4
        d1 = d[:, None] * sc.astype(F32)
        mm = dmin[:, None] * m.astype(F32)
        vals = d1[:, :, None] * q.astype(F32) - mm[:, :, None]
        return vals.reshape(-1)[:n]
    if ty == 14:  # Q6_K: ql[128], qh[64], sc[16] (i8), d
        b = _blocks(data, 210)
        d = f16(b[:, 208], b[:, 209])
        sc = b[:, 192:208].view(np.int8).astype(F32)
        out = np.empty((b.shape[0], 256), F32)
        for h in range(2):
            ql = b[:, 64 * h:64 * h + 64].astype(np.uint32)
            qh = b[:, 128 + 32 * h:128 + 32 * h + 32].astype(np.uint32)
            # quarter k of the 128-value half: low/high nibble of ql[0:32]/ql[32:64], bits 2k..2k+1 of qh
            nib = [ql[:, :32] & 0xF, ql[:, 32:] & 0xF, ql[:, :32] >> 4, ql[:, 32:] >> 4]
            for k in range(4):
                u = nib[k] | (((qh >> (2 * k)) & 3) << 4)
                q = u.astype(np.int32) - 32
                for half16 in range(2):
                    s = sc[:, 8 * h + 2 * k + half16]
                    seg = slice(16 * half16, 16 * half16 + 16)
                    out[:, 128 * h + 32 * k + 16 * half16:128 * h + 32 * k + 16 * half16 + 16] = (
                        (d * s)[:, None] * q[:, seg].astype(F32))
        return out.reshape(-1)[:n]
    raise ValueError(f"type {ty}")


def int_values(ty, data):
    """Per-weight integers the integer dots use, with the 32/16-value grouping:
    Q4_K -> nibble (0..15) per value; Q6_K -> u = q + 32 (0..63);
    Q8_0 -> signed byte; Q4_0 -> nibble (0..15)."""
    if ty == 12:
        b = _blocks(data, 144)
        qs = b[:, 16:144]
        q = np.empty((b.shape[0], 256), np.int64)
        for g in range(4):
            q[:, 64 * g:64 * g + 32] = qs[:, 32 * g:32 * g + 32] & 0xF
            q[:, 64 * g + 32:64 * g + 64] = qs[:, 32 * g:32 * g + 32] >> 4
        return q.reshape(-1)
    if ty == 14:
        b = _blocks(data, 210)
        out = np.empty((b.shape[0], 256), np.int64)
        for h in range(2):
            ql = b[:, 64 * h:64 * h + 64].astype(np.int64)
            qh = b[:, 128 + 32 * h:128 + 32 * h + 32].astype(np.int64)
            nib = [ql[:, :32] & 0xF, ql[:, 32:] & 0xF, ql[:, :32] >> 4, ql[:, 32:] >> 4]
            for k in range(4):
                out[:, 128 * h + 32 * k:128 * h + 32 * k + 32] = nib[k] | (((qh >> (2 * k)) & 3) << 4)
        return out.reshape(-1)
    if ty == 8:
        return _blocks(data, 34)[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
    if ty == 2:
        b = _blocks(data, 18)[:, 2:]
        return np.concatenate([b & 0xF, b >> 4], axis=1).astype(np.int64).reshape(-1)
    raise ValueError(ty)


def quantize_q8_closed_form(x, rounding="even"):
    """Q8 activation blocks from their definition: per 32 values
    d = amax/127 (f32), inv = 1/d (0 if d == 0), q = round(x*inv) saturated
    to int8; rounding 'even' (AVX2 cvtps) or 'away' (f32::round)."""
    x = np.asarray(x, F32).reshape(-1, 32)
    amax = np.max(np.abs(x), axis=1)
    d = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv = np.where(d > 0, F32(1.0) / np.where(d > 0, d, F32(1.0)), F32(0.0)).astype(F32)
    v = (x * inv[:, None]).astype(F32)
    if rounding == "even":
        r = np.rint(v)
    else:
        r = np.sign(v) * np.floor(np.abs(v) + F32(0.5))
    q = np.clip(r, -128, 127).astype(np.int8)
    s = q.astype(np.int32).sum(axis=1)
    s16 = q.astype(np.int32).reshape(-1, 2, 16).sum(axis=2).reshape(-1)
    return q.reshape(-1), d, s.astype(np.int32), s16.astype(np.int32)
