"""An independent GGUF v2/v3 encoder and decoder (test infrastructure),
written from the published GGUF format description, not from any code:

  file     = "GGUF" u32:version u64:n_tensors u64:n_kv kv[n_kv] tinfo[n_tensors]
             pad to `alignment` tensor data
  kv       = str:key u32:type value
  value    = scalar by type (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32,
             7 bool (1 byte), 10 u64, 11 i64, 12 f64), 8 str, or 9 array =
             u32:elem_type u64:count elem[count] (elements without a tag)
  str      = u64:len bytes
  tinfo    = str:name u32:n_dims u64:dim[n_dims] u32:ggml_type u64:offset
  alignment = the u32 value of "general.alignment" if present, else 32; each
             tensor's offset is relative to the aligned start of the data.

All integers little-endian. Values are represented as (type, value) with
arrays as (9, (elem_type, [values])).
"""
import struct

SCALAR_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q",
              12: "<d"}


def _enc_str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _enc_payload(ty, v):
    if ty == 8:
        return _enc_str(v)
    if ty == 9:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_enc_payload(et, x) for x in items)
    if ty == 7:
        return struct.pack("<B", 1 if v else 0)
    return struct.pack(SCALAR_FMT[ty], v)


def encode(meta, tensors, version=3, alignment=32, sort_keys=True):
    """meta: {key: (type, value)}; tensors: [(name, ggml_type, dims, bytes)].
    Offsets are assigned in order, each aligned."""
    keys = sorted(meta, key=lambda k: k.encode()) if sort_keys else list(meta)
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for k in keys:
        ty, v = meta[k]
        out += _enc_str(k) + struct.pack("<I", ty) + _enc_payload(ty, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(data)
    for (name, ty, dims, _), o in zip(tensors, offs):
        out += _enc_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, o)
    start = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (start - len(out))
    for (_, _, _, data), o in zip(tensors, offs):
        out += b"\0" * (start + o - len(out))
        out += bytes(data)
    return bytes(out)


def decode(buf):
    """Returns (version, {key: (type, value)}, [(name, type, dims, offset)], data_start)."""
    pos = 0

    def take(n):
        nonlocal pos
        if pos + n > len(buf):
            raise ValueError("eof")
        b = buf[pos:pos + n]
        pos += n
        return b

    def scalar(ty):
        f = SCALAR_FMT[ty]
        v = struct.unpack(f, take(struct.calcsize(f)))[0]
        return bool(v) if ty == 7 else v

    def string():
        n = struct.unpack("<Q", take(8))[0]
        return take(n).decode("utf-8", "replace")

    def value(ty):
        if ty == 8:
            return string()
        if ty == 9:
            et, n = struct.unpack("<IQ", take(12))
            return (et, [value(et) for _ in range(n)])
        return scalar(ty)

    if take(4) != b"GGUF":
        raise ValueError("magic")
    version, nt, nkv = struct.unpack("<IQQ", take(20))
    meta = {}
    for _ in range(nkv):
        k = string()
        ty = struct.unpack("<I", take(4))[0]
        meta[k] = (ty, value(ty))
    infos = []
    for _ in range(nt):
        name = string()
        nd = struct.unpack("<I", take(4))[0]
        dims = [struct.unpack("<Q", take(8))[0] for _ in range(nd)]
        ty, off = struct.unpack("<IQ", take(12))
        infos.append((name, ty, dims, off))
    align = meta.get("general.alignment", (4, 32))[1]
    start = (pos + align - 1) // align * align
    return version, meta, infos, start
