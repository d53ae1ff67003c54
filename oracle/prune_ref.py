"""CPU restatement of the reference's vocabulary pruning (prune::prune_vocab,
src/prune.rs:127-291) — test infrastructure only: the parity tests compare
librlh's rlh_prune_vocab with it, output file against output file. Nothing in
the product imports it.

It works on a decoded GGUF in the plain representation of
tests/golden/gguf_format.py: metadata {key: (type, value)} with arrays as
(9, (element type, [values])), tensor infos [(name, ggml type, dims)] in file
order and a function returning a tensor's bytes. It returns the metadata and
tensors of the pruned file (for gguf_format.encode) and the PruneStats
counts.
"""

# Scripts dropped (prune.rs:39-90) and the notation blocks kept inside them
# (prune.rs:94): the reference's table.
DROP_RANGES = [
    (0x0400, 0x052F), (0x0530, 0x058F), (0x0590, 0x05FF), (0x0700, 0x07FF), (0x0800, 0x089F),
    (0x0900, 0x0DFF), (0x0E00, 0x0EFF), (0x0F00, 0x0FFF), (0x1000, 0x109F), (0x10A0, 0x10FF),
    (0x1100, 0x11FF), (0x1200, 0x139F), (0x13A0, 0x13FF), (0x1400, 0x167F), (0x1680, 0x16FF),
    (0x1700, 0x18FF), (0x1900, 0x1DFF), (0x1F00, 0x1FFF), (0x2C00, 0x2C5F), (0x2C80, 0x2CFF),
    (0x2D00, 0x2D7F), (0x2D80, 0x2DDF), (0x2DE0, 0x2DFF), (0x2E80, 0x2FFF), (0x3000, 0x303F),
    (0x3040, 0x30FF), (0x3100, 0x312F), (0x3130, 0x318F), (0x3190, 0x31FF), (0x3200, 0x33FF),
    (0x3400, 0x4DBF), (0x4DC0, 0x4DFF), (0x4E00, 0x9FFF), (0xA000, 0xA71F), (0xA800, 0xAFFF),
    (0xAB00, 0xAB2F), (0xAB70, 0xABFF), (0xAC00, 0xD7FF), (0xF900, 0xFAFF), (0xFE30, 0xFE4F),
    (0xFE50, 0xFE6F), (0xFF00, 0xFFEF), (0x10000, 0x1D0FF), (0x1D200, 0x1D3FF), (0x1D800, 0x1EFFF),
    (0x20000, 0x2FFFF), (0x30000, 0x3FFFF),
]
KEEP_ASTRAL = [(0x1D100, 0x1D1FF), (0x1D400, 0x1D7FF)]

# GGUF value types (gguf.rs:204-235) and ggml block geometry (quant.rs:44-66)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GEOM = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
        12: (256, 144), 13: (256, 176), 14: (256, 210)}


def char_dropped(cp):
    """char_dropped (prune.rs:96-102)."""
    if any(a <= cp <= b for a, b in KEEP_ASTRAL):
        return False
    return any(a <= cp <= b for a, b in DROP_RANGES)


def _unicode_to_byte():
    """The inverse of bytes_to_unicode (tokenizer.rs:7-32): printable Latin-1
    bytes stand for themselves, the other 68 bytes for 256, 257, ... in
    byte order."""
    direct = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    out, n = {}, 0
    for b in range(256):
        if b in direct:
            out[chr(b)] = b
        else:
            out[chr(256 + n)] = b
            n += 1
    return out


_U2B = _unicode_to_byte()


def decode_token_bytes(s):
    """decode_token_bytes (tokenizer.rs:362-383): a character of the
    byte-level alphabet is its byte, any other character its UTF-8 bytes."""
    out = bytearray()
    for ch in s:
        b = _U2B.get(ch)
        if b is not None:
            out.append(b)
        else:
            out += ch.encode("utf-8")
    return bytes(out)


def surface_kept(token):
    """surface_kept (prune.rs:104-108): the token's bytes read as lossy UTF-8
    hold no character of a dropped script."""
    text = decode_token_bytes(token).decode("utf-8", "replace")
    return not any(char_dropped(ord(c)) for c in text)


def as_u32(tv):
    """MetaValue::as_u32 (gguf.rs:32-44): integer types with Rust's `as`."""
    ty, v = tv
    if ty in (U8, I8, U16, I16, U32, I32, U64, I64):
        return int(v) & 0xFFFFFFFF
    return None


def as_string_vec(tv):
    """MetaValue::as_string_vec (gguf.rs:82-89)."""
    if tv is None or tv[0] != ARR:
        return None
    et, items = tv[1]
    if et != STR:
        return None
    return list(items)


def prune(meta, infos, tensor_bytes):
    """prune_vocab (prune.rs:127-291) on a decoded file. Returns (meta,
    tensors, alignment, stats) of the output, tensors as (name, type, dims,
    bytes); raises ValueError("prune: ...") where the reference returns its
    InvalidData errors."""
    def bad(msg):
        return ValueError("prune: " + msg)

    tokens = as_string_vec(meta.get("tokenizer.ggml.tokens"))
    if tokens is None:
        raise bad("tokenizer.ggml.tokens")
    tt = meta.get("tokenizer.ggml.token_type")
    if tt is not None and tt[0] == ARR:
        et, items = tt[1]
        types = [as_u32((et, x)) if as_u32((et, x)) is not None else 1 for x in items]
    else:
        types = [1] * len(tokens)
    merges = as_string_vec(meta.get("tokenizer.ggml.merges")) or []
    if len(types) != len(tokens):
        raise bad("tokenizer.ggml.token_type length mismatch")
    vocab = len(tokens)

    pinned = [False] * vocab
    for key, tv in meta.items():
        if key.endswith("_token_id"):
            i = as_u32(tv)
            if i is not None and i < vocab:
                pinned[i] = True

    keep = [False] * vocab
    stats = dict(kept_special=0, kept_byte=0, kept_normal=0)
    for i, t in enumerate(tokens):
        ty = types[i]
        if ty in (2, 3, 4, 6) or pinned[i]:
            keep[i] = True
            if ty in (3, 4):
                stats["kept_special"] += 1
            elif ty == 6:
                stats["kept_byte"] += 1
            else:
                stats["kept_normal"] += 1
        elif surface_kept(t):
            keep[i] = True
            stats["kept_normal"] += 1
    new_vocab = sum(keep)
    if new_vocab == 0:
        raise bad("prune would remove the entire vocabulary")
    new_id, nxt = [None] * vocab, 0
    for i in range(vocab):
        if keep[i]:
            new_id[i] = nxt
            nxt += 1

    old_to_id = {}
    for i, t in enumerate(tokens):
        old_to_id[t] = i  # a repeated string keeps its last id
    merges_new = []
    for m in merges:
        if " " not in m:
            continue
        l, r = m.split(" ", 1)
        li, ri, mi = old_to_id.get(l), old_to_id.get(r), old_to_id.get(l + r)
        if li is not None and ri is not None and mi is not None and keep[li] and keep[ri] and keep[mi]:
            merges_new.append(m)

    out = {}
    for key, (ty, v) in meta.items():
        if ty == ARR:
            et, items = v
            if et == ARR and items:
                raise bad("nested arrays are not supported by the writer")
            if not items:
                et = STR  # an empty array is written with the string tag
            v = (et, items)
        out[key] = (ty, v)
    out["tokenizer.ggml.tokens"] = (ARR, (STR, [t for i, t in enumerate(tokens) if keep[i]]))
    out["tokenizer.ggml.token_type"] = (ARR, (I32, [_i32(types[i]) for i in range(vocab) if keep[i]]))
    out["tokenizer.ggml.merges"] = (ARR, (STR, merges_new))
    for key, tv in meta.items():
        if key.endswith("_token_id"):
            i = as_u32(tv)
            if i is None:
                continue
            if i >= vocab or new_id[i] is None:
                raise bad(f"special token id {i} ('{key}') was pruned")
            out[key] = (U32, new_id[i])

    tensors, saved = [], 0
    for name, ty, dims in infos:
        data = tensor_bytes(name)
        rows = 1
        for d in dims[1:]:
            rows *= d
        cols = dims[0] if dims else 1
        if name in ("token_embd.weight", "output.weight") and rows == vocab:
            bs, ts = GEOM[ty]
            rb = cols // bs * ts
            sliced = b"".join(data[i * rb:(i + 1) * rb] for i in range(vocab) if keep[i])
            saved += len(data) - len(sliced)
            tensors.append((name, ty, [cols, new_vocab], sliced))
        else:
            tensors.append((name, ty, list(dims), data))
    align = as_u32(meta["general.alignment"]) if "general.alignment" in meta else None
    stats.update(old_vocab=vocab, new_vocab=new_vocab, dropped=vocab - new_vocab, merges_old=len(merges),
                 merges_new=len(merges_new), embd_bytes_saved=saved)
    return out, tensors, 32 if align is None else align, stats


def _i32(u):
    """`u32 as i32`."""
    u &= 0xFFFFFFFF
    return u - (1 << 32) if u >= 1 << 31 else u
