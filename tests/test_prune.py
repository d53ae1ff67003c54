"""Vocabulary pruning (prune::prune_vocab, src/prune.rs:127-291):
rlh_prune_vocab against the oracle's restatement (oracle/prune_ref.py) on
synthetic GGUF files, output file against output file, byte for byte, and
the PruneStats counts. CPU only (host code).

The vocabularies mix the byte-level encodings of kept scripts (Latin,
Arabic, Greek, emoji, musical symbols and mathematical alphanumerics inside
the dropped astral range) and dropped ones (CJK, Cyrillic, Devanagari,
Hangul, Greek Extended, Linear B), UTF-8 fragments (lossy decoding keeps
them), characters outside the byte-level alphabet, every token type, tokens
named by *_token_id keys (kept whatever their script), repeated strings and
merges that do and do not survive. The script table itself is pinned by
code points at the edges of its ranges."""
import os

import numpy as np
import pytest

import prune_ref
import rlh
from golden import gguf_format as gf


def _b2u():
    direct = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    out, n = {}, 0
    for b in range(256):
        if b in direct:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + n)
            n += 1
    return out


B2U = _b2u()


def bl(text):
    """The byte-level token string of `text` (bytes_to_unicode of its UTF-8)."""
    raw = text.encode("utf-8") if isinstance(text, str) else bytes(text)
    return "".join(B2U[b] for b in raw)


KEPT = ["the", " world", "ab", "abc", " Hello", "123", "!", "سلام", "αβ",
        "\U0001F600", "\U0001D11E", "\U0001D400", "été", "�", "؀", "Ⱡ"]
DROPPED = ["中文", "при", "नम", "한", "ἀ", "\U00010000", "あ",
           "Ａ", "Ѐ", "ԯ", "\U0003FFFF", "\U0001D0FF", "\U0001D800", "a一"]


def _vocab():
    """(tokens, types, merges, metadata extras)."""
    toks, types = [], []

    def add(s, ty=1):
        toks.append(s)
        types.append(ty)
        return len(toks) - 1

    for t in KEPT:
        add(bl(t))
    for t in DROPPED:
        add(bl(t))
    add(bl(b"\xe4\xb8"))               # the first two bytes of a CJK character: lossy -> U+FFFD, kept
    add(bl(b"\x80abc"))                 # a stray continuation byte, then Latin
    add(bl(b"\xe4\xb8\xad\xe4"))        # a whole CJK character and a fragment: dropped
    add("x中y")                     # a character outside the byte-level alphabet, as its UTF-8: dropped
    add("<|im_start|>", 3)
    add("<|im_end|>", 3)
    add(bl("中国"), 4)          # user-defined CJK token: kept
    add(bl("ж"), 2)                # unknown: kept
    for b in (0x41, 0xE4, 0x0A):
        add(f"<0x{b:02X}>", 6)
    bos = add(bl("日"))             # pinned by bos_token_id although CJK
    add(bl("the"))                      # a repeated string (the map keeps the last id)
    add(bl(" "))
    add(bl("中"))
    add(bl("文"))
    eos = toks.index("<|im_end|>")
    merges = [bl("a") + " " + bl("b"), bl("ab") + " " + bl("c"), bl("中") + " " + bl("文"),
              bl(" ") + " " + bl("world"), "nospace", bl("t") + " " + bl("he"), bl("a") + " " + bl("bc"),
              bl("ab") + " " + bl("c") + " x"]
    # the single characters the merges name
    for ch in ("a", "b", "c", "t", "he", "world", "bc"):
        if bl(ch) not in toks:
            add(bl(ch))
    extra = {"tokenizer.ggml.bos_token_id": (gf_u32, bos), "tokenizer.ggml.eos_token_id": (gf_u32, eos),
             "tokenizer.ggml.padding_token_id": (gf_i32, eos),
             "tokenizer.ggml.unknown_token_id": (gf_u64, types.index(2)),
             "general.name_token_id": (gf_str, "not a number"), "general.empty": (gf_arr, (gf_i32, [])),
             "general.flag": (gf_bool, True), "general.f": (gf_f32, 0.25)}
    return toks, types, merges, extra


gf_u8, gf_i8, gf_u16, gf_i16, gf_u32, gf_i32, gf_f32, gf_bool, gf_str, gf_arr, gf_u64, gf_i64, gf_f64 = range(13)


def _write(path, toks, types, merges, extra, tensors, version=3, alignment=32, with_types=True):
    meta = {"general.architecture": (gf_str, "qwen3"), "tokenizer.ggml.model": (gf_str, "gpt2"),
            "tokenizer.ggml.tokens": (gf_arr, (gf_str, toks)),
            "tokenizer.ggml.merges": (gf_arr, (gf_str, merges))}
    if with_types:
        meta["tokenizer.ggml.token_type"] = (gf_arr, (gf_i32, types))
    if alignment != 32:
        meta["general.alignment"] = (gf_u32, alignment)
    meta.update(extra)
    with open(path, "wb") as f:
        f.write(gf.encode(meta, tensors, version=version, alignment=alignment))


def _tensors(vocab, rng):
    e = 256
    embd = rng.integers(0, 256, vocab * e // 256 * 144, dtype=np.uint8)     # Q4_K rows
    out = rng.integers(0, 256, vocab * e // 256 * 210, dtype=np.uint8)      # Q6_K rows
    norm = rng.standard_normal(e).astype(np.float32)
    other = rng.integers(0, 256, vocab * 34, dtype=np.uint8)                # Q8_0, vocab rows, another name
    return [("token_embd.weight", 12, [e, vocab], embd.tobytes()), ("output_norm.weight", 0, [e], norm.tobytes()),
            ("blk.0.ffn_gate.weight", 8, [32, vocab], other.tobytes()),
            ("output.weight", 14, [e, vocab], out.tobytes())]


def _oracle(path):
    buf = open(path, "rb").read()
    version, meta, infos, start = gf.decode(buf)
    geom = prune_ref.GEOM

    def tb(name):
        for n, ty, dims, off in infos:
            if n == name:
                cnt = int(np.prod(dims)) if dims else 1
                bs, ts = geom[ty]
                return buf[start + off:start + off + cnt // bs * ts]
        raise KeyError(name)

    m, tensors, align, stats = prune_ref.prune(meta, [(n, ty, d) for n, ty, d, _ in infos], tb)
    return gf.encode(m, tensors, version=version, alignment=align), stats


@pytest.mark.parametrize("version,alignment", [(3, 32), (2, 64)])
def test_prune_matches_oracle_file_bytes(tmp_path, version, alignment):
    toks, types, merges, extra = _vocab()
    rng = np.random.default_rng(version)
    src = tmp_path / "in.gguf"
    _write(src, toks, types, merges, extra, _tensors(len(toks), rng), version, alignment)
    dst = tmp_path / "out.gguf"
    st = rlh.prune_vocab(src, dst)
    want, wst = _oracle(src)
    got = open(dst, "rb").read()
    assert got == want
    for k, v in wst.items():
        assert st[k] == v, k
    assert st["out_bytes"] == os.path.getsize(dst) == len(want)
    # the classification itself: every KEPT string kept, every DROPPED string dropped
    _, meta, _, _ = gf.decode(got)
    kept = set(meta["tokenizer.ggml.tokens"][1][1])
    for t in KEPT:
        assert bl(t) in kept, t
    for t in DROPPED:
        assert bl(t) not in kept, t
    assert st["kept_special"] == 3 and st["kept_byte"] == 3 and st["dropped"] == len(DROPPED) + 4
    # the bos token (CJK) survived and every *_token_id names its old token
    new_toks = meta["tokenizer.ggml.tokens"][1][1]
    for key in ("tokenizer.ggml.bos_token_id", "tokenizer.ggml.eos_token_id", "tokenizer.ggml.padding_token_id",
                "tokenizer.ggml.unknown_token_id"):
        ty, nid = meta[key]
        assert ty == gf_u32 and new_toks[nid] == toks[extra[key][1]]
    assert meta["general.name_token_id"] == (gf_str, "not a number")
    assert meta["general.empty"] == (gf_arr, (gf_str, []))  # an empty array takes the string tag
    merged = meta["tokenizer.ggml.merges"][1][1]
    assert bl("a") + " " + bl("b") in merged and bl("中") + " " + bl("文") not in merged
    assert "nospace" not in merged


def test_prune_row_slices_and_reload(tmp_path):
    """token_embd and output keep exactly the kept tokens' rows; a tensor
    with one row per token but another name is copied whole; the output
    reads back through the product's own reader."""
    toks, types, merges, extra = _vocab()
    rng = np.random.default_rng(5)
    ts = _tensors(len(toks), rng)
    src = tmp_path / "in.gguf"
    _write(src, toks, types, merges, extra, ts)
    dst = tmp_path / "out.gguf"
    st = rlh.prune_vocab(src, dst)
    with rlh.Gguf(dst) as g:
        kept = g.meta("tokenizer.ggml.tokens")
        keep_ids = []
        seen = {}
        for i, t in enumerate(toks):
            seen.setdefault(t, []).append(i)
        # kept ids in order: walk the old vocabulary, matching the new list
        j = 0
        for i, t in enumerate(toks):
            if j < len(kept) and kept[j] == t:
                keep_ids.append(i)
                j += 1
        assert len(keep_ids) == st["new_vocab"] == len(kept)
        embd = np.frombuffer(ts[0][3], np.uint8).reshape(len(toks), 144)
        out = np.frombuffer(ts[3][3], np.uint8).reshape(len(toks), 210)
        assert np.array_equal(g.tensor_bytes("token_embd.weight").reshape(-1, 144), embd[keep_ids])
        assert np.array_equal(g.tensor_bytes("output.weight").reshape(-1, 210), out[keep_ids])
        assert g.tensor_bytes("blk.0.ffn_gate.weight").tobytes() == ts[2][3]
        assert st["embd_bytes_saved"] == (len(toks) - len(kept)) * (144 + 210)


def test_prune_without_token_types_and_merges(tmp_path):
    """No token_type key (every token normal) and no merges key (the output
    gets an empty merges array)."""
    toks, types, merges, extra = _vocab()
    rng = np.random.default_rng(9)
    src = tmp_path / "in.gguf"
    _write(src, toks, types, [], {"tokenizer.ggml.bos_token_id": (gf_u32, 3)}, _tensors(len(toks), rng),
           with_types=False)
    dst = tmp_path / "out.gguf"
    st = rlh.prune_vocab(src, dst)
    want, wst = _oracle(src)
    assert open(dst, "rb").read() == want
    assert st["kept_special"] == 0 and st["kept_byte"] == 0 and st["merges_old"] == 0


def test_prune_errors(tmp_path):
    """The reference's InvalidData cases: no vocabulary, a token_type array
    of another length, an id key beyond the vocabulary, everything dropped."""
    rng = np.random.default_rng(1)
    toks, types, merges, extra = _vocab()
    lib = rlh.load()
    cases = [
        ({"tokenizer.ggml.tokens": (gf_arr, (gf_i32, [1, 2]))}, b"tokenizer.ggml.tokens"),
        ({"tokenizer.ggml.token_type": (gf_arr, (gf_i32, [1]))}, b"length mismatch"),
        ({"tokenizer.ggml.eos_token_id": (gf_u32, 10 ** 6)}, b"was pruned"),
    ]
    for i, (over, msg) in enumerate(cases):
        src = tmp_path / f"bad{i}.gguf"
        _write(src, toks, types, merges, dict(extra, **over), _tensors(len(toks), rng))
        with pytest.raises(rlh.RlhError) as e:
            rlh.prune_vocab(src, tmp_path / "o.gguf")
        assert e.value.code == rlh.RLH_EFORMAT and msg in lib.rlh_last_error(), msg
        with pytest.raises(ValueError):
            _oracle(src)
    cjk = [bl(t) for t in DROPPED]
    src = tmp_path / "allcjk.gguf"
    _write(src, cjk, [1] * len(cjk), [], {}, _tensors(len(cjk), rng))
    with pytest.raises(rlh.RlhError) as e:
        rlh.prune_vocab(src, tmp_path / "o.gguf")
    assert b"entire vocabulary" in lib.rlh_last_error()
    with pytest.raises(rlh.RlhError) as e:
        rlh.prune_vocab(tmp_path / "missing.gguf", tmp_path / "o.gguf")
    assert e.value.code == rlh.RLH_EIO


def test_script_table_edges():
    """Code points at both edges of every dropped range (and one past them)
    and of the kept astral blocks, through a one-token vocabulary each:
    kept exactly when the oracle's table keeps it."""
    pts = set()
    for a, b in prune_ref.DROP_RANGES + prune_ref.KEEP_ASTRAL:
        pts.update((a - 1, a, b, b + 1))
    pts = sorted(p for p in pts if 0 < p < 0x110000 and not 0xD800 <= p <= 0xDFFF)
    toks = ["<|x|>"] + [bl(chr(p)) for p in pts]
    types = [3] + [1] * len(pts)
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        src, dst = os.path.join(d, "in.gguf"), os.path.join(d, "out.gguf")
        _write(src, toks, types, [], {}, [])
        rlh.prune_vocab(src, dst)
        _, meta, _, _ = gf.decode(open(dst, "rb").read())
    kept = set(meta["tokenizer.ggml.tokens"][1][1])
    for p in pts:
        assert (bl(chr(p)) in kept) == (not prune_ref.char_dropped(p)), hex(p)
    # a few fixed points of the reference's table
    assert prune_ref.char_dropped(0x4E00) and prune_ref.char_dropped(0x0400)
    assert not prune_ref.char_dropped(0x0600) and not prune_ref.char_dropped(0x1D11E)
    assert not prune_ref.char_dropped(0x03B1) and prune_ref.char_dropped(0x1F00)
