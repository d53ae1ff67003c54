"""GGUF reader and writer of librlh (GgufFile, src/gguf.rs; write_gguf,
src/prune.rs:381-442; Model::read_config, src/model.rs:241-293) against an
independent encoder/decoder written from the format description
(tests/golden/gguf_format.py). CPU only."""
import ctypes
import math
import os
import struct
import time

import numpy as np
import pytest

import rlh
from golden import gguf_format as gf

META = {
    "general.architecture": (rlh.GGUF_STR, "qwen3"),
    "a.u8": (rlh.GGUF_U8, 200), "a.i8": (rlh.GGUF_I8, -5), "a.u16": (rlh.GGUF_U16, 60000),
    "a.i16": (rlh.GGUF_I16, -300), "a.u32": (rlh.GGUF_U32, 4000000000), "a.i32": (rlh.GGUF_I32, -7),
    "a.f32": (rlh.GGUF_F32, 1.5), "a.bool": (rlh.GGUF_BOOL, True), "a.u64": (rlh.GGUF_U64, 2 ** 40 + 3),
    "a.i64": (rlh.GGUF_I64, -(2 ** 40)), "a.f64": (rlh.GGUF_F64, 0.1), "a.str": (rlh.GGUF_STR, "héllo"),
    "a.arr_str": (rlh.GGUF_ARR, (rlh.GGUF_STR, ["x", "", "yz"])),
    "a.arr_i32": (rlh.GGUF_ARR, (rlh.GGUF_I32, [1, -2, 3])),
    "a.arr_empty": (rlh.GGUF_ARR, (rlh.GGUF_F32, [])),
}


def _tensors(rng):
    return [("w0", rlh.Q4_K, [512, 3], rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8)),
            ("norm", rlh.F32, [7], rng.standard_normal(7).astype(np.float32).view(np.uint8)),
            ("w1", rlh.Q8_0, [64, 2], rng.integers(0, 256, 2 * 2 * 34, dtype=np.uint8)),
            ("e", rlh.F16, [0], np.zeros(0, np.uint8))]


def test_writer_matches_independent_encoder(tmp_path):
    """Same bytes as the independent encoder: keys in byte order, aligned
    tensor offsets, aligned data section."""
    rng = np.random.default_rng(1)
    ts = _tensors(rng)
    for version, align in ((3, 32), (2, 64)):
        p = tmp_path / f"w{version}.gguf"
        rlh.write_gguf(p, META, ts, version=version, alignment=align)
        want = gf.encode(META, [(n, t, d, b.tobytes()) for n, t, d, b in ts], version=version, alignment=align)
        assert p.read_bytes() == want


def test_round_trip_through_reader(tmp_path):
    rng = np.random.default_rng(2)
    ts = _tensors(rng)
    p = tmp_path / "rt.gguf"
    rlh.write_gguf(p, META, ts)
    with rlh.Gguf(p) as g:
        assert g.version == 3 and g.n_files == 1
        assert g.keys() == sorted(META, key=lambda k: k.encode())
        for k, (ty, v) in META.items():
            got = g.meta(k)
            assert g.meta_type(k)[0] == ty
            if ty == rlh.GGUF_ARR:
                assert got == list(v[1]) and g.meta_type(k)[1] == v[0]
            elif ty == rlh.GGUF_F32:
                assert got == np.float32(v)
            else:
                assert got == v, k
        infos = g.tensors()
        assert [(n, t, d) for n, t, d, _, _ in infos] == [(n, t, d) for n, t, d, _ in ts]
        for n, _, _, b in ts:
            assert np.array_equal(g.tensor_bytes(n), b)
        with pytest.raises(rlh.RlhError) as e:
            g.tensor_bytes("nope")
        assert e.value.code == rlh.RLH_ENOENT
        with pytest.raises(rlh.RlhError) as e:
            g.meta("missing.key")
        assert e.value.code == rlh.RLH_ENOENT


def test_reader_parses_independent_file(tmp_path):
    """A file from the independent encoder with general.alignment 128 and keys
    in insertion order (a reader must not assume sorted keys)."""
    rng = np.random.default_rng(3)
    ts = [(n, t, d, b.tobytes()) for n, t, d, b in _tensors(rng)]
    meta = dict(META)
    meta["general.alignment"] = (rlh.GGUF_U32, 128)
    raw = gf.encode(meta, ts, version=2, alignment=128, sort_keys=False)
    p = tmp_path / "ind.gguf"
    p.write_bytes(raw)
    _, _, infos, start = gf.decode(raw)
    with rlh.Gguf(p) as g:
        assert g.version == 2
        assert g.keys() == list(meta)
        for (n, t, d, off), (gn, gt, gd, goff, gfi) in zip(infos, g.tensors()):
            assert (n, t, d, off, 0) == (gn, gt, gd, goff, gfi)
        for n, _, _, b in ts:
            assert g.tensor_bytes(n).tobytes() == b


def test_as_u32_and_as_f32_conversions(tmp_path):
    """MetaValue::as_u32 / as_f32 (gguf.rs:32-56): Rust `as` conversions."""
    meta = {"i8": (rlh.GGUF_I8, -1), "i64": (rlh.GGUF_I64, -(2 ** 33) + 5), "u64": (rlh.GGUF_U64, 2 ** 32 + 9),
            "f64": (rlh.GGUF_F64, 0.1), "b": (rlh.GGUF_BOOL, True), "s": (rlh.GGUF_STR, "7")}
    p = tmp_path / "c.gguf"
    rlh.write_gguf(p, meta, [])
    lib = rlh.load()
    with rlh.Gguf(p) as g:
        v = ctypes.c_uint32()
        for k, want in (("i8", 0xFFFFFFFF), ("i64", (-(2 ** 33) + 5) & 0xFFFFFFFF), ("u64", 9)):
            assert lib.rlh_gguf_meta_u32(g.h, k.encode(), ctypes.byref(v)) == 0 and v.value == want
        for k in ("f64", "b", "s"):
            assert lib.rlh_gguf_meta_u32(g.h, k.encode(), ctypes.byref(v)) == rlh.RLH_EINVAL
        f = ctypes.c_float()
        assert lib.rlh_gguf_meta_f32(g.h, b"f64", ctypes.byref(f)) == 0 and f.value == np.float32(0.1)
        assert lib.rlh_gguf_meta_f32(g.h, b"i8", ctypes.byref(f)) == rlh.RLH_EINVAL


def _open_code(path):
    h = ctypes.c_void_p()
    lib = rlh.load()
    rc = lib.rlh_gguf_open(os.fsencode(path), ctypes.byref(h))
    if rc == 0:
        lib.rlh_gguf_close(h)
    return rc, lib.rlh_last_error().decode()


def test_malformed_inputs_fail_without_abort(tmp_path):
    """gguf.rs:433-464 (empty file, absurd counts failing fast, an absurd
    string length) plus bad magic, other versions, unknown value and tensor
    types, deep nesting, truncation inside the tensor table, and a missing
    file."""
    cases = {
        "empty": b"",
        "huge": b"GGUF" + struct.pack("<IQQ", 3, 2 ** 64 - 1, 2 ** 64 - 1),
        "trunc_key": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2 ** 64 - 1),
        "magic": b"GGUX" + struct.pack("<IQQ", 3, 0, 0),
        "v1": b"GGUF" + struct.pack("<IQQ", 1, 0, 0),
        "v4": b"GGUF" + struct.pack("<IQQ", 4, 0, 0),
        "value_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf._enc_str("k") + struct.pack("<I", 13),
        "elem_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf._enc_str("k") + struct.pack("<IIQ", 9, 77, 1),
        "huge_array": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf._enc_str("k") + struct.pack("<IIQ", 9, 0, 2 ** 62),
        "nested": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf._enc_str("k")
                  + struct.pack("<I", 9) + struct.pack("<IQ", 9, 1) * 20 + struct.pack("<IQ", 0, 0),
        "tensor_type": gf.encode({}, [("t", 99, [32], b"")]),
        "tensor_trunc": gf.encode({}, [("t", 0, [4], b"\0" * 16)])[:40],
    }
    for name, raw in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(raw)
        t0 = time.time()
        rc, msg = _open_code(p)
        assert rc == rlh.RLH_EFORMAT, (name, rc, msg)
        assert time.time() - t0 < 10, name
        assert msg.startswith("gguf:"), (name, msg)
    assert _open_code(tmp_path / "does-not-exist.gguf")[0] == rlh.RLH_EIO


def test_tensor_out_of_range(tmp_path):
    """A tensor whose offset or size runs past the end of the file: the
    table parses, its bytes do not (tensor_bytes_info, gguf.rs:405-413)."""
    raw = gf.encode({}, [("a", rlh.F32, [4], np.arange(4, dtype=np.float32).tobytes())])
    p = tmp_path / "oor.gguf"
    p.write_bytes(raw[:-4])
    with rlh.Gguf(p) as g:
        with pytest.raises(rlh.RlhError) as e:
            g.tensor_bytes("a")
        assert e.value.code == rlh.RLH_EFORMAT


def test_split_files(tmp_path):
    """split.count > 1: the siblings named -0000k-of-0000n.gguf are opened
    and their tensors resolved (gguf.rs:259-293); a missing sibling is
    skipped as the reference skips it."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal(8).astype(np.float32)
    b = rng.standard_normal(16).astype(np.float32)
    c = rng.standard_normal(4).astype(np.float32)
    base = tmp_path / "m"
    rlh.write_gguf(f"{base}-00001-of-00003.gguf", {"split.count": (rlh.GGUF_U16, 3)}, [("a", rlh.F32, [8], a)])
    rlh.write_gguf(f"{base}-00002-of-00003.gguf", {"split.count": (rlh.GGUF_U16, 3)}, [("b", rlh.F32, [16], b)])
    with rlh.Gguf(f"{base}-00001-of-00003.gguf") as g:
        assert g.n_files == 2
        assert [t[0] for t in g.tensors()] == ["a", "b"]
        assert [t[4] for t in g.tensors()] == [0, 1]
        assert np.array_equal(g.tensor_bytes("b").view(np.float32), b)
    rlh.write_gguf(f"{base}-00003-of-00003.gguf", {}, [("c", rlh.F32, [4], c)])
    with rlh.Gguf(f"{base}-00001-of-00003.gguf") as g:
        assert g.n_files == 3
        assert np.array_equal(g.tensor_bytes("c").view(np.float32), c)


def _config_of(tmp_path, meta, tensors=None):
    p = tmp_path / "cfg.gguf"
    rlh.write_gguf(p, meta, tensors or [("token_embd.weight", rlh.F32, [4, 11], np.zeros(44, np.float32))])
    with rlh.Gguf(p) as g:
        return g.config()


def test_read_config_keys_and_defaults(tmp_path):
    """Model::read_config (model.rs:241-293): "{arch}.{key}" first, then the
    bare key; defaults for head_count_kv (head_count), key_length
    (embedding_length / head_count), rope theta 10000, eps 1e-5, context
    4096; vocab = rows of token_embd; QK-norm and output from the tensors."""
    meta = {"general.architecture": (rlh.GGUF_STR, "qwen3"), "qwen3.block_count": (rlh.GGUF_U32, 2),
            "qwen3.embedding_length": (rlh.GGUF_U64, 512), "feed_forward_length": (rlh.GGUF_I32, 768),
            "qwen3.attention.head_count": (rlh.GGUF_U32, 4)}
    c, arch = _config_of(tmp_path, meta)
    assert arch == "qwen3"
    assert (c.n_layer, c.n_embd, c.n_ff, c.n_head, c.n_head_kv, c.head_dim) == (2, 512, 768, 4, 4, 128)
    assert c.rope_theta == 10000.0 and c.rms_eps == np.float32(1e-5) and c.n_ctx == 4096
    assert c.vocab_size == 11 and c.has_qk_norm == 0 and c.has_output == 0
    meta.update({"qwen3.attention.head_count_kv": (rlh.GGUF_U32, 2), "qwen3.attention.key_length": (rlh.GGUF_U32, 64),
                 "qwen3.rope.freq_base": (rlh.GGUF_F64, 1e6), "qwen3.context_length": (rlh.GGUF_U32, 40960),
                 "qwen3.attention.layer_norm_rms_epsilon": (rlh.GGUF_F32, 1e-6),
                 "feed_forward_length": (rlh.GGUF_I32, 1), "qwen3.feed_forward_length": (rlh.GGUF_U32, 1024)})
    ts = [("token_embd.weight", rlh.F32, [4, 3], np.zeros(12, np.float32)),
          ("blk.0.attn_q_norm.weight", rlh.F32, [4], np.zeros(4, np.float32)),
          ("output.weight", rlh.F32, [4, 3], np.zeros(12, np.float32))]
    c, _ = _config_of(tmp_path, meta, ts)
    assert (c.n_ff, c.n_head_kv, c.head_dim, c.n_ctx) == (1024, 2, 64, 40960)
    assert c.rope_theta == 1e6 and c.rms_eps == np.float32(1e-6)
    assert c.vocab_size == 3 and c.has_qk_norm == 1 and c.has_output == 1


def test_architecture_gate_and_missing_keys(tmp_path):
    """check_arch (model.rs:794-808): qwen3 and qwen2 only (no architecture
    key means "llama", refused); a missing required key is an error."""
    base = {"qwen2.block_count": (rlh.GGUF_U32, 1), "qwen2.embedding_length": (rlh.GGUF_U32, 256),
            "qwen2.feed_forward_length": (rlh.GGUF_U32, 256), "qwen2.attention.head_count": (rlh.GGUF_U32, 2)}
    c, arch = _config_of(tmp_path, dict(base, **{"general.architecture": (rlh.GGUF_STR, "qwen2")}))
    assert arch == "qwen2" and c.n_layer == 1
    for a in ("llama", "mistral", "gemma", ""):
        with pytest.raises(rlh.RlhError) as e:
            _config_of(tmp_path, dict(base, **{"general.architecture": (rlh.GGUF_STR, a)}))
        assert e.value.code == rlh.RLH_EUNSUP
    with pytest.raises(rlh.RlhError) as e:
        _config_of(tmp_path, base)  # defaults to "llama"
    assert e.value.code == rlh.RLH_EUNSUP and b"'llama'" in rlh.load().rlh_last_error()
    bad = dict(base, **{"general.architecture": (rlh.GGUF_STR, "qwen2")})
    del bad["qwen2.embedding_length"]
    with pytest.raises(rlh.RlhError) as e:
        _config_of(tmp_path, bad)
    assert e.value.code == rlh.RLH_EFORMAT and b"embedding_length" in rlh.load().rlh_last_error()


def _qwen2_meta(n_embd, n_ff, n_head, n_head_kv, key_length=None):
    m = {"general.architecture": (rlh.GGUF_STR, "qwen2"), "qwen2.block_count": (rlh.GGUF_U32, 1),
         "qwen2.embedding_length": (rlh.GGUF_U32, n_embd), "qwen2.feed_forward_length": (rlh.GGUF_U32, n_ff),
         "qwen2.attention.head_count": (rlh.GGUF_U32, n_head),
         "qwen2.attention.head_count_kv": (rlh.GGUF_U32, n_head_kv),
         "tokenizer.ggml.tokens": (rlh.GGUF_ARR, (rlh.GGUF_STR, ["a", "b", "c"]))}
    if key_length is not None:
        m["qwen2.attention.key_length"] = (rlh.GGUF_U32, key_length)
    return m


@pytest.mark.parametrize("shape,reason", [
    ((896, 4864, 14, 2, None), b"head_dim 64"),      # Qwen2.5-0.5B: head_dim 896 / 14
    ((1024, 3072, 16, 8, 64), b"head_dim 64"),       # key_length given explicitly
    ((2048, 5000, 16, 2, 128), b"multiples of 256"),  # n_ff not a multiple of 256
    ((1152, 3072, 9, 3, 128), b"multiples of 256"),   # n_embd 1152 = 4.5 x 256
    ((2048, 4096, 16, 1, 128), b"more than 8 query heads")])
def test_unsupported_shapes_refused_before_upload(tmp_path, shape, reason):
    """Shapes Model::read_config accepts (model.rs:249-268: any head_dim;
    rows of any whole number of blocks, tensor.rs:28-30) but this path does
    not run are refused by rlh_config_check, which rlh_model_load_gguf
    applies right after reading the config: RLH_EUNSUP with the reason,
    before the vocabulary or any tensor is read and before a device is
    needed (this test runs without a GPU). The config itself still reads."""
    n_embd, n_ff, n_head, n_head_kv, kl = shape
    meta = _qwen2_meta(n_embd, n_ff, n_head, n_head_kv, kl)
    p = tmp_path / "shape.gguf"
    rlh.write_gguf(p, meta, [("token_embd.weight", rlh.F32, [4, 3], np.zeros(12, np.float32))])
    lib = rlh.load()
    with rlh.Gguf(p) as g:
        c, arch = g.config()
        assert arch == "qwen2" and c.n_embd == n_embd and c.head_dim == (kl or n_embd // n_head)
        assert lib.rlh_config_check(ctypes.byref(c)) == rlh.RLH_EUNSUP
        assert reason in lib.rlh_last_error()
        h = ctypes.c_void_p()
        assert lib.rlh_model_load_gguf(g.h, ctypes.byref(h)) == rlh.RLH_EUNSUP
        assert reason in lib.rlh_last_error() and not h.value
        hm = ctypes.c_void_p()
        assert lib.rlh_model_create(ctypes.byref(c), ctypes.byref(hm)) == rlh.RLH_EUNSUP and not hm.value


def test_supported_shapes_pass_config_check():
    """Every benchmark model and every test spec passes rlh_config_check, and
    the checks on zero dimensions and head divisibility come first."""
    lib = rlh.load()
    for name, spec in rlh.SPECS.items():
        c = spec.config()
        assert lib.rlh_config_check(ctypes.byref(c)) == rlh.RLH_OK, (name, lib.rlh_last_error())
    c = rlh.SPECS["tiny-q4km"].config()
    c.n_head_kv = 3
    assert lib.rlh_config_check(ctypes.byref(c)) == rlh.RLH_EINVAL
    c.n_head_kv = 0
    assert lib.rlh_config_check(ctypes.byref(c)) == rlh.RLH_EINVAL
    assert lib.rlh_config_check(None) == rlh.RLH_EINVAL


def test_synthetic_model_file(tmp_path):
    """A seeded synthetic model written as a Qwen3 GGUF: the config it
    resolves is the spec's, every tensor is found by its GGUF name with the
    same bytes, and loading without the vocabulary fails as read_tokenizer
    does (model.rs:295-300)."""
    spec = rlh.SPECS["tiny-q4km-untied"]
    tensors = rlh.synth_model(spec, 9)
    p = tmp_path / "tiny.gguf"
    rlh.write_model_gguf(p, spec, tensors)
    with rlh.Gguf(p) as g:
        c, arch = g.config()
        assert arch == "qwen3"
        want = spec.config()
        for f, _ in rlh.Config._fields_:
            assert getattr(c, f) == getattr(want, f), f
        names = {t[0]: t for t in g.tensors()}
        for kind, layer, ty, cols, rows, buf in tensors:
            n = rlh.gguf_tensor_name(kind, layer)
            assert names[n][1] == ty
            assert np.array_equal(g.tensor_bytes(n), buf)
        assert len(g.meta("tokenizer.ggml.tokens")) == spec.vocab
    meta = rlh.model_gguf_meta(spec)
    del meta["tokenizer.ggml.tokens"]
    p2 = tmp_path / "novocab.gguf"
    rlh.write_gguf(p2, meta, rlh.model_gguf_tensors(tensors))
    lib = rlh.load()
    with rlh.Gguf(p2) as g:
        h = ctypes.c_void_p()
        assert lib.rlh_model_load_gguf(g.h, ctypes.byref(h)) == rlh.RLH_EFORMAT
        assert b"tokenizer.ggml.tokens" in lib.rlh_last_error()


def test_writer_argument_checks(tmp_path):
    lib = rlh.load()
    w = ctypes.c_void_p()
    assert lib.rlh_gguf_writer_create(1, 32, ctypes.byref(w)) == rlh.RLH_EINVAL
    assert lib.rlh_gguf_writer_create(3, 32, ctypes.byref(w)) == 0
    try:
        assert lib.rlh_gguf_writer_set_array(w, b"k", rlh.GGUF_ARR, None, 0) == rlh.RLH_EINVAL
        assert b"nested arrays" in lib.rlh_last_error()
        dims = np.array([256, 2], np.uint64)
        data = np.zeros(100, np.uint8)  # a 2 x 256 Q4_K tensor needs 288 bytes
        assert lib.rlh_gguf_writer_add_tensor(w, b"t", rlh.Q4_K, 2, dims.ctypes.data, data.ctypes.data, 100) \
            == rlh.RLH_EINVAL
        assert lib.rlh_gguf_writer_write(w, os.fsencode(tmp_path / "no" / "such" / "dir.gguf")) == rlh.RLH_EIO
    finally:
        lib.rlh_gguf_writer_destroy(w)
