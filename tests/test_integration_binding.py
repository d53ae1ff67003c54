"""The Rust FFI binding in the repository's integration guide mirrors
include/rlh.h one to one: the same entry points, each with the same
parameter count and order, parameter types and return type under the C ->
Rust type mapping of std::os::raw. CPU only (the binding text is not
compiled here: no Rust toolchain)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

C_SCALARS = {"int": "c_int", "uint32_t": "u32", "uint64_t": "u64", "int32_t": "i32", "int8_t": "i8", "int64_t": "i64",
             "float": "f32", "double": "f64", "char": "c_char", "void": "c_void",
             "rlh_config": "RlhConfig", "rlh_model": "RlhModel", "rlh_cache": "RlhCache",
             "rlh_sampling_params": "RlhSamplingParams", "rlh_gguf": "RlhGguf", "rlh_prune_stats": "RlhPruneStats",
             "rlh_gguf_writer": "RlhGgufWriter", "rlh_tokenizer": "RlhTokenizer", "rlh_dsampler": "RlhDsampler"}


def c_to_rust(ctype):
    """'const float*' -> '*const f32', 'rlh_model**' -> '*mut *mut RlhModel',
    'const char* const*' -> '*const *const c_char': each '*' becomes *const
    when what it points to is const-qualified, else *mut."""
    toks = ctype.replace("*", " * ").split()
    base = [t for t in toks if t not in ("const", "*")]
    assert len(base) == 1, ctype
    levels, pending = [], False
    for t in toks:
        if t == "const":
            pending = True
        elif t == "*":
            levels.append(pending)
            pending = False
    out = C_SCALARS[base[0]]
    for const in levels:
        out = ("*const " if const else "*mut ") + out
    return out


def header_decls():
    text = open(os.path.join(ROOT, "include", "rlh.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"#.*", "", text)
    decls = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(rlh_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = " ".join(m.group(1).split()), m.group(2), " ".join(m.group(3).split())
        params = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                pm = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", a)
                params.append(c_to_rust(pm.group(1).strip()))
        decls[name] = (None if ret == "void" else c_to_rust(ret), params)
    return decls


def binding_decls():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```rust\n(.*?)```", text, flags=re.S)
    ext = [b for b in blocks if 'extern "C"' in b]
    assert len(ext) == 1, "the integration guide must hold exactly one extern \"C\" Rust block"
    body = re.sub(r"//.*", "", ext[0])
    decls = {}
    for m in re.finditer(r"pub fn (rlh_[a-z0-9_]+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", body, flags=re.S):
        name, args, ret = m.group(1), " ".join(m.group(2).split()), m.group(4)
        params = []
        if args:
            for a in args.split(","):
                a = a.strip()
                if a:
                    params.append(" ".join(a.split(":", 1)[1].split()))
        decls[name] = (" ".join(ret.split()) if ret else None, params)
    return decls


def test_type_mapping():
    assert c_to_rust("const float*") == "*const f32"
    assert c_to_rust("rlh_model**") == "*mut *mut RlhModel"
    assert c_to_rust("const rlh_model*") == "*const RlhModel"
    assert c_to_rust("uint64_t") == "u64"
    assert c_to_rust("const char* const*") == "*const *const c_char"


def test_binding_mirrors_header():
    h = header_decls()
    b = binding_decls()
    assert len(h) >= 30
    assert sorted(h) == sorted(b), (sorted(set(h) - set(b)), sorted(set(b) - set(h)))
    for name, (ret, params) in h.items():
        bret, bparams = b[name]
        assert bret == ret, (name, ret, bret)
        assert bparams == params, (name, params, bparams)
