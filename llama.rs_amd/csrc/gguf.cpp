// gguf.cpp — GGUF v2/v3 reader and writer, and Model::load's resolution of
// a GGUF file onto the device model (host C++, part of librlh).
//
// Reader: GgufFile::open (src/gguf.rs:246-307) — the file is memory-mapped;
// metadata is parsed eagerly; tensor bytes are borrowed from the mapping.
// Split models (split.count > 1) open their sibling files the way
// gguf.rs:259-293 names them. Every read is bounds-checked: a malformed file
// (bad magic, unsupported version, truncated data, absurd counts or
// lengths, unknown value or tensor types, nesting beyond kMaxDepth) returns
// RLH_EFORMAT and never aborts (gguf.rs:433-464's failure modes).
// Writer: write_gguf (src/prune.rs:381-442) — keys in byte order, tensor
// data offsets aligned, the data section aligned.
// Model: Model::read_config (model.rs:241-293) with the architecture gate
// (model.rs:794-808) and Model::load's tensor resolution (model.rs:150-239).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <list>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rlh.h"
#include "sampler.h"
#include "utf8.h"

namespace {

using rlh::set_error;

// GGUF metadata value types (gguf.rs:204-235).
enum : uint32_t {
  V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
  V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};
constexpr int kMaxDepth = 8;  // arrays of arrays deeper than this are refused
constexpr uint64_t kMaxElems = 1ull << 25;  // metadata array elements per file

struct Meta {
  uint32_t type = V_U8;
  uint64_t u = 0;   // unsigned and boolean payloads
  int64_t i = 0;    // signed payloads
  double f = 0.0;   // F64 (and F32 widened)
  float f32 = 0.f;  // F32 as stored
  std::string s;
  uint32_t elem = V_STR;  // array element type
  std::vector<Meta> arr;
};

struct Info {
  std::string name;
  std::vector<uint64_t> dims;  // dims[0] is the row length (fastest varying)
  uint32_t ty = 0;
  uint64_t offset = 0;  // from the start of the file's data section
  uint32_t file = 0;
};

// Block size / bytes per block of the ggml types GgmlType::from_u32 accepts
// (quant.rs:26-90).
bool type_geom(uint32_t ty, uint64_t* bs, uint64_t* ts) {
  switch (ty) {
    case RLH_TYPE_F32: *bs = 1; *ts = 4; return true;
    case RLH_TYPE_F16: case RLH_TYPE_BF16: *bs = 1; *ts = 2; return true;
    case RLH_TYPE_Q4_0: *bs = 32; *ts = 18; return true;
    case RLH_TYPE_Q4_1: *bs = 32; *ts = 20; return true;
    case RLH_TYPE_Q5_0: *bs = 32; *ts = 22; return true;
    case RLH_TYPE_Q5_1: *bs = 32; *ts = 24; return true;
    case RLH_TYPE_Q8_0: *bs = 32; *ts = 34; return true;
    case RLH_TYPE_Q4_K: *bs = 256; *ts = 144; return true;
    case RLH_TYPE_Q5_K: *bs = 256; *ts = 176; return true;
    case RLH_TYPE_Q6_K: *bs = 256; *ts = 210; return true;
    default: return false;
  }
}

// Elements of a tensor (0 and false on overflow).
bool n_elements(const Info& t, uint64_t* n) {
  uint64_t p = 1;
  for (uint64_t d : t.dims) {
    if (d != 0 && p > UINT64_MAX / d) return false;
    p *= d;
  }
  *n = p;
  return true;
}

// TensorInfo::nbytes (gguf.rs:105-108): whole blocks of the element count.
bool n_bytes(const Info& t, uint64_t* nb) {
  uint64_t n = 0, bs = 0, ts = 0;
  if (!n_elements(t, &n) || !type_geom(t.ty, &bs, &ts)) return false;
  const uint64_t blocks = n / bs;
  if (ts != 0 && blocks > UINT64_MAX / ts) return false;
  *nb = blocks * ts;
  return true;
}

uint64_t align_up(uint64_t x, uint64_t a) { return a == 0 ? x : (x + a - 1) / a * a; }

// Bounds-checked little-endian reader over one mapping.
struct Cursor {
  const uint8_t* p;
  uint64_t n, pos = 0;
  uint64_t elems = 0;  // metadata array elements read so far
  std::string err;
  bool take(uint64_t k, const uint8_t** out) {
    if (k > n - pos) {  // pos <= n always; no addition to overflow
      err = "gguf: unexpected eof";
      return false;
    }
    *out = p + pos;
    pos += k;
    return true;
  }
  template <class T>
  bool get(T* v) {
    const uint8_t* b;
    if (!take(sizeof(T), &b)) return false;
    std::memcpy(v, b, sizeof(T));
    return true;
  }
  // strings as String::from_utf8_lossy makes them (gguf.rs:191-195)
  bool str(std::string* s) {
    uint64_t len;
    const uint8_t* b;
    if (!get(&len) || !take(len, &b)) return false;
    *s = rlh::utf8_lossy(b, (size_t)len);
    return true;
  }
  bool value(uint32_t ty, Meta* m, int depth) {
    m->type = ty;
    switch (ty) {
      case V_U8: { uint8_t v; if (!get(&v)) return false; m->u = v; return true; }
      case V_I8: { int8_t v; if (!get(&v)) return false; m->i = v; return true; }
      case V_U16: { uint16_t v; if (!get(&v)) return false; m->u = v; return true; }
      case V_I16: { int16_t v; if (!get(&v)) return false; m->i = v; return true; }
      case V_U32: { uint32_t v; if (!get(&v)) return false; m->u = v; return true; }
      case V_I32: { int32_t v; if (!get(&v)) return false; m->i = v; return true; }
      case V_F32: { float v; if (!get(&v)) return false; m->f32 = v; m->f = v; return true; }
      case V_BOOL: { uint8_t v; if (!get(&v)) return false; m->u = v != 0; return true; }
      case V_STR: return str(&m->s);
      case V_U64: { uint64_t v; if (!get(&v)) return false; m->u = v; return true; }
      case V_I64: { int64_t v; if (!get(&v)) return false; m->i = v; return true; }
      case V_F64: { double v; if (!get(&v)) return false; m->f = v; return true; }
      case V_ARR: {
        if (depth >= kMaxDepth) {
          err = "gguf: metadata arrays nested too deeply";
          return false;
        }
        uint32_t et;
        uint64_t cnt;
        if (!get(&et) || !get(&cnt)) return false;
        if (et > V_F64) {
          err = "gguf: unknown metadata value type " + std::to_string(et);
          return false;
        }
        m->elem = et;
        // every element takes at least one byte: no reservation ahead of the
        // data, so an absurd count fails at the end of the file; the element
        // total is capped so that a huge file cannot exhaust host memory
        for (uint64_t k = 0; k < cnt; k++) {
          if (++elems > kMaxElems) {
            err = "gguf: metadata arrays hold more than 2^25 elements";
            return false;
          }
          m->arr.emplace_back();
          if (!value(et, &m->arr.back(), depth + 1)) return false;
        }
        return true;
      }
      default:
        err = "gguf: unknown metadata value type " + std::to_string(ty);
        return false;
    }
  }
};

// MetaValue::as_u32 (gguf.rs:32-44): integer types convert with Rust's `as`
// (sign-extended, then truncated to 32 bits); others have no u32 value.
bool as_u32(const Meta* m, uint32_t* out) {
  switch (m->type) {
    case V_U8: case V_U16: case V_U32: case V_U64: *out = (uint32_t)m->u; return true;
    case V_I8: case V_I16: case V_I32: case V_I64: *out = (uint32_t)(uint64_t)m->i; return true;
    default: return false;
  }
}

struct Mapping {
  void* base = nullptr;
  uint64_t size = 0;
};

}  // namespace

struct rlh_gguf {
  uint32_t version = 0;
  std::vector<Mapping> maps;
  std::vector<uint64_t> data_off;
  std::vector<std::string> meta_order;  // keys in file order (first occurrence)
  std::unordered_map<std::string, Meta> meta;
  std::vector<std::string> order;  // tensor_order (gguf.rs:127)
  std::unordered_map<std::string, Info> tensors;
};

namespace {

void unmap_all(rlh_gguf* g) {
  for (auto& m : g->maps)
    if (m.base) munmap(m.base, m.size);
  g->maps.clear();
}

int map_file(const std::string& path, Mapping* out) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return set_error(RLH_EIO, ("cannot open '" + path + "': " + std::strerror(errno)).c_str());
  struct stat st {};
  if (fstat(fd, &st) != 0) {
    close(fd);
    return set_error(RLH_EIO, ("cannot stat '" + path + "'").c_str());
  }
  out->size = (uint64_t)st.st_size;
  out->base = nullptr;
  if (out->size > 0) {
    void* p = mmap(nullptr, (size_t)out->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      close(fd);
      return set_error(RLH_EIO, ("cannot map '" + path + "'").c_str());
    }
    out->base = p;
  }
  close(fd);
  return RLH_OK;
}

// parse_header_and_tensors (gguf.rs:244-311) for mapping `file`.
int parse(rlh_gguf* g, uint32_t file, bool keep_meta) {
  const Mapping& mp = g->maps[file];
  Cursor c{(const uint8_t*)mp.base, mp.size};
  auto bad = [&](const std::string& msg) { return set_error(RLH_EFORMAT, msg.c_str()); };
  const uint8_t* magic;
  if (!c.take(4, &magic) || std::memcmp(magic, "GGUF", 4) != 0) return bad("gguf: bad magic");
  uint32_t version;
  uint64_t n_tensors, n_kv;
  if (!c.get(&version)) return bad(c.err);
  if (version < 2 || version > 3) return bad("gguf: unsupported version " + std::to_string(version));
  if (!c.get(&n_tensors) || !c.get(&n_kv)) return bad(c.err);
  std::unordered_map<std::string, Meta> meta;
  std::vector<std::string> meta_order;
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key;
    uint32_t ty;
    Meta v;
    if (!c.str(&key) || !c.get(&ty) || !c.value(ty, &v, 0)) return bad(c.err);
    if (!meta.count(key)) meta_order.push_back(key);
    meta[key] = std::move(v);  // a repeated key keeps its last value, as a map insert
  }
  std::vector<Info> list;
  for (uint64_t k = 0; k < n_tensors; k++) {
    Info t;
    uint32_t nd;
    if (!c.str(&t.name) || !c.get(&nd)) return bad(c.err);
    for (uint32_t d = 0; d < nd; d++) {
      uint64_t v;
      if (!c.get(&v)) return bad(c.err);
      t.dims.push_back(v);
    }
    if (!c.get(&t.ty) || !c.get(&t.offset)) return bad(c.err);
    uint64_t bs, ts;
    if (!type_geom(t.ty, &bs, &ts))
      return bad("gguf: unsupported tensor type " + std::to_string(t.ty) + " for '" + t.name + "'");
    t.file = file;
    list.push_back(std::move(t));
  }
  uint64_t alignment = 32;
  auto it = meta.find("general.alignment");
  if (it != meta.end()) {
    uint32_t a = 0;
    if (as_u32(&it->second, &a)) alignment = a;
  }
  g->data_off.push_back(align_up(c.pos, alignment));
  if (keep_meta) {
    g->version = version;
    g->meta = std::move(meta);
    g->meta_order = std::move(meta_order);
  }
  for (auto& t : list) {
    g->order.push_back(t.name);
    g->tensors[t.name] = std::move(t);  // a repeated name keeps its last entry
  }
  return RLH_OK;
}

std::string replace_all(std::string s, const std::string& from, const std::string& to) {
  if (from.empty()) return s;
  size_t p = 0;
  while ((p = s.find(from, p)) != std::string::npos) {
    s.replace(p, from.size(), to);
    p += to.size();
  }
  return s;
}

const Meta* find_meta(const rlh_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->meta.find(key);
  return it == g->meta.end() ? nullptr : &it->second;
}

int no_key(const char* key) { return set_error(RLH_ENOENT, (std::string("missing metadata key: ") + (key ? key : "")).c_str()); }

}  // namespace

extern "C" {

int rlh_gguf_open(const char* path, rlh_gguf** out) {
  if (!path || !out) return set_error(RLH_EINVAL, "null argument");
  *out = nullptr;
  rlh_gguf* g = new rlh_gguf();
  g->maps.emplace_back();
  int rc = map_file(path, &g->maps[0]);
  if (!rc) rc = parse(g, 0, true);
  if (rc) {
    unmap_all(g);
    delete g;
    return rc;
  }
  // split models: sibling files named as gguf.rs:262-273 names them
  auto sc = g->meta.find("split.count");
  uint32_t count = 0;
  if (sc != g->meta.end() && as_u32(&sc->second, &count) && count > 1) {
    const std::string p(path);
    char from[64], to[64];
    for (uint32_t part = 2; part <= count; part++) {
      std::snprintf(from, sizeof from, "-%05u-of-%05u.gguf", 1u, count);
      std::snprintf(to, sizeof to, "-%05u-of-%05u.gguf", part, count);
      std::string sib;
      if (p.find(from) != std::string::npos) {
        sib = replace_all(p, from, to);
      } else {
        std::snprintf(from, sizeof from, "-00001-of-0000%u.gguf", count);
        std::snprintf(to, sizeof to, "-%05u-of-0000%u.gguf", part, count);
        sib = replace_all(p, from, to);
      }
      struct stat st {};
      if (stat(sib.c_str(), &st) != 0) continue;  // a missing sibling is skipped, as the reference does
      g->maps.emplace_back();
      rc = map_file(sib, &g->maps.back());
      if (!rc) rc = parse(g, (uint32_t)(g->maps.size() - 1), false);
      if (rc) {
        unmap_all(g);
        delete g;
        return rc;
      }
    }
  }
  *out = g;
  return RLH_OK;
}

void rlh_gguf_close(rlh_gguf* g) {
  if (!g) return;
  unmap_all(g);
  delete g;
}

uint32_t rlh_gguf_version(const rlh_gguf* g) { return g ? g->version : 0; }
uint64_t rlh_gguf_n_files(const rlh_gguf* g) { return g ? g->maps.size() : 0; }
uint64_t rlh_gguf_n_tensors(const rlh_gguf* g) { return g ? g->order.size() : 0; }
uint64_t rlh_gguf_n_meta(const rlh_gguf* g) { return g ? g->meta_order.size() : 0; }

int rlh_gguf_meta_key(const rlh_gguf* g, uint64_t index, const char** key) {
  if (!g || !key) return set_error(RLH_EINVAL, "null argument");
  if (index >= g->meta_order.size()) return set_error(RLH_EINVAL, "metadata index out of range");
  *key = g->meta_order[index].c_str();
  return RLH_OK;
}

int rlh_gguf_tensor_info(const rlh_gguf* g, uint64_t index, const char** name, uint32_t* ggml_type,
                         uint32_t* n_dims, uint64_t* dims, uint32_t max_dims, uint64_t* offset, uint32_t* file_index) {
  if (!g || !name || !ggml_type || !n_dims) return set_error(RLH_EINVAL, "null argument");
  if (index >= g->order.size()) return set_error(RLH_EINVAL, "tensor index out of range");
  const Info& t = g->tensors.at(g->order[index]);
  *name = t.name.c_str();
  *ggml_type = t.ty;
  *n_dims = (uint32_t)t.dims.size();
  for (uint32_t d = 0; dims && d < max_dims && d < t.dims.size(); d++) dims[d] = t.dims[d];
  if (offset) *offset = t.offset;
  if (file_index) *file_index = t.file;
  return RLH_OK;
}

int rlh_gguf_tensor_bytes(const rlh_gguf* g, const char* name, const void** data, uint64_t* nbytes) {
  if (!g || !name || !data || !nbytes) return set_error(RLH_EINVAL, "null argument");
  auto it = g->tensors.find(name);
  if (it == g->tensors.end()) return set_error(RLH_ENOENT, (std::string("tensor '") + name + "'").c_str());
  const Info& t = it->second;
  uint64_t nb = 0;
  if (!n_bytes(t, &nb) || t.file >= g->maps.size())
    return set_error(RLH_EFORMAT, (std::string("tensor '") + name + "' out of range").c_str());
  const Mapping& mp = g->maps[t.file];
  const uint64_t d0 = g->data_off[t.file];
  // start = data_offset + offset, end = start + nbytes, both within the file
  if (t.offset > mp.size || d0 > mp.size - t.offset || nb > mp.size - d0 - t.offset)
    return set_error(RLH_EFORMAT, (std::string("tensor '") + name + "' out of range").c_str());
  *data = (const uint8_t*)mp.base + d0 + t.offset;
  *nbytes = nb;
  return RLH_OK;
}

int rlh_gguf_meta_type(const rlh_gguf* g, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* n_elems) {
  const Meta* m = find_meta(g, key);
  if (!m) return no_key(key);
  if (type) *type = m->type;
  if (elem_type) *elem_type = m->type == V_ARR ? m->elem : 0;
  if (n_elems) *n_elems = m->type == V_ARR ? m->arr.size() : 1;
  return RLH_OK;
}

int rlh_gguf_meta_u32(const rlh_gguf* g, const char* key, uint32_t* v) {
  const Meta* m = find_meta(g, key);
  if (!v) return set_error(RLH_EINVAL, "null argument");
  if (!m) return no_key(key);
  if (!as_u32(m, v)) return set_error(RLH_EINVAL, (std::string("metadata '") + key + "' is not an integer").c_str());
  return RLH_OK;
}

// MetaValue::as_f32 (gguf.rs:50-56): F32, or F64 rounded to f32.
int rlh_gguf_meta_f32(const rlh_gguf* g, const char* key, float* v) {
  const Meta* m = find_meta(g, key);
  if (!v) return set_error(RLH_EINVAL, "null argument");
  if (!m) return no_key(key);
  if (m->type == V_F32) *v = m->f32;
  else if (m->type == V_F64) *v = (float)m->f;
  else return set_error(RLH_EINVAL, (std::string("metadata '") + key + "' is not a float").c_str());
  return RLH_OK;
}

int rlh_gguf_meta_scalar(const rlh_gguf* g, const char* key, uint64_t* u, int64_t* i, double* f) {
  const Meta* m = find_meta(g, key);
  if (!m) return no_key(key);
  if (m->type == V_STR || m->type == V_ARR) return set_error(RLH_EINVAL, (std::string("metadata '") + key + "' is not a scalar").c_str());
  if (u) *u = m->u;
  if (i) *i = m->i;
  if (f) *f = m->f;
  return RLH_OK;
}

int rlh_gguf_meta_str(const rlh_gguf* g, const char* key, const char** s, uint64_t* len) {
  const Meta* m = find_meta(g, key);
  if (!s) return set_error(RLH_EINVAL, "null argument");
  if (!m) return no_key(key);
  if (m->type != V_STR) return set_error(RLH_EINVAL, (std::string("metadata '") + key + "' is not a string").c_str());
  *s = m->s.c_str();
  if (len) *len = m->s.size();
  return RLH_OK;
}

int rlh_gguf_meta_arr_str(const rlh_gguf* g, const char* key, uint64_t index, const char** s, uint64_t* len) {
  const Meta* m = find_meta(g, key);
  if (!s) return set_error(RLH_EINVAL, "null argument");
  if (!m) return no_key(key);
  if (m->type != V_ARR || index >= m->arr.size() || m->arr[index].type != V_STR)
    return set_error(RLH_EINVAL, (std::string("metadata '") + key + "' has no string at that index").c_str());
  *s = m->arr[index].s.c_str();
  if (len) *len = m->arr[index].s.size();
  return RLH_OK;
}

int rlh_gguf_meta_arr_scalar(const rlh_gguf* g, const char* key, uint64_t index, uint64_t* u, int64_t* i, double* f) {
  const Meta* m = find_meta(g, key);
  if (!m) return no_key(key);
  if (m->type != V_ARR || index >= m->arr.size() || m->arr[index].type == V_STR || m->arr[index].type == V_ARR)
    return set_error(RLH_EINVAL, (std::string("metadata '") + key + "' has no scalar at that index").c_str());
  const Meta& e = m->arr[index];
  if (u) *u = e.u;
  if (i) *i = e.i;
  if (f) *f = e.f;
  return RLH_OK;
}

// ---- Model::read_config / Model::load -------------------------------------

int rlh_gguf_config(const rlh_gguf* g, rlh_config* cfg, char* arch, uint64_t arch_cap) {
  if (!g || !cfg) return set_error(RLH_EINVAL, "null argument");
  std::string a = "llama";  // model.rs:243-247
  if (const Meta* m = find_meta(g, "general.architecture"))
    if (m->type == V_STR) a = m->s;
  if (arch && arch_cap) {
    std::strncpy(arch, a.c_str(), (size_t)arch_cap - 1);
    arch[arch_cap - 1] = 0;
  }
  if (a != "qwen3" && a != "qwen2")  // check_arch (model.rs:794-808)
    return set_error(RLH_EUNSUP, ("unsupported architecture '" + a + "': this path implements qwen3 and qwen2").c_str());
  // "{arch}.{k}" first, then the bare key (model.rs:250-259)
  auto getu = [&](const char* k, uint32_t* v) -> bool {
    const Meta* m = find_meta(g, (a + "." + k).c_str());
    if (!m) m = find_meta(g, k);
    return m && as_u32(m, v);
  };
  auto getf = [&](const char* k, float* v) -> bool {
    const Meta* m = find_meta(g, (a + "." + k).c_str());
    if (!m) m = find_meta(g, k);
    if (!m) return false;
    if (m->type == V_F32) *v = m->f32;
    else if (m->type == V_F64) *v = (float)m->f;
    else return false;
    return true;
  };
  rlh_config c{};
  const char* req[4] = {"block_count", "embedding_length", "feed_forward_length", "attention.head_count"};
  uint32_t* dst[4] = {&c.n_layer, &c.n_embd, &c.n_ff, &c.n_head};
  for (int k = 0; k < 4; k++)
    if (!getu(req[k], dst[k])) return set_error(RLH_EFORMAT, (std::string("missing metadata key: ") + req[k]).c_str());
  if (!getu("attention.head_count_kv", &c.n_head_kv)) c.n_head_kv = c.n_head;
  if (!getu("attention.key_length", &c.head_dim)) c.head_dim = c.n_head ? c.n_embd / c.n_head : 0;
  if (!getf("rope.freq_base", &c.rope_theta)) c.rope_theta = 10000.0f;
  if (!getf("attention.layer_norm_rms_epsilon", &c.rms_eps)) c.rms_eps = 1e-5f;
  if (!getu("context_length", &c.n_ctx)) c.n_ctx = 4096;
  auto te = g->tensors.find("token_embd.weight");
  c.vocab_size = 0;
  if (te != g->tensors.end()) {
    uint64_t r = 1;
    for (size_t d = 1; d < te->second.dims.size(); d++) r *= te->second.dims[d];
    c.vocab_size = (uint32_t)r;  // TensorInfo::n_rows (gguf.rs:111-117)
  }
  c.has_qk_norm = g->tensors.count("blk.0.attn_q_norm.weight") ? 1u : 0u;
  c.has_output = g->tensors.count("output.weight") ? 1u : 0u;
  *cfg = c;
  return RLH_OK;
}

int rlh_model_load_gguf(const rlh_gguf* g, rlh_model** out) {
  if (!g || !out) return set_error(RLH_EINVAL, "null argument");
  *out = nullptr;
  rlh_config cfg{};
  int rc = rlh_gguf_config(g, &cfg, nullptr, 0);
  if (rc) return rc;
  // shapes the device path cannot run are refused before anything is read
  if ((rc = rlh_config_check(&cfg))) return rc;
  // Model::read_tokenizer requires the vocabulary (model.rs:295-300)
  const Meta* toks = find_meta(g, "tokenizer.ggml.tokens");
  if (!toks || toks->type != V_ARR || toks->elem != V_STR)
    return set_error(RLH_EFORMAT, "missing metadata key: tokenizer.ggml.tokens");
  rlh_model* m = nullptr;
  if ((rc = rlh_model_create(&cfg, &m))) return rc;
  // one tensor by GGUF name: rows = n_rows, cols = n_cols (gguf.rs:111-123)
  auto put = [&](const std::string& name, int kind, int layer, bool required) -> int {
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) {
      if (!required) return RLH_OK;
      return set_error(RLH_ESTATE, ("model is missing required tensor '" + name + "'").c_str());
    }
    const Info& t = it->second;
    const void* data = nullptr;
    uint64_t nb = 0;
    int r = rlh_gguf_tensor_bytes(g, name.c_str(), &data, &nb);
    if (r) return r;
    const uint64_t cols = t.dims.empty() ? 1 : t.dims[0];
    uint64_t rows = 1;
    for (size_t d = 1; d < t.dims.size(); d++) rows *= t.dims[d];
    r = rlh_model_set_tensor(m, kind, layer, t.ty, data, cols, rows);
    if (r) return set_error(r, ("tensor '" + name + "': " + rlh_last_error()).c_str());
    return RLH_OK;
  };
  rc = put("token_embd.weight", RLH_T_TOKEN_EMBD, 0, true);
  if (!rc) rc = put("output_norm.weight", RLH_T_OUTPUT_NORM, 0, true);
  if (!rc) rc = put("output.weight", RLH_T_OUTPUT, 0, false);
  for (uint32_t l = 0; !rc && l < cfg.n_layer; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    const int li = (int)l;
    struct {
      const char* n;
      int kind;
      bool req;
    } spec[] = {{"attn_norm.weight", RLH_T_ATTN_NORM, true},      {"ffn_norm.weight", RLH_T_FFN_NORM, true},
                {"attn_q_norm.weight", RLH_T_ATTN_Q_NORM, cfg.has_qk_norm != 0},
                {"attn_k_norm.weight", RLH_T_ATTN_K_NORM, cfg.has_qk_norm != 0},
                {"attn_q.bias", RLH_T_ATTN_Q_BIAS, false},        {"attn_k.bias", RLH_T_ATTN_K_BIAS, false},
                {"attn_v.bias", RLH_T_ATTN_V_BIAS, false},        {"attn_q.weight", RLH_T_ATTN_Q, true},
                {"attn_k.weight", RLH_T_ATTN_K, true},            {"attn_v.weight", RLH_T_ATTN_V, true},
                {"attn_output.weight", RLH_T_ATTN_OUTPUT, true},  {"ffn_gate.weight", RLH_T_FFN_GATE, true},
                {"ffn_up.weight", RLH_T_FFN_UP, true},            {"ffn_down.weight", RLH_T_FFN_DOWN, true}};
    for (auto& s : spec) {
      // QK-norm weights only when blk.0 has them (model.rs:185-196)
      if ((s.kind == RLH_T_ATTN_Q_NORM || s.kind == RLH_T_ATTN_K_NORM) && !cfg.has_qk_norm) continue;
      if ((rc = put(p + s.n, s.kind, li, s.req))) break;
    }
  }
  if (!rc) rc = rlh_model_finalize(m);
  if (rc) {
    std::string msg = rlh_last_error();
    rlh_model_destroy(m);
    return set_error(rc, msg.c_str());
  }
  *out = m;
  return RLH_OK;
}

}  // extern "C"

// ---- writer (write_gguf, prune.rs:381-442) -----------------------------------

namespace {
struct WTensor {
  std::string name;
  uint32_t ty;
  std::vector<uint64_t> dims;
  const void* data;
  uint64_t nbytes;
};
}  // namespace

struct rlh_gguf_writer {
  uint32_t version = 3;
  uint64_t alignment = 32;
  std::map<std::string, Meta> meta;  // written in key order (prune.rs:405-410)
  std::vector<WTensor> tensors;
};

namespace {

uint64_t scalar_size(uint32_t ty) {
  switch (ty) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
  }
}

// A scalar Meta of type ty from `size` bytes of raw little-endian value.
Meta scalar_meta(uint32_t ty, const uint8_t* p) {
  Meta m;
  m.type = ty;
  switch (ty) {
    case V_U8: m.u = p[0]; break;
    case V_I8: m.i = (int8_t)p[0]; break;
    case V_BOOL: m.u = p[0] != 0; break;
    case V_U16: { uint16_t v; std::memcpy(&v, p, 2); m.u = v; break; }
    case V_I16: { int16_t v; std::memcpy(&v, p, 2); m.i = v; break; }
    case V_U32: { uint32_t v; std::memcpy(&v, p, 4); m.u = v; break; }
    case V_I32: { int32_t v; std::memcpy(&v, p, 4); m.i = v; break; }
    case V_F32: { float v; std::memcpy(&v, p, 4); m.f32 = v; m.f = v; break; }
    case V_U64: { uint64_t v; std::memcpy(&v, p, 8); m.u = v; break; }
    case V_I64: { int64_t v; std::memcpy(&v, p, 8); m.i = v; break; }
    case V_F64: { double v; std::memcpy(&v, p, 8); m.f = v; break; }
  }
  return m;
}

struct Out {
  FILE* f;
  uint64_t pos = 0;
  bool ok = true;
  void bytes(const void* p, uint64_t n) {
    if (ok && n && std::fwrite(p, 1, (size_t)n, f) != (size_t)n) ok = false;
    pos += n;
  }
  template <class T>
  void put(T v) { bytes(&v, sizeof v); }
  void str(const std::string& s) {
    put<uint64_t>(s.size());
    bytes(s.data(), s.size());
  }
  void zeros(uint64_t n) {
    static const uint8_t z[4096] = {};
    while (n) {
      const uint64_t k = std::min<uint64_t>(n, sizeof z);
      bytes(z, k);
      n -= k;
    }
  }
  // a value's payload without its type tag (write_array_elem, prune.rs:360-379)
  void payload(const Meta& m) {
    switch (m.type) {
      case V_U8: case V_BOOL: put<uint8_t>((uint8_t)m.u); break;
      case V_I8: put<int8_t>((int8_t)m.i); break;
      case V_U16: put<uint16_t>((uint16_t)m.u); break;
      case V_I16: put<int16_t>((int16_t)m.i); break;
      case V_U32: put<uint32_t>((uint32_t)m.u); break;
      case V_I32: put<int32_t>((int32_t)m.i); break;
      case V_F32: put<float>(m.f32); break;
      case V_STR: str(m.s); break;
      case V_U64: put<uint64_t>(m.u); break;
      case V_I64: put<int64_t>(m.i); break;
      case V_F64: put<double>(m.f); break;
      case V_ARR:
        put<uint32_t>(m.elem);
        put<uint64_t>(m.arr.size());
        for (const Meta& e : m.arr) payload(e);
        break;
    }
  }
};

}  // namespace

extern "C" {

int rlh_gguf_writer_create(uint32_t version, uint64_t alignment, rlh_gguf_writer** out) {
  if (!out) return set_error(RLH_EINVAL, "null argument");
  *out = nullptr;
  if (version < 2 || version > 3) return set_error(RLH_EINVAL, "GGUF version must be 2 or 3");
  rlh_gguf_writer* w = new rlh_gguf_writer();
  w->version = version;
  w->alignment = alignment;
  *out = w;
  return RLH_OK;
}

void rlh_gguf_writer_destroy(rlh_gguf_writer* w) { delete w; }

int rlh_gguf_writer_set_scalar(rlh_gguf_writer* w, const char* key, uint32_t type, const void* value) {
  if (!w || !key || !value) return set_error(RLH_EINVAL, "null argument");
  if (scalar_size(type) == 0) return set_error(RLH_EINVAL, "not a scalar GGUF value type");
  w->meta[key] = scalar_meta(type, (const uint8_t*)value);
  return RLH_OK;
}

int rlh_gguf_writer_set_string(rlh_gguf_writer* w, const char* key, const char* s, uint64_t len) {
  if (!w || !key || (!s && len)) return set_error(RLH_EINVAL, "null argument");
  Meta m;
  m.type = V_STR;
  m.s.assign(s ? s : "", (size_t)len);
  w->meta[key] = std::move(m);
  return RLH_OK;
}

int rlh_gguf_writer_set_array(rlh_gguf_writer* w, const char* key, uint32_t elem_type, const void* values, uint64_t n) {
  if (!w || !key || (!values && n)) return set_error(RLH_EINVAL, "null argument");
  if (elem_type == V_ARR) return set_error(RLH_EINVAL, "nested arrays are not supported by the writer");
  Meta m;
  m.type = V_ARR;
  m.elem = elem_type;
  if (elem_type == V_STR) {
    const char* const* strs = (const char* const*)values;
    for (uint64_t k = 0; k < n; k++) {
      if (!strs[k]) return set_error(RLH_EINVAL, "null string in a string array");
      Meta e;
      e.type = V_STR;
      e.s = strs[k];
      m.arr.push_back(std::move(e));
    }
  } else {
    const uint64_t sz = scalar_size(elem_type);
    if (!sz) return set_error(RLH_EINVAL, "unknown GGUF element type");
    for (uint64_t k = 0; k < n; k++) m.arr.push_back(scalar_meta(elem_type, (const uint8_t*)values + k * sz));
  }
  w->meta[key] = std::move(m);
  return RLH_OK;
}

int rlh_gguf_writer_add_tensor(rlh_gguf_writer* w, const char* name, uint32_t ggml_type, uint32_t n_dims,
                               const uint64_t* dims, const void* data, uint64_t nbytes) {
  if (!w || !name || (!dims && n_dims) || (!data && nbytes)) return set_error(RLH_EINVAL, "null argument");
  Info t;
  t.ty = ggml_type;
  t.dims.assign(dims, dims + n_dims);
  uint64_t nb = 0;
  if (!n_bytes(t, &nb)) return set_error(RLH_EINVAL, "unknown ggml type or element count overflow");
  if (nb != nbytes)
    return set_error(RLH_EINVAL, ("tensor '" + std::string(name) + "': " + std::to_string(nbytes) +
                                  " bytes given, its shape and type need " + std::to_string(nb)).c_str());
  w->tensors.push_back(WTensor{name, ggml_type, t.dims, data, nbytes});
  return RLH_OK;
}

int rlh_gguf_writer_write(rlh_gguf_writer* w, const char* path) {
  if (!w || !path) return set_error(RLH_EINVAL, "null argument");
  std::vector<uint64_t> offs;
  uint64_t off = 0;
  for (const WTensor& t : w->tensors) {
    off = align_up(off, w->alignment);
    offs.push_back(off);
    off += t.nbytes;
  }
  FILE* f = std::fopen(path, "wb");
  if (!f) return set_error(RLH_EIO, ("cannot create '" + std::string(path) + "'").c_str());
  Out o{f};
  o.bytes("GGUF", 4);
  o.put<uint32_t>(w->version);
  o.put<uint64_t>(w->tensors.size());
  o.put<uint64_t>(w->meta.size());
  for (const auto& kv : w->meta) {
    o.str(kv.first);
    o.put<uint32_t>(kv.second.type);
    o.payload(kv.second);
  }
  for (size_t k = 0; k < w->tensors.size(); k++) {
    const WTensor& t = w->tensors[k];
    o.str(t.name);
    o.put<uint32_t>((uint32_t)t.dims.size());
    for (uint64_t d : t.dims) o.put<uint64_t>(d);
    o.put<uint32_t>(t.ty);
    o.put<uint64_t>(offs[k]);
  }
  const uint64_t data_start = align_up(o.pos, w->alignment);
  o.zeros(data_start - o.pos);
  for (size_t k = 0; k < w->tensors.size(); k++) {
    o.zeros(data_start + offs[k] - o.pos);
    o.bytes(w->tensors[k].data, w->tensors[k].nbytes);
  }
  const bool ok = o.ok && std::fclose(f) == 0;
  if (!ok) return set_error(RLH_EIO, ("write to '" + std::string(path) + "' failed").c_str());
  return RLH_OK;
}

}  // extern "C"

// ---- prune_vocab (src/prune.rs:127-291) ---------------------------------------
// Rewrites a GGUF file keeping only the vocabulary of a Latin + Arabic/Persian
// (+ symbols, emoji) deployment, with the matching rows of the vocabulary-sized
// tensors (token_embd, output): the model then decodes over a smaller logits
// matrix. Host code; the pruned file loads like any other.

namespace {

// Code point ranges of the scripts the pruning drops (prune.rs:39-90) and the
// notation blocks kept inside them (prune.rs:94). These tables decide which
// rows the pruned file holds, so they are the reference's.
const uint32_t kDropRanges[][2] = {
    {0x0400, 0x052F},   {0x0530, 0x058F},   {0x0590, 0x05FF},   {0x0700, 0x07FF},   {0x0800, 0x089F},
    {0x0900, 0x0DFF},   {0x0E00, 0x0EFF},   {0x0F00, 0x0FFF},   {0x1000, 0x109F},   {0x10A0, 0x10FF},
    {0x1100, 0x11FF},   {0x1200, 0x139F},   {0x13A0, 0x13FF},   {0x1400, 0x167F},   {0x1680, 0x16FF},
    {0x1700, 0x18FF},   {0x1900, 0x1DFF},   {0x1F00, 0x1FFF},   {0x2C00, 0x2C5F},   {0x2C80, 0x2CFF},
    {0x2D00, 0x2D7F},   {0x2D80, 0x2DDF},   {0x2DE0, 0x2DFF},   {0x2E80, 0x2FFF},   {0x3000, 0x303F},
    {0x3040, 0x30FF},   {0x3100, 0x312F},   {0x3130, 0x318F},   {0x3190, 0x31FF},   {0x3200, 0x33FF},
    {0x3400, 0x4DBF},   {0x4DC0, 0x4DFF},   {0x4E00, 0x9FFF},   {0xA000, 0xA71F},   {0xA800, 0xAFFF},
    {0xAB00, 0xAB2F},   {0xAB70, 0xABFF},   {0xAC00, 0xD7FF},   {0xF900, 0xFAFF},   {0xFE30, 0xFE4F},
    {0xFE50, 0xFE6F},   {0xFF00, 0xFFEF},   {0x10000, 0x1D0FF}, {0x1D200, 0x1D3FF}, {0x1D800, 0x1EFFF},
    {0x20000, 0x2FFFF}, {0x30000, 0x3FFFF}};
const uint32_t kKeepAstral[][2] = {{0x1D100, 0x1D1FF}, {0x1D400, 0x1D7FF}};

bool char_dropped(uint32_t u) {  // prune.rs:96-102
  for (const auto& r : kKeepAstral)
    if (u >= r[0] && u <= r[1]) return false;
  for (const auto& r : kDropRanges)
    if (u >= r[0] && u <= r[1]) return true;
  return false;
}

// surface_kept (prune.rs:104-108): the token string is undone through the
// byte-level alphabet (decode_token_bytes, tokenizer.rs:362-383: a character
// of the alphabet is its byte, any other character its own UTF-8), the bytes
// are read as lossy UTF-8, and no character may be in a dropped script.
// U+FFFD (what lossy decoding puts for invalid bytes) is never dropped, so
// invalid bytes are simply passed over.
bool surface_kept(const std::string& tok, const int16_t (&cp_to_byte)[324]) {
  std::string bytes;
  bytes.reserve(tok.size());
  const uint8_t* s = (const uint8_t*)tok.data();
  for (size_t i = 0; i < tok.size();) {
    int bad = 1;
    const int len = rlh::utf8_seq(s, tok.size(), i, &bad);  // the string is valid UTF-8 (read lossily)
    if (len == 0) {
      i += (size_t)bad;
      continue;
    }
    const uint32_t cp = rlh::utf8_cp(s + i, len);
    if (cp < 324 && cp_to_byte[cp] >= 0) bytes += (char)cp_to_byte[cp];
    else bytes.append(tok, i, (size_t)len);
    i += (size_t)len;
  }
  const uint8_t* b = (const uint8_t*)bytes.data();
  for (size_t i = 0; i < bytes.size();) {
    int bad = 1;
    const int len = rlh::utf8_seq(b, bytes.size(), i, &bad);
    if (len == 0) {
      i += (size_t)bad;
      continue;
    }
    if (char_dropped(rlh::utf8_cp(b + i, len))) return false;
    i += (size_t)len;
  }
  return true;
}

// MetaValue::as_string_vec (gguf.rs:82-89): an array whose elements are all strings.
bool as_string_vec(const Meta* m, std::vector<const std::string*>* out) {
  if (!m || m->type != V_ARR) return false;
  out->clear();
  for (const Meta& e : m->arr) {
    if (e.type != V_STR) return false;
    out->push_back(&e.s);
  }
  return true;
}

bool ends_with(const std::string& s, const char* suf) {
  const size_t n = std::strlen(suf);
  return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

Meta str_array(const std::vector<std::string>& v) {
  Meta m;
  m.type = V_ARR;
  m.elem = V_STR;
  for (const std::string& s : v) {
    Meta e;
    e.type = V_STR;
    e.s = s;
    m.arr.push_back(std::move(e));
  }
  return m;
}

}  // namespace

extern "C" {

int rlh_prune_vocab(const char* in_path, const char* out_path, rlh_prune_stats* stats) {
  if (!in_path || !out_path) return set_error(RLH_EINVAL, "null argument");
  rlh_gguf* g = nullptr;
  int rc = rlh_gguf_open(in_path, &g);
  if (rc) return rc;
  struct Closer {
    rlh_gguf* g;
    ~Closer() { rlh_gguf_close(g); }
  } closer{g};
  auto bad = [](const std::string& msg) { return set_error(RLH_EFORMAT, ("prune: " + msg).c_str()); };

  std::vector<const std::string*> tokens, merges;
  if (!as_string_vec(find_meta(g, "tokenizer.ggml.tokens"), &tokens)) return bad("tokenizer.ggml.tokens");
  const uint64_t vocab = tokens.size();
  std::vector<uint32_t> types(vocab, 1u);  // absent or not an array: every token normal
  if (const Meta* tt = find_meta(g, "tokenizer.ggml.token_type"); tt && tt->type == V_ARR) {
    types.assign(tt->arr.size(), 1u);
    for (size_t k = 0; k < tt->arr.size(); k++) {
      uint32_t v = 1;
      if (as_u32(&tt->arr[k], &v)) types[k] = v;
    }
  }
  if (!as_string_vec(find_meta(g, "tokenizer.ggml.merges"), &merges)) merges.clear();
  if (types.size() != vocab) return bad("tokenizer.ggml.token_type length mismatch");

  // token ids named by *_token_id keys always survive
  std::vector<bool> pinned(vocab, false);
  for (const auto& kv : g->meta) {
    uint32_t id = 0;
    if (ends_with(kv.first, "_token_id") && as_u32(&kv.second, &id) && id < vocab) pinned[id] = true;
  }
  int16_t cp_to_byte[324];
  {
    std::fill(std::begin(cp_to_byte), std::end(cp_to_byte), (int16_t)-1);
    uint32_t n = 0;
    for (uint32_t b = 0; b < 256; b++) {  // bytes_to_unicode (tokenizer.rs:7-32)
      const bool direct = (b >= 0x21 && b <= 0x7e) || (b >= 0xa1 && b <= 0xac) || (b >= 0xae && b <= 0xff);
      cp_to_byte[direct ? b : 256 + n++] = (int16_t)b;
    }
  }
  rlh_prune_stats st{};
  std::vector<bool> keep(vocab, false);
  for (uint64_t i = 0; i < vocab; i++) {
    const uint32_t ty = types[i];  // 2 unknown, 3 control, 4 user-defined, 6 byte
    if (ty == 2 || ty == 3 || ty == 4 || ty == 6 || pinned[i]) {
      keep[i] = true;
      if (ty == 3 || ty == 4) st.kept_special++;
      else if (ty == 6) st.kept_byte++;
      else st.kept_normal++;
    } else if (surface_kept(*tokens[i], cp_to_byte)) {
      keep[i] = true;
      st.kept_normal++;
    }
  }
  std::vector<uint32_t> new_id(vocab, UINT32_MAX);
  uint32_t next = 0;
  for (uint64_t i = 0; i < vocab; i++)
    if (keep[i]) new_id[i] = next++;
  const uint64_t new_vocab = next;
  if (new_vocab == 0) return bad("prune would remove the entire vocabulary");

  // merges that still resolve inside the kept set; a token string maps to
  // its last id, as a map built in id order keeps it
  std::unordered_map<std::string, uint32_t> to_id;
  for (uint64_t i = 0; i < vocab; i++) to_id[*tokens[i]] = (uint32_t)i;
  std::vector<std::string> merges_new;
  for (const std::string* m : merges) {
    const size_t sp = m->find(' ');
    if (sp == std::string::npos) continue;
    const std::string l = m->substr(0, sp), r = m->substr(sp + 1);
    auto li = to_id.find(l), ri = to_id.find(r), mi = to_id.find(l + r);
    if (li != to_id.end() && ri != to_id.end() && mi != to_id.end() && keep[li->second] && keep[ri->second] &&
        keep[mi->second])
      merges_new.push_back(*m);
  }

  // metadata: every key of the input, then the new vocabulary, types,
  // merges and remapped *_token_id values (written as u32)
  rlh_gguf_writer w;
  w.version = g->version;
  uint32_t align = 32;
  if (const Meta* a = find_meta(g, "general.alignment")) {
    uint32_t v = 0;
    if (as_u32(a, &v)) align = v;
  }
  w.alignment = align;
  for (const auto& kv : g->meta) {
    Meta m = kv.second;
    if (m.type == V_ARR) {
      for (const Meta& e : m.arr)
        if (e.type == V_ARR) return bad("nested arrays are not supported by the writer");
      if (m.arr.empty()) m.elem = V_STR;  // an empty array is written with the string tag
    }
    w.meta[kv.first] = std::move(m);
  }
  {
    std::vector<std::string> kept_tokens;
    Meta types_new;
    types_new.type = V_ARR;
    types_new.elem = V_I32;
    for (uint64_t i = 0; i < vocab; i++) {
      if (!keep[i]) continue;
      kept_tokens.push_back(*tokens[i]);
      Meta e;
      e.type = V_I32;
      e.i = (int32_t)types[i];
      types_new.arr.push_back(e);
    }
    w.meta["tokenizer.ggml.tokens"] = str_array(kept_tokens);
    w.meta["tokenizer.ggml.token_type"] = std::move(types_new);
    w.meta["tokenizer.ggml.merges"] = str_array(merges_new);
  }
  for (const auto& kv : g->meta) {
    uint32_t id = 0;
    if (!ends_with(kv.first, "_token_id") || !as_u32(&kv.second, &id)) continue;
    if (id >= vocab || new_id[id] == UINT32_MAX)
      return bad("special token id " + std::to_string(id) + " ('" + kv.first + "') was pruned");
    Meta m;
    m.type = V_U32;
    m.u = new_id[id];
    w.meta[kv.first] = m;
  }

  // tensors in file order; token_embd / output with one row per token keep
  // the rows of the kept tokens
  std::list<std::vector<uint8_t>> owned;  // stable addresses for the writer
  for (const std::string& name : g->order) {
    const Info& t = g->tensors.at(name);
    const void* data = nullptr;
    uint64_t nb = 0;
    if ((rc = rlh_gguf_tensor_bytes(g, name.c_str(), &data, &nb))) return rc;
    uint64_t rows = 1, bs = 0, ts = 0;
    for (size_t d = 1; d < t.dims.size(); d++) rows *= t.dims[d];
    const uint64_t cols = t.dims.empty() ? 1 : t.dims[0];
    type_geom(t.ty, &bs, &ts);
    if ((name == "token_embd.weight" || name == "output.weight") && rows == vocab) {
      const uint64_t rb = cols / bs * ts;
      Info ni = t;
      ni.dims = {cols, new_vocab};
      uint64_t nb_new = 0;
      n_bytes(ni, &nb_new);
      std::vector<uint8_t> sliced;
      sliced.reserve(std::max<uint64_t>(nb_new, new_vocab * rb));
      for (uint64_t i = 0; i < vocab; i++)
        if (keep[i]) sliced.insert(sliced.end(), (const uint8_t*)data + i * rb, (const uint8_t*)data + i * rb + rb);
      st.embd_bytes_saved += nb - sliced.size();
      // rows of whole blocks (every ggml file): the sliced rows are the
      // tensor's bytes; otherwise zeros fill it up to its size
      if (sliced.size() < nb_new) sliced.resize(nb_new, 0);
      owned.push_back(std::move(sliced));
      w.tensors.push_back(WTensor{name, t.ty, ni.dims, owned.back().data(), nb_new});
    } else {
      w.tensors.push_back(WTensor{name, t.ty, t.dims, data, nb});
    }
  }
  if ((rc = rlh_gguf_writer_write(&w, out_path))) return rc;
  struct stat sb {};
  if (stat(out_path, &sb) != 0) return set_error(RLH_EIO, ("cannot stat '" + std::string(out_path) + "'").c_str());
  st.old_vocab = vocab;
  st.new_vocab = new_vocab;
  st.dropped = vocab - new_vocab;
  st.merges_old = merges.size();
  st.merges_new = merges_new.size();
  st.out_bytes = (uint64_t)sb.st_size;
  if (stats) *stats = st;
  return RLH_OK;
}

}  // extern "C"
