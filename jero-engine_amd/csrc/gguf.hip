// gguf.hip -- GGUF v3 model files: map, parse, look tensors up, upload them (host code).
//
// The weight source of LockedModelWeights: the file mapped read-only and its GGUF v3 header,
// metadata and tensor descriptors parsed (src/weights.rs:338-570; the parser itself is jero-core's
// GgufFile, outside this repository), tensors found by name (ModelWeights::tensor,
// src/weights.rs:1097-1144) with the tied-embedding fallback: a missing `output.weight` of a
// non-BitNet model is `token_embd.weight` (:1110-1126).  flock, mlock and memory admission are host
// residency policy and stay out.  Uploads go through the device registry (registry.hip), the
// RepackedTensorStore counterpart, so a tensor is copied to HBM once.
//
// Layout (the public GGUF v3 format, little-endian): magic "GGUF", u32 version, u64 tensor count,
// u64 metadata count; metadata entries (string key, u32 type, value); tensor descriptors (string
// name, u32 n_dims, u64 dims[n_dims] with dims[0] the row length, u32 ggml type, u64 offset); the
// data section starts at the next multiple of general.alignment (default 32) and every offset is
// relative to it.  Strings are u64 length + bytes.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "jero_common.h"
#include "runtime.h"

extern "C" int jero_hip_weights_register(const void* host, size_t nbytes, const void** dev_out);

namespace {

enum GgufType : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
  kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

int scalar_size(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return -1;
  }
}

// Well-formed UTF-8 (RFC 3629: shortest forms only, no surrogates, at most U+10FFFF).  GGUF
// strings are UTF-8; the reference's parser builds Rust Strings from them, which rejects the rest.
bool valid_utf8(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    int len;
    uint32_t cp;
    if (c < 0x80) { i++; continue; }
    if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
    else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
    else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
    else return false;
    if (n - i < size_t(len)) return false;
    for (int k = 1; k < len; k++) {
      if ((s[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3F);
    }
    static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
    if (cp < kMin[len] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += size_t(len);
  }
  return true;
}

struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;
  bool ok = true;
  template <typename T>
  T get() {
    T v{};
    if (!ok || n - pos < sizeof(T)) {
      ok = false;
      return v;
    }
    std::memcpy(&v, p + pos, sizeof(T));
    pos += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (!ok || len > n - pos || !valid_utf8(p + pos, size_t(len))) {
      ok = false;
      return {};
    }
    std::string s(reinterpret_cast<const char*>(p + pos), size_t(len));
    pos += size_t(len);
    return s;
  }
  void skip(uint64_t k) {
    if (!ok || k > n - pos) ok = false;
    else pos += size_t(k);
  }
};

struct Meta {
  uint32_t type = 0;
  int64_t i = 0;   // integer and bool values
  double f = 0.0;  // float values (and integers, converted)
  std::string s;
  uint64_t count = 0;  // arrays: element count (elements are skipped)
};

struct Tensor {
  int quant = 0;
  std::vector<int64_t> dims;
  uint64_t offset = 0;
  size_t nbytes = 0;
};

}  // namespace

struct jero_gguf {
  void* map = nullptr;
  size_t len = 0;
  uint32_t version = 0;
  std::string arch;
  std::map<std::string, Meta> meta;
  std::map<std::string, Tensor> tensors;
  std::vector<std::string> order;  // file order
  size_t data_start = 0;
  const uint8_t* bytes() const { return static_cast<const uint8_t*>(map); }
};

namespace {

using jero::fail;

// One metadata value at the reader (type already read).
bool read_value(Reader& r, uint32_t t, Meta& m) {
  m.type = t;
  switch (t) {
    case kU8: m.i = r.get<uint8_t>(); break;
    case kI8: m.i = r.get<int8_t>(); break;
    case kU16: m.i = r.get<uint16_t>(); break;
    case kI16: m.i = r.get<int16_t>(); break;
    case kU32: m.i = r.get<uint32_t>(); break;
    case kI32: m.i = r.get<int32_t>(); break;
    case kBool: m.i = r.get<uint8_t>() != 0; break;
    case kU64: m.i = int64_t(r.get<uint64_t>()); break;
    case kI64: m.i = r.get<int64_t>(); break;
    case kF32: m.f = r.get<float>(); return r.ok;
    case kF64: m.f = r.get<double>(); return r.ok;
    case kString: m.s = r.str(); return r.ok;
    case kArray: {
      const uint32_t et = r.get<uint32_t>();
      m.count = r.get<uint64_t>();
      if (!r.ok) return false;
      if (et == kString) {
        for (uint64_t k = 0; k < m.count && r.ok; k++) r.str();
      } else if (scalar_size(et) > 0) {
        if (m.count > (r.n - r.pos) / uint64_t(scalar_size(et))) return false;
        r.skip(m.count * uint64_t(scalar_size(et)));
      } else {
        return false;  // nested arrays: not used by model files
      }
      return r.ok;
    }
    default: return false;
  }
  m.f = double(m.i);
  return r.ok;
}

int parse(jero_gguf& g) {
  Reader r{g.bytes(), g.len};
  if (r.get<uint32_t>() != 0x46554747u) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: not a GGUF file (bad magic)");
  g.version = r.get<uint32_t>();
  if (!r.ok) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: truncated header");
  if (g.version < 2 || g.version > 3)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "gguf: version " + std::to_string(g.version) + " (2 or 3 expected)");
  const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
  if (!r.ok || n_tensors > g.len || n_kv > g.len) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: truncated header");
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key = r.str();
    const uint32_t t = r.get<uint32_t>();
    Meta m;
    if (!r.ok || !read_value(r, t, m))
      return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: bad or truncated metadata entry " + std::to_string(k));
    g.meta[key] = m;
  }
  for (uint64_t k = 0; k < n_tensors; k++) {
    std::string name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok || nd == 0 || nd > 4) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: bad tensor descriptor " + std::to_string(k));
    Tensor t;
    for (uint32_t d = 0; d < nd; d++) t.dims.push_back(int64_t(r.get<uint64_t>()));
    t.quant = int(r.get<uint32_t>());
    t.offset = r.get<uint64_t>();
    if (!r.ok) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: truncated tensor descriptor " + std::to_string(k));
    int64_t rows = 1;
    for (uint32_t d = 1; d < nd; d++) {
      if (t.dims[d] <= 0 || rows > (int64_t(1) << 40) / t.dims[d])
        return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: bad dims of tensor '" + name + "'");
      rows *= t.dims[d];
    }
    if (t.dims[0] <= 0 || t.dims[0] > (int64_t(1) << 40))
      return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: bad row length of tensor '" + name + "'");
    const int64_t rb = jero::row_bytes(t.quant, t.dims[0]);
    if (rb > 0 && rows > INT64_MAX / rb)
      return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: tensor '" + name + "' too large");
    // tensors in other formats are listed with no byte size and cannot be fetched
    t.nbytes = rb > 0 ? size_t(rb) * size_t(rows) : 0;
    if (g.tensors.count(name)) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: tensor '" + name + "' listed twice");
    g.order.push_back(name);
    g.tensors[name] = t;
  }
  uint64_t align = 32;
  auto it = g.meta.find("general.alignment");
  if (it != g.meta.end() && it->second.type != kString && it->second.type != kArray) align = uint64_t(it->second.i);
  if (align == 0 || (align & (align - 1))) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: alignment not a power of two");
  g.data_start = size_t((r.pos + align - 1) / align * align);
  for (const auto& [name, t] : g.tensors) {
    if (t.offset % align) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: tensor '" + name + "' misaligned");
    if (t.offset > g.len || g.data_start > g.len - t.offset || t.nbytes > g.len - g.data_start - t.offset)
      return fail(JERO_ERR_TENSOR_BOUNDS, "gguf: tensor '" + name + "' runs past the end of the file");
  }
  auto a = g.meta.find("general.architecture");
  if (a != g.meta.end() && a->second.type == kString) g.arch = a->second.s;
  return JERO_OK;
}

// Encoder-style architectures keep no KV cache and get no tied LM head
// (architecture_requires_kv_cache, src/memory.rs:863-868).
bool architecture_requires_kv_cache(const std::string& arch) {
  static const char* const kNoCache[] = {"modernbert", "bert", "deberta-v3", "ttm", "ft-transformer", "tabpfn-v2"};
  for (const char* a : kNoCache)
    if (arch == a) return false;
  return true;
}

// The descriptor of `name`, with the tied-embedding fallback of the reference.
const Tensor* find_tensor(const jero_gguf* g, const std::string& name) {
  auto it = g->tensors.find(name);
  if (it != g->tensors.end()) return &it->second;
  if (name == "output.weight" && architecture_requires_kv_cache(g->arch) && g->arch.rfind("bitnet", 0) != 0) {
    auto e = g->tensors.find("token_embd.weight");
    if (e != g->tensors.end()) return &e->second;
  }
  return nullptr;
}

const Meta* find_meta(const jero_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->meta.find(key);
  return it == g->meta.end() ? nullptr : &it->second;
}

}  // namespace

using namespace jero;

extern "C" int jero_hip_gguf_open(const char* path, jero_gguf** out) {
  if (!path || !out) return fail(JERO_ERR_INVALID_ARGUMENT, "gguf_open: null pointer");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf_open: cannot open ") + path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    ::close(fd);
    return fail(JERO_ERR_TENSOR_BOUNDS, std::string("gguf_open: empty or unreadable file ") + path);
  }
  void* map = mmap(nullptr, size_t(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf_open: cannot map ") + path);
  auto* g = new jero_gguf;
  g->map = map;
  g->len = size_t(st.st_size);
  const int rc = parse(*g);
  if (rc) {
    munmap(g->map, g->len);
    delete g;
    return rc;
  }
  *out = g;
  return JERO_OK;
}

extern "C" void jero_hip_gguf_close(jero_gguf* g) {
  if (!g) return;
  (void)jero_hip_weights_release(g->map, g->len);
  munmap(g->map, g->len);
  delete g;
}

extern "C" int jero_hip_gguf_info(const jero_gguf* g, int64_t* n_tensors, const char** arch) {
  if (!g) return fail(JERO_ERR_INVALID_ARGUMENT, "gguf_info: null handle");
  if (n_tensors) *n_tensors = int64_t(g->order.size());
  if (arch) *arch = g->arch.c_str();
  return JERO_OK;
}

extern "C" int jero_hip_gguf_meta_int(const jero_gguf* g, const char* key, int64_t* v) {
  const Meta* m = find_meta(g, key);
  if (!m || !v) return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf: no metadata key ") + (key ? key : "(null)"));
  if (m->type == kString || m->type == kArray || m->type == kF32 || m->type == kF64)
    return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf: metadata ") + key + " is not an integer");
  *v = m->i;
  return JERO_OK;
}

extern "C" int jero_hip_gguf_meta_float(const jero_gguf* g, const char* key, double* v) {
  const Meta* m = find_meta(g, key);
  if (!m || !v) return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf: no metadata key ") + (key ? key : "(null)"));
  if (m->type == kString || m->type == kArray)
    return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf: metadata ") + key + " is not a number");
  *v = m->f;
  return JERO_OK;
}

extern "C" int jero_hip_gguf_meta_str(const jero_gguf* g, const char* key, const char** v) {
  const Meta* m = find_meta(g, key);
  if (!m || !v) return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf: no metadata key ") + (key ? key : "(null)"));
  if (m->type != kString) return fail(JERO_ERR_INVALID_ARGUMENT, std::string("gguf: metadata ") + key + " is not a string");
  *v = m->s.c_str();
  return JERO_OK;
}

extern "C" int jero_hip_gguf_tensor_name(const jero_gguf* g, int64_t i, const char** name) {
  if (!g || !name) return fail(JERO_ERR_INVALID_ARGUMENT, "gguf_tensor_name: null pointer");
  if (i < 0 || i >= int64_t(g->order.size())) return fail(JERO_ERR_TENSOR_BOUNDS, "gguf_tensor_name: index out of range");
  *name = g->order[size_t(i)].c_str();
  return JERO_OK;
}

extern "C" int jero_hip_gguf_tensor(const jero_gguf* g, const char* name, int* quant, int* n_dims, int64_t* dims,
                                    const void** host, size_t* nbytes) {
  if (!g || !name) return fail(JERO_ERR_INVALID_ARGUMENT, "gguf_tensor: null pointer");
  const Tensor* t = find_tensor(g, name);
  if (!t) return fail(JERO_ERR_TENSOR_BOUNDS, std::string("tensor '") + name + "' not found in the model file");
  if (quant) *quant = t->quant;
  if (n_dims) *n_dims = int(t->dims.size());
  if (dims)
    for (size_t d = 0; d < 4; d++) dims[d] = d < t->dims.size() ? t->dims[d] : 1;
  if (host) *host = g->bytes() + g->data_start + t->offset;
  if (nbytes) *nbytes = t->nbytes;
  if (t->nbytes == 0)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, std::string("tensor '") + name + "': ggml type " +
                                                  std::to_string(t->quant) + " has no block size here");
  return JERO_OK;
}

extern "C" int jero_hip_gguf_upload(const jero_gguf* g, const char* name, const void** dev) {
  const void* host = nullptr;
  size_t nbytes = 0;
  const int rc = jero_hip_gguf_tensor(g, name, nullptr, nullptr, nullptr, &host, &nbytes);
  if (rc) return rc;
  return jero_hip_weights_register(host, nbytes, dev);
}
