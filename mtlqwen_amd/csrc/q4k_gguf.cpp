// GGUF reader for the Q4_K path: maps a model file read-only, indexes its
// metadata and tensor table, and uploads Q4_K tensors as q4k_weight handles.
//
// Replaces the reference's use of ggml's gguf_init_from_buffer over the
// mapped model file (model/qwen35/forward.cpp:12-23, loadWeights): tensor
// name, type, shape (ne[0] = k fastest, ne[1] = n) and byte range.  The
// container layout follows the published GGUF format (versions 2 and 3,
// little-endian):
//   "GGUF", u32 version, u64 tensor count, u64 metadata count,
//   metadata: string key, u32 value type, value
//     (strings are u64 length + bytes; arrays are u32 element type,
//      u64 count, elements),
//   tensor infos: string name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
//     u64 offset within the data section,
//   padding to general.alignment (default 32), then the data section.
// Every read is bounds-checked against the mapping, so a truncated or
// malformed file yields Q4K_EFORMAT, never an out-of-range access.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/q4k.h"

// Defined in q4k_api.hip: records the thread's last error message.
int q4k_internal_fail(int code, const char* msg);

namespace {

int gfail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return q4k_internal_fail(code, buf);
}

enum GgufType : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
  kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};

// Bytes of one scalar metadata value (0: not a fixed-size scalar).
size_t scalar_bytes(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

// (elements per block, bytes per block) of the ggml tensor types the reader
// sizes; the values are the ggml file format's block records.
bool ggml_block(uint32_t type, uint64_t* elems, uint64_t* bytes) {
  struct B { uint32_t type; uint64_t elems, bytes; };
  static const B table[] = {
      {0, 1, 4},      // F32
      {1, 1, 2},      // F16
      {2, 32, 18},    // Q4_0
      {3, 32, 20},    // Q4_1
      {6, 32, 22},    // Q5_0
      {7, 32, 24},    // Q5_1
      {8, 32, 34},    // Q8_0
      {9, 32, 36},    // Q8_1
      {10, 256, 84},  // Q2_K
      {11, 256, 110}, // Q3_K
      {12, 256, 144}, // Q4_K
      {13, 256, 176}, // Q5_K
      {14, 256, 210}, // Q6_K
      {15, 256, 292}, // Q8_K
      {23, 256, 136}, // IQ4_XS
      {24, 1, 1},     // I8
      {25, 1, 2},     // I16
      {26, 1, 4},     // I32
      {27, 1, 8},     // I64
      {28, 1, 8},     // F64
      {30, 1, 2},     // BF16
  };
  for (const B& b : table)
    if (b.type == type) {
      *elems = b.elems;
      *bytes = b.bytes;
      return true;
    }
  return false;
}

struct Meta {
  uint32_t type = 0;
  uint64_t pos = 0;  // file offset of the value
  int64_t ival = 0;  // integer / bool value
  bool has_int = false;
  std::string sval;
  bool has_str = false;
};

struct Tensor {
  std::string name;
  uint32_t type = 0, n_dims = 0;
  uint64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0;  // within the data section
  uint64_t bytes = 0;   // 0 when the type's block size is unknown
};

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t* base;
  uint64_t size, pos = 0;
  bool ok = true;

  bool take(void* dst, uint64_t n) {
    if (!ok || n > size - pos) {
      ok = false;
      return false;
    }
    memcpy(dst, base + pos, n);
    pos += n;
    return true;
  }
  bool skip(uint64_t n) {
    if (!ok || n > size - pos) {
      ok = false;
      return false;
    }
    pos += n;
    return true;
  }
  uint32_t u32() {
    uint32_t v = 0;
    take(&v, 4);
    return v;
  }
  uint64_t u64() {
    uint64_t v = 0;
    take(&v, 8);
    return v;
  }
  bool str(std::string* s) {
    const uint64_t n = u64();
    if (!ok || n > size - pos) {
      ok = false;
      return false;
    }
    if (s)
      s->assign(reinterpret_cast<const char*>(base + pos), (size_t)n);
    pos += n;
    return true;
  }
};

}  // namespace

struct q4k_gguf {
  void* map = nullptr;
  uint64_t size = 0;
  uint32_t version = 0;
  uint64_t data_offset = 0;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, uint64_t> by_name;
  std::unordered_map<std::string, Meta> meta;
};

namespace {

// Skips (or reads, for scalars and strings) one metadata value of type t.
bool read_value(Cursor& c, uint32_t t, Meta* m) {
  if (t == kString) {
    std::string s;
    if (!c.str(m ? &s : nullptr))
      return false;
    if (m) {
      m->sval = std::move(s);
      m->has_str = true;
    }
    return true;
  }
  if (t == kArray) {
    const uint32_t et = c.u32();
    const uint64_t n = c.u64();
    if (!c.ok)
      return false;
    if (et == kString) {
      for (uint64_t i = 0; i < n; ++i)
        if (!c.str(nullptr))
          return false;
      return true;
    }
    if (et == kArray) {  // arrays of arrays of scalars
      for (uint64_t i = 0; i < n; ++i) {
        const uint32_t t2 = c.u32();
        const uint64_t n2 = c.u64();
        const size_t sb = scalar_bytes(t2);
        if (!c.ok || sb == 0 || n2 > (c.size - c.pos) / sb)
          return c.ok = false;
        c.skip(n2 * sb);
      }
      return c.ok;
    }
    const size_t sb = scalar_bytes(et);
    if (sb == 0 || n > (c.size - c.pos) / sb)
      return c.ok = false;
    return c.skip(n * sb);
  }
  const size_t sb = scalar_bytes(t);
  if (sb == 0)
    return c.ok = false;
  uint8_t raw[8] = {0};
  if (!c.take(raw, sb))
    return false;
  if (m && t != kF32 && t != kF64) {
    int64_t v = 0;
    switch (t) {
      case kU8: case kBool: v = raw[0]; break;
      case kI8: v = (int8_t)raw[0]; break;
      case kU16: { uint16_t x; memcpy(&x, raw, 2); v = x; break; }
      case kI16: { int16_t x; memcpy(&x, raw, 2); v = x; break; }
      case kU32: { uint32_t x; memcpy(&x, raw, 4); v = x; break; }
      case kI32: { int32_t x; memcpy(&x, raw, 4); v = x; break; }
      case kU64: { uint64_t x; memcpy(&x, raw, 8); v = (int64_t)x; break; }
      case kI64: { int64_t x; memcpy(&x, raw, 8); v = x; break; }
    }
    m->ival = v;
    m->has_int = true;
  }
  return true;
}

int parse(q4k_gguf* g) {
  Cursor c{static_cast<const uint8_t*>(g->map), g->size};
  char magic[4];
  if (!c.take(magic, 4) || memcmp(magic, "GGUF", 4) != 0)
    return gfail(Q4K_EFORMAT, "not a GGUF file (bad magic)");
  g->version = c.u32();
  if (!c.ok || (g->version != 2 && g->version != 3))
    return gfail(Q4K_EFORMAT, "unsupported GGUF version %u", g->version);
  const uint64_t n_tensors = c.u64(), n_kv = c.u64();
  if (!c.ok)
    return gfail(Q4K_EFORMAT, "truncated GGUF header");
  // Every metadata entry and tensor info takes at least 12 / 24 bytes.
  if (n_kv > g->size / 12 || n_tensors > g->size / 24)
    return gfail(Q4K_EFORMAT, "GGUF counts exceed the file size");
  uint64_t alignment = 32;
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key;
    if (!c.str(&key))
      return gfail(Q4K_EFORMAT, "truncated metadata key %llu", (unsigned long long)i);
    Meta m;
    m.type = c.u32();
    m.pos = c.pos;
    if (!c.ok || !read_value(c, m.type, &m))
      return gfail(Q4K_EFORMAT, "bad or truncated metadata value for '%s'", key.c_str());
    if (key == "general.alignment") {
      if (!m.has_int || m.ival <= 0 || (m.ival & (m.ival - 1)) != 0)
        return gfail(Q4K_EFORMAT, "general.alignment must be a power of two");
      alignment = (uint64_t)m.ival;
    }
    g->meta[key] = std::move(m);
  }
  g->tensors.resize((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Tensor& t = g->tensors[(size_t)i];
    if (!c.str(&t.name))
      return gfail(Q4K_EFORMAT, "truncated tensor info %llu", (unsigned long long)i);
    t.n_dims = c.u32();
    if (!c.ok || t.n_dims == 0 || t.n_dims > 4)
      return gfail(Q4K_EFORMAT, "tensor '%s': %u dimensions", t.name.c_str(), t.n_dims);
    uint64_t elems = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      t.ne[d] = c.u64();
      if (t.ne[d] == 0 || elems > (UINT64_MAX >> 1) / t.ne[d])
        return gfail(Q4K_EFORMAT, "tensor '%s': bad dimension", t.name.c_str());
      elems *= t.ne[d];
    }
    t.type = c.u32();
    t.offset = c.u64();
    if (!c.ok)
      return gfail(Q4K_EFORMAT, "truncated tensor info '%s'", t.name.c_str());
    if (t.offset % alignment != 0)
      return gfail(Q4K_EFORMAT, "tensor '%s': offset not aligned to %llu", t.name.c_str(), (unsigned long long)alignment);
    uint64_t be = 0, bb = 0;
    if (ggml_block(t.type, &be, &bb)) {
      if (t.ne[0] % be != 0)
        return gfail(Q4K_EFORMAT, "tensor '%s': row of %llu elements is not whole blocks", t.name.c_str(), (unsigned long long)t.ne[0]);
      if (elems / be > UINT64_MAX / bb)
        return gfail(Q4K_EFORMAT, "tensor '%s': size overflows", t.name.c_str());
      t.bytes = elems / be * bb;
    }
    if (!g->by_name.emplace(t.name, i).second)
      return gfail(Q4K_EFORMAT, "duplicate tensor name '%s'", t.name.c_str());
  }
  g->data_offset = (c.pos + alignment - 1) / alignment * alignment;
  if (g->data_offset > g->size && n_tensors > 0)
    return gfail(Q4K_EFORMAT, "data section starts past the end of the file");
  for (const Tensor& t : g->tensors) {
    const uint64_t avail = g->size - (g->data_offset < g->size ? g->data_offset : g->size);
    if (t.offset > avail || t.bytes > avail - t.offset)
      return gfail(Q4K_EFORMAT, "tensor '%s' extends past the end of the file", t.name.c_str());
  }
  return Q4K_OK;
}

}  // namespace

extern "C" {

int q4k_gguf_open(const char* path, q4k_gguf** out) {
  if (!path || !out)
    return gfail(Q4K_EINVAL, "null argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0)
    return gfail(Q4K_ENOTFOUND, "cannot open '%s'", path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return gfail(Q4K_EFORMAT, "'%s' is empty or unreadable", path);
  }
  void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED)
    return gfail(Q4K_ENOMEM, "cannot map '%s'", path);
  q4k_gguf* g = new (std::nothrow) q4k_gguf;
  if (!g) {
    munmap(map, (size_t)st.st_size);
    return gfail(Q4K_ENOMEM, "out of host memory");
  }
  g->map = map;
  g->size = (uint64_t)st.st_size;
  int rc = parse(g);
  if (rc) {
    q4k_gguf_close(g);
    return rc;
  }
  *out = g;
  return Q4K_OK;
}

int q4k_gguf_close(q4k_gguf* g) {
  if (!g)
    return gfail(Q4K_EINVAL, "null handle");
  if (g->map)
    munmap(g->map, (size_t)g->size);
  delete g;
  return Q4K_OK;
}

int q4k_gguf_info(const q4k_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv, uint64_t* data_offset, uint64_t* file_bytes) {
  if (!g)
    return gfail(Q4K_EINVAL, "null handle");
  if (version)
    *version = g->version;
  if (n_tensors)
    *n_tensors = g->tensors.size();
  if (n_kv)
    *n_kv = g->meta.size();
  if (data_offset)
    *data_offset = g->data_offset;
  if (file_bytes)
    *file_bytes = g->size;
  return Q4K_OK;
}

int q4k_gguf_tensor(const q4k_gguf* g, uint64_t i, char* name, size_t name_len, uint32_t* ggml_type, uint32_t* n_dims, uint64_t ne[4],
                    uint64_t* file_offset, uint64_t* bytes) {
  if (!g)
    return gfail(Q4K_EINVAL, "null handle");
  if (i >= g->tensors.size())
    return gfail(Q4K_ENOTFOUND, "tensor index %llu out of range", (unsigned long long)i);
  const Tensor& t = g->tensors[(size_t)i];
  if (name && name_len) {
    if (t.name.size() >= name_len)
      return gfail(Q4K_EINVAL, "name buffer of %zu bytes is too small for '%s'", name_len, t.name.c_str());
    memcpy(name, t.name.c_str(), t.name.size() + 1);
  }
  if (ggml_type)
    *ggml_type = t.type;
  if (n_dims)
    *n_dims = t.n_dims;
  if (ne)
    for (int d = 0; d < 4; ++d)
      ne[d] = t.ne[d];
  if (file_offset)
    *file_offset = g->data_offset + t.offset;
  if (bytes)
    *bytes = t.bytes;
  return Q4K_OK;
}

int q4k_gguf_find(const q4k_gguf* g, const char* name, uint64_t* index) {
  if (!g || !name || !index)
    return gfail(Q4K_EINVAL, "null argument");
  auto it = g->by_name.find(name);
  if (it == g->by_name.end())
    return gfail(Q4K_ENOTFOUND, "missing weight %s", name);  // forward.cpp:39-40
  *index = it->second;
  return Q4K_OK;
}

int q4k_gguf_tensor_data(const q4k_gguf* g, uint64_t i, const void** data, uint64_t* bytes) {
  if (!g || !data)
    return gfail(Q4K_EINVAL, "null argument");
  if (i >= g->tensors.size())
    return gfail(Q4K_ENOTFOUND, "tensor index %llu out of range", (unsigned long long)i);
  const Tensor& t = g->tensors[(size_t)i];
  *data = static_cast<const uint8_t*>(g->map) + g->data_offset + t.offset;
  if (bytes)
    *bytes = t.bytes;
  return Q4K_OK;
}

int q4k_gguf_meta_int(const q4k_gguf* g, const char* key, int64_t* value) {
  if (!g || !key || !value)
    return gfail(Q4K_EINVAL, "null argument");
  auto it = g->meta.find(key);
  if (it == g->meta.end())
    return gfail(Q4K_ENOTFOUND, "missing metadata key %s", key);
  if (!it->second.has_int)
    return gfail(Q4K_EINVAL, "metadata key %s is not an integer", key);
  *value = it->second.ival;
  return Q4K_OK;
}

int q4k_gguf_meta_str(const q4k_gguf* g, const char* key, char* buf, size_t len) {
  if (!g || !key || !buf || len == 0)
    return gfail(Q4K_EINVAL, "null argument");
  auto it = g->meta.find(key);
  if (it == g->meta.end())
    return gfail(Q4K_ENOTFOUND, "missing metadata key %s", key);
  if (!it->second.has_str)
    return gfail(Q4K_EINVAL, "metadata key %s is not a string", key);
  if (it->second.sval.size() >= len)
    return gfail(Q4K_EINVAL, "buffer of %zu bytes is too small for metadata key %s", len, key);
  memcpy(buf, it->second.sval.c_str(), it->second.sval.size() + 1);
  return Q4K_OK;
}

int q4k_weight_from_gguf(const q4k_gguf* g, const char* name, int device, q4k_weight** out) {
  if (!g || !name || !out)
    return gfail(Q4K_EINVAL, "null argument");
  uint64_t i = 0;
  int rc = q4k_gguf_find(g, name, &i);
  if (rc)
    return rc;
  const Tensor& t = g->tensors[(size_t)i];
  if (t.type != Q4K_GGML_TYPE_Q4_K && t.type != Q4K_GGML_TYPE_Q6_K && t.type != Q4K_GGML_TYPE_Q8_0 && t.type != Q4K_GGML_TYPE_Q5_K &&
      t.type != Q4K_GGML_TYPE_IQ4_XS)
    return gfail(Q4K_ETYPE, "tensor %s has ggml type %u, not one the linear path serves", name, t.type);
  if (t.n_dims != 2 || t.ne[0] > UINT32_MAX || t.ne[1] > UINT32_MAX)
    return gfail(Q4K_ESHAPE, "tensor %s is not a 2-D matrix within 32-bit dimensions", name);
  const void* data = static_cast<const uint8_t*>(g->map) + g->data_offset + t.offset;
  // Weight{view, n = ne[1], k = ne[0], type} (forward.cpp:18-21).
  return q4k_weight_create(data, (size_t)t.bytes, (uint32_t)t.ne[1], (uint32_t)t.ne[0], t.type, device, out);
}

}  // extern "C"
