// GGUF (v2, v3) reader: the file's metadata and tensor infos, as the
// reference's readGgufHeader (src/gguf.ts:276-328), over a read-only memory
// map, so tensor bytes are handed to the device repackers without a copy
// through user memory. Arrays are kept as their offset and length and
// decoded element by element on request (readGgufArray, :346-360).
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "status.h"

namespace {

// [weights per block, bytes per block] of the ggml types (src/gguf.ts:49-71).
bool type_layout(int type, uint64_t *weights, uint64_t *bytes) {
  struct L {
    int type;
    uint64_t w, b;
  };
  static const L table[] = {{0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},
                            {6, 32, 22},   {7, 32, 24},   {8, 32, 34},   {9, 32, 36},
                            {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
                            {14, 256, 210}, {15, 256, 292}, {24, 1, 1},    {25, 1, 2},
                            {26, 1, 4},    {27, 1, 8},    {28, 1, 8},    {30, 1, 2}};
  for (const L &l : table)
    if (l.type == type) {
      *weights = l.w;
      *bytes = l.b;
      return true;
    }
  return false;
}

// Bytes of a scalar metadata value type (src/gguf.ts:117-129); 0 otherwise.
uint64_t scalar_size(uint32_t t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
  }
}

struct Meta {
  std::string key;
  uint32_t type;     // a GGUF value type
  uint32_t elem;     // arrays: element type
  uint64_t length;   // arrays: element count; strings: bytes
  uint64_t offset;   // file offset of the value (arrays: first element)
};

struct Tensor {
  std::string name;
  std::vector<int64_t> dims;
  int32_t type;
  uint64_t offset, bytes;
};

}  // namespace

struct wg_gguf {
  const uint8_t *map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  std::vector<Meta> meta;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int64_t> by_name, by_key;
  uint64_t data_offset = 0;
};

namespace {

// Sequential little-endian reads over the map; any read past the end fails.
struct Cursor {
  const uint8_t *p;
  size_t size, pos;
  bool ok = true;
  bool need(uint64_t n) {
    if (!ok || n > size - pos) ok = false;
    return ok;
  }
  uint32_t u32() {
    if (!need(4)) return 0;
    uint32_t v;
    memcpy(&v, p + pos, 4);
    pos += 4;
    return v;
  }
  uint64_t u64() {
    if (!need(8)) return 0;
    uint64_t v;
    memcpy(&v, p + pos, 8);
    pos += 8;
    return v;
  }
  void skip(uint64_t n) {
    if (need(n)) pos += n;
  }
  std::string str() {
    uint64_t n = u64();
    if (!need(n)) return std::string();
    std::string s(reinterpret_cast<const char *>(p + pos), n);
    pos += n;
    return s;
  }
};

// Skips one value of `type` (recursing into arrays), recording nothing.
bool skip_value(Cursor &c, uint32_t type, int depth) {
  if (type == 8) {
    c.skip(c.u64());
  } else if (type == 9) {
    if (depth > 0) return false;  // nested arrays (the reference rejects them too)
    uint32_t elem = c.u32();
    uint64_t n = c.u64();
    uint64_t sz = scalar_size(elem);
    if (elem == 8) {
      for (uint64_t i = 0; i < n && c.ok; i++) c.skip(c.u64());
    } else if (sz) {
      if (n > (c.size - c.pos) / sz) return c.ok = false;
      c.skip(n * sz);
    } else {
      return false;
    }
  } else {
    uint64_t sz = scalar_size(type);
    if (!sz) return false;
    c.skip(sz);
  }
  return c.ok;
}

int parse(wg_gguf *g) {
  Cursor c{g->map, g->size, 0};
  if (g->size < 24 || memcmp(g->map, "GGUF", 4) != 0)
    return wg::fail(WG_ERR_INVALID, "not a GGUF file");
  c.pos = 4;
  g->version = c.u32();
  if (g->version != 2 && g->version != 3)
    return wg::fail(WG_ERR_UNSUPPORTED, "GGUF version %u is not supported", g->version);
  uint64_t n_tensors = c.u64(), n_kv = c.u64();
  if (n_tensors > g->size / 24 || n_kv > g->size / 13)
    return wg::fail(WG_ERR_INVALID, "GGUF: counts beyond the file (%llu tensors, %llu keys)",
                    (unsigned long long)n_tensors, (unsigned long long)n_kv);
  for (uint64_t i = 0; i < n_kv; i++) {
    Meta m;
    m.key = c.str();
    m.type = c.u32();
    m.elem = 0;
    m.length = 0;
    m.offset = c.pos;
    if (m.type == 9) {
      m.elem = c.u32();
      m.length = c.u64();
      m.offset = c.pos;
      c.pos = m.offset - 12;
    } else if (m.type == 8) {
      m.length = c.u64();
      m.offset = c.pos;
      c.pos = m.offset - 8;
    }
    if (!skip_value(c, m.type, 0) || !c.ok)
      return wg::fail(WG_ERR_INVALID, "GGUF: bad metadata value %s (type %u)", m.key.c_str(),
                      m.type);
    g->by_key[m.key] = (int64_t)g->meta.size();
    g->meta.push_back(std::move(m));
  }
  for (uint64_t i = 0; i < n_tensors; i++) {
    Tensor t;
    t.name = c.str();
    uint32_t nd = c.u32();
    if (nd > 4) return wg::fail(WG_ERR_INVALID, "GGUF: %s has %u dimensions", t.name.c_str(), nd);
    for (uint32_t d = 0; d < nd; d++) t.dims.push_back((int64_t)c.u64());
    t.type = (int32_t)c.u32();
    t.offset = c.u64();  // relative to the data section for now
    if (!c.ok) return wg::fail(WG_ERR_INVALID, "GGUF: truncated tensor infos");
    g->by_name[t.name] = (int64_t)g->tensors.size();
    g->tensors.push_back(std::move(t));
  }
  // general.alignment (default 32) sets where the data section starts.
  uint64_t align = 32;
  auto a = g->by_key.find("general.alignment");
  if (a != g->by_key.end()) {
    const Meta &m = g->meta[a->second];
    if (m.type == 4 || m.type == 5) {
      uint32_t v;
      memcpy(&v, g->map + m.offset, 4);
      align = v ? v : 32;
    }
  }
  g->data_offset = (c.pos + align - 1) / align * align;
  for (Tensor &t : g->tensors) {
    uint64_t bw, bb;
    t.offset += g->data_offset;
    if (type_layout(t.type, &bw, &bb)) {
      uint64_t rows = 1, bytes = 0;
      bool over = false;
      for (size_t d = 1; d < t.dims.size(); d++)
        over |= __builtin_mul_overflow(rows, (uint64_t)t.dims[d], &rows);
      uint64_t first = t.dims.empty() ? 1 : (uint64_t)t.dims[0];
      over |= first > (1ull << 62) ||
              __builtin_mul_overflow((first + bw - 1) / bw * bb, rows, &bytes);
      t.bytes = bytes;
      if (over || t.offset > g->size || t.bytes > g->size - t.offset)
        return wg::fail(WG_ERR_INVALID, "GGUF: %s runs past the end of the file", t.name.c_str());
    } else {
      t.bytes = 0;
    }
  }
  return WG_OK;
}

void fill_value(const wg_gguf *g, const Meta &m, wg_gguf_value *out) {
  memset(out, 0, sizeof *out);
  out->key = m.key.c_str();
  out->type = (int32_t)m.type;
  out->elem_type = (int32_t)m.elem;
  out->length = m.length;
  out->offset = m.offset;
  const uint8_t *p = g->map + m.offset;
  switch (m.type) {
    case 0: out->i = p[0]; break;
    case 1: out->i = (int8_t)p[0]; break;
    case 2: { uint16_t v; memcpy(&v, p, 2); out->i = v; break; }
    case 3: { int16_t v; memcpy(&v, p, 2); out->i = v; break; }
    case 4: { uint32_t v; memcpy(&v, p, 4); out->i = v; break; }
    case 5: { int32_t v; memcpy(&v, p, 4); out->i = v; break; }
    case 6: { float v; memcpy(&v, p, 4); out->f = v; break; }
    case 7: out->i = p[0] != 0; break;
    case 8: out->s = reinterpret_cast<const char *>(p); break;
    case 10: { uint64_t v; memcpy(&v, p, 8); out->i = (int64_t)v; break; }
    case 11: { int64_t v; memcpy(&v, p, 8); out->i = v; break; }
    case 12: { double v; memcpy(&v, p, 8); out->f = v; break; }
    default: break;
  }
  if (m.type != 6 && m.type != 12) out->f = (double)out->i;
  else out->i = (int64_t)out->f;
}

}  // namespace

extern "C" {

int wg_gguf_open(const char *path, wg_gguf **out) {
  WG_REQUIRE(path && out, "wg_gguf_open: bad arguments");
  *out = nullptr;
  int fd = open(path, O_RDONLY);
  if (fd < 0) return wg::fail(WG_ERR_INVALID, "wg_gguf_open: %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return wg::fail(WG_ERR_INVALID, "wg_gguf_open: %s: empty or unreadable", path);
  }
  void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) return wg::fail(WG_ERR_OOM, "wg_gguf_open: mmap: %s", strerror(errno));
  wg_gguf *g = new wg_gguf;
  g->map = static_cast<const uint8_t *>(map);
  g->size = (size_t)st.st_size;
  int rc = parse(g);
  if (rc) {
    munmap(const_cast<uint8_t *>(g->map), g->size);
    delete g;
    return rc;
  }
  *out = g;
  return WG_OK;
}

int wg_gguf_close(wg_gguf *g) {
  if (!g) return WG_OK;
  munmap(const_cast<uint8_t *>(g->map), g->size);
  delete g;
  return WG_OK;
}

int32_t wg_gguf_version(const wg_gguf *g) { return g ? (int32_t)g->version : 0; }
int64_t wg_gguf_data_offset(const wg_gguf *g) { return g ? (int64_t)g->data_offset : -1; }
int64_t wg_gguf_tensor_count(const wg_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }
int64_t wg_gguf_meta_count(const wg_gguf *g) { return g ? (int64_t)g->meta.size() : 0; }

int64_t wg_gguf_find_tensor(const wg_gguf *g, const char *name) {
  if (!g || !name) return -1;
  auto it = g->by_name.find(name);
  return it == g->by_name.end() ? -1 : it->second;
}

int64_t wg_gguf_find_meta(const wg_gguf *g, const char *key) {
  if (!g || !key) return -1;
  auto it = g->by_key.find(key);
  return it == g->by_key.end() ? -1 : it->second;
}

int wg_gguf_tensor(const wg_gguf *g, int64_t i, wg_gguf_tensor_info *out) {
  WG_REQUIRE(g && out && i >= 0 && i < (int64_t)g->tensors.size(),
             "wg_gguf_tensor: no tensor %lld", (long long)i);
  const Tensor &t = g->tensors[i];
  memset(out, 0, sizeof *out);
  out->name = t.name.c_str();
  out->n_dims = (int32_t)t.dims.size();
  for (size_t d = 0; d < t.dims.size(); d++) out->dims[d] = t.dims[d];
  out->type = t.type;
  out->offset = t.offset;
  out->bytes = t.bytes;
  out->data = t.bytes ? g->map + t.offset : nullptr;
  return WG_OK;
}

int wg_gguf_meta(const wg_gguf *g, int64_t i, wg_gguf_value *out) {
  WG_REQUIRE(g && out && i >= 0 && i < (int64_t)g->meta.size(), "wg_gguf_meta: no key %lld",
             (long long)i);
  fill_value(g, g->meta[i], out);
  return WG_OK;
}

int wg_gguf_meta_element(const wg_gguf *g, int64_t i, uint64_t j, wg_gguf_value *out) {
  WG_REQUIRE(g && out && i >= 0 && i < (int64_t)g->meta.size(), "wg_gguf_meta_element: no key");
  const Meta &m = g->meta[i];
  WG_REQUIRE(m.type == 9, "wg_gguf_meta_element: %s is not an array", m.key.c_str());
  WG_REQUIRE(j < m.length, "wg_gguf_meta_element: %s has %llu elements", m.key.c_str(),
             (unsigned long long)m.length);
  Meta e;
  e.key = m.key;
  e.type = m.elem;
  e.elem = 0;
  e.length = 0;
  uint64_t sz = scalar_size(m.elem);
  if (sz) {
    e.offset = m.offset + j * sz;
  } else if (m.elem == 8) {
    // Strings: walk the length prefixes (bounded by the parse above).
    uint64_t pos = m.offset;
    for (uint64_t k = 0; k < j; k++) {
      uint64_t n;
      memcpy(&n, g->map + pos, 8);
      pos += 8 + n;
    }
    memcpy(&e.length, g->map + pos, 8);
    e.offset = pos + 8;
  } else {
    return wg::fail(WG_ERR_UNSUPPORTED, "wg_gguf_meta_element: element type %u", m.elem);
  }
  fill_value(g, e, out);
  out->key = m.key.c_str();
  return WG_OK;
}

}  // extern "C"
