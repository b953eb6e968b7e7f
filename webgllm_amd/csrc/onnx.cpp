// An ONNX ModelProto reader (the reference's parseOnnxModel, src/onnx.ts:
// 71-282): the graph's nodes with their attributes, and its initializers
// with where their bytes are (inline in the memory-mapped file, or in an
// external data file). It reads the protobuf wire format directly; nothing
// in the graph is run.
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "status.h"

struct wg_onnx {};

namespace {

struct Tensor {
  std::string name;
  std::vector<int64_t> dims;
  int32_t data_type = 0;
  const uint8_t *raw = nullptr;
  uint64_t raw_bytes = 0;
  bool external = false;
  std::string location;
  int64_t offset = 0, length = -1;
  std::vector<int64_t> int64_data;
  std::vector<float> float_data;
};

struct Attr {
  std::string name;
  int32_t type = 0;
  float f = 0.0f;
  int64_t i = 0;
  std::string s;
  std::vector<int64_t> ints;
  std::vector<float> floats;
  int64_t strings = 0;
  int64_t tensor = -1;
};

struct Node {
  std::string name, op_type, domain;
  std::vector<std::string> inputs, outputs;
  std::vector<Attr> attrs;
};

struct File {
  const uint8_t *map = nullptr;
  size_t size = 0;
  std::string graph_name;
  std::vector<Node> nodes;
  std::vector<Tensor> tensors;  // initializers first, then attribute tensors
  size_t n_init = 0;
};

struct Truncated {};

// Wire-format reads over bytes [pos, end) of one message.
struct Reader {
  const uint8_t *p, *end;

  bool done() const { return p >= end; }
  uint64_t varint() {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p >= end) throw Truncated{};
      const uint8_t b = *p++;
      v |= (uint64_t)(b & 0x7f) << shift;
      if (b < 0x80) return v;
    }
    throw Truncated{};
  }
  Reader sub() {
    const uint64_t n = varint();
    if (n > (uint64_t)(end - p)) throw Truncated{};
    Reader r{p, p + n};
    p += n;
    return r;
  }
  std::string string() {
    Reader r = sub();
    return std::string((const char *)r.p, (size_t)(r.end - r.p));
  }
  float f32() {
    if (end - p < 4) throw Truncated{};
    float f;
    memcpy(&f, p, 4);
    p += 4;
    return f;
  }
  void skip(int wire) {
    switch (wire) {
      case 0: varint(); break;
      case 1:
        if (end - p < 8) throw Truncated{};
        p += 8;
        break;
      case 2: sub(); break;
      case 5:
        if (end - p < 4) throw Truncated{};
        p += 4;
        break;
      default: throw wire;  // groups (3, 4) and unknown types
    }
  }
  // A repeated varint or float field, packed (wire 2) or one element.
  void varints(int wire, std::vector<int64_t> &out) {
    if (wire == 2) {
      Reader r = sub();
      while (!r.done()) out.push_back((int64_t)r.varint());
    } else {
      out.push_back((int64_t)varint());
    }
  }
  void floats(int wire, std::vector<float> &out) {
    if (wire == 2) {
      Reader r = sub();
      while (!r.done()) out.push_back(r.f32());
    } else {
      out.push_back(f32());
    }
  }
};

// TensorProto (onnx.proto: dims 1, data_type 2, float_data 4, int64_data 7,
// name 8, raw_data 9, external_data 13, data_location 14).
Tensor read_tensor(Reader r) {
  Tensor t;
  while (!r.done()) {
    const uint64_t key = r.varint();
    const int field = (int)(key >> 3), wire = (int)(key & 7);
    if (field == 1) {
      r.varints(wire, t.dims);
    } else if (field == 2) {
      t.data_type = (int32_t)r.varint();
    } else if (field == 8) {
      t.name = r.string();
    } else if (field == 9) {
      Reader b = r.sub();
      t.raw = b.p;
      t.raw_bytes = (uint64_t)(b.end - b.p);
    } else if (field == 4) {
      r.floats(wire, t.float_data);
    } else if (field == 7) {
      r.varints(wire, t.int64_data);
    } else if (field == 13) {
      Reader e = r.sub();
      std::string k, v;
      while (!e.done()) {
        const uint64_t ek = e.varint();
        if ((ek >> 3) == 1) k = e.string();
        else if ((ek >> 3) == 2) v = e.string();
        else e.skip((int)(ek & 7));
      }
      t.external = true;
      if (k == "location") t.location = v;
      else if (k == "offset") t.offset = strtoll(v.c_str(), nullptr, 10);
      else if (k == "length") t.length = strtoll(v.c_str(), nullptr, 10);
    } else {
      r.skip(wire);
    }
  }
  return t;
}

// AttributeProto (name 1, f 2, i 3, s 4, t 5, floats 7, ints 8, strings 9, type 20).
Attr read_attr(Reader r, File &f) {
  Attr a;
  while (!r.done()) {
    const uint64_t key = r.varint();
    const int field = (int)(key >> 3), wire = (int)(key & 7);
    if (field == 1) a.name = r.string();
    else if (field == 20) a.type = (int32_t)r.varint();
    else if (field == 2) a.f = r.f32();
    else if (field == 3) a.i = (int64_t)r.varint();
    else if (field == 4) a.s = r.string();
    else if (field == 5) {
      f.tensors.push_back(read_tensor(r.sub()));
      a.tensor = (int64_t)f.tensors.size() - 1;
    } else if (field == 7) r.floats(wire, a.floats);
    else if (field == 8) r.varints(wire, a.ints);
    else if (field == 9) {
      r.sub();
      a.strings++;
    } else r.skip(wire);
  }
  return a;
}

// NodeProto (input 1, output 2, name 3, op_type 4, attribute 5, domain 7).
Node read_node(Reader r, File &f) {
  Node n;
  while (!r.done()) {
    const uint64_t key = r.varint();
    const int field = (int)(key >> 3), wire = (int)(key & 7);
    if (field == 1) n.inputs.push_back(r.string());
    else if (field == 2) n.outputs.push_back(r.string());
    else if (field == 3) n.name = r.string();
    else if (field == 4) n.op_type = r.string();
    else if (field == 7) n.domain = r.string();
    else if (field == 5) n.attrs.push_back(read_attr(r.sub(), f));
    else r.skip(wire);
  }
  return n;
}

// ModelProto's graph (field 7): GraphProto node 1, name 2, initializer 5.
// Attribute tensors read while the nodes are parsed go after the
// initializers, so initializers keep indices 0 .. n_init - 1.
int parse(File &f) {
  Reader top{f.map, f.map + f.size};
  while (!top.done()) {
    const uint64_t key = top.varint();
    if ((key >> 3) != 7 || (key & 7) != 2) {
      top.skip((int)(key & 7));
      continue;
    }
    Reader g = top.sub();
    std::vector<Tensor> attr_tensors;
    while (!g.done()) {
      const uint64_t k = g.varint();
      const int field = (int)(k >> 3), wire = (int)(k & 7);
      if (field == 1) {
        File scratch;
        f.nodes.push_back(read_node(g.sub(), scratch));
        for (auto &a : f.nodes.back().attrs)
          if (a.tensor >= 0) {
            attr_tensors.push_back(std::move(scratch.tensors[(size_t)a.tensor]));
            a.tensor = -2 - (int64_t)(attr_tensors.size() - 1);  // fixed below
          }
      } else if (field == 2) {
        f.graph_name = g.string();
      } else if (field == 5) {
        f.tensors.push_back(read_tensor(g.sub()));
      } else {
        g.skip(wire);
      }
    }
    f.n_init = f.tensors.size();
    for (auto &n : f.nodes)
      for (auto &a : n.attrs)
        if (a.tensor <= -2) a.tensor = (int64_t)f.n_init + (-2 - a.tensor);
    for (auto &t : attr_tensors) f.tensors.push_back(std::move(t));
    return WG_OK;
  }
  return wg::fail(WG_ERR_INVALID, "ONNX: no graph in the model");
}

File *as_file(const wg_onnx *h) {
  return reinterpret_cast<File *>(const_cast<wg_onnx *>(h));
}

}  // namespace

extern "C" {

int wg_onnx_open(const char *path, wg_onnx **out) {
  WG_REQUIRE(path && out, "wg_onnx_open: bad arguments");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return wg::fail(WG_ERR_INVALID, "ONNX: %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return wg::fail(WG_ERR_INVALID, "ONNX: %s: %s", path, strerror(errno));
  }
  File *f = new File;
  f->size = (size_t)st.st_size;
  if (f->size) {
    void *m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      close(fd);
      delete f;
      return wg::fail(WG_ERR_INVALID, "ONNX: %s: %s", path, strerror(errno));
    }
    f->map = static_cast<const uint8_t *>(m);
  }
  close(fd);
  int rc;
  try {
    rc = parse(*f);
  } catch (Truncated) {
    rc = wg::fail(WG_ERR_INVALID, "ONNX: truncated message");
  } catch (int wire) {
    rc = wg::fail(WG_ERR_INVALID, "ONNX: unsupported wire type %d", wire);
  } catch (...) {  // no exception leaves the C ABI (a huge count: bad_alloc)
    rc = wg::fail(WG_ERR_OOM, "ONNX: %s: out of host memory while parsing", path);
  }
  if (rc != WG_OK) {
    if (f->map) munmap((void *)f->map, f->size);
    delete f;
    return rc;
  }
  *out = reinterpret_cast<wg_onnx *>(f);
  return WG_OK;
}

int wg_onnx_close(wg_onnx *h) {
  File *f = as_file(h);
  if (!f) return WG_OK;
  if (f->map) munmap((void *)f->map, f->size);
  delete f;
  return WG_OK;
}

const char *wg_onnx_graph_name(const wg_onnx *h) { return h ? as_file(h)->graph_name.c_str() : nullptr; }

int64_t wg_onnx_node_count(const wg_onnx *h) { return h ? (int64_t)as_file(h)->nodes.size() : -1; }

int64_t wg_onnx_tensor_count(const wg_onnx *h) { return h ? (int64_t)as_file(h)->tensors.size() : -1; }

int64_t wg_onnx_init_count(const wg_onnx *h) { return h ? (int64_t)as_file(h)->n_init : -1; }

int64_t wg_onnx_find_init(const wg_onnx *h, const char *name) {
  if (!h || !name) return -1;
  File *f = as_file(h);
  for (size_t i = 0; i < f->n_init; i++)
    if (f->tensors[i].name == name) return (int64_t)i;
  return -1;
}

int wg_onnx_tensor(const wg_onnx *h, int64_t i, wg_onnx_tensor_info *out) {
  WG_REQUIRE(h && out, "wg_onnx_tensor: bad arguments");
  File *f = as_file(h);
  WG_REQUIRE(i >= 0 && (size_t)i < f->tensors.size(), "wg_onnx_tensor: no tensor %lld",
             (long long)i);
  const Tensor &t = f->tensors[(size_t)i];
  WG_REQUIRE(t.dims.size() <= 8, "ONNX: %s has %zu dims (at most 8)", t.name.c_str(),
             t.dims.size());
  memset(out, 0, sizeof(*out));
  out->name = t.name.c_str();
  out->n_dims = (int32_t)t.dims.size();
  for (size_t d = 0; d < t.dims.size(); d++) out->dims[d] = t.dims[d];
  out->data_type = t.data_type;
  out->raw = t.raw;
  out->raw_bytes = t.raw_bytes;
  out->location = t.external ? t.location.c_str() : nullptr;
  out->offset = t.offset;
  out->length = t.length;
  out->int64_data = t.int64_data.empty() ? nullptr : t.int64_data.data();
  out->n_int64 = (int64_t)t.int64_data.size();
  out->float_data = t.float_data.empty() ? nullptr : t.float_data.data();
  out->n_float = (int64_t)t.float_data.size();
  return WG_OK;
}

int wg_onnx_node(const wg_onnx *h, int64_t i, wg_onnx_node_info *out) {
  WG_REQUIRE(h && out, "wg_onnx_node: bad arguments");
  File *f = as_file(h);
  WG_REQUIRE(i >= 0 && (size_t)i < f->nodes.size(), "wg_onnx_node: no node %lld", (long long)i);
  const Node &n = f->nodes[(size_t)i];
  out->name = n.name.c_str();
  out->op_type = n.op_type.c_str();
  out->domain = n.domain.c_str();
  out->n_inputs = (int32_t)n.inputs.size();
  out->n_outputs = (int32_t)n.outputs.size();
  out->n_attrs = (int32_t)n.attrs.size();
  return WG_OK;
}

const char *wg_onnx_node_input(const wg_onnx *h, int64_t i, int32_t j) {
  if (!h || i < 0 || (size_t)i >= as_file(h)->nodes.size()) return nullptr;
  const Node &n = as_file(h)->nodes[(size_t)i];
  return j >= 0 && (size_t)j < n.inputs.size() ? n.inputs[(size_t)j].c_str() : nullptr;
}

const char *wg_onnx_node_output(const wg_onnx *h, int64_t i, int32_t j) {
  if (!h || i < 0 || (size_t)i >= as_file(h)->nodes.size()) return nullptr;
  const Node &n = as_file(h)->nodes[(size_t)i];
  return j >= 0 && (size_t)j < n.outputs.size() ? n.outputs[(size_t)j].c_str() : nullptr;
}

int wg_onnx_node_attr(const wg_onnx *h, int64_t i, int32_t j, wg_onnx_attr *out) {
  WG_REQUIRE(h && out, "wg_onnx_node_attr: bad arguments");
  File *f = as_file(h);
  WG_REQUIRE(i >= 0 && (size_t)i < f->nodes.size(), "wg_onnx_node_attr: no node %lld",
             (long long)i);
  const Node &n = f->nodes[(size_t)i];
  WG_REQUIRE(j >= 0 && (size_t)j < n.attrs.size(), "wg_onnx_node_attr: no attribute %d", j);
  const Attr &a = n.attrs[(size_t)j];
  out->name = a.name.c_str();
  out->type = a.type;
  out->f = a.f;
  out->i = a.i;
  out->s = a.s.data();
  out->s_len = (uint64_t)a.s.size();
  out->ints = a.ints.empty() ? nullptr : a.ints.data();
  out->n_ints = (int64_t)a.ints.size();
  out->floats = a.floats.empty() ? nullptr : a.floats.data();
  out->n_floats = (int64_t)a.floats.size();
  out->n_strings = a.strings;
  out->tensor = a.tensor;
  return WG_OK;
}

}  // extern "C"
