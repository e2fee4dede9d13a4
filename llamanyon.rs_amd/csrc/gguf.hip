// gguf.hip -- GGUF reader (host) and tensor upload to the device.
//
// Replaces GgufFile::open / parse / tensor / tensor_raw_bytes
// (swamp-gguf/src/mmap.rs:27-117), TensorInfo (tensor_info.rs:8-27) and
// the metadata reader (metadata.rs:117-243) for what the matmul path needs.
// The file is mapped read-only and never copied on the host: tensor bytes
// go from the mapping to the device in one hipMemcpyAsync.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "swamp_common.hpp"
#include "swamp_gguf.h"

namespace {

constexpr uint64_t kAlign = 32;  // GGUF_ALIGNMENT (mmap.rs:13); general.alignment is not read

struct Tensor {
  std::string name;
  std::vector<uint64_t> shape;
  uint32_t dtype;
  uint64_t offset;  // absolute, in the file
  uint64_t nbytes;
};

struct Value {
  uint32_t type;
  uint64_t u = 0;  // integer types, bool (as stored)
  int64_t i = 0;   // signed types
  double f = 0;    // f32 / f64
  std::string s;   // string
};

// Cursor over the mapping; every read checks the end (UnexpectedEof).
struct Reader {
  const uint8_t *p;
  size_t n, pos = 0;
  bool ok = true;
  bool take(size_t k) {
    if (!ok || k > n - pos) return ok = false;
    return true;
  }
  template <typename T>
  T get() {
    T v{};
    if (take(sizeof(T))) {
      std::memcpy(&v, p + pos, sizeof(T));  // little-endian host, as the file
      pos += sizeof(T);
    }
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (!ok || !take(len)) return {};
    std::string s(reinterpret_cast<const char *>(p + pos), size_t(len));
    pos += size_t(len);
    return s;
  }
};

}  // namespace

struct swamp_gguf {
  int fd = -1;
  const uint8_t *map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t data_offset = 0;
  uint64_t n_kv = 0;
  std::vector<std::pair<std::string, Value>> kv;  // file order; lookups take the last
  std::vector<Tensor> tensors;
};

namespace {

// parse_metadata_value / parse_metadata_array (metadata.rs:202-243).
// Arrays are walked (their elements validated and skipped); only scalars
// are kept for lookup.
int read_value(Reader &r, uint32_t type, Value &v, int depth) {
  v.type = type;
  switch (type) {
  case SWAMP_GGUF_U8: v.u = r.get<uint8_t>(); break;
  case SWAMP_GGUF_I8: v.i = r.get<int8_t>(); break;
  case SWAMP_GGUF_U16: v.u = r.get<uint16_t>(); break;
  case SWAMP_GGUF_I16: v.i = r.get<int16_t>(); break;
  case SWAMP_GGUF_U32: v.u = r.get<uint32_t>(); break;
  case SWAMP_GGUF_I32: v.i = r.get<int32_t>(); break;
  case SWAMP_GGUF_F32: v.f = r.get<float>(); break;
  case SWAMP_GGUF_BOOL: v.u = r.get<uint8_t>(); break;
  case SWAMP_GGUF_STRING: v.s = r.str(); break;
  case SWAMP_GGUF_U64: v.u = r.get<uint64_t>(); break;
  case SWAMP_GGUF_I64: v.i = r.get<int64_t>(); break;
  case SWAMP_GGUF_F64: v.f = r.get<double>(); break;
  case SWAMP_GGUF_ARRAY: {
    const uint32_t et = r.get<uint32_t>();
    const uint64_t count = r.get<uint64_t>();
    if (!r.ok) return SWAMP_EIO;
    // the reference's array reader has no nested-array case (:226-242)
    if (et == SWAMP_GGUF_ARRAY || et > SWAMP_GGUF_F64 || depth > 0) return SWAMP_EDTYPE;
    Value e;
    for (uint64_t k = 0; k < count && r.ok; k++)
      if (int rc = read_value(r, et, e, depth + 1)) return rc;
    v.u = count;
    break;
  }
  default:
    return SWAMP_EDTYPE;
  }
  return r.ok ? SWAMP_OK : SWAMP_EIO;
}

// GgufFile::parse (mmap.rs:34-94).
int parse(swamp_gguf &g) {
  Reader r{g.map, g.size};
  if (g.size < 4) return SWAMP_EIO;
  if (std::memcmp(g.map, "GGUF", 4) != 0) return SWAMP_EMAGIC;
  r.pos = 4;
  g.version = r.get<uint32_t>();
  if (!r.ok) return SWAMP_EIO;
  if (g.version < 1 || g.version > 3) return SWAMP_EVERSION;
  const bool wide = g.version >= 2;
  const uint64_t n_t = wide ? r.get<uint64_t>() : r.get<uint32_t>();
  const uint64_t n_kv = wide ? r.get<uint64_t>() : r.get<uint32_t>();
  if (!r.ok) return SWAMP_EIO;
  g.n_kv = n_kv;
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key = r.str();
    const uint32_t type = r.get<uint32_t>();
    if (!r.ok) return SWAMP_EIO;
    Value v;
    if (int rc = read_value(r, type, v, 0)) return rc;
    g.kv.emplace_back(std::move(key), std::move(v));
  }
  for (uint64_t t = 0; t < n_t; t++) {
    Tensor ti;
    ti.name = r.str();
    const uint32_t n_dims = r.get<uint32_t>();
    if (!r.ok) return SWAMP_EIO;
    uint64_t n_elems = 1;
    for (uint32_t d = 0; d < n_dims && r.ok; d++) {
      const uint64_t dim = wide ? r.get<uint64_t>() : r.get<uint32_t>();
      ti.shape.push_back(dim);
      n_elems *= dim;
    }
    ti.dtype = r.get<uint32_t>();
    ti.offset = r.get<uint64_t>();
    if (!r.ok) return SWAMP_EIO;
    if (swamp_block_size(ti.dtype) == 0) return SWAMP_EDTYPE;  // GgmlDType::from_u32
    ti.nbytes = swamp_nbytes_for(ti.dtype, size_t(n_elems));
    g.tensors.push_back(std::move(ti));
  }
  g.data_offset = (uint64_t(r.pos) + kAlign - 1) / kAlign * kAlign;
  for (auto &t : g.tensors) t.offset += g.data_offset;
  return SWAMP_OK;
}

const Value *lookup(const swamp_gguf *g, const char *key) {
  if (!g || !key) return nullptr;
  for (size_t k = g->kv.size(); k-- > 0;)  // HashMap insert: the last duplicate wins
    if (g->kv[k].first == key) return &g->kv[k].second;
  return nullptr;
}

}  // namespace

extern "C" {

int swamp_gguf_open(const char *path, swamp_gguf **out) {
  if (!path || !out) return SWAMP_EINVAL;
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return SWAMP_EIO;
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return SWAMP_EIO;
  }
  auto *g = new swamp_gguf;
  g->fd = fd;
  g->size = size_t(st.st_size);
  if (g->size > 0) {
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      swamp_gguf_close(g);
      return SWAMP_EIO;
    }
    g->map = static_cast<const uint8_t *>(m);
  }
  if (int rc = parse(*g)) {
    swamp_gguf_close(g);
    return rc;
  }
  *out = g;
  return SWAMP_OK;
}

void swamp_gguf_close(swamp_gguf *g) {
  if (!g) return;
  if (g->map) munmap(const_cast<uint8_t *>(g->map), g->size);
  if (g->fd >= 0) ::close(g->fd);
  delete g;
}

uint32_t swamp_gguf_version(const swamp_gguf *g) { return g ? g->version : 0; }
int64_t swamp_gguf_n_tensors(const swamp_gguf *g) { return g ? int64_t(g->tensors.size()) : 0; }
int64_t swamp_gguf_n_kv(const swamp_gguf *g) { return g ? int64_t(g->n_kv) : 0; }
uint64_t swamp_gguf_data_offset(const swamp_gguf *g) { return g ? g->data_offset : 0; }
uint64_t swamp_gguf_file_size(const swamp_gguf *g) { return g ? uint64_t(g->size) : 0; }

int swamp_gguf_tensor_info(const swamp_gguf *g, int64_t i, const char **name, uint32_t *dtype,
                           int *n_dims, uint64_t dims[4], uint64_t *offset, uint64_t *nbytes) {
  if (!g || i < 0 || i >= int64_t(g->tensors.size())) return SWAMP_EINVAL;
  const Tensor &t = g->tensors[size_t(i)];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype;
  if (n_dims) *n_dims = int(t.shape.size());
  if (dims)
    for (size_t d = 0; d < 4; d++) dims[d] = d < t.shape.size() ? t.shape[d] : 0;
  if (offset) *offset = t.offset;
  if (nbytes) *nbytes = t.nbytes;
  return SWAMP_OK;
}

int64_t swamp_gguf_find(const swamp_gguf *g, const char *name) {
  if (!g || !name) return SWAMP_EINVAL;
  for (size_t i = 0; i < g->tensors.size(); i++)
    if (g->tensors[i].name == name) return int64_t(i);
  return SWAMP_ENOTFOUND;
}

int swamp_gguf_tensor_raw(const swamp_gguf *g, int64_t i, const void **ptr, size_t *len) {
  if (!g || i < 0 || i >= int64_t(g->tensors.size()) || !ptr || !len) return SWAMP_EINVAL;
  const Tensor &t = g->tensors[size_t(i)];
  if (t.offset > g->size || t.nbytes > g->size - t.offset) return SWAMP_ETENSOR;
  *ptr = g->map + t.offset;
  *len = size_t(t.nbytes);
  return SWAMP_OK;
}

int swamp_gguf_upload(const swamp_gguf *g, int64_t i, void *d_dst, size_t dst_len, void *stream) {
  const void *src = nullptr;
  size_t len = 0;
  if (!d_dst) return SWAMP_EINVAL;
  if (int rc = swamp_gguf_tensor_raw(g, i, &src, &len)) return rc;
  if (dst_len < len) return SWAMP_ESHAPE;
  if (len == 0) return SWAMP_OK;
  if (int rc = swamp_gpu_init()) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(d_dst, src, len, hipMemcpyHostToDevice, s) != hipSuccess) return SWAMP_ELAUNCH;
  // the source is the caller's mapping: finish before returning
  return hipStreamSynchronize(s) == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

int swamp_gguf_meta_type(const swamp_gguf *g, const char *key, uint32_t *type) {
  const Value *v = lookup(g, key);
  if (!v) return SWAMP_ENOTFOUND;
  if (type) *type = v->type;
  return SWAMP_OK;
}

// MetadataValue::as_u32 (metadata.rs:60-68): U8, U16, U32, I32 (bit cast).
int swamp_gguf_meta_u32(const swamp_gguf *g, const char *key, uint32_t *out) {
  const Value *v = lookup(g, key);
  if (!v || !out) return v ? SWAMP_EINVAL : SWAMP_ENOTFOUND;
  switch (v->type) {
  case SWAMP_GGUF_U8: case SWAMP_GGUF_U16: case SWAMP_GGUF_U32: *out = uint32_t(v->u); return SWAMP_OK;
  case SWAMP_GGUF_I32: *out = uint32_t(int32_t(v->i)); return SWAMP_OK;
  default: return SWAMP_ENOTFOUND;
  }
}

// MetadataValue::as_u64 (:70-80): U8, U16, U32, U64, I32 and I64 (sign-extended).
int swamp_gguf_meta_u64(const swamp_gguf *g, const char *key, uint64_t *out) {
  const Value *v = lookup(g, key);
  if (!v || !out) return v ? SWAMP_EINVAL : SWAMP_ENOTFOUND;
  switch (v->type) {
  case SWAMP_GGUF_U8: case SWAMP_GGUF_U16: case SWAMP_GGUF_U32: case SWAMP_GGUF_U64:
    *out = v->u;
    return SWAMP_OK;
  case SWAMP_GGUF_I32: case SWAMP_GGUF_I64: *out = uint64_t(v->i); return SWAMP_OK;
  default: return SWAMP_ENOTFOUND;
  }
}

// MetadataValue::as_f32 (:82-90): F32, F64 (rounded), U32, I32.
int swamp_gguf_meta_f32(const swamp_gguf *g, const char *key, float *out) {
  const Value *v = lookup(g, key);
  if (!v || !out) return v ? SWAMP_EINVAL : SWAMP_ENOTFOUND;
  switch (v->type) {
  case SWAMP_GGUF_F32: case SWAMP_GGUF_F64: *out = float(v->f); return SWAMP_OK;
  case SWAMP_GGUF_U32: *out = float(uint32_t(v->u)); return SWAMP_OK;
  case SWAMP_GGUF_I32: *out = float(int32_t(v->i)); return SWAMP_OK;
  default: return SWAMP_ENOTFOUND;
  }
}

// MetadataValue::as_str (:92-97): strings only.
int swamp_gguf_meta_str(const swamp_gguf *g, const char *key, const char **str, size_t *len) {
  const Value *v = lookup(g, key);
  if (!v || !str || !len) return v ? SWAMP_EINVAL : SWAMP_ENOTFOUND;
  if (v->type != SWAMP_GGUF_STRING) return SWAMP_ENOTFOUND;
  *str = v->s.data();
  *len = v->s.size();
  return SWAMP_OK;
}

}  // extern "C"
