// gguf_host.hip -- GGUF (v2/v3) shard reader and multi-shard tensor manifest,
// host code only: the ingest side of the library (replaces the reference's
// gguf_load_shard / gguf_load_manifest / gguf_find / gguf_tensor_pread,
// gguf.h:163-192, gguf.c:285-551).
//
// File layout (the public GGUF format): "GGUF" magic, u32 version, u64
// tensor count, u64 metadata count; metadata entries (string key, u32 value
// type, value; strings are u64 length + bytes, arrays are u32 element type +
// u64 count + elements); tensor infos (string name, u32 n_dims, u64 dims,
// u32 ggml type, u64 offset relative to the data section); the data section
// starts at the end of the infos rounded up to general.alignment (32 when
// absent).  Observable behaviour kept from the reference: versions 2 and 3
// only, 1..4 dims, a tensor whose element count is not a whole number of
// its type's blocks or whose bytes run past the end of its file is an
// error, and so is a tensor name present in two shards.
//
// The header is read through a small buffered cursor (pread windows), so a
// shard of any header size parses in one pass; tensor payloads are never
// touched here.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/fdm.h"
#include "fdm_internal.h"

namespace fdm {

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kDefaultAlign = 32;
constexpr uint64_t kMaxString = 64ull << 20;   // sanity caps on header fields
constexpr uint64_t kMaxArray = 64ull << 20;

// ggml block geometry: elements per block and bytes per block, by ggml type
// id (the ids and sizes are the ggml format's; 0 = unknown or removed id).
struct TypeGeom {
  const char* name;
  uint32_t blck, bytes;
};
constexpr TypeGeom kTypes[] = {
    {"F32", 1, 4},       {"F16", 1, 2},         {"Q4_0", 32, 18},      {"Q4_1", 32, 20},
    {nullptr, 0, 0},     {nullptr, 0, 0},       {"Q5_0", 32, 22},      {"Q5_1", 32, 24},
    {"Q8_0", 32, 34},    {"Q8_1", 32, 36},      {"Q2_K", 256, 84},     {"Q3_K", 256, 110},
    {"Q4_K", 256, 144},  {"Q5_K", 256, 176},    {"Q6_K", 256, 210},    {"Q8_K", 256, 292},
    {"IQ2_XXS", 256, 66}, {"IQ2_XS", 256, 74},  {"IQ3_XXS", 256, 98},  {"IQ1_S", 256, 50},
    {"IQ4_NL", 32, 18},  {"IQ3_S", 256, 110},   {"IQ2_S", 256, 82},    {"IQ4_XS", 256, 136},
    {"I8", 1, 1},        {"I16", 1, 2},         {"I32", 1, 4},         {"I64", 1, 8},
    {"F64", 1, 8},       {"IQ1_M", 256, 56},    {"BF16", 1, 2},
};
constexpr uint32_t kNumTypes = sizeof(kTypes) / sizeof(kTypes[0]);

int gfail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int gfail(int code, const char* fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  set_last_error(msg);
  return code;
}

// Sequential reader over a file descriptor through a refillable window.
class Cursor {
 public:
  Cursor(int fd, uint64_t size) : fd_(fd), size_(size) {}
  uint64_t pos() const { return pos_; }
  bool read(void* dst, uint64_t n) {
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n) {
      if (pos_ >= win_off_ + win_len_ || pos_ < win_off_) {
        if (!refill()) return false;
      }
      const uint64_t have = win_off_ + win_len_ - pos_;
      const uint64_t take = n < have ? n : have;
      memcpy(d, buf_.data() + (pos_ - win_off_), take);
      d += take;
      pos_ += take;
      n -= take;
    }
    return true;
  }
  bool skip(uint64_t n) {
    if (n > size_ - pos_) return false;
    pos_ += n;
    return true;
  }
  template <typename T>
  bool get(T* v) { return read(v, sizeof(T)); }
  bool str(std::string* s) {
    uint64_t n;
    if (!get(&n) || n > kMaxString || n > size_ - pos_) return false;
    s->resize(n);
    return read(&(*s)[0], n);
  }

 private:
  bool refill() {
    if (pos_ >= size_) return false;
    buf_.resize(kWindow);
    const uint64_t want = size_ - pos_ < kWindow ? size_ - pos_ : kWindow;
    uint64_t got = 0;
    while (got < want) {
      const ssize_t r = pread(fd_, buf_.data() + got, want - got, (off_t)(pos_ + got));
      if (r < 0 && errno == EINTR) continue;
      if (r <= 0) return false;
      got += (uint64_t)r;
    }
    win_off_ = pos_;
    win_len_ = got;
    return true;
  }
  static constexpr uint64_t kWindow = 1u << 20;
  int fd_;
  uint64_t size_, pos_ = 0, win_off_ = 0, win_len_ = 0;
  std::vector<uint8_t> buf_;
};

uint64_t scalar_size(uint32_t t) {
  switch (t) {
    case FDM_GGUF_UINT8: case FDM_GGUF_INT8: case FDM_GGUF_BOOL: return 1;
    case FDM_GGUF_UINT16: case FDM_GGUF_INT16: return 2;
    case FDM_GGUF_UINT32: case FDM_GGUF_INT32: case FDM_GGUF_FLOAT32: return 4;
    case FDM_GGUF_UINT64: case FDM_GGUF_INT64: case FDM_GGUF_FLOAT64: return 8;
    default: return 0;
  }
}

}  // namespace

uint64_t ggml_nbytes(uint32_t type, const uint64_t* dims, uint32_t n_dims) {
  if (type >= kNumTypes || !kTypes[type].blck || n_dims == 0 || n_dims > 4) return 0;
  uint64_t n = 1;
  for (uint32_t i = 0; i < n_dims; ++i) {
    if (dims[i] && n > UINT64_MAX / dims[i]) return 0;
    n *= dims[i];
  }
  if (n == 0 || n % kTypes[type].blck) return 0;
  return n / kTypes[type].blck * kTypes[type].bytes;
}

static int parse_kv(Cursor& c, GgufKv* kv) {
  uint32_t t;
  if (!c.str(&kv->key) || !c.get(&t)) return -1;
  kv->type = t;
  if (t == FDM_GGUF_ARRAY) {
    uint32_t et;
    uint64_t n;
    if (!c.get(&et) || !c.get(&n) || n > kMaxArray) return -1;
    kv->arr_type = et;
    kv->arr_n = n;
    if (et == FDM_GGUF_STRING) {
      for (uint64_t i = 0; i < n; ++i) {
        std::string s;
        if (!c.str(&s)) return -1;
      }
      return 0;
    }
    const uint64_t es = scalar_size(et);
    if (!es) return -1;  // nested arrays are not part of the format
    return c.skip(es * n) ? 0 : -1;
  }
  if (t == FDM_GGUF_STRING) return c.str(&kv->str) ? 0 : -1;
  const uint64_t es = scalar_size(t);
  if (!es) return -1;
  uint8_t raw[8] = {};
  if (!c.read(raw, es)) return -1;
  memcpy(&kv->raw, raw, 8);
  return 0;
}

int gguf_open_shard(GgufShard* s, const char* path) {
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return gfail(FDM_E_IO, "open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return gfail(FDM_E_IO, "fstat %s: %s", path, strerror(errno));
  }
  s->path = path;
  s->fd = fd;
  s->file_size = (uint64_t)st.st_size;
  s->alignment = kDefaultAlign;
  Cursor c(fd, s->file_size);
  uint32_t magic = 0, version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!c.get(&magic) || !c.get(&version) || !c.get(&n_tensors) || !c.get(&n_kv))
    return gfail(FDM_E_FORMAT, "%s: short header", path);
  if (magic != kGgufMagic) return gfail(FDM_E_FORMAT, "%s: bad magic 0x%08x", path, magic);
  if (version != 2 && version != 3)
    return gfail(FDM_E_FORMAT, "%s: unsupported GGUF version %u", path, version);
  s->version = version;
  if (n_kv > kMaxArray || n_tensors > kMaxArray)
    return gfail(FDM_E_FORMAT, "%s: implausible counts (%llu kv, %llu tensors)", path,
                 (unsigned long long)n_kv, (unsigned long long)n_tensors);
  s->kvs.resize(n_kv);
  for (uint64_t i = 0; i < n_kv; ++i) {
    GgufKv& kv = s->kvs[i];
    if (parse_kv(c, &kv) != 0) return gfail(FDM_E_FORMAT, "%s: bad metadata entry %llu", path, (unsigned long long)i);
    if (kv.key == "general.alignment") {
      if (kv.type == FDM_GGUF_UINT32) s->alignment = (uint32_t)kv.raw;
      else if (kv.type == FDM_GGUF_UINT64) s->alignment = kv.raw;
    }
  }
  s->tensors.resize(n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor& t = s->tensors[i];
    if (!c.str(&t.name) || !c.get(&t.n_dims))
      return gfail(FDM_E_FORMAT, "%s: bad tensor info %llu", path, (unsigned long long)i);
    if (t.n_dims == 0 || t.n_dims > 4)
      return gfail(FDM_E_FORMAT, "%s: tensor %s has %u dims", path, t.name.c_str(), t.n_dims);
    for (uint32_t d = 0; d < t.n_dims; ++d)
      if (!c.get(&t.dims[d])) return gfail(FDM_E_FORMAT, "%s: bad tensor info %s", path, t.name.c_str());
    if (!c.get(&t.type) || !c.get(&t.rel_offset))
      return gfail(FDM_E_FORMAT, "%s: bad tensor info %s", path, t.name.c_str());
    t.nbytes = ggml_nbytes(t.type, t.dims, t.n_dims);
    if (!t.nbytes)
      return gfail(FDM_E_FORMAT, "%s: tensor %s: type %u / shape is not whole blocks", path,
                   t.name.c_str(), t.type);
  }
  const uint64_t align = s->alignment ? s->alignment : kDefaultAlign;
  s->data_start = (c.pos() + align - 1) / align * align;
  for (GgufTensor& t : s->tensors) {
    t.abs_offset = s->data_start + t.rel_offset;
    if (t.abs_offset < s->data_start || t.abs_offset > s->file_size ||
        t.nbytes > s->file_size - t.abs_offset)
      return gfail(FDM_E_FORMAT, "%s: tensor %s runs past the end of the file", path, t.name.c_str());
  }
  return FDM_OK;
}

GgufManifest::~GgufManifest() {
  for (GgufShard& s : shards)
    if (s.fd >= 0) close(s.fd);
}

const GgufTensor* GgufManifest::find(const char* name) const {
  const auto it = index.find(name);
  return it == index.end() ? nullptr : &shards[it->second.first].tensors[it->second.second];
}

const GgufKv* GgufManifest::find_kv(int shard, const char* key) const {
  if (shard < 0 || shard >= (int)shards.size()) return nullptr;
  for (const GgufKv& kv : shards[shard].kvs)
    if (kv.key == key) return &kv;
  return nullptr;
}

int GgufManifest::read(const GgufTensor& t, void* dst, uint64_t n, uint64_t rel) const {
  if (rel > t.nbytes || n > t.nbytes - rel)
    return gfail(FDM_E_INVAL, "read of %llu bytes at %llu past the end of %s (%llu bytes)",
                 (unsigned long long)n, (unsigned long long)rel, t.name.c_str(),
                 (unsigned long long)t.nbytes);
  const int fd = shards[t.shard].fd;
  uint8_t* d = static_cast<uint8_t*>(dst);
  uint64_t got = 0;
  while (got < n) {
    const ssize_t r = pread(fd, d + got, n - got, (off_t)(t.abs_offset + rel + got));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0)
      return gfail(FDM_E_IO, "read of %s: %s", t.name.c_str(), r < 0 ? strerror(errno) : "end of file");
    got += (uint64_t)r;
  }
  return FDM_OK;
}

}  // namespace fdm

using fdm::GgufKv;
using fdm::GgufManifest;
using fdm::GgufTensor;

struct fdm_gguf {
  GgufManifest m;
};

extern "C" {

int fdm_gguf_open(const char* const* paths, int n_paths, fdm_gguf** out) {
  if (!out || !paths || n_paths <= 0) return fdm::gfail(FDM_E_INVAL, "no shard paths");
  *out = nullptr;
  fdm_gguf* g = new fdm_gguf;
  g->m.shards.resize(n_paths);
  for (int i = 0; i < n_paths; ++i) {
    if (!paths[i]) {
      delete g;
      return fdm::gfail(FDM_E_INVAL, "shard path %d is null", i);
    }
    if (int rc = fdm::gguf_open_shard(&g->m.shards[i], paths[i])) {
      delete g;
      return rc;
    }
  }
  for (int i = 0; i < n_paths; ++i) {
    std::vector<GgufTensor>& ts = g->m.shards[i].tensors;
    for (size_t j = 0; j < ts.size(); ++j) {
      ts[j].shard = i;
      const auto ins = g->m.index.emplace(ts[j].name, std::make_pair(i, j));
      if (!ins.second) {
        const int other = ins.first->second.first;
        const std::string name = ts[j].name;
        const std::string pa = g->m.shards[other].path, pb = g->m.shards[i].path;
        delete g;
        return fdm::gfail(FDM_E_FORMAT, "tensor %s is in two shards (%s and %s)", name.c_str(),
                          pa.c_str(), pb.c_str());
      }
      g->m.order.push_back({i, j});
    }
  }
  *out = g;
  return FDM_OK;
}

int fdm_gguf_close(fdm_gguf* g) {
  delete g;
  return FDM_OK;
}

int fdm_gguf_count(const fdm_gguf* g, int* n_shards, uint64_t* n_tensors) {
  if (!g) return fdm::gfail(FDM_E_INVAL, "null manifest");
  if (n_shards) *n_shards = (int)g->m.shards.size();
  if (n_tensors) *n_tensors = g->m.order.size();
  return FDM_OK;
}

int fdm_gguf_shard_info(const fdm_gguf* g, int shard, uint32_t* version, uint64_t* alignment,
                        uint64_t* data_start, uint64_t* n_kv, uint64_t* n_tensors) {
  if (!g || shard < 0 || shard >= (int)g->m.shards.size())
    return fdm::gfail(FDM_E_INVAL, "shard %d out of range", shard);
  const fdm::GgufShard& s = g->m.shards[shard];
  if (version) *version = s.version;
  if (alignment) *alignment = s.alignment;
  if (data_start) *data_start = s.data_start;
  if (n_kv) *n_kv = s.kvs.size();
  if (n_tensors) *n_tensors = s.tensors.size();
  return FDM_OK;
}

static void fill_info(const GgufTensor& t, fdm_gguf_tensor_info* info) {
  info->type = (int)t.type;
  info->n_dims = (int)t.n_dims;
  for (int d = 0; d < 4; ++d) info->dims[d] = d < (int)t.n_dims ? t.dims[d] : 1;
  info->nbytes = t.nbytes;
  info->offset = t.abs_offset;
  info->shard = t.shard;
}

int fdm_gguf_find(const fdm_gguf* g, const char* name, fdm_gguf_tensor_info* info) {
  if (!g || !name || !info) return fdm::gfail(FDM_E_INVAL, "null argument");
  const GgufTensor* t = g->m.find(name);
  if (!t) return fdm::gfail(FDM_E_STATE, "no tensor %s", name);
  fill_info(*t, info);
  return FDM_OK;
}

int fdm_gguf_tensor_at(const fdm_gguf* g, uint64_t i, char* name, size_t cap, fdm_gguf_tensor_info* info) {
  if (!g || i >= g->m.order.size()) return fdm::gfail(FDM_E_INVAL, "tensor index out of range");
  const auto& o = g->m.order[i];
  const GgufTensor& t = g->m.shards[o.first].tensors[o.second];
  if (name) {
    if (cap <= t.name.size()) return fdm::gfail(FDM_E_INVAL, "name buffer of %zu bytes too small", cap);
    memcpy(name, t.name.c_str(), t.name.size() + 1);
  }
  if (info) fill_info(t, info);
  return FDM_OK;
}

int fdm_gguf_find_kv(const fdm_gguf* g, int shard, const char* key, int* type, int* arr_type,
                     uint64_t* arr_n) {
  if (!g || !key) return fdm::gfail(FDM_E_INVAL, "null argument");
  const GgufKv* kv = g->m.find_kv(shard, key);
  if (!kv) return fdm::gfail(FDM_E_STATE, "no metadata key %s in shard %d", key, shard);
  if (type) *type = (int)kv->type;
  if (arr_type) *arr_type = kv->type == FDM_GGUF_ARRAY ? (int)kv->arr_type : -1;
  if (arr_n) *arr_n = kv->type == FDM_GGUF_ARRAY ? kv->arr_n : 0;
  return FDM_OK;
}

int fdm_gguf_kv_int(const fdm_gguf* g, int shard, const char* key, int64_t* v) {
  const GgufKv* kv = g && key ? g->m.find_kv(shard, key) : nullptr;
  if (!kv || !v) return fdm::gfail(FDM_E_STATE, "no metadata key %s", key ? key : "(null)");
  switch (kv->type) {
    case FDM_GGUF_UINT8: *v = (uint8_t)kv->raw; break;
    case FDM_GGUF_INT8: *v = (int8_t)kv->raw; break;
    case FDM_GGUF_UINT16: *v = (uint16_t)kv->raw; break;
    case FDM_GGUF_INT16: *v = (int16_t)kv->raw; break;
    case FDM_GGUF_UINT32: *v = (uint32_t)kv->raw; break;
    case FDM_GGUF_INT32: *v = (int32_t)kv->raw; break;
    case FDM_GGUF_UINT64: case FDM_GGUF_INT64: *v = (int64_t)kv->raw; break;
    case FDM_GGUF_BOOL: *v = (uint8_t)kv->raw != 0; break;
    default: return fdm::gfail(FDM_E_INVAL, "metadata %s is not an integer", key);
  }
  return FDM_OK;
}

int fdm_gguf_kv_float(const fdm_gguf* g, int shard, const char* key, double* v) {
  const GgufKv* kv = g && key ? g->m.find_kv(shard, key) : nullptr;
  if (!kv || !v) return fdm::gfail(FDM_E_STATE, "no metadata key %s", key ? key : "(null)");
  if (kv->type == FDM_GGUF_FLOAT32) {
    float f;
    uint32_t b = (uint32_t)kv->raw;
    memcpy(&f, &b, 4);
    *v = f;
  } else if (kv->type == FDM_GGUF_FLOAT64) {
    memcpy(v, &kv->raw, 8);
  } else {
    return fdm::gfail(FDM_E_INVAL, "metadata %s is not a float", key);
  }
  return FDM_OK;
}

int fdm_gguf_kv_str(const fdm_gguf* g, int shard, const char* key, char* buf, size_t cap) {
  const GgufKv* kv = g && key ? g->m.find_kv(shard, key) : nullptr;
  if (!kv || !buf) return fdm::gfail(FDM_E_STATE, "no metadata key %s", key ? key : "(null)");
  if (kv->type != FDM_GGUF_STRING) return fdm::gfail(FDM_E_INVAL, "metadata %s is not a string", key);
  if (cap <= kv->str.size()) return fdm::gfail(FDM_E_INVAL, "string buffer of %zu bytes too small", cap);
  memcpy(buf, kv->str.c_str(), kv->str.size() + 1);
  return FDM_OK;
}

int fdm_gguf_read(const fdm_gguf* g, const char* name, void* h_buf, uint64_t n, uint64_t rel) {
  if (!g || !name || (!h_buf && n)) return fdm::gfail(FDM_E_INVAL, "null argument");
  const GgufTensor* t = g->m.find(name);
  if (!t) return fdm::gfail(FDM_E_STATE, "no tensor %s", name);
  return g->m.read(*t, h_buf, n, rel);
}

int fdm_ggml_type_geometry(int type, uint64_t* block_elems, uint64_t* block_bytes) {
  if (type < 0 || (uint32_t)type >= fdm::kNumTypes || !fdm::kTypes[type].blck)
    return fdm::gfail(FDM_E_INVAL, "unknown ggml type %d", type);
  if (block_elems) *block_elems = fdm::kTypes[type].blck;
  if (block_bytes) *block_bytes = fdm::kTypes[type].bytes;
  return FDM_OK;
}

}  // extern "C"

namespace fdm {
const GgufManifest* gguf_manifest(const fdm_gguf* g) { return g ? &g->m : nullptr; }
}  // namespace fdm
