// GGUF container reader: header, metadata and tensor table, with the tensor bytes left in a
// read-only memory mapping until one is asked for.
//
// Restates GGUFFile (Sources/IshizukiKit/Config/GGUFFile.swift:179-397) and the GGMLType geometry
// (:13-121): the same checks in the same order, the same shape convention (GGUF stores dims
// fastest-varying first; shapes here are row-major, so the table's [K, N] reads as N rows of K),
// and the same data offset (the header's end rounded up to general.alignment, default 32).
// Uploading a tensor's blocks to device memory is GGUFWeights.load's packed path
// (Sources/IshizukiKit/Core/GGUFWeights.swift:47-85) minus the model-specific renaming.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ishizuki_hip.h"

namespace ishz {
void set_error(const std::string &msg);
int fail(const char *what, hipError_t e);
int decline(const std::string &why);
int einval(const std::string &why);
}  // namespace ishz

using namespace ishz;

// ---------------------------------------------------------------- GGMLType geometry
// GGMLType.blockSize / typeSize (GGUFFile.swift:39-88); 0 for raw values outside the enum.
extern "C" int ishz_ggml_type_known(uint32_t t) {
  switch (t) {
  case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 9: case 10: case 11: case 12:
  case 13: case 14: case 15: case 16: case 17: case 18: case 19: case 20: case 21: case 22:
  case 23: case 24: case 25: case 26: case 27: case 28: case 29: case 30:
    return 1;
  }
  return 0;
}

extern "C" int ishz_ggml_geometry(uint32_t t, int *block_size, int *type_size) {
  int bs = 256, ts = 0;
  switch (t) {
  case 0: bs = 1; ts = 4; break;    // F32
  case 1: bs = 1; ts = 2; break;    // F16
  case 30: bs = 1; ts = 2; break;   // BF16
  case 28: bs = 1; ts = 8; break;   // F64
  case 24: bs = 1; ts = 1; break;   // I8
  case 25: bs = 1; ts = 2; break;   // I16
  case 26: bs = 1; ts = 4; break;   // I32
  case 27: bs = 1; ts = 8; break;   // I64
  case 2: bs = 32; ts = 18; break;  // Q4_0
  case 3: bs = 32; ts = 20; break;  // Q4_1
  case 6: bs = 32; ts = 22; break;  // Q5_0
  case 7: bs = 32; ts = 24; break;  // Q5_1
  case 8: bs = 32; ts = 34; break;  // Q8_0
  case 9: bs = 32; ts = 36; break;  // Q8_1
  case 20: bs = 32; ts = 18; break; // IQ4_NL
  case 10: ts = 84; break;          // Q2_K
  case 11: ts = 110; break;         // Q3_K
  case 12: ts = 144; break;         // Q4_K
  case 13: ts = 176; break;         // Q5_K
  case 14: ts = 210; break;         // Q6_K
  case 15: ts = 292; break;         // Q8_K
  case 16: ts = 66; break;          // IQ2_XXS
  case 17: ts = 74; break;          // IQ2_XS
  case 18: ts = 98; break;          // IQ3_XXS
  case 19: ts = 50; break;          // IQ1_S
  case 21: ts = 110; break;         // IQ3_S
  case 22: ts = 82; break;          // IQ2_S
  case 23: ts = 136; break;         // IQ4_XS
  case 29: ts = 56; break;          // IQ1_M
  default: return decline("unknown GGML type " + std::to_string(t));
  }
  if (block_size) *block_size = bs;
  if (type_size) *type_size = ts;
  return ISHZ_OK;
}

// ---------------------------------------------------------------- the reader
struct ishz_gguf_value {
  uint32_t type = 0;  // GGUF value type (0..12)
  uint64_t u = 0;
  int64_t i = 0;
  double d = 0.0;
  std::string s;
  uint32_t elem = 0;  // array element type
  std::vector<ishz_gguf_value> arr;
};

struct ishz_gguf_tensor {
  std::string name;
  int rank = 0;
  int64_t shape[4] = {0, 0, 0, 0};  // row-major (GGUF order reversed)
  uint32_t type = 0;
  uint64_t offset = 0, nbytes = 0;
};

struct ishz_gguf {
  std::string path;
  int fd = -1;
  const uint8_t *map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t data_offset = 0;
  std::vector<std::string> keys;
  std::vector<ishz_gguf_value> values;
  std::unordered_map<std::string, int64_t> kv_index;
  std::vector<ishz_gguf_tensor> tensors;
  std::unordered_map<std::string, int64_t> tensor_index;
  ~ishz_gguf() {
    if (map) munmap((void *)map, size);
    if (fd >= 0) close(fd);
  }
};

namespace {

struct ParseError {
  std::string msg;
};

struct Reader {
  const uint8_t *p;
  size_t n, pos = 0;
  void need(size_t k) {
    if (k > n - pos) throw ParseError{"GGUF header ends mid-field"};
  }
  template <class T>
  T scalar() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, p + pos, sizeof(T));  // little-endian host
    pos += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t len = scalar<uint64_t>();
    if (len >= (1ull << 28)) throw ParseError{"GGUF string length " + std::to_string(len) + " is implausible"};
    need(len);
    std::string s((const char *)p + pos, len);
    pos += len;
    return s;
  }
  ishz_gguf_value value(uint32_t type) {
    ishz_gguf_value v;
    v.type = type;
    switch (type) {
    case 0: v.u = scalar<uint8_t>(); break;
    case 1: v.i = scalar<int8_t>(); break;
    case 2: v.u = scalar<uint16_t>(); break;
    case 3: v.i = scalar<int16_t>(); break;
    case 4: v.u = scalar<uint32_t>(); break;
    case 5: v.i = scalar<int32_t>(); break;
    case 6: v.d = (double)scalar<float>(); break;
    case 7: v.u = scalar<uint8_t>() != 0; break;
    case 8: v.s = str(); break;
    case 9: {
      v.elem = scalar<uint32_t>();
      const uint64_t count = scalar<uint64_t>();
      if (count >= (1ull << 26)) throw ParseError{"GGUF array of " + std::to_string(count) + " is implausible"};
      v.arr.reserve(count);
      for (uint64_t k = 0; k < count; k++) v.arr.push_back(value(v.elem));
      break;
    }
    case 10: v.u = scalar<uint64_t>(); break;
    case 11: v.i = scalar<int64_t>(); break;
    case 12: v.d = scalar<double>(); break;
    default: throw ParseError{"GGUF metadata type " + std::to_string(type) + " is unknown"};
    }
    return v;
  }
};

const char *base_name(const std::string &path) {
  const size_t s = path.find_last_of('/');
  return path.c_str() + (s == std::string::npos ? 0 : s + 1);
}

// intValue (GGUFFile.swift:133-141): exact integers, rounded doubles, bools
bool int_value(const ishz_gguf_value &v, int64_t *out) {
  switch (v.type) {
  case 0: case 2: case 4: case 10:
    if (v.u > (uint64_t)INT64_MAX) return false;
    *out = (int64_t)v.u;
    return true;
  case 7: *out = v.u ? 1 : 0; return true;
  case 1: case 3: case 5: case 11: *out = v.i; return true;
  case 6: case 12: {
    const double r = __builtin_round(v.d);
    if (!(r >= -9.2233720368547758e18 && r < 9.2233720368547758e18)) return false;
    *out = (int64_t)r;
    return true;
  }
  }
  return false;
}

}  // namespace

extern "C" int ishz_gguf_open(const char *path, ishz_gguf **out) {
  if (!path || !out) return einval("null pointer");
  *out = nullptr;
  ishz_gguf *f = new ishz_gguf();
  f->path = path;
  f->fd = open(path, O_RDONLY);
  if (f->fd < 0) {
    delete f;
    return einval(std::string("cannot open ") + path);
  }
  struct stat st;
  if (fstat(f->fd, &st) != 0) {
    delete f;
    return einval(std::string("cannot stat ") + path);
  }
  f->size = (size_t)st.st_size;
  if (f->size) {
    void *m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) {
      delete f;
      return einval(std::string("cannot map ") + path);
    }
    f->map = (const uint8_t *)m;
  }
  try {
    Reader r{f->map, f->size};
    if (r.scalar<uint32_t>() != 0x46554747u) throw ParseError{std::string(base_name(f->path)) + " is not a GGUF file"};
    f->version = r.scalar<uint32_t>();
    if (f->version != 2 && f->version != 3)
      throw ParseError{"GGUF version " + std::to_string(f->version) + " is not supported"};
    const uint64_t tensor_count = r.scalar<uint64_t>(), kv_count = r.scalar<uint64_t>();
    if (tensor_count >= 1000000 || kv_count >= 1000000) throw ParseError{"GGUF header counts are implausible"};
    for (uint64_t k = 0; k < kv_count; k++) {
      std::string key = r.str();
      const uint32_t type = r.scalar<uint32_t>();
      ishz_gguf_value v = r.value(type);
      auto it = f->kv_index.find(key);
      if (it != f->kv_index.end()) {  // a repeated key keeps the last value, as a dictionary would
        f->values[it->second] = std::move(v);
      } else {
        f->kv_index[key] = (int64_t)f->keys.size();
        f->keys.push_back(std::move(key));
        f->values.push_back(std::move(v));
      }
    }
    int64_t alignment = 32;
    auto al = f->kv_index.find("general.alignment");
    if (al != f->kv_index.end() && !int_value(f->values[al->second], &alignment)) alignment = 32;
    if (alignment <= 0 || (alignment & (alignment - 1)))
      throw ParseError{"GGUF alignment " + std::to_string(alignment) + " is not a power of two"};
    for (uint64_t k = 0; k < tensor_count; k++) {
      ishz_gguf_tensor t;
      t.name = r.str();
      const uint32_t rank = r.scalar<uint32_t>();
      if (rank < 1 || rank > 4) throw ParseError{t.name + " has rank " + std::to_string(rank)};
      t.rank = (int)rank;
      uint64_t dims[4];
      for (uint32_t d = 0; d < rank; d++) dims[d] = r.scalar<uint64_t>();
      for (uint32_t d = 0; d < rank; d++) t.shape[d] = (int64_t)dims[rank - 1 - d];
      t.type = r.scalar<uint32_t>();
      if (!ishz_ggml_type_known(t.type)) throw ParseError{t.name + " has unknown GGML type " + std::to_string(t.type)};
      t.offset = r.scalar<uint64_t>();
      int bs = 1, ts = 1;
      ishz_ggml_geometry(t.type, &bs, &ts);
      unsigned __int128 elements = 1;
      for (uint32_t d = 0; d < rank; d++) elements *= dims[d];
      if (elements % (unsigned)bs)
        throw ParseError{t.name + " has " + std::to_string((uint64_t)elements) + " elements, not a multiple of its " +
                         std::to_string(bs) + "-element block"};
      t.nbytes = (uint64_t)(elements / (unsigned)bs * (unsigned)ts);
      f->tensor_index[t.name] = (int64_t)f->tensors.size();
      f->tensors.push_back(std::move(t));
    }
    f->data_offset = (r.pos + (uint64_t)alignment - 1) / (uint64_t)alignment * (uint64_t)alignment;
  } catch (const ParseError &e) {
    delete f;
    return einval(e.msg);
  }
  *out = f;
  return ISHZ_OK;
}

extern "C" void ishz_gguf_close(ishz_gguf *f) { delete f; }
extern "C" uint32_t ishz_gguf_version(const ishz_gguf *f) { return f ? f->version : 0; }
extern "C" uint64_t ishz_gguf_data_offset(const ishz_gguf *f) { return f ? f->data_offset : 0; }
extern "C" int64_t ishz_gguf_tensor_count(const ishz_gguf *f) { return f ? (int64_t)f->tensors.size() : 0; }

extern "C" int64_t ishz_gguf_find_tensor(const ishz_gguf *f, const char *name) {
  if (!f || !name) return -1;
  auto it = f->tensor_index.find(name);
  return it == f->tensor_index.end() ? -1 : it->second;
}

extern "C" int ishz_gguf_tensor_info(const ishz_gguf *f, int64_t i, const char **name, int *rank, int64_t *shape,
                                     uint32_t *type, uint64_t *offset, uint64_t *nbytes) {
  if (!f || i < 0 || i >= (int64_t)f->tensors.size()) return einval("tensor index out of range");
  const ishz_gguf_tensor &t = f->tensors[i];
  if (name) *name = t.name.c_str();
  if (rank) *rank = t.rank;
  if (shape)
    for (int d = 0; d < 4; d++) shape[d] = d < t.rank ? t.shape[d] : 0;
  if (type) *type = t.type;
  if (offset) *offset = t.offset;
  if (nbytes) *nbytes = t.nbytes;
  return ISHZ_OK;
}

// data(for:) (GGUFFile.swift:289-301): the bytes at data_offset + offset, or an error when they
// run past the end of the file.
extern "C" const void *ishz_gguf_tensor_data(const ishz_gguf *f, int64_t i) {
  if (!f || i < 0 || i >= (int64_t)f->tensors.size()) {
    einval("tensor index out of range");
    return nullptr;
  }
  const ishz_gguf_tensor &t = f->tensors[i];
  const uint64_t at = f->data_offset + t.offset;
  if (at > f->size || t.nbytes > f->size - at) {
    einval(t.name + " runs past the end of " + base_name(f->path));
    return nullptr;
  }
  return f->map + at;
}

// GGUFWeights.load's packed path: a quantized tensor's blocks as they lie on disk, into device
// memory the caller owns (dst_bytes >= the tensor's byte count), ordered on `stream`. The host
// side is the read-only mapping; the copy is synchronous with respect to the host buffer.
extern "C" int ishz_gguf_tensor_upload(const ishz_gguf *f, int64_t i, void *dst, size_t dst_bytes,
                                       ishz_stream_t stream) {
  const void *src = ishz_gguf_tensor_data(f, i);
  if (!src) return ISHZ_EINVAL;
  const uint64_t n = f->tensors[i].nbytes;
  if (!dst || dst_bytes < n) return einval("destination too small for " + f->tensors[i].name);
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail("gguf tensor upload", e);
  return ISHZ_OK;
}

// ---------------------------------------------------------------- metadata
extern "C" int64_t ishz_gguf_kv_count(const ishz_gguf *f) { return f ? (int64_t)f->keys.size() : 0; }

extern "C" const char *ishz_gguf_kv_key(const ishz_gguf *f, int64_t i) {
  return f && i >= 0 && i < (int64_t)f->keys.size() ? f->keys[i].c_str() : nullptr;
}

extern "C" int64_t ishz_gguf_find_kv(const ishz_gguf *f, const char *key) {
  if (!f || !key) return -1;
  auto it = f->kv_index.find(key);
  return it == f->kv_index.end() ? -1 : it->second;
}

extern "C" const ishz_gguf_value *ishz_gguf_kv_value(const ishz_gguf *f, int64_t i) {
  return f && i >= 0 && i < (int64_t)f->values.size() ? &f->values[i] : nullptr;
}

extern "C" int ishz_gguf_value_type(const ishz_gguf_value *v) { return v ? (int)v->type : -1; }

extern "C" int64_t ishz_gguf_value_len(const ishz_gguf_value *v) {
  return v && v->type == 9 ? (int64_t)v->arr.size() : -1;
}

extern "C" const ishz_gguf_value *ishz_gguf_value_elem(const ishz_gguf_value *v, int64_t j) {
  return v && v->type == 9 && j >= 0 && j < (int64_t)v->arr.size() ? &v->arr[j] : nullptr;
}

// Scalars as the reference's accessors see them: intValue, floatValue, boolValue, stringValue
// (GGUFFile.swift:133-167). ISHZ_DECLINED when the value has no such reading.
extern "C" int ishz_gguf_value_int(const ishz_gguf_value *v, int64_t *out) {
  if (!v || !out) return einval("null pointer");
  return int_value(*v, out) ? ISHZ_OK : ISHZ_DECLINED;
}

extern "C" int ishz_gguf_value_float(const ishz_gguf_value *v, double *out) {
  if (!v || !out) return einval("null pointer");
  switch (v->type) {
  case 0: case 2: case 4: case 10: *out = (double)(float)v->u; return ISHZ_OK;
  case 1: case 3: case 5: case 11: *out = (double)(float)v->i; return ISHZ_OK;
  case 6: case 12: *out = (double)(float)v->d; return ISHZ_OK;
  }
  return ISHZ_DECLINED;
}

extern "C" int ishz_gguf_value_bool(const ishz_gguf_value *v, int *out) {
  if (!v || !out) return einval("null pointer");
  switch (v->type) {
  case 7: case 0: case 2: case 4: case 10: *out = v->u != 0; return ISHZ_OK;
  case 1: case 3: case 5: case 11: *out = v->i != 0; return ISHZ_OK;
  }
  return ISHZ_DECLINED;
}

extern "C" int ishz_gguf_value_string(const ishz_gguf_value *v, const char **s, size_t *len) {
  if (!v || !s) return einval("null pointer");
  if (v->type != 8) return ISHZ_DECLINED;
  *s = v->s.data();
  if (len) *len = v->s.size();
  return ISHZ_OK;
}

// The raw payload of a scalar (for a caller that wants the exact stored bits): u for unsigned
// and bool types, i for signed, d for floats.
extern "C" int ishz_gguf_value_raw(const ishz_gguf_value *v, uint64_t *u, int64_t *i, double *d) {
  if (!v) return einval("null pointer");
  if (u) *u = v->u;
  if (i) *i = v->i;
  if (d) *d = v->d;
  return ISHZ_OK;
}
