// gqk_gguf.cpp - GGUF v3 file reader and the load path from a file's tensor to device tiles.
//
// The reference gets its tensors from vLLM's GGUF loader (gguf-py 0.17.1's GGUFReader,
// gguf-plugin/requirements.txt:1) and repacks them at load time in _create_tiles
// (gguf-plugin/patches/gguf-tiles-all-types.patch:59-131).  Here the file is read by this C++
// reader (memory-mapped, read only, no copies of tensor data) and a tensor goes from the mapping
// to the caller's device tiles with one host-to-device copy into a caller-provided staging buffer
// and one repack launch.
//
// Format (GGUF version 3, little endian): magic "GGUF", u32 version, u64 tensor count, u64
// key/value count, the key/values (string key, u32 value type, value), the tensor infos (string
// name, u32 n_dims, u64 dims[n_dims], u32 ggml type, u64 offset), padding to the alignment
// (metadata key general.alignment, default 32), then the data section; a tensor's offset is
// relative to the data section.  Strings are u64 length + bytes.  Arrays are u32 element type +
// u64 count + elements.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "gguf_hip.h"
#include "gqk_common.h"

namespace {

// (block size, bytes per block) of every GGML type id with a fixed size, as gguf-py's
// GGML_QUANT_SIZES; {0, 0} for ids without one (removed or unknown types)
struct TypeSize {
  int32_t block, bytes;
};
TypeSize type_size(int t) {
  switch (t) {
    case 0: return {1, 4};       // F32
    case 1: return {1, 2};       // F16
    case 2: return {32, 18};     // Q4_0
    case 3: return {32, 20};     // Q4_1
    case 6: return {32, 22};     // Q5_0
    case 7: return {32, 24};     // Q5_1
    case 8: return {32, 34};     // Q8_0
    case 9: return {32, 36};     // Q8_1
    case 10: return {256, 84};   // Q2_K
    case 11: return {256, 110};  // Q3_K
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 15: return {256, 292};  // Q8_K
    case 16: return {256, 66};   // IQ2_XXS
    case 17: return {256, 74};   // IQ2_XS
    case 18: return {256, 98};   // IQ3_XXS
    case 19: return {256, 50};   // IQ1_S
    case 20: return {32, 18};    // IQ4_NL
    case 21: return {256, 110};  // IQ3_S
    case 22: return {256, 82};   // IQ2_S
    case 23: return {256, 136};  // IQ4_XS
    case 24: return {1, 1};      // I8
    case 25: return {1, 2};      // I16
    case 26: return {1, 4};      // I32
    case 27: return {1, 8};      // I64
    case 28: return {1, 8};      // F64
    case 29: return {256, 56};   // IQ1_M
    case 30: return {1, 2};      // BF16
    case 34: return {256, 54};   // TQ1_0
    case 35: return {256, 66};   // TQ2_0
    case 39: return {32, 17};    // MXFP4
    default: return {0, 0};
  }
}

// GGUF value types
enum { V_U8 = 0, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };
int scalar_bytes(int vt) {
  switch (vt) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
  }
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  gqk_set_last_error(buf);
  return code;
}

}  // namespace

struct gqk_gguf {
  const uint8_t* base = nullptr;   // the mapping
  size_t size = 0;
  int32_t version = 0;
  int64_t alignment = 32;
  int64_t data_offset = 0;
  std::vector<std::string> tensor_names, keys;
  std::vector<gqk_gguf_tensor> tensors;
  std::vector<gqk_gguf_kv> kvs;
  std::vector<std::vector<std::pair<const char*, int64_t>>> kv_strings;   // per kv: its string(s)
  std::unordered_map<std::string, int64_t> tensor_index, kv_index;
  ~gqk_gguf() {
    if (base) munmap((void*)base, size);
  }
};

namespace {

// bounds-checked little-endian cursor over the mapping
struct Cursor {
  const uint8_t* p;
  size_t pos, end;
  bool ok = true;
  template <class T>
  T get() {
    T v{};
    if (!ok || end - pos < sizeof(T)) {
      ok = false;
      return v;
    }
    memcpy(&v, p + pos, sizeof(T));
    pos += sizeof(T);
    return v;
  }
  // a GGUF string: pointer into the mapping and its length
  std::pair<const char*, int64_t> str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > end - pos) {
      ok = false;
      return {nullptr, 0};
    }
    const char* s = (const char*)(p + pos);
    pos += n;
    return {s, (int64_t)n};
  }
  bool skip(uint64_t n) {
    if (!ok || n > end - pos) return ok = false;
    pos += n;
    return true;
  }
};

// one value of type vt at the cursor into kv (scalars, strings; arrays by reference)
bool read_value(Cursor& c, int vt, gqk_gguf_kv& kv, std::vector<std::pair<const char*, int64_t>>& strs, int depth) {
  kv.type = vt;
  kv.count = 1;
  switch (vt) {
    case V_U8: kv.i64 = c.get<uint8_t>(); break;
    case V_I8: kv.i64 = c.get<int8_t>(); break;
    case V_U16: kv.i64 = c.get<uint16_t>(); break;
    case V_I16: kv.i64 = c.get<int16_t>(); break;
    case V_U32: kv.i64 = c.get<uint32_t>(); break;
    case V_I32: kv.i64 = c.get<int32_t>(); break;
    case V_U64: kv.i64 = (int64_t)c.get<uint64_t>(); break;
    case V_I64: kv.i64 = c.get<int64_t>(); break;
    case V_BOOL: kv.i64 = c.get<uint8_t>() != 0; break;
    case V_F32: kv.f64 = c.get<float>(); break;
    case V_F64: kv.f64 = c.get<double>(); break;
    case V_STR: {
      const auto s = c.str();
      kv.data = s.first;
      kv.count = s.second;
      strs.push_back(s);
      break;
    }
    case V_ARR: {
      if (depth > 0) return false;   // arrays of arrays: not in GGUF files written by GGML
      const int et = (int)c.get<uint32_t>();
      const uint64_t n = c.get<uint64_t>();
      if (!c.ok) return false;
      kv.array_type = et;
      kv.count = (int64_t)n;
      kv.data = c.p + c.pos;
      if (et == V_STR) {
        for (uint64_t i = 0; i < n && c.ok; ++i) strs.push_back(c.str());
      } else {
        const int b = scalar_bytes(et);
        if (b == 0 || n > (c.end - c.pos) / b) return false;
        c.skip(n * b);
      }
      break;
    }
    default: return false;
  }
  return c.ok;
}

int parse(gqk_gguf* f) {
  Cursor c{f->base, 0, f->size};
  const uint32_t magic = c.get<uint32_t>();
  if (!c.ok || magic != 0x46554747u) return fail(GQK_ERR_ARG, "gguf: not a GGUF file (magic %08x)", magic);
  f->version = (int32_t)c.get<uint32_t>();
  if (f->version != 3) return fail(GQK_ERR_ARG, "gguf: version %d (this reader takes version 3)", f->version);
  const uint64_t nt = c.get<uint64_t>(), nkv = c.get<uint64_t>();
  // every tensor info and key/value takes at least 8 bytes: a count beyond that is corrupt
  if (!c.ok || nt > f->size / 8 || nkv > f->size / 8)
    return fail(GQK_ERR_ARG, "gguf: corrupt header (%llu tensors, %llu keys)", (unsigned long long)nt,
                (unsigned long long)nkv);
  f->kvs.resize(nkv);
  f->kv_strings.resize(nkv);
  f->keys.resize(nkv);
  for (uint64_t i = 0; i < nkv; ++i) {
    const auto k = c.str();
    const int vt = (int)c.get<uint32_t>();
    if (!c.ok) return fail(GQK_ERR_ARG, "gguf: truncated key/value %llu", (unsigned long long)i);
    f->keys[i].assign(k.first, k.second);
    gqk_gguf_kv& kv = f->kvs[i];
    kv = gqk_gguf_kv{};
    if (!read_value(c, vt, kv, f->kv_strings[i], 0))
      return fail(GQK_ERR_ARG, "gguf: bad value of key '%s' (type %d)", f->keys[i].c_str(), vt);
    f->kv_index[f->keys[i]] = (int64_t)i;
  }
  for (uint64_t i = 0; i < nkv; ++i) f->kvs[i].key = f->keys[i].c_str();
  auto al = f->kv_index.find("general.alignment");
  if (al != f->kv_index.end()) {
    const gqk_gguf_kv& kv = f->kvs[al->second];
    if (kv.type != V_U32 || kv.i64 <= 0 || (kv.i64 & (kv.i64 - 1)))
      return fail(GQK_ERR_ARG, "gguf: general.alignment must be a power-of-two u32");
    f->alignment = kv.i64;
  }
  f->tensors.resize(nt);
  f->tensor_names.resize(nt);
  for (uint64_t i = 0; i < nt; ++i) {
    const auto nm = c.str();
    const uint32_t nd = c.get<uint32_t>();
    if (!c.ok || nd < 1 || nd > 4) return fail(GQK_ERR_ARG, "gguf: bad tensor info %llu", (unsigned long long)i);
    gqk_gguf_tensor& t = f->tensors[i];
    t = gqk_gguf_tensor{};
    t.n_dims = (int32_t)nd;
    int64_t elems = 1;
    for (uint32_t d = 0; d < 4; ++d) t.dims[d] = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint64_t v = c.get<uint64_t>();
      if (v == 0 || v > ((uint64_t)1 << 40) || (uint64_t)elems > ((uint64_t)1 << 62) / v)
        return fail(GQK_ERR_ARG, "gguf: tensor %llu: bad dimension", (unsigned long long)i);
      t.dims[d] = (int64_t)v;
      elems *= (int64_t)v;
    }
    t.ggml_type = (int32_t)c.get<uint32_t>();
    t.offset = (int64_t)c.get<uint64_t>();
    if (!c.ok) return fail(GQK_ERR_ARG, "gguf: truncated tensor info %llu", (unsigned long long)i);
    f->tensor_names[i].assign(nm.first, nm.second);
    const TypeSize ts = type_size(t.ggml_type);
    t.nbytes = ts.block == 0 || t.dims[0] % ts.block ? -1 : elems / ts.block * ts.bytes;
  }
  f->data_offset = (int64_t)((c.pos + f->alignment - 1) / f->alignment * f->alignment);
  for (uint64_t i = 0; i < nt; ++i) {
    gqk_gguf_tensor& t = f->tensors[i];
    t.name = f->tensor_names[i].c_str();
    if (t.offset % f->alignment)
      return fail(GQK_ERR_ARG, "gguf: tensor '%s' at unaligned offset %lld", t.name, (long long)t.offset);
    const int64_t at = f->data_offset + t.offset;
    if (t.nbytes >= 0) {
      if (at < f->data_offset || at > (int64_t)f->size || t.nbytes > (int64_t)f->size - at)
        return fail(GQK_ERR_ARG, "gguf: tensor '%s' runs past the end of the file", t.name);
      t.data = f->base + at;
    }
    t.offset = at;   // absolute from here on
    if (!f->tensor_index.emplace(f->tensor_names[i], (int64_t)i).second)
      return fail(GQK_ERR_ARG, "gguf: duplicate tensor name '%s'", t.name);
  }
  return GQK_OK;
}

}  // namespace

extern "C" {

int gqk_ggml_type_size(int ggml_type, int32_t* block, int32_t* bytes) {
  const TypeSize ts = type_size(ggml_type);
  if (ts.block == 0) return fail(GQK_ERR_TYPE, "ggml type %d has no fixed block size", ggml_type);
  if (block) *block = ts.block;
  if (bytes) *bytes = ts.bytes;
  return GQK_OK;
}

int gqk_gguf_open(const char* path, gqk_gguf** out) {
  if (!path || !out) return fail(GQK_ERR_ARG, "gguf_open: null argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(GQK_ERR_ARG, "gguf_open: cannot open '%s'", path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    return fail(GQK_ERR_ARG, "gguf_open: '%s' is too short for a GGUF header", path);
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) return fail(GQK_ERR_ARG, "gguf_open: cannot map '%s'", path);
  gqk_gguf* f = new gqk_gguf;
  f->base = (const uint8_t*)m;
  f->size = (size_t)st.st_size;
  const int rc = parse(f);
  if (rc != GQK_OK) {
    delete f;
    return rc;
  }
  *out = f;
  return GQK_OK;
}

void gqk_gguf_close(gqk_gguf* f) { delete f; }

int gqk_gguf_info(const gqk_gguf* f, int64_t* n_tensors, int64_t* n_kv, int64_t* alignment, int64_t* data_offset,
                  int32_t* version) {
  if (!f) return fail(GQK_ERR_ARG, "gguf_info: null handle");
  if (n_tensors) *n_tensors = (int64_t)f->tensors.size();
  if (n_kv) *n_kv = (int64_t)f->kvs.size();
  if (alignment) *alignment = f->alignment;
  if (data_offset) *data_offset = f->data_offset;
  if (version) *version = f->version;
  return GQK_OK;
}

int gqk_gguf_tensor_at(const gqk_gguf* f, int64_t i, gqk_gguf_tensor* out) {
  if (!f || !out) return fail(GQK_ERR_ARG, "gguf_tensor_at: null argument");
  if (i < 0 || i >= (int64_t)f->tensors.size()) return fail(GQK_ERR_ARG, "gguf_tensor_at: index %lld", (long long)i);
  *out = f->tensors[i];
  return GQK_OK;
}

int64_t gqk_gguf_find_tensor(const gqk_gguf* f, const char* name) {
  if (!f || !name) return fail(GQK_ERR_ARG, "gguf_find_tensor: null argument");
  auto it = f->tensor_index.find(name);
  return it == f->tensor_index.end() ? -1 : it->second;
}

int gqk_gguf_kv_at(const gqk_gguf* f, int64_t i, gqk_gguf_kv* out) {
  if (!f || !out) return fail(GQK_ERR_ARG, "gguf_kv_at: null argument");
  if (i < 0 || i >= (int64_t)f->kvs.size()) return fail(GQK_ERR_ARG, "gguf_kv_at: index %lld", (long long)i);
  *out = f->kvs[i];
  return GQK_OK;
}

int64_t gqk_gguf_find_kv(const gqk_gguf* f, const char* key) {
  if (!f || !key) return fail(GQK_ERR_ARG, "gguf_find_kv: null argument");
  auto it = f->kv_index.find(key);
  return it == f->kv_index.end() ? -1 : it->second;
}

int gqk_gguf_kv_string(const gqk_gguf* f, int64_t i, int64_t j, const char** s, int64_t* len) {
  if (!f || !s || !len) return fail(GQK_ERR_ARG, "gguf_kv_string: null argument");
  if (i < 0 || i >= (int64_t)f->kvs.size()) return fail(GQK_ERR_ARG, "gguf_kv_string: index %lld", (long long)i);
  const auto& strs = f->kv_strings[i];
  if (j < 0 || j >= (int64_t)strs.size())
    return fail(GQK_ERR_ARG, "gguf_kv_string: key '%s' has no string %lld", f->keys[i].c_str(), (long long)j);
  *s = strs[j].first;
  *len = strs[j].second;
  return GQK_OK;
}

int gqk_gguf_upload_tiles(const gqk_gguf* f, int64_t i, void* staging, int64_t staging_bytes, void* tiles,
                          void* stream) {
  if (!f || !staging || !tiles) return fail(GQK_ERR_ARG, "gguf_upload_tiles: null argument");
  if (i < 0 || i >= (int64_t)f->tensors.size())
    return fail(GQK_ERR_ARG, "gguf_upload_tiles: index %lld", (long long)i);
  const gqk_gguf_tensor& t = f->tensors[i];
  if (t.n_dims != 2) return fail(GQK_ERR_SHAPE, "gguf_upload_tiles: '%s' is not a matrix", t.name);
  if (t.nbytes < 0) return fail(GQK_ERR_TYPE, "gguf_upload_tiles: '%s' has ggml type %d", t.name, t.ggml_type);
  if (staging_bytes < t.nbytes)
    return fail(GQK_ERR_SHAPE, "gguf_upload_tiles: staging %lld bytes < %lld", (long long)staging_bytes,
                (long long)t.nbytes);
  hipStream_t st = (hipStream_t)stream;
  // the rows are pageable (the mapping): the copy is staged by the runtime
  if (hipMemcpyAsync(staging, t.data, (size_t)t.nbytes, hipMemcpyHostToDevice, st) != hipSuccess)
    return fail(GQK_ERR_HIP, "gguf_upload_tiles: host-to-device copy of '%s' failed", t.name);
  const int64_t K = t.dims[0], n = t.dims[1];
  return gqk_repack(staging, t.nbytes / n, t.ggml_type, n, K, tiles, stream);
}

}  // extern "C"
