// GGUF (ggml's on-disk model format, versions 2 and 3) reader: maps the file
// read-only, parses the header, the metadata key/value pairs and the tensor
// table, and hands out tensor bytes for upload.  The reference has no loader
// ("GGUF file parsing - separate", ROADMAP.md:230-234); the layout follows
// the published GGUF specification (ggml docs/gguf.md):
//
//   u32 magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x { string key | u32 value_type | value }
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 ggml_type | u64 offset }
//   padding to `general.alignment` (u32 metadata, default 32) | tensor data
//
// strings are u64 length + bytes (no terminator); arrays are u32 item type +
// u64 count + items; all little-endian.  Tensor offsets are relative to the
// aligned data section and must be multiples of the alignment.
//
// The file is untrusted input: every read is bounds-checked against the
// mapping, counts and lengths are checked before anything is allocated for
// them, and every tensor's byte range must lie inside the file.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "axh_gguf.h"
#include "axh_internal.h"

using axh::fail;
using axh::ok;

namespace {

enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
  kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

constexpr uint32_t kMaxDims = 4;         // GGML_MAX_DIMS
constexpr uint64_t kMaxString = 1u << 30;

// Block geometry of the ggml types (elements per block, bytes per block);
// {0, 0} for types this reader does not size.
struct TypeSize {
  uint32_t elems, bytes;
};

TypeSize type_size(uint32_t t) {
  switch (t) {
  case AXH_GGML_F32: return {1, 4};
  case AXH_GGML_F16: return {1, 2};
  case AXH_GGML_Q4_0: return {32, 18};
  case AXH_GGML_Q4_1: return {32, 20};
  case AXH_GGML_Q5_0: return {32, 22};
  case AXH_GGML_Q5_1: return {32, 24};
  case AXH_GGML_Q8_0: return {32, 34};
  case AXH_GGML_Q8_1: return {32, 36};
  case AXH_GGML_Q2_K: return {256, 84};
  case AXH_GGML_Q3_K: return {256, 110};
  case AXH_GGML_Q4_K: return {256, 144};
  case AXH_GGML_Q5_K: return {256, 176};
  case AXH_GGML_Q6_K: return {256, 210};
  case AXH_GGML_Q8_K: return {256, 292};
  case AXH_GGML_I8: return {1, 1};
  case AXH_GGML_I16: return {1, 2};
  case AXH_GGML_I32: return {1, 4};
  case AXH_GGML_I64: return {1, 8};
  case AXH_GGML_F64: return {1, 8};
  case AXH_GGML_BF16: return {1, 2};
  default: return {0, 0};
  }
}

struct Cursor {
  const uint8_t *p;
  uint64_t n, at = 0;
  bool ok = true;

  bool need(uint64_t k) {
    if (!ok || k > n - at) ok = false;
    return ok;
  }
  template <typename T> T get() {
    T v{};
    if (need(sizeof(T))) {
      std::memcpy(&v, p + at, sizeof(T));
      at += sizeof(T);
    }
    return v;
  }
  // A string as (offset, length) into the mapping.
  bool str(uint64_t *off, uint64_t *len) {
    const uint64_t l = get<uint64_t>();
    if (!ok || l > kMaxString || !need(l)) return ok = false;
    *off = at;
    *len = l;
    at += l;
    return true;
  }
};

struct Kv {
  std::string key;
  uint32_t type = 0;       // value type
  uint32_t item_type = 0;  // arrays: item type
  uint64_t count = 0;      // arrays: items; strings: bytes
  uint64_t value_off = 0;  // file offset of the value (array: of the first item)
};

struct Tensor {
  std::string name;
  uint32_t type = 0, n_dims = 0;
  uint64_t ne[kMaxDims] = {1, 1, 1, 1};
  uint64_t rel_off = 0, offset = 0, nbytes = 0;
};

uint64_t scalar_bytes(uint32_t t) {
  switch (t) {
  case kU8: case kI8: case kBool: return 1;
  case kU16: case kI16: return 2;
  case kU32: case kI32: case kF32: return 4;
  case kU64: case kI64: case kF64: return 8;
  default: return 0;
  }
}

// Skips one value of type t (nested arrays allowed up to a small depth).
bool skip_value(Cursor &c, uint32_t t, int depth) {
  if (const uint64_t b = scalar_bytes(t)) return c.need(b) && (c.at += b, true);
  if (t == kString) {
    uint64_t o, l;
    return c.str(&o, &l);
  }
  if (t == kArray && depth < 4) {
    const uint32_t it = c.get<uint32_t>();
    const uint64_t cnt = c.get<uint64_t>();
    if (!c.ok) return false;
    if (const uint64_t b = scalar_bytes(it)) {
      if (cnt > (c.n - c.at) / b) return c.ok = false;
      c.at += cnt * b;
      return true;
    }
    if (cnt > c.n - c.at) return c.ok = false; // each item takes at least one byte
    for (uint64_t i = 0; i < cnt; ++i)
      if (!skip_value(c, it, depth + 1)) return false;
    return true;
  }
  return c.ok = false;
}

} // namespace

struct axh_gguf {
  void *map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint32_t alignment = 32;
  uint64_t data_off = 0;
  std::vector<Kv> kvs;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, uint64_t> by_name;
  std::unordered_map<std::string, uint64_t> kv_by_key;

  ~axh_gguf() {
    if (map) munmap(map, size);
  }
  const uint8_t *bytes() const { return static_cast<const uint8_t *>(map); }
};

static axh_status parse(axh_gguf *g) {
  Cursor c{g->bytes(), g->size};
  if (c.get<uint32_t>() != 0x46554747u || !c.ok)
    return fail(AXH_ERR_METADATA_PARSE, "not a GGUF file (bad magic)");
  g->version = c.get<uint32_t>();
  if (!c.ok || (g->version != 2 && g->version != 3))
    return fail(AXH_ERR_METADATA_SCHEMA_MISMATCH, "unsupported GGUF version (2 and 3 are read)");
  const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
  // Every KV takes at least 12 bytes and every tensor info at least 24.
  if (!c.ok || n_kv > g->size / 12 || n_tensors > g->size / 24)
    return fail(AXH_ERR_METADATA_PARSE, "GGUF counts exceed the file size");
  g->kvs.reserve(n_kv);
  for (uint64_t i = 0; i < n_kv; ++i) {
    Kv kv;
    uint64_t ko, kl;
    if (!c.str(&ko, &kl)) return fail(AXH_ERR_METADATA_PARSE, "truncated GGUF metadata key");
    kv.key.assign(reinterpret_cast<const char *>(g->bytes() + ko), kl);
    kv.type = c.get<uint32_t>();
    if (!c.ok) return fail(AXH_ERR_METADATA_PARSE, "truncated GGUF metadata");
    const uint64_t start = c.at;
    if (kv.type == kArray) {
      kv.item_type = c.get<uint32_t>();
      kv.count = c.get<uint64_t>();
      kv.value_off = c.at;
      c.at = start;
    } else if (kv.type == kString) {
      kv.count = c.get<uint64_t>();
      kv.value_off = c.at;
      c.at = start;
    } else {
      kv.value_off = start;
    }
    if (!skip_value(c, kv.type, 0))
      return fail(AXH_ERR_METADATA_PARSE, "malformed or truncated GGUF value for " + kv.key);
    if (g->kv_by_key.count(kv.key))
      return fail(AXH_ERR_METADATA_PARSE, "duplicate GGUF metadata key " + kv.key);
    g->kv_by_key.emplace(kv.key, g->kvs.size());
    g->kvs.push_back(std::move(kv));
  }
  auto al = g->kv_by_key.find("general.alignment");
  if (al != g->kv_by_key.end()) {
    const Kv &kv = g->kvs[al->second];
    if (kv.type != kU32) return fail(AXH_ERR_METADATA_PARSE, "general.alignment must be a u32");
    std::memcpy(&g->alignment, g->bytes() + kv.value_off, 4);
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1)) != 0)
      return fail(AXH_ERR_METADATA_PARSE, "general.alignment must be a power of two");
  }
  g->tensors.reserve(n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Tensor t;
    uint64_t no, nl;
    if (!c.str(&no, &nl)) return fail(AXH_ERR_METADATA_PARSE, "truncated GGUF tensor name");
    t.name.assign(reinterpret_cast<const char *>(g->bytes() + no), nl);
    t.n_dims = c.get<uint32_t>();
    if (!c.ok || t.n_dims == 0 || t.n_dims > kMaxDims)
      return fail(AXH_ERR_METADATA_PARSE, "GGUF tensor " + t.name + ": n_dims must be 1..4");
    uint64_t n_elems = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      t.ne[d] = c.get<uint64_t>();
      if (t.ne[d] == 0 || (n_elems > 0 && t.ne[d] > (1ull << 62) / n_elems))
        return fail(AXH_ERR_METADATA_PARSE, "GGUF tensor " + t.name + ": bad dimension");
      n_elems *= t.ne[d];
    }
    t.type = c.get<uint32_t>();
    t.rel_off = c.get<uint64_t>();
    if (!c.ok) return fail(AXH_ERR_METADATA_PARSE, "truncated GGUF tensor info");
    const TypeSize ts = type_size(t.type);
    if (ts.elems) {
      if (t.ne[0] % ts.elems != 0)
        return fail(AXH_ERR_METADATA_PARSE,
                    "GGUF tensor " + t.name + ": row length is not a whole number of blocks");
      // Element counts reach 2^62, so blocks * block bytes can wrap in 64
      // bits: such a tensor cannot lie inside any file.
      if (__builtin_mul_overflow(n_elems / ts.elems, (uint64_t)ts.bytes, &t.nbytes) ||
          t.nbytes > g->size)
        return fail(AXH_ERR_METADATA_PARSE,
                    "GGUF tensor " + t.name + ": byte size exceeds the file");
    }
    if (t.rel_off % g->alignment != 0)
      return fail(AXH_ERR_METADATA_PARSE, "GGUF tensor " + t.name + ": misaligned offset");
    if (g->by_name.count(t.name))
      return fail(AXH_ERR_METADATA_PARSE, "duplicate GGUF tensor name " + t.name);
    g->by_name.emplace(t.name, g->tensors.size());
    g->tensors.push_back(std::move(t));
  }
  const uint64_t a = g->alignment;
  g->data_off = (c.at + a - 1) / a * a;
  for (Tensor &t : g->tensors) {
    if (t.rel_off > g->size || g->data_off > g->size - t.rel_off ||
        t.nbytes > g->size - g->data_off - t.rel_off)
      return fail(AXH_ERR_METADATA_PARSE, "GGUF tensor " + t.name + " extends past the file end");
    t.offset = g->data_off + t.rel_off;
  }
  return ok();
}

extern "C" {

axh_status axh_ggml_type_size(uint32_t type, uint32_t *block_elems, uint32_t *block_bytes) {
  const TypeSize ts = type_size(type);
  if (!ts.elems) return fail(AXH_ERR_INVALID_ARGUMENT, "ggml type without a known block size");
  if (block_elems) *block_elems = ts.elems;
  if (block_bytes) *block_bytes = ts.bytes;
  return ok();
}

axh_status axh_gguf_open(const char *path, axh_gguf **out) {
  if (!path || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(AXH_ERR_METADATA_IO, std::string("cannot open ") + path);
  struct stat st{};
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    return fail(AXH_ERR_METADATA_PARSE, std::string("not a GGUF file (too short): ") + path);
  }
  void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) return fail(AXH_ERR_METADATA_IO, std::string("cannot map ") + path);
  auto *g = new axh_gguf();
  g->map = m;
  g->size = (size_t)st.st_size;
  const axh_status s = parse(g);
  if (s != AXH_OK) {
    delete g;
    return s;
  }
  *out = g;
  return ok();
}

void axh_gguf_close(axh_gguf *g) { delete g; }

uint32_t axh_gguf_version(const axh_gguf *g) { return g ? g->version : 0; }
uint32_t axh_gguf_alignment(const axh_gguf *g) { return g ? g->alignment : 0; }
uint64_t axh_gguf_data_offset(const axh_gguf *g) { return g ? g->data_off : 0; }
uint64_t axh_gguf_tensor_count(const axh_gguf *g) { return g ? g->tensors.size() : 0; }
uint64_t axh_gguf_kv_count(const axh_gguf *g) { return g ? g->kvs.size() : 0; }

axh_status axh_gguf_tensor_at(const axh_gguf *g, uint64_t i, axh_gguf_tensor_info *out) {
  if (!g || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (i >= g->tensors.size()) return fail(AXH_ERR_INVALID_ARGUMENT, "tensor index out of range");
  const Tensor &t = g->tensors[i];
  out->name = t.name.c_str();
  out->type = t.type;
  out->n_dims = t.n_dims;
  for (uint32_t d = 0; d < kMaxDims; ++d) out->ne[d] = t.ne[d];
  out->offset = t.offset;
  out->nbytes = t.nbytes;
  return ok();
}

axh_status axh_gguf_find_tensor(const axh_gguf *g, const char *name, uint64_t *index) {
  if (!g || !name || !index) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  auto it = g->by_name.find(name);
  if (it == g->by_name.end()) return fail(AXH_ERR_INVALID_ARGUMENT, std::string("no tensor ") + name);
  *index = it->second;
  return ok();
}

const void *axh_gguf_tensor_data(const axh_gguf *g, uint64_t i) {
  if (!g || i >= g->tensors.size()) return nullptr;
  return g->bytes() + g->tensors[i].offset;
}

axh_status axh_gguf_upload_tensor(axh_context *ctx, const axh_gguf *g, uint64_t i, void *dst,
                                  uint64_t capacity) {
  if (!ctx || !g || !dst) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (i >= g->tensors.size()) return fail(AXH_ERR_INVALID_ARGUMENT, "tensor index out of range");
  const Tensor &t = g->tensors[i];
  if (!type_size(t.type).elems)
    return fail(AXH_ERR_INVALID_ARGUMENT, "GGUF tensor " + t.name + " has an unsized ggml type");
  if (t.nbytes > capacity)
    return fail(AXH_ERR_INVALID_ARGUMENT, "destination smaller than GGUF tensor " + t.name);
  return axh_upload(ctx, dst, g->bytes() + t.offset, t.nbytes);
}

axh_status axh_gguf_kv_at(const axh_gguf *g, uint64_t i, axh_gguf_kv_info *out) {
  if (!g || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (i >= g->kvs.size()) return fail(AXH_ERR_INVALID_ARGUMENT, "metadata index out of range");
  const Kv &kv = g->kvs[i];
  out->key = kv.key.c_str();
  out->type = kv.type;
  out->item_type = kv.item_type;
  out->count = kv.count;
  out->value = g->bytes() + kv.value_off;
  return ok();
}

axh_status axh_gguf_find_kv(const axh_gguf *g, const char *key, uint64_t *index) {
  if (!g || !key || !index) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  auto it = g->kv_by_key.find(key);
  if (it == g->kv_by_key.end()) return fail(AXH_ERR_INVALID_ARGUMENT, std::string("no key ") + key);
  *index = it->second;
  return ok();
}

} // extern "C"
