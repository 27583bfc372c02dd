// loader.cpp — checkpoint reading for lisa_runner_load: the safetensors
// container ([u64 LE header length][JSON header][tensor bytes], offsets
// relative to the end of the header; the reference's
// src/format/safetensor.rs:27-89) memory-mapped read-only, and the index of
// every tensor name over the shards of a snapshot (src/model/weights.rs:22-42).
// Host-only: nothing here touches the GPU, so hosts can open and validate a
// snapshot (lisa_weight_index_validate) before creating a device.
//
// Unlike the reference, which trusts the header, every tensor's byte range is
// checked against its shard's data region and against dtype size x shape, so
// a truncated or inconsistent shard is an error rather than an out-of-bounds
// read.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstring>
#include <memory>
#include <unordered_map>

#include "bridge.h"
#include "loader.h"

namespace {

struct Shard {
  std::string path;
  const uint8_t* map = nullptr;
  size_t size = 0;
  uint64_t data_start = 0, data_len = 0;
};

// dtype names and element sizes in the order of the reference's Dtype enum
// (src/format/dtype.rs:3-33)
const char* kDtypeNames[] = {"BOOL", "U8", "U16", "I16", "F16", "BF16", "U32", "I32", "F32", "U64", "F64"};
const uint64_t kDtypeBytes[] = {1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8};
constexpr int kDtypes = 11;

int dtype_from_name(const std::string& s) {
  for (int i = 0; i < kDtypes; ++i)
    if (s == kDtypeNames[i]) return i;
  return -1;
}

// ---- a JSON reader for the header: objects, arrays, strings, integers ----
struct Json {
  const char* p;
  const char* end;
  std::string err;

  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  static void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xc0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      s += (char)(0xe0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3f));
      s += (char)(0x80 | (cp & 0x3f));
    } else {
      s += (char)(0xf0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3f));
      s += (char)(0x80 | ((cp >> 6) & 0x3f));
      s += (char)(0x80 | (cp & 0x3f));
    }
  }
  bool hex4(uint32_t* v) {
    if (end - p < 4) return fail("truncated \\u escape");
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      x <<= 4;
      if (c >= '0' && c <= '9') x |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') x |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') x |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    *v = x;
    return true;
  }
  bool string(std::string* out) {
    ws();
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    std::string s;
    while (p < end && *p != '"') {
      char c = *p++;
      if ((unsigned char)c < 0x20) return fail("control character in a string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p >= end) return fail("truncated escape");
      c = *p++;
      switch (c) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xd800 && cp < 0xdc00) {  // surrogate pair
            uint32_t lo;
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("unpaired surrogate");
            p += 2;
            if (!hex4(&lo) || lo < 0xdc00 || lo >= 0xe000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          put_utf8(s, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    *out = std::move(s);
    return true;
  }
  // a non-negative integer (shapes and offsets)
  bool uint(uint64_t* out) {
    ws();
    if (p >= end || *p < '0' || *p > '9') return fail("expected a non-negative integer");
    uint64_t v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const uint64_t d = (uint64_t)(*p++ - '0');
      if (v > (UINT64_MAX - d) / 10) return fail("integer overflow");
      v = v * 10 + d;
    }
    if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return fail("expected an integer");
    *out = v;
    return true;
  }
  bool uint_array(std::vector<uint64_t>* out) {
    if (!eat('[')) return fail("expected an array");
    out->clear();
    if (eat(']')) return true;
    do {
      uint64_t v;
      if (!uint(&v)) return false;
      out->push_back(v);
    } while (eat(','));
    return eat(']') ? true : fail("expected ']'");
  }
  // skips any value (the __metadata__ object, unknown fields)
  bool skip(int depth = 0) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    if (*p == '"') {
      std::string s;
      return string(&s);
    }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      ++p;
      if (eat(close)) return true;
      do {
        if (obj) {
          std::string k;
          if (!string(&k) || !eat(':')) return fail("bad object");
        }
        if (!skip(depth + 1)) return false;
      } while (eat(','));
      return eat(close) ? true : fail("unterminated object or array");
    }
    const char* s = p;
    while (p < end && (std::isalnum((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.')) ++p;
    return p > s ? true : fail("bad value");
  }
};

struct RawTensor {
  std::string name;
  int dtype = -1;
  std::vector<uint64_t> shape;
  uint64_t start = 0, end = 0;
};

// The tensor table of one header (parse_header, safetensor.rs:61-89):
// top-level keys beginning with "__" are metadata and skipped.
bool parse_header(const char* text, size_t len, std::vector<RawTensor>* out, std::string* err) {
  Json j{text, text + len, {}};
  if (!j.eat('{')) {
    *err = "safetensors header must be an object";
    return false;
  }
  if (!j.eat('}')) {
    do {
      RawTensor t;
      if (!j.string(&t.name) || !j.eat(':')) {
        *err = j.err.empty() ? "bad header entry" : j.err;
        return false;
      }
      if (t.name.rfind("__", 0) == 0) {
        if (!j.skip()) {
          *err = j.err;
          return false;
        }
        continue;
      }
      if (!j.eat('{')) {
        *err = "tensor " + t.name + ": expected an object";
        return false;
      }
      bool have_dtype = false, have_shape = false, have_off = false;
      if (!j.eat('}')) {
        do {
          std::string key;
          if (!j.string(&key) || !j.eat(':')) {
            *err = "tensor " + t.name + ": " + j.err;
            return false;
          }
          if (key == "dtype") {
            std::string d;
            if (!j.string(&d)) {
              *err = "tensor " + t.name + ": " + j.err;
              return false;
            }
            t.dtype = dtype_from_name(d);
            if (t.dtype < 0) {
              *err = "unknown dtype " + d;  // dtype_from_name panics with this (dtype.rs:31)
              return false;
            }
            have_dtype = true;
          } else if (key == "shape") {
            if (!j.uint_array(&t.shape)) {
              *err = "tensor " + t.name + ": shape: " + j.err;
              return false;
            }
            have_shape = true;
          } else if (key == "data_offsets") {
            std::vector<uint64_t> o;
            if (!j.uint_array(&o) || o.size() != 2) {
              *err = "tensor " + t.name + ": data_offsets must be two integers";
              return false;
            }
            t.start = o[0];
            t.end = o[1];
            have_off = true;
          } else if (!j.skip()) {
            *err = "tensor " + t.name + ": " + j.err;
            return false;
          }
        } while (j.eat(','));
        if (!j.eat('}')) {
          *err = "tensor " + t.name + ": expected '}'";
          return false;
        }
      }
      if (!have_dtype || !have_shape || !have_off) {
        *err = "tensor " + t.name + ": dtype, shape and data_offsets are required";
        return false;
      }
      out->push_back(std::move(t));
    } while (j.eat(','));
    if (!j.eat('}')) {
      *err = j.err.empty() ? "expected '}' after the last header entry" : j.err;
      return false;
    }
  }
  return true;
}

}  // namespace

struct LisaWeightIndex {
  std::vector<Shard> shards;
  std::unordered_map<std::string, LisaSlotInfo> slots;
  ~LisaWeightIndex() {
    for (Shard& s : shards)
      if (s.map) munmap(const_cast<uint8_t*>(s.map), s.size);
  }
};

namespace {

// open (safetensor.rs:27-40): map the file and read its tensor table.
int open_shard(const std::string& path, Shard* sh, std::vector<RawTensor>* tensors) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return lisa_fail(LISA_E_ARG, "open shard %s: %s", path.c_str(), std::strerror(errno));
  struct stat st {};
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    return lisa_fail(LISA_E_ARG, "stat shard %s: %s", path.c_str(), std::strerror(e));
  }
  const size_t size = (size_t)st.st_size;
  if (size < 8) {
    ::close(fd);
    return lisa_fail(LISA_E_ARG, "shard %s: %zu bytes, shorter than the header length", path.c_str(), size);
  }
  void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return lisa_fail(LISA_E_ARG, "map shard %s: %s", path.c_str(), std::strerror(errno));
  sh->path = path;
  sh->map = static_cast<const uint8_t*>(m);
  sh->size = size;
  uint64_t hl = 0;
  for (int i = 7; i >= 0; --i) hl = (hl << 8) | sh->map[i];  // u64 little endian
  if (hl > size - 8) return lisa_fail(LISA_E_ARG, "shard %s: header length %llu past the end of the file",
                                      path.c_str(), (unsigned long long)hl);
  sh->data_start = 8 + hl;
  sh->data_len = size - sh->data_start;
  std::string err;
  if (!parse_header(reinterpret_cast<const char*>(sh->map + 8), (size_t)hl, tensors, &err))
    return lisa_fail(LISA_E_ARG, "parse safetensors header of %s: %s", path.c_str(), err.c_str());
  for (const RawTensor& t : *tensors) {
    if (t.end < t.start || t.end > sh->data_len)
      return lisa_fail(LISA_E_ARG, "shard %s: tensor %s data_offsets [%llu, %llu) outside the %llu-byte data region",
                       path.c_str(), t.name.c_str(), (unsigned long long)t.start, (unsigned long long)t.end,
                       (unsigned long long)sh->data_len);
    uint64_t n = kDtypeBytes[t.dtype];
    for (uint64_t d : t.shape) {
      if (d && n > UINT64_MAX / d) return lisa_fail(LISA_E_ARG, "shard %s: tensor %s shape overflows", path.c_str(), t.name.c_str());
      n *= d;
    }
    if (n != t.end - t.start)
      return lisa_fail(LISA_E_ARG, "shard %s: tensor %s holds %llu bytes, its dtype and shape need %llu",
                       path.c_str(), t.name.c_str(), (unsigned long long)(t.end - t.start), (unsigned long long)n);
  }
  return LISA_OK;
}

}  // namespace

int lisa_index_open_paths(const std::vector<std::string>& paths, LisaWeightIndex** out) {
  std::unique_ptr<LisaWeightIndex> idx(new LisaWeightIndex());
  for (size_t si = 0; si < paths.size(); ++si) {
    idx->shards.emplace_back();
    std::vector<RawTensor> ts;
    LISA_TRY(open_shard(paths[si], &idx->shards.back(), &ts));
    for (RawTensor& t : ts) {
      LisaSlotInfo s;
      s.shard = (int)si;
      s.offset = t.start;
      s.len = t.end - t.start;
      s.dtype = t.dtype;
      s.shape = t.shape;
      // WeightIndex::open asserts on a name seen twice (weights.rs:26-37)
      if (!idx->slots.emplace(t.name, std::move(s)).second)
        return lisa_fail(LISA_E_ARG, "duplicate tensor %s", t.name.c_str());
    }
  }
  *out = idx.release();
  return LISA_OK;
}

const LisaSlotInfo* lisa_index_find(const LisaWeightIndex* idx, const std::string& name) {
  auto it = idx->slots.find(name);
  return it == idx->slots.end() ? nullptr : &it->second;
}

const uint8_t* lisa_index_bytes(const LisaWeightIndex* idx, const LisaSlotInfo& s) {
  const Shard& sh = idx->shards[(size_t)s.shard];
  return sh.map + sh.data_start + s.offset;
}

const char* lisa_dtype_name(int dtype) { return dtype >= 0 && dtype < kDtypes ? kDtypeNames[dtype] : "?"; }

namespace {
std::string shape_str(const std::vector<uint64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}
}  // namespace

int lisa_index_expect(const LisaWeightIndex* idx, const std::string& name, int dtype,
                      const std::vector<uint64_t>& shape, const LisaSlotInfo** out) {
  const LisaSlotInfo* s = lisa_index_find(idx, name);
  if (!s) return lisa_fail(LISA_E_ARG, "missing tensor %s", name.c_str());
  if (s->dtype != dtype || s->shape != shape)
    return lisa_fail(LISA_E_ARG, "invalid tensor %s: %s %s, expected %s %s", name.c_str(), lisa_dtype_name(s->dtype),
                     shape_str(s->shape).c_str(), lisa_dtype_name(dtype), shape_str(shape).c_str());
  if (out) *out = s;
  return LISA_OK;
}

int lisa_snapshot_paths(const char* dir, std::vector<std::string>* out) {
  DIR* d = opendir(dir);
  if (!d) return lisa_fail(LISA_E_ARG, "read snapshot %s: %s", dir, std::strerror(errno));
  out->clear();
  while (struct dirent* e = readdir(d)) {
    const std::string n = e->d_name;
    const std::string ext = ".safetensors";
    if (n.size() > ext.size() && n.compare(n.size() - ext.size(), ext.size(), ext) == 0)
      out->push_back(std::string(dir) + "/" + n);
  }
  closedir(d);
  std::sort(out->begin(), out->end());
  if (out->empty()) return lisa_fail(LISA_E_ARG, "no safetensors shards in %s", dir);
  return LISA_OK;
}

// ---- C ABI ------------------------------------------------------------------
extern "C" int lisa_weight_index_open(const char* const* paths, int32_t n, LisaWeightIndex** out) {
  if (!out || n < 0 || (n && !paths)) return lisa_fail(LISA_E_ARG, "lisa_weight_index_open: bad argument");
  std::vector<std::string> ps;
  for (int32_t i = 0; i < n; ++i) {
    if (!paths[i]) return lisa_fail(LISA_E_ARG, "lisa_weight_index_open: null path %d", i);
    ps.emplace_back(paths[i]);
  }
  return lisa_index_open_paths(ps, out);
}

extern "C" int lisa_weight_index_open_snapshot(const char* dir, LisaWeightIndex** out) {
  if (!dir || !out) return lisa_fail(LISA_E_ARG, "lisa_weight_index_open_snapshot: null argument");
  std::vector<std::string> ps;
  LISA_TRY(lisa_snapshot_paths(dir, &ps));
  return lisa_index_open_paths(ps, out);
}

extern "C" void lisa_weight_index_free(LisaWeightIndex* idx) { delete idx; }

extern "C" int32_t lisa_weight_index_len(const LisaWeightIndex* idx) { return idx ? (int32_t)idx->slots.size() : 0; }

extern "C" int32_t lisa_weight_index_shard_count(const LisaWeightIndex* idx) {
  return idx ? (int32_t)idx->shards.size() : 0;
}

extern "C" int lisa_weight_index_slot(const LisaWeightIndex* idx, const char* name, LisaWeightSlot* out) {
  if (!idx || !name || !out) return lisa_fail(LISA_E_ARG, "lisa_weight_index_slot: null argument");
  const LisaSlotInfo* s = lisa_index_find(idx, name);
  if (!s) return lisa_fail(LISA_E_ARG, "missing tensor %s", name);
  if (s->shape.size() > LISA_MAX_DIMS) return lisa_fail(LISA_E_ARG, "tensor %s has %zu dimensions", name, s->shape.size());
  std::memset(out, 0, sizeof *out);
  out->shard = s->shard;
  out->dtype = s->dtype;
  out->ndim = (int32_t)s->shape.size();
  out->offset = s->offset;
  out->data_start = idx->shards[(size_t)s->shard].data_start;
  out->len = s->len;
  for (size_t i = 0; i < s->shape.size(); ++i) out->shape[i] = s->shape[i];
  return LISA_OK;
}
