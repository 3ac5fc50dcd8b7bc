// Host side of the safetensors loader: header parsing and the bulk copy of the data section to
// device memory (SafeTensors.open / has / info and the uploads of app/weights.js:38-118).
//
// File layout (the safetensors format, as app/weights.js:40-47 reads it): an 8-byte little-endian
// header length N, N bytes of a UTF-8 JSON object, then the data section. Each header entry is
// name -> {"dtype": "F32", "shape": [..], "data_offsets": [begin, end]} with byte offsets relative
// to the data section; "__metadata__" holds string -> string pairs. The reference hands the parsed
// object to JSON.parse semantics: a repeated key keeps its first position and takes its last value;
// anything after the object other than whitespace is an error.

#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <exception>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "supra_weights.h"
#include "status.h"

struct sa_st_file {
  const uint8_t* base = nullptr;  // the whole file
  int64_t size = 0;
  void* map = nullptr;            // our mapping (nullptr for sa_st_open_memory)
  int64_t data_start = 0;
  std::vector<std::pair<std::string, sa_st_tensor>> tensors;
  std::unordered_map<std::string, size_t> index;
  std::vector<std::pair<std::string, std::string>> meta;
};

namespace {

using sa::fail;
using sa::ok;

struct DtypeName {
  const char* name;
  int32_t code;
  int32_t bytes;
};

// The safetensors dtype names; the first ten are the ones app/weights.js:4 sizes and decodes.
constexpr DtypeName kDtypes[] = {
    {"F32", SA_DT_F32, 4},   {"F16", SA_DT_F16, 2},   {"BF16", SA_DT_BF16, 2},        {"F64", SA_DT_F64, 8},
    {"I64", SA_DT_I64, 8},   {"I32", SA_DT_I32, 4},   {"I16", SA_DT_I16, 2},          {"I8", SA_DT_I8, 1},
    {"U8", SA_DT_U8, 1},     {"BOOL", SA_DT_BOOL, 1}, {"U16", SA_DT_U16, 2},          {"U32", SA_DT_U32, 4},
    {"U64", SA_DT_U64, 8},   {"F8_E4M3", SA_DT_F8_E4M3, 1}, {"F8_E5M2", SA_DT_F8_E5M2, 1},
};

constexpr int kMaxDepth = 64;  // nesting accepted inside values this loader skips

// Recursive-descent JSON reader over [p, end) for the subset a header needs, with a skipper for
// the values it does not interpret. Every method returns false on malformed input and leaves a
// message in `err`.
struct Json {
  const char* p;
  const char* end;
  std::string err;

  bool bad(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end - p < 4) return bad("truncated \\u escape");
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return bad("bad \\u escape");
    }
    return true;
  }
  bool str(std::string& out) {
    out.clear();
    if (!lit('"')) return bad("expected a string");
    while (p < end) {
      const unsigned char c = (unsigned char)*p++;
      if (c == '"') return true;
      if (c < 0x20) return bad("control character in a string");
      if (c != '\\') {
        out += (char)c;
        continue;
      }
      if (p >= end) break;
      const char e = *p++;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            const char* save = p;
            p += 2;
            uint32_t lo;
            if (!hex4(lo)) return false;
            if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            else p = save;  // a lone high surrogate followed by another escape
          }
          utf8(out, cp);  // lone surrogates are kept as their code units, as JSON.parse keeps them
          break;
        }
        default: return bad("bad escape in a string");
      }
    }
    return bad("unterminated string");
  }
  // A non-negative integer (no sign, fraction or exponent) that fits in int64.
  bool uint(int64_t& v) {
    ws();
    if (p >= end || *p < '0' || *p > '9') return bad("expected a non-negative integer");
    uint64_t acc = 0;
    const char* start = p;
    while (p < end && *p >= '0' && *p <= '9') {
      acc = acc * 10 + (uint64_t)(*p++ - '0');
      if (acc > (uint64_t)INT64_MAX / 10 && p < end && *p >= '0' && *p <= '9') return bad("integer too large");
    }
    if (p - start > 1 && *start == '0') return bad("integer with a leading zero");
    if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return bad("expected an integer, found a fraction");
    if (acc > (uint64_t)INT64_MAX) return bad("integer too large");
    v = (int64_t)acc;
    return true;
  }
  // Skips any JSON value; [b, p) is its text afterwards.
  bool skip(int depth = 0) {
    if (depth > kMaxDepth) return bad("JSON nested too deeply");
    ws();
    if (p >= end) return bad("expected a value");
    const char c = *p;
    if (c == '"') {
      std::string s;
      return str(s);
    }
    if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      ++p;
      if (lit(close)) return true;
      do {
        if (c == '{') {
          std::string k;
          if (!str(k) || !lit(':')) return bad("expected key: value");
        }
        if (!skip(depth + 1)) return false;
      } while (lit(','));
      return lit(close) ? true : bad("unterminated object or array");
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      ++p;
      while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) ++p;
      return true;
    }
    for (const char* w : {"true", "false", "null"}) {
      const size_t n = strlen(w);
      if ((size_t)(end - p) >= n && memcmp(p, w, n) == 0) {
        p += n;
        return true;
      }
    }
    return bad("unexpected character");
  }
};

const DtypeName* find_dtype(const std::string& s) {
  for (const DtypeName& d : kDtypes)
    if (s == d.name) return &d;
  return nullptr;
}

// One tensor entry {"dtype": .., "shape": [..], "data_offsets": [b, e]} (other keys ignored).
bool parse_entry(Json& j, sa_st_tensor& t) {
  memset(&t, 0, sizeof t);
  t.struct_size = sizeof(sa_st_tensor);
  bool have_dtype = false, have_shape = false, have_offsets = false;
  if (!j.lit('{')) return j.bad("a tensor entry is not an object");
  if (!j.lit('}')) {
    do {
      std::string key;
      if (!j.str(key) || !j.lit(':')) return j.bad("expected key: value in a tensor entry");
      if (key == "dtype") {
        std::string s;
        if (!j.str(s)) return j.bad("dtype is not a string");
        const DtypeName* d = find_dtype(s);
        t.dtype = d ? d->code : SA_DT_OTHER;
        t.elem_bytes = d ? d->bytes : 0;
        const size_t n = std::min(s.size(), sizeof(t.dtype_name) - 1);
        memcpy(t.dtype_name, s.data(), n);
        t.dtype_name[n] = '\0';
        have_dtype = true;
      } else if (key == "shape") {
        if (!j.lit('[')) return j.bad("shape is not an array");
        t.ndim = 0;
        t.numel = 1;
        bool overflow = false;
        if (!j.lit(']')) {
          do {
            int64_t v;
            if (!j.uint(v)) return false;
            if (t.ndim >= SA_ST_MAX_DIMS) return j.bad("more than 8 dimensions");
            t.shape[t.ndim++] = v;
            if (v != 0 && t.numel > INT64_MAX / v) overflow = true;
            else t.numel *= v;
          } while (j.lit(','));
          if (!j.lit(']')) return j.bad("unterminated shape");
        }
        if (overflow) return j.bad("shape element count overflows");
        have_shape = true;
      } else if (key == "data_offsets") {
        if (!j.lit('[') || !j.uint(t.begin) || !j.lit(',') || !j.uint(t.end) || !j.lit(']'))
          return j.bad("data_offsets is not [begin, end]");
        have_offsets = true;
      } else if (!j.skip()) {
        return false;
      }
    } while (j.lit(','));
    if (!j.lit('}')) return j.bad("unterminated tensor entry");
  }
  if (!have_dtype || !have_shape || !have_offsets) return j.bad("a tensor entry lacks dtype, shape or data_offsets");
  return true;
}

int parse(sa_st_file* f) {
  if (f->size < 8) return fail(SA_ERR_FORMAT, "file of %lld bytes has no header length", (long long)f->size);
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | f->base[i];
  if (n > (uint64_t)(f->size - 8))
    return fail(SA_ERR_FORMAT, "header length %llu exceeds the file (%lld bytes)", (unsigned long long)n, (long long)f->size);
  f->data_start = 8 + (int64_t)n;
  const int64_t data_bytes = f->size - f->data_start;
  Json j{reinterpret_cast<const char*>(f->base) + 8, reinterpret_cast<const char*>(f->base) + 8 + n, {}};
  if (!j.lit('{')) return fail(SA_ERR_FORMAT, "header is not a JSON object");
  if (!j.lit('}')) {
    do {
      std::string name;
      if (!j.str(name) || !j.lit(':')) return fail(SA_ERR_FORMAT, "header: %s", j.err.empty() ? "expected key: value" : j.err.c_str());
      if (name == "__metadata__") {
        f->meta.clear();  // a repeated key takes its last value
        if (!j.lit('{')) return fail(SA_ERR_FORMAT, "__metadata__ is not an object");
        if (!j.lit('}')) {
          do {
            std::string k, v;
            if (!j.str(k) || !j.lit(':')) return fail(SA_ERR_FORMAT, "__metadata__: %s", j.err.c_str());
            j.ws();
            if (j.p < j.end && *j.p == '"') {
              if (!j.str(v)) return fail(SA_ERR_FORMAT, "__metadata__: %s", j.err.c_str());
            } else {
              const char* b = j.p;
              if (!j.skip()) return fail(SA_ERR_FORMAT, "__metadata__: %s", j.err.c_str());
              v.assign(b, j.p);
            }
            auto it = std::find_if(f->meta.begin(), f->meta.end(), [&](const auto& kv) { return kv.first == k; });
            if (it != f->meta.end()) it->second = v;
            else f->meta.emplace_back(std::move(k), std::move(v));
          } while (j.lit(','));
          if (!j.lit('}')) return fail(SA_ERR_FORMAT, "unterminated __metadata__");
        }
        continue;
      }
      sa_st_tensor t;
      if (!parse_entry(j, t)) return fail(SA_ERR_FORMAT, "tensor %s: %s", name.c_str(), j.err.c_str());
      if (t.begin > t.end || t.end > data_bytes)
        return fail(SA_ERR_FORMAT, "tensor %s: data_offsets [%lld, %lld] outside the %lld-byte data section", name.c_str(),
                    (long long)t.begin, (long long)t.end, (long long)data_bytes);
      if (t.elem_bytes > 0 && (t.numel > INT64_MAX / t.elem_bytes || t.numel * t.elem_bytes != t.end - t.begin))
        return fail(SA_ERR_FORMAT, "tensor %s: %lld bytes for %lld elements of %s", name.c_str(),
                    (long long)(t.end - t.begin), (long long)t.numel, t.dtype_name);
      auto it = f->index.find(name);
      if (it != f->index.end()) {
        f->tensors[it->second].second = t;
      } else {
        f->index.emplace(name, f->tensors.size());
        f->tensors.emplace_back(std::move(name), t);
      }
    } while (j.lit(','));
    if (!j.lit('}')) return fail(SA_ERR_FORMAT, "header: %s", j.err.empty() ? "unterminated object" : j.err.c_str());
  }
  j.ws();
  if (j.p != j.end) return fail(SA_ERR_FORMAT, "header has %lld bytes after its JSON object", (long long)(j.end - j.p));
  return ok();
}

// memcpy split over up to kCopyThreads host threads (slices of at least 1 MiB): one thread cannot
// read a page-cache mapping as fast as the DMA drains pinned memory.
constexpr int kCopyThreads = 8;

void parallel_copy(uint8_t* dst, const uint8_t* src, int64_t len) {
  constexpr int64_t kMinSlice = 1 << 20;
  const int64_t want = std::min<int64_t>(kCopyThreads, std::max<int64_t>(1, len / kMinSlice));
  const int64_t slice = ((len + want - 1) / want + 4095) & ~(int64_t)4095;
  std::vector<std::thread> pool;
  int64_t done = slice;  // bytes [slice, done) are handed to started threads
  try {
    pool.reserve((size_t)want);
    for (; done < len; done += slice) {
      const int64_t off = done, n = std::min(slice, len - done);
      pool.emplace_back([=] { memcpy(dst + off, src + off, (size_t)n); });
    }
  } catch (...) {
    // a thread could not start: this thread copies what was not handed out
  }
  memcpy(dst, src, (size_t)std::min(slice, len));
  if (done < len) memcpy(dst + done, src + done, (size_t)(len - done));
  for (std::thread& t : pool) t.join();
}

int finish_open(sa_st_file* f, sa_st_file** out) {
  int rc;
  try {
    rc = parse(f);
  } catch (...) {
    if (f->map) munmap(f->map, (size_t)f->size);
    delete f;
    throw;
  }
  if (rc != SA_OK) {
    if (f->map) munmap(f->map, (size_t)f->size);
    delete f;
    return rc;
  }
  *out = f;
  return ok();
}

int open_file(const char* path, sa_st_file** out);
int open_memory(const void* bytes, int64_t size, sa_st_file** out);
int upload(const sa_st_file* f, int64_t begin, int64_t end, void* dst, void* staging, int64_t staging_bytes,
           void* stream);

// Runs `body` and turns a C++ exception (host allocation failure) into an error status: nothing
// propagates across the C ABI.
template <class F>
int guarded(F body) {
  try {
    return body();
  } catch (const std::exception& e) {
    return fail(SA_ERR_IO, "host allocation failed: %s", e.what());
  } catch (...) {
    return fail(SA_ERR_IO, "host allocation failed");
  }
}

}  // namespace

extern "C" {

int sa_st_open(const char* path, sa_st_file** out) {
  return guarded([&] { return open_file(path, out); });
}

int sa_st_open_memory(const void* bytes, int64_t size, sa_st_file** out) {
  return guarded([&] { return open_memory(bytes, size, out); });
}

}  // extern "C"

namespace {

int open_file(const char* path, sa_st_file** out) {
  if (!out) return fail(SA_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (!path) return fail(SA_ERR_INVALID, "path is NULL");
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(SA_ERR_IO, "open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    close(fd);
    return fail(SA_ERR_IO, "stat %s: %s", path, strerror(e));
  }
  if (st.st_size < 8) {
    close(fd);
    return fail(SA_ERR_FORMAT, "%s: %lld bytes, no header length", path, (long long)st.st_size);
  }
  void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  const int e = errno;
  close(fd);
  if (map == MAP_FAILED) return fail(SA_ERR_IO, "mmap %s: %s", path, strerror(e));
  madvise(map, (size_t)st.st_size, MADV_SEQUENTIAL);
  sa_st_file* f = new (std::nothrow) sa_st_file;
  if (!f) {
    munmap(map, (size_t)st.st_size);
    return fail(SA_ERR_IO, "out of host memory");
  }
  f->base = static_cast<const uint8_t*>(map);
  f->size = st.st_size;
  f->map = map;
  return finish_open(f, out);
}

int open_memory(const void* bytes, int64_t size, sa_st_file** out) {
  if (!out) return fail(SA_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (!bytes || size < 0) return fail(SA_ERR_INVALID, "bytes is NULL or size is negative");
  sa_st_file* f = new (std::nothrow) sa_st_file;
  if (!f) return fail(SA_ERR_IO, "out of host memory");
  f->base = static_cast<const uint8_t*>(bytes);
  f->size = size;
  return finish_open(f, out);
}

}  // namespace

extern "C" {

int sa_st_close(sa_st_file* f) {
  if (!f) return ok();
  if (f->map) munmap(f->map, (size_t)f->size);
  delete f;
  return ok();
}

int64_t sa_st_count(const sa_st_file* f) { return f ? (int64_t)f->tensors.size() : 0; }

const char* sa_st_name(const sa_st_file* f, int64_t i) {
  if (!f || i < 0 || i >= (int64_t)f->tensors.size()) return nullptr;
  return f->tensors[(size_t)i].first.c_str();
}

int sa_st_info(const sa_st_file* f, const char* name, sa_st_tensor* out) {
  if (!f || !name || !out) return fail(SA_ERR_INVALID, "NULL argument");
  if (out->struct_size != sizeof(sa_st_tensor))
    return fail(SA_ERR_INVALID, "struct_size %u != sizeof(sa_st_tensor) %zu", out->struct_size, sizeof(sa_st_tensor));
  return guarded([&] {
    auto it = f->index.find(name);
    if (it == f->index.end()) return fail(SA_ERR_NOT_FOUND, "missing tensor %s", name);
    *out = f->tensors[it->second].second;
    return ok();
  });
}

int64_t sa_st_metadata_count(const sa_st_file* f) { return f ? (int64_t)f->meta.size() : 0; }

const char* sa_st_metadata_key(const sa_st_file* f, int64_t i) {
  if (!f || i < 0 || i >= (int64_t)f->meta.size()) return nullptr;
  return f->meta[(size_t)i].first.c_str();
}

const char* sa_st_metadata_value(const sa_st_file* f, const char* key) {
  if (!f || !key) return nullptr;
  for (const auto& kv : f->meta)
    if (kv.first == key) return kv.second.c_str();
  return nullptr;
}

int64_t sa_st_data_bytes(const sa_st_file* f) { return f ? f->size - f->data_start : 0; }

const void* sa_st_data(const sa_st_file* f) { return f ? f->base + f->data_start : nullptr; }

int sa_st_upload(const sa_st_file* f, int64_t begin, int64_t end, void* dst, void* staging, int64_t staging_bytes,
                 void* stream) {
  return guarded([&] { return upload(f, begin, end, dst, staging, staging_bytes, stream); });
}

}  // extern "C"

namespace {

int upload(const sa_st_file* f, int64_t begin, int64_t end, void* dst, void* staging, int64_t staging_bytes,
           void* stream) {
  if (!f) return fail(SA_ERR_INVALID, "file is NULL");
  const int64_t data_bytes = f->size - f->data_start;
  if (begin < 0 || begin > end || end > data_bytes)
    return fail(SA_ERR_INVALID, "range [%lld, %lld) outside the %lld-byte data section", (long long)begin, (long long)end,
                (long long)data_bytes);
  if (begin == end) return ok();
  if (!dst) return fail(SA_ERR_INVALID, "dst is NULL");
  const uint8_t* src = f->base + f->data_start + begin;
  const int64_t n = end - begin;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (!staging) {
    e = hipMemcpyAsync(dst, src, (size_t)n, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? ok() : sa::hip_fail(e, "upload");
  }
  constexpr int64_t kMinStaging = 2 << 20;
  if (staging_bytes < kMinStaging)
    return fail(SA_ERR_INVALID, "staging of %lld bytes (at least %lld)", (long long)staging_bytes, (long long)kMinStaging);
  const int64_t half = (staging_bytes / 2) & ~(int64_t)4095;
  hipEvent_t done[2] = {nullptr, nullptr};
  for (hipEvent_t& ev : done) {
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) break;
  }
  // chunk i fills staging half i % 2 from the mapping, then queues its DMA; before a half is
  // refilled, the DMA that last read it must have finished
  int64_t i = 0;
  for (int64_t off = 0; e == hipSuccess && off < n; off += half, ++i) {
    const int b = (int)(i & 1);
    const int64_t len = std::min(half, n - off);
    uint8_t* stage = static_cast<uint8_t*>(staging) + b * half;
    if (i >= 2) e = hipEventSynchronize(done[b]);
    if (e != hipSuccess) break;
    parallel_copy(stage, src + off, len);
    e = hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, stage, (size_t)len, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipEventRecord(done[b], s);
  }
  const hipError_t sync = hipStreamSynchronize(s);  // the staging buffer is the caller's again on return
  if (e == hipSuccess) e = sync;
  for (hipEvent_t ev : done)
    if (ev) (void)hipEventDestroy(ev);
  return e == hipSuccess ? ok() : sa::hip_fail(e, "staged upload");
}

}  // namespace
