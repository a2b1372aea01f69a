// mxq_safetensors.cpp — read-only access to .safetensors files holding the
// quantized triples (`prefix.weight` U32 packed codes + bf16 scales/biases).
//
// Follows the reference's own loaders: H3Weights parses the header once and
// reads tensors on demand (`model/minimax h3/H3Common.swift:181-260`), and
// MappedSafetensors maps the file read-only so that a tensor's bytes come from
// the page cache instead of a second heap copy
// (`model/3模块/Safetensors-mmap映射-通用.swift:40-135`). On MI355X the bytes
// then have to cross PCIe into HBM: mxq_st_read streams them through two
// pinned staging buffers, so the copy out of the mapping (which takes the page
// faults / disk reads; several threads per chunk) of chunk i+1 overlaps the
// DMA of chunk i, with MADV_WILLNEED readahead one chunk ahead.
//
// File format (safetensors): 8-byte little-endian header length n, n bytes of
// JSON {"key": {"dtype": "U32", "shape": [..], "data_offsets": [lo, hi]}, ...,
// "__metadata__": {...}}, then the data area; offsets are relative to it.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "mxq.h"

// the library's error reporting (mxq_api.cpp)
namespace mxq {
int set_error(int status, const char* fmt, ...);
int clear_error();
}  // namespace mxq

namespace {

constexpr size_t kChunk = 16u << 20;  // bytes per staging buffer
constexpr unsigned kMaxCopyThreads = 8;  // threads copying a chunk out of the mapping

// dst[0, n) = src[0, n) with up to kMaxCopyThreads threads (one copy thread
// is far below the host link: the page faults and memcpy of the mapped bytes
// would bound the upload)
void parallel_copy(void* dst, const void* src, size_t n) {
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const unsigned t = static_cast<unsigned>(
      std::min<size_t>({kMaxCopyThreads, hw, std::max<size_t>(1, n >> 20)}));
  if (t <= 1) {
    std::memcpy(dst, src, n);
    return;
  }
  const size_t part = (n / t + 4095) & ~size_t(4095);
  std::vector<std::thread> pool;
  pool.reserve(t - 1);
  for (unsigned i = 1; i < t; ++i) {
    const size_t a = std::min(n, i * part), b = std::min(n, a + part);
    if (a < b)
      pool.emplace_back([=] {
        std::memcpy(static_cast<uint8_t*>(dst) + a, static_cast<const uint8_t*>(src) + a, b - a);
      });
  }
  std::memcpy(dst, src, std::min(n, part));
  for (auto& th : pool) th.join();
}

struct Entry {
  std::string key;
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t offset = 0;  // absolute byte offset in the file
  int64_t nbytes = 0;
};

int64_t itemsize(const std::string& d) {
  if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  if (d == "U16" || d == "I16" || d == "F16" || d == "BF16") return 2;
  if (d == "U32" || d == "I32" || d == "F32") return 4;
  if (d == "U64" || d == "I64" || d == "F64") return 8;
  return 0;  // unknown: size not checked
}

// ---- a small JSON reader for the header (objects, arrays, strings, numbers,
// literals); values that are not needed are parsed and skipped
class Json {
 public:
  Json(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool ok() const { return err_.empty(); }
  const std::string& error() const { return err_; }

  bool header(std::vector<Entry>& out) {
    ws();
    if (!eat('{')) return fail("header is not a JSON object");
    ws();
    if (eat('}')) return true;
    for (;;) {
      std::string key;
      if (!string(key)) return false;
      ws();
      if (!eat(':')) return fail("expected ':'");
      ws();
      if (key == "__metadata__") {
        if (!skip()) return false;
      } else {
        Entry e;
        e.key = key;
        if (!tensor(e)) return false;
        out.push_back(std::move(e));
      }
      ws();
      if (eat(',')) {
        ws();
        continue;
      }
      if (eat('}')) break;
      return fail("expected ',' or '}'");
    }
    ws();
    if (p_ != end_) return fail("trailing bytes after the header object");
    return true;
  }

 private:
  bool tensor(Entry& e) {
    if (!eat('{')) return fail("tensor entry is not an object");
    bool have_dtype = false, have_shape = false, have_offsets = false;
    int64_t lo = 0, hi = 0;
    ws();
    if (!eat('}')) {
      for (;;) {
        std::string f;
        ws();
        if (!string(f)) return false;
        ws();
        if (!eat(':')) return fail("expected ':'");
        ws();
        if (f == "dtype") {
          if (!string(e.dtype)) return false;
          have_dtype = true;
        } else if (f == "shape") {
          if (!ints(e.shape)) return false;
          have_shape = true;
        } else if (f == "data_offsets") {
          std::vector<int64_t> o;
          if (!ints(o)) return false;
          if (o.size() != 2) return fail("data_offsets must have two entries");
          lo = o[0];
          hi = o[1];
          have_offsets = true;
        } else if (!skip()) {
          return false;
        }
        ws();
        if (eat(',')) continue;
        if (eat('}')) break;
        return fail("expected ',' or '}' in a tensor entry");
      }
    }
    if (!have_dtype || !have_shape || !have_offsets)
      return fail("tensor '" + e.key + "' lacks dtype, shape or data_offsets");
    if (lo < 0 || hi < lo) return fail("tensor '" + e.key + "' has bad data_offsets");
    e.offset = lo;
    e.nbytes = hi - lo;
    return true;
  }
  bool ints(std::vector<int64_t>& v) {
    if (!eat('[')) return fail("expected an array");
    ws();
    if (eat(']')) return true;
    for (;;) {
      ws();
      int64_t x = 0;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("expected a non-negative integer");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
        if (x > (INT64_MAX - 9) / 10) return fail("integer too large");
        x = x * 10 + (*p_++ - '0');
      }
      v.push_back(x);
      ws();
      if (eat(',')) continue;
      if (eat(']')) return true;
      return fail("expected ',' or ']'");
    }
  }
  bool string(std::string& s) {
    if (!eat('"')) return fail("expected a string");
    while (p_ < end_ && *p_ != '"') {
      if (*p_ == '\\') {
        if (++p_ >= end_) break;
        const char c = *p_++;
        switch (c) {
          case 'n': s += '\n'; break;
          case 't': s += '\t'; break;
          case 'r': s += '\r'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'u': {  // keep the code unit as UTF-8 (BMP; surrogates pass through)
            if (end_ - p_ < 4) return fail("bad \\u escape");
            unsigned cp = 0;
            for (int i = 0; i < 4; ++i) {
              const char h = *p_++;
              cp = cp * 16 + (h >= '0' && h <= '9' ? h - '0'
                              : h >= 'a' && h <= 'f' ? h - 'a' + 10
                              : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
              if (cp > 0xFFFF) return fail("bad \\u escape");
            }
            if (cp < 0x80) {
              s += static_cast<char>(cp);
            } else if (cp < 0x800) {
              s += static_cast<char>(0xC0 | (cp >> 6));
              s += static_cast<char>(0x80 | (cp & 0x3F));
            } else {
              s += static_cast<char>(0xE0 | (cp >> 12));
              s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
              s += static_cast<char>(0x80 | (cp & 0x3F));
            }
            break;
          }
          default: s += c;  // \" \\ \/
        }
      } else {
        s += *p_++;
      }
    }
    if (!eat('"')) return fail("unterminated string");
    return true;
  }
  bool skip(int depth = 0) {  // any value
    ws();
    if (p_ >= end_) return fail("unexpected end of header");
    if (depth > 64) return fail("header nested too deeply");
    if (*p_ == '"') {
      std::string t;
      return string(t);
    }
    if (*p_ == '{' || *p_ == '[') {
      const char close = *p_ == '{' ? '}' : ']';
      const bool obj = *p_ == '{';
      ++p_;
      ws();
      if (eat(close)) return true;
      for (;;) {
        ws();
        if (obj) {
          std::string k;
          if (!string(k)) return false;
          ws();
          if (!eat(':')) return fail("expected ':'");
        }
        if (!skip(depth + 1)) return false;
        ws();
        if (eat(',')) continue;
        if (eat(close)) return true;
        return fail("unbalanced header JSON");
      }
    }
    // number or literal
    const char* s = p_;
    while (p_ < end_ && *p_ != '\0' &&
           (std::strchr("+-.0123456789", *p_) || std::isalpha(static_cast<unsigned char>(*p_))))
      ++p_;
    if (p_ == s) return fail("unexpected character in header");
    return true;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  bool eat(char c) {
    if (p_ < end_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  bool fail(const std::string& m) {
    if (err_.empty()) err_ = m;
    return false;
  }
  const char* p_;
  const char* end_;
  std::string err_;
};

}  // namespace

struct mxq_safetensors {
  int fd = -1;
  uint8_t* base = nullptr;
  size_t size = 0;
  std::string path;
  std::vector<Entry> entries;
  std::unordered_map<std::string, size_t> index;
  // pinned staging for device reads, created on the first one
  void* pinned[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  bool pending[2] = {false, false};
};

namespace {

int st_fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return mxq::set_error(status, "%s", buf);
}

const Entry* find(const mxq_safetensors* st, const char* key) {
  if (!st || !key) return nullptr;
  auto it = st->index.find(key);
  return it == st->index.end() ? nullptr : &st->entries[it->second];
}

void release(mxq_safetensors* st) {
  for (int k = 0; k < 2; ++k) {
    if (st->done[k]) {
      if (st->pending[k]) (void)hipEventSynchronize(st->done[k]);
      (void)hipEventDestroy(st->done[k]);
    }
    if (st->pinned[k]) (void)hipHostFree(st->pinned[k]);
  }
  if (st->base) munmap(st->base, st->size);
  if (st->fd >= 0) close(st->fd);
  delete st;
}

}  // namespace

extern "C" {

int mxq_st_open(const char* path, mxq_safetensors** out) {
  if (!path || !out) return st_fail(MXQ_ERR_NULL, "[safetensors] path and out must be non-NULL.");
  *out = nullptr;
  auto* st = new mxq_safetensors();
  st->path = path;
  st->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (st->fd < 0) {
    release(st);
    return st_fail(MXQ_ERR_INVALID, "[safetensors] open failed: %s", path);
  }
  struct stat sb;
  if (fstat(st->fd, &sb) != 0 || sb.st_size < 8) {
    release(st);
    return st_fail(MXQ_ERR_INVALID, "[safetensors] bad header: file too small: %s", path);
  }
  st->size = static_cast<size_t>(sb.st_size);
  void* m = mmap(nullptr, st->size, PROT_READ, MAP_PRIVATE, st->fd, 0);
  if (m == MAP_FAILED) {
    release(st);
    return st_fail(MXQ_ERR_INVALID, "[safetensors] mmap failed: %s", path);
  }
  st->base = static_cast<uint8_t*>(m);
  uint64_t n = 0;
  std::memcpy(&n, st->base, 8);  // little-endian host
  if (n == 0 || n > st->size - 8) {
    release(st);
    return st_fail(MXQ_ERR_INVALID, "[safetensors] bad header: length out of range: %s", path);
  }
  Json j(reinterpret_cast<const char*>(st->base + 8), n);
  if (!j.header(st->entries)) {
    const std::string e = j.error();
    release(st);
    return st_fail(MXQ_ERR_INVALID, "[safetensors] bad header: %s: %s", e.c_str(), path);
  }
  // data region [start, size); the parser guarantees 0 <= offset (lo) and
  // 0 <= nbytes (hi - lo), so both comparisons below are between non-negative
  // values no larger than the file, and no sum can overflow
  const uint64_t start = 8 + n;
  const uint64_t data = st->size - start;
  for (size_t i = 0; i < st->entries.size(); ++i) {
    Entry& e = st->entries[i];
    const bool in_file = static_cast<uint64_t>(e.offset) <= data &&
                         static_cast<uint64_t>(e.nbytes) <= data - static_cast<uint64_t>(e.offset);
    if (in_file) e.offset += static_cast<int64_t>(start);
    int64_t count = 1;
    for (int64_t d : e.shape)  // -1 once the product overflows
      count = count < 0 ? -1 : d == 0 || count <= INT64_MAX / d ? count * d : -1;
    // a dtype this reader does not know is kept as raw bytes (range-checked above,
    // element count unchecked)
    const int64_t isz = itemsize(e.dtype);
    int64_t want = 0;
    const bool size_ok = count >= 0 && (isz == 0 || (!__builtin_mul_overflow(count, isz, &want) &&
                                                      want == e.nbytes));
    if (!in_file || !size_ok || !st->index.emplace(e.key, i).second) {
      const std::string k = e.key;
      release(st);
      return st_fail(MXQ_ERR_INVALID,
                     "[safetensors] bad header: tensor '%s' has a bad size, range or a "
                     "duplicate key: %s", k.c_str(), path);
    }
  }
  *out = st;
  return mxq::clear_error();
}

void mxq_st_close(mxq_safetensors* st) {
  if (st) release(st);
}

int64_t mxq_st_count(const mxq_safetensors* st) {
  return st ? static_cast<int64_t>(st->entries.size()) : 0;
}

const char* mxq_st_key(const mxq_safetensors* st, int64_t i) {
  if (!st || i < 0 || i >= static_cast<int64_t>(st->entries.size())) return nullptr;
  return st->entries[static_cast<size_t>(i)].key.c_str();
}

int mxq_st_info(const mxq_safetensors* st, const char* key, char dtype[16], int* ndim,
                int64_t shape[MXQ_ST_MAX_DIMS], int64_t* nbytes) {
  const Entry* e = find(st, key);
  if (!st || !key) return st_fail(MXQ_ERR_NULL, "[safetensors] handle and key must be non-NULL.");
  if (!e) return st_fail(MXQ_ERR_INVALID, "[safetensors] no tensor '%s'.", key);
  if (e->shape.size() > MXQ_ST_MAX_DIMS)
    return st_fail(MXQ_ERR_UNSUPPORTED, "[safetensors] tensor '%s' has more than %d dims.", key,
                   MXQ_ST_MAX_DIMS);
  if (dtype) {
    std::memset(dtype, 0, 16);
    std::strncpy(dtype, e->dtype.c_str(), 15);
  }
  if (ndim) *ndim = static_cast<int>(e->shape.size());
  if (shape)
    for (size_t i = 0; i < e->shape.size(); ++i) shape[i] = e->shape[i];
  if (nbytes) *nbytes = e->nbytes;
  return mxq::clear_error();
}

int mxq_st_read_host(const mxq_safetensors* st, const char* key, void* dst) {
  const Entry* e = find(st, key);
  if (!st || !key) return st_fail(MXQ_ERR_NULL, "[safetensors] handle and key must be non-NULL.");
  if (!e) return st_fail(MXQ_ERR_INVALID, "[safetensors] no tensor '%s'.", key);
  if (e->nbytes && !dst) return st_fail(MXQ_ERR_NULL, "[safetensors] dst must be non-NULL.");
  if (e->nbytes) std::memcpy(dst, st->base + e->offset, static_cast<size_t>(e->nbytes));
  return mxq::clear_error();
}

int mxq_st_read(mxq_safetensors* st, const char* key, void* dst, mxq_stream stream) {
  const Entry* e = find(st, key);
  if (!st || !key) return st_fail(MXQ_ERR_NULL, "[safetensors] handle and key must be non-NULL.");
  if (!e) return st_fail(MXQ_ERR_INVALID, "[safetensors] no tensor '%s'.", key);
  if (e->nbytes == 0) return mxq::clear_error();
  if (!dst) return st_fail(MXQ_ERR_NULL, "[safetensors] dst must be non-NULL.");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int k = 0; k < 2; ++k) {
    if (!st->pinned[k]) {
      hipError_t r = hipHostMalloc(&st->pinned[k], kChunk, hipHostMallocDefault);
      if (r == hipSuccess)
        r = hipEventCreateWithFlags(&st->done[k], hipEventDisableTiming);
      if (r != hipSuccess)
        return st_fail(MXQ_ERR_HIP, "[safetensors] HIP error: %s", hipGetErrorString(r));
    }
  }
  const uint8_t* src = st->base + e->offset;
  const size_t total = static_cast<size_t>(e->nbytes);
  const uintptr_t page = static_cast<uintptr_t>(sysconf(_SC_PAGESIZE));
  auto advise = [&](size_t off) {  // read ahead the chunk at `off`
    if (off >= total) return;
    const uintptr_t a = reinterpret_cast<uintptr_t>(src + off) & ~(page - 1);
    const size_t len = std::min(kChunk, total - off) + (reinterpret_cast<uintptr_t>(src + off) - a);
    (void)madvise(reinterpret_cast<void*>(a), len, MADV_WILLNEED);
  };
  advise(0);
  int k = 0;
  for (size_t off = 0; off < total; off += kChunk, k ^= 1) {
    const size_t n = std::min(kChunk, total - off);
    advise(off + kChunk);
    if (st->pending[k]) {
      const hipError_t r = hipEventSynchronize(st->done[k]);
      st->pending[k] = false;
      if (r != hipSuccess)
        return st_fail(MXQ_ERR_HIP, "[safetensors] HIP error: %s", hipGetErrorString(r));
    }
    parallel_copy(st->pinned[k], src + off, n);
    hipError_t r = hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, st->pinned[k], n,
                                  hipMemcpyHostToDevice, s);
    if (r == hipSuccess) r = hipEventRecord(st->done[k], s);
    if (r != hipSuccess)
      return st_fail(MXQ_ERR_HIP, "[safetensors] HIP error: %s", hipGetErrorString(r));
    st->pending[k] = true;
  }
  return mxq::clear_error();
}

}  // extern "C"
