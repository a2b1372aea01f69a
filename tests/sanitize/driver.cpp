// Driver for the host-only sanitizer build of libmxq's C ABI (see
// tests/test_sanitize.py). Built with g++ -fsanitize=address,undefined against
// mxq_api.cpp, mxq_safetensors.cpp, a HIP stand-in (hip/hip_runtime.h here)
// and counting launchers (launch_stub.cpp), so any out-of-bounds access or
// undefined behaviour in the header parser or the argument checks aborts the
// run.
//
//   driver files PATH...       open, inspect and read every tensor of each file
//   driver fuzz SEED COUNT DIR  COUNT random and mutated headers, bounded, fixed seed
//   driver api SEED COUNT       every entry point with COUNT random edge-case argument sets
//
// Prints one line per file or case; exits 0 unless a sanitizer aborts first.
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mxq.h"

extern int g_launches;

namespace {

uint64_t g_state = 0;
uint64_t next() {  // splitmix64
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint64_t below(uint64_t n) { return n ? next() % n : 0; }

int read_all(const char* path) {
  mxq_safetensors* st = nullptr;
  const int rc = mxq_st_open(path, &st);
  if (rc != MXQ_OK) return rc;
  const int64_t n = mxq_st_count(st);
  for (int64_t i = 0; i < n; ++i) {
    const char* key = mxq_st_key(st, i);
    char dtype[16];
    int ndim = 0;
    int64_t shape[MXQ_ST_MAX_DIMS], nbytes = 0;
    if (mxq_st_info(st, key, dtype, &ndim, shape, &nbytes) != MXQ_OK) continue;
    std::vector<unsigned char> host(static_cast<size_t>(nbytes) + 1), dev(host.size());
    mxq_st_read_host(st, key, host.data());
    mxq_st_read(st, key, dev.data(), nullptr);  // "device" memory is host memory here
    if (nbytes && std::memcmp(host.data(), dev.data(), static_cast<size_t>(nbytes)) != 0) {
      std::printf("read mismatch: %s %s\n", path, key);
      std::exit(3);
    }
  }
  mxq_st_info(st, "no such key", nullptr, nullptr, nullptr, nullptr);
  mxq_st_key(st, -1);
  mxq_st_key(st, n);
  mxq_st_close(st);
  return MXQ_OK;
}

// ---- header fuzz
const char* kDtypes[] = {"F32", "BF16", "U32", "U8", "F64", "I64", "BOOL", "F8_E4M3", "XX", ""};
const uint64_t kBig[] = {0, 1, 2, 3, 7, 8, 64, 255, 256, 4096, (1ull << 31) - 1, 1ull << 31,
                         (1ull << 62), (1ull << 63) - 1, (1ull << 63) - 37, (1ull << 63) - 101,
                         9223372036854775808ull, 18446744073709551615ull};

uint64_t pick_number(uint64_t data) {
  switch (below(4)) {
    case 0: return below(data + 2);
    case 1: return data + below(3);
    case 2: return kBig[below(sizeof(kBig) / sizeof(kBig[0]))];
    default: return next() >> below(64);
  }
}

std::string header(uint64_t data) {
  std::string h = "{";
  const int tensors = static_cast<int>(below(4));
  if (below(4) == 0) h += "\"__metadata__\": {\"format\": \"pt\", \"x\": [1, {\"y\": null}]}, ";
  for (int t = 0; t < tensors; ++t) {
    if (t) h += ", ";
    h += "\"t" + std::to_string(below(3) == 0 ? 0 : t) + "\": {";
    h += std::string("\"dtype\": \"") + kDtypes[below(sizeof(kDtypes) / sizeof(kDtypes[0]))] + "\"";
    h += ", \"shape\": [";
    const int nd = static_cast<int>(below(10));
    for (int d = 0; d < nd; ++d) h += (d ? ", " : "") + std::to_string(pick_number(data));
    h += "], \"data_offsets\": [";
    const uint64_t lo = pick_number(data), hi = below(3) ? lo + below(data + 2) : pick_number(data);
    h += std::to_string(lo) + ", " + std::to_string(hi) + "]";
    if (below(6) == 0) h += ", \"extra\": [true, false, \"\\u00e9\\n\"]";
    h += "}";
  }
  h += "}";
  // byte-level mutations
  const int muts = below(3) ? 0 : static_cast<int>(below(4)) + 1;
  for (int m = 0; m < muts && !h.empty(); ++m) {
    const size_t at = below(h.size());
    switch (below(4)) {
      case 0: h[at] = static_cast<char>(next()); break;
      case 1: h.erase(at, 1); break;
      case 2: h.insert(at, 1, "{}[]\",:\\ 0e-"[below(13)]); break;
      default: h.resize(at); break;
    }
  }
  return h;
}

int fuzz(uint64_t seed, int count, const char* dir) {
  g_state = seed;
  const std::string path = std::string(dir) + "/fuzz.safetensors";
  int accepted = 0;
  for (int i = 0; i < count; ++i) {
    const uint64_t data = below(200);
    const std::string h = header(data);
    uint64_t n = h.size();
    if (below(10) == 0) n = pick_number(h.size() + data);  // a wrong length field
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return 2;
    std::fwrite(&n, 8, 1, f);
    std::fwrite(h.data(), 1, h.size(), f);
    for (uint64_t j = 0; j < data; ++j) std::fputc(static_cast<int>(j * 7 + i), f);
    std::fclose(f);
    if (read_all(path.c_str()) == MXQ_OK) ++accepted;
  }
  std::printf("fuzz seed=%" PRIu64 " cases=%d accepted=%d\n", seed, count, accepted);
  return 0;
}

// ---- argument checks of every entry point
const int64_t kDims[] = {-1, 0, 1, 2, 8, 9, 31, 32, 33, 63, 64, 96, 128, 4096, 16384,
                         (1ll << 22), (1ll << 22) + 64, (1ll << 31) - 1, (1ll << 31),
                         (1ll << 40), (1ll << 62), INT64_MAX};
const int kBits[] = {-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 16};
const int kGs[] = {-64, 0, 16, 32, 64, 100, 128, 256};

int64_t dim() { return kDims[below(sizeof(kDims) / sizeof(kDims[0]))]; }
int bits() { return kBits[below(sizeof(kBits) / sizeof(kBits[0]))]; }
int gsz() { return kGs[below(sizeof(kGs) / sizeof(kGs[0]))]; }
// a pointer that is never dereferenced in this build: NULL, aligned or misaligned
void* ptr() {
  static unsigned char arena[64] __attribute__((aligned(256)));
  switch (below(6)) {
    case 0: return nullptr;
    case 1: return arena + 2;
    case 2: return arena + 4;
    default: return arena;
  }
}

int api(uint64_t seed, int count) {
  g_state = seed;
  for (int i = 0; i < count; ++i) {
    const int64_t M = dim(), N = dim(), K = dim(), R = dim();
    const int b = bits(), gs = gsz(), act = static_cast<int>(below(4)) - 1;
    const int dt = static_cast<int>(below(3));
    void *x = ptr(), *w = ptr(), *s = ptr(), *c = ptr(), *y = ptr(), *t = ptr();
    const uint32_t* wq = static_cast<const uint32_t*>(w);
    mxq_quantize(x, dt, M, K, gs, b, static_cast<int>(below(3)), static_cast<uint32_t*>(w), s, c,
                 dt, nullptr);
    mxq_dequantize(wq, s, c, dt, M, K, gs, b, y, dt, nullptr);
    mxq_pack(static_cast<const uint8_t*>(x), M, K, b, static_cast<uint32_t*>(w), nullptr);
    mxq_unpack(wq, M, K, b, static_cast<uint8_t*>(y), nullptr);
    mxq_quantized_matmul(x, M, K, wq, s, c, N, static_cast<int>(below(2)), gs, b,
                         below(2) ? t : nullptr, y, nullptr);
    mxq_quantized_matmul_workspace_size(M, N, K, gs, b);
    mxq_quantized_matmul_ws(x, M, K, wq, s, c, N, 1, gs, b, nullptr, y, t,
                            static_cast<size_t>(below(1u << 20)), nullptr);
    mxq_quantized_matmul_noalloc(x, M, K, wq, s, c, N, static_cast<int>(below(2)), gs, b,
                                 nullptr, y, nullptr);
    mxq_qmm(x, M, K, wq, s, c, N, gs, b, nullptr, y, nullptr);
    mxq_qmv(x, M, K, wq, s, c, N, gs, b, nullptr, y, nullptr);
    mxq_tiled_bytes(N, K, gs, b);
    mxq_tile(wq, s, c, N, K, gs, b, t, nullptr);
    mxq_tile_swiglu(wq, s, c, N, K, gs, b, t, nullptr);
    mxq_untile(t, N, K, gs, b, static_cast<uint32_t*>(w), s, c, nullptr);
    mxq_untile_swiglu(t, N, K, gs, b, static_cast<uint32_t*>(w), s, c, nullptr);
    mxq_quantized_matmul_tiled(x, M, K, t, N, gs, b, nullptr, y, nullptr);
    mxq_qmm_tiled(x, M, K, t, N, gs, b, nullptr, y, nullptr);
    mxq_qmv_tiled(x, M, K, t, N, gs, b, nullptr, y, nullptr);
    mxq_qmm_tiled_act(x, M, K, t, N, gs, b, nullptr, act, y, nullptr);
    mxq_qmm_tiled_lora(x, M, K, t, N, gs, b, nullptr, act, s, c, R, y, nullptr);
    mxq_norm_modscale(x, M, K, w, s, c, N, static_cast<const uint32_t*>(t), 1e-6f, y, nullptr);
    mxq_mod_gate(x, w, M, K, s, N, static_cast<const uint32_t*>(t), y, nullptr);
    mxq_rmsnorm_rope(x, M, N, K, w, s, c, dt, static_cast<int>(R & 1023), 1e-6f, y, nullptr);
    {  // the memory and stream helpers ("device" memory is host memory in this build)
      mxq_stream st = nullptr;
      void* d = nullptr;
      unsigned char h[32] = {0};
      const size_t n = static_cast<size_t>(below(3)) * 16;
      mxq_stream_create(below(8) ? &st : nullptr);
      mxq_malloc(below(8) ? &d : nullptr, n);
      mxq_copy_to_device(below(6) ? d : nullptr, h, n, st);
      mxq_copy_to_host(h, below(6) ? d : nullptr, n, st);
      mxq_stream_synchronize(st);
      mxq_free(d);
      mxq_stream_destroy(st);
    }
    mxq_status_string(static_cast<int>(below(12)) - 8);
    (void)mxq_last_error();
  }
  std::printf("api seed=%" PRIu64 " cases=%d launches=%d\n", seed, count, g_launches);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 3 && std::strcmp(argv[1], "files") == 0) {
    for (int i = 2; i < argc; ++i) std::printf("%s %d\n", argv[i], read_all(argv[i]));
    return 0;
  }
  if (argc == 5 && std::strcmp(argv[1], "fuzz") == 0)
    return fuzz(std::strtoull(argv[2], nullptr, 10), std::atoi(argv[3]), argv[4]);
  if (argc == 4 && std::strcmp(argv[1], "api") == 0)
    return api(std::strtoull(argv[2], nullptr, 10), std::atoi(argv[3]));
  std::fprintf(stderr, "usage: driver files PATH... | fuzz SEED COUNT DIR | api SEED COUNT\n");
  return 2;
}
