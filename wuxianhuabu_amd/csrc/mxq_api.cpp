// mxq_api.cpp — the C ABI declared in include/mxq.h.
//
// Argument checking mirrors what mlx rejects before it launches anything
// (unsupported bits / group size, K not a multiple of the group size, shape
// mismatches between the packed weight and scales/biases), and each message
// names the mlx operation it stands in for, as mlx's own messages do
// ("[quantize] ...", "[quantized_matmul] ..."). The reference reaches these
// checks through MLX-Swift (`model/minimax h3/H3Common.swift:358-359`).
// Device memory is allocated only by mxq_malloc (for hosts without HIP) and, for
// mxq_quantized_matmul's large-M calls, as a stream-ordered workspace from a memory pool
// this library owns (one per GPU).
#include "../../include/mxq.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>

#include "mxq_internal.hpp"
#include "mxq_tiled.hpp"

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = '\0';
  return MXQ_OK;
}

bool bits_supported(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}
bool gs_supported(int gs) { return gs == 32 || gs == 64 || gs == 128; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
// rows x cols elements (both non-negative): their bit counts, and rows or cols
// rounded up to a block of 64, stay within int64
bool fits(int64_t rows, int64_t cols) {
  return rows <= INT64_MAX / 64 && cols <= INT64_MAX / 64 &&
         (rows == 0 || cols <= INT64_MAX / 64 / rows);
}

int check_bits_gs(const char* op, int bits, int gs, int64_t cols) {
  if (!bits_supported(bits))
    return fail(MXQ_ERR_INVALID,
                "[%s] The requested number of bits %d is not supported. The supported "
                "bits are 2, 3, 4, 5, 6 and 8.",
                op, bits);
  if (!gs_supported(gs))
    return fail(MXQ_ERR_INVALID,
                "[%s] The requested group size %d is not supported. The supported group "
                "sizes are 32, 64, and 128.",
                op, gs);
  if (cols < 0 || cols % gs != 0)
    return fail(MXQ_ERR_INVALID,
                "[%s] The last dimension of the matrix needs to be divisible by the "
                "quantization group size %d. However the provided matrix has last "
                "dimension %lld.",
                op, gs, static_cast<long long>(cols));
  return MXQ_OK;
}

int hip_status(const char* op, hipError_t e) {
  if (e == hipSuccess) return ok();
  return fail(MXQ_ERR_HIP, "[%s] HIP error: %s", op, hipGetErrorString(e));
}

}  // namespace

// the thread-local error text, shared with mxq_safetensors.cpp
namespace mxq {
int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}
int clear_error() { return ok(); }
}  // namespace mxq

namespace {

bool dtype_ok(int d) { return d == MXQ_FLOAT32 || d == MXQ_BFLOAT16; }

// The matmul kernels address a tile of up to 256 activation rows with 32-bit
// byte offsets (row * K * 2) and 32-bit buffer sizes (rows * K * 2): K up to
// 2^22 keeps both below 2^31.
constexpr int64_t kMaxK = int64_t{1} << 22;

int check_matmul(const char* op, const void* x, int64_t M, int64_t K, const uint32_t* wq,
                 const void* scales, const void* biases, int64_t N, int gs, int bits,
                 const void* bias, const void* y) {
  if (M < 0 || N < 0 || K < 0)
    return fail(MXQ_ERR_INVALID, "[%s] Negative dimension (M=%lld, N=%lld, K=%lld).", op,
                static_cast<long long>(M), static_cast<long long>(N),
                static_cast<long long>(K));
  int rc = check_bits_gs(op, bits, gs, K);
  if (rc) return rc;
  if (K == 0)
    return fail(MXQ_ERR_INVALID, "[%s] K must be positive (got 0).", op);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXQ_ERR_INVALID, "[%s] Dimensions above 2^31-1 are not supported.", op);
  if (K > kMaxK)
    return fail(MXQ_ERR_INVALID, "[%s] K above 2^22 (%lld) is not supported (got %lld).", op,
                static_cast<long long>(kMaxK), static_cast<long long>(K));
  if (M == 0 || N == 0) return MXQ_OK;
  if (!x || !wq || !scales || !biases || !y)
    return fail(MXQ_ERR_NULL, "[%s] x, w, scales, biases and y must be non-NULL.", op);
  if (!aligned4(x) || !aligned4(wq) || !aligned4(y) || !aligned4(scales) ||
      !aligned4(biases) || (bias && !aligned4(bias)))
    return fail(MXQ_ERR_ALIGNMENT, "[%s] All tensor pointers must be 4-byte aligned.", op);
  return MXQ_OK;
}

}  // namespace

extern "C" {

int mxq_abi_version(void) { return MXQ_ABI_VERSION; }

const char* mxq_last_error(void) { return g_last_error; }

const char* mxq_status_string(int status) {
  switch (status) {
    case MXQ_OK: return "MXQ_OK";
    case MXQ_ERR_INVALID: return "MXQ_ERR_INVALID";
    case MXQ_ERR_UNSUPPORTED: return "MXQ_ERR_UNSUPPORTED";
    case MXQ_ERR_ALIGNMENT: return "MXQ_ERR_ALIGNMENT";
    case MXQ_ERR_NULL: return "MXQ_ERR_NULL";
    case MXQ_ERR_HIP: return "MXQ_ERR_HIP";
    default: return "MXQ_ERR_UNKNOWN";
  }
}

int mxq_stream_synchronize(mxq_stream stream) {
  return hip_status("synchronize", hipStreamSynchronize(static_cast<hipStream_t>(stream)));
}

int mxq_stream_create(mxq_stream* stream) {
  if (!stream) return fail(MXQ_ERR_NULL, "[stream_create] stream must be non-NULL.");
  hipStream_t s = nullptr;
  const int rc = hip_status("stream_create", hipStreamCreate(&s));  // default priority
  *stream = rc == MXQ_OK ? static_cast<mxq_stream>(s) : nullptr;
  return rc;
}

int mxq_stream_destroy(mxq_stream stream) {
  if (!stream) return ok();
  return hip_status("stream_destroy", hipStreamDestroy(static_cast<hipStream_t>(stream)));
}

int mxq_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(MXQ_ERR_NULL, "[malloc] ptr must be non-NULL.");
  *ptr = nullptr;
  if (bytes == 0) return ok();
  const int rc = hip_status("malloc", hipMalloc(ptr, bytes));
  if (rc != MXQ_OK) *ptr = nullptr;
  return rc;
}

int mxq_free(void* ptr) {
  if (!ptr) return ok();
  return hip_status("free", hipFree(ptr));
}

namespace {
int copy_sync(const char* op, void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
              mxq_stream stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return fail(MXQ_ERR_NULL, "[%s] dst and src must be non-NULL.", op);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return hip_status(op, e);
}
}  // namespace

int mxq_copy_to_device(void* dst, const void* src, size_t bytes, mxq_stream stream) {
  return copy_sync("copy_to_device", dst, src, bytes, hipMemcpyHostToDevice, stream);
}

int mxq_copy_to_host(void* dst, const void* src, size_t bytes, mxq_stream stream) {
  return copy_sync("copy_to_host", dst, src, bytes, hipMemcpyDeviceToHost, stream);
}

int mxq_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq,
             mxq_stream stream) {
  if (!bits_supported(bits))
    return fail(MXQ_ERR_INVALID, "[pack] The requested number of bits %d is not supported.",
                bits);
  if (rows < 0 || cols < 0 || !fits(rows, cols) || (cols * bits) % 32 != 0)
    return fail(MXQ_ERR_INVALID,
                "[pack] cols*bits must be a non-negative multiple of 32 (rows=%lld, "
                "cols=%lld, bits=%d).",
                static_cast<long long>(rows), static_cast<long long>(cols), bits);
  if (rows == 0 || cols == 0) return ok();
  if (!codes || !wq) return fail(MXQ_ERR_NULL, "[pack] codes and wq must be non-NULL.");
  if (!aligned4(wq)) return fail(MXQ_ERR_ALIGNMENT, "[pack] wq must be 4-byte aligned.");
  return hip_status("pack", mxq::detail::launch_pack(codes, rows, cols, bits, wq,
                                                     static_cast<hipStream_t>(stream)));
}

int mxq_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits, uint8_t* codes,
               mxq_stream stream) {
  if (!bits_supported(bits))
    return fail(MXQ_ERR_INVALID, "[unpack] The requested number of bits %d is not supported.",
                bits);
  if (rows < 0 || cols < 0 || !fits(rows, cols) || (cols * bits) % 32 != 0)
    return fail(MXQ_ERR_INVALID,
                "[unpack] cols*bits must be a non-negative multiple of 32 (rows=%lld, "
                "cols=%lld, bits=%d).",
                static_cast<long long>(rows), static_cast<long long>(cols), bits);
  if (rows == 0 || cols == 0) return ok();
  if (!codes || !wq) return fail(MXQ_ERR_NULL, "[unpack] codes and wq must be non-NULL.");
  if (!aligned4(wq)) return fail(MXQ_ERR_ALIGNMENT, "[unpack] wq must be 4-byte aligned.");
  return hip_status("unpack", mxq::detail::launch_unpack(wq, rows, cols, bits, codes,
                                                         static_cast<hipStream_t>(stream)));
}

int mxq_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols, int group_size,
                 int bits, int mode, uint32_t* wq, void* scales, void* biases, int sb_dtype,
                 mxq_stream stream) {
  int rc = check_bits_gs("quantize", bits, group_size, cols);
  if (rc) return rc;
  if (rows < 0) return fail(MXQ_ERR_INVALID, "[quantize] rows must be non-negative.");
  if (!fits(rows, cols)) return fail(MXQ_ERR_INVALID, "[quantize] rows x cols out of range.");
  if (!dtype_ok(w_dtype) || !dtype_ok(sb_dtype))
    return fail(MXQ_ERR_INVALID,
                "[quantize] Only float32 and bfloat16 weights, scales and biases are "
                "supported.");
  if (mode != MXQ_MODE_MINMAX && mode != MXQ_MODE_MLX_EDGE)
    return fail(MXQ_ERR_INVALID, "[quantize] Unknown quantization mode %d.", mode);
  if (rows == 0 || cols == 0) return ok();
  if (!w || !wq || !scales || !biases)
    return fail(MXQ_ERR_NULL, "[quantize] w, wq, scales and biases must be non-NULL.");
  if (!aligned4(w) || !aligned4(wq) || !aligned4(scales) || !aligned4(biases))
    return fail(MXQ_ERR_ALIGNMENT, "[quantize] All tensor pointers must be 4-byte aligned.");
  return hip_status("quantize",
                    mxq::detail::launch_quantize(w, w_dtype, rows, cols, group_size, bits, mode,
                                                 wq, scales, biases, sb_dtype,
                                                 static_cast<hipStream_t>(stream)));
}

int mxq_dequantize(const uint32_t* wq, const void* scales, const void* biases, int sb_dtype,
                   int64_t rows, int64_t cols, int group_size, int bits, void* out,
                   int out_dtype, mxq_stream stream) {
  int rc = check_bits_gs("dequantize", bits, group_size, cols);
  if (rc) return rc;
  if (rows < 0) return fail(MXQ_ERR_INVALID, "[dequantize] rows must be non-negative.");
  if (!fits(rows, cols)) return fail(MXQ_ERR_INVALID, "[dequantize] rows x cols out of range.");
  if (!dtype_ok(sb_dtype) || !dtype_ok(out_dtype))
    return fail(MXQ_ERR_INVALID,
                "[dequantize] Only float32 and bfloat16 scales, biases and outputs are "
                "supported.");
  if (rows == 0 || cols == 0) return ok();
  if (!wq || !scales || !biases || !out)
    return fail(MXQ_ERR_NULL, "[dequantize] w, scales, biases and out must be non-NULL.");
  if (!aligned4(wq) || !aligned4(scales) || !aligned4(biases) || !aligned4(out))
    return fail(MXQ_ERR_ALIGNMENT, "[dequantize] All tensor pointers must be 4-byte aligned.");
  return hip_status("dequantize",
                    mxq::detail::launch_dequantize(wq, scales, biases, sb_dtype, rows, cols,
                                                   group_size, bits, out, out_dtype,
                                                   static_cast<hipStream_t>(stream)));
}

int mxq_qmv(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* scales,
            const void* biases, int64_t N, int group_size, int bits, const void* bias, void* y,
            mxq_stream stream) {
  int rc = check_matmul("quantized_matmul", x, M, K, wq, scales, biases, N, group_size, bits,
                        bias, y);
  if (rc) return rc;
  if (M > MXQ_QMV_MAX_M)
    return fail(MXQ_ERR_INVALID, "[qmv] M=%lld exceeds the GEMV limit %d.",
                static_cast<long long>(M), MXQ_QMV_MAX_M);
  if (M == 0 || N == 0) return ok();
  return hip_status(
      "quantized_matmul",
      mxq::detail::launch_qmv(static_cast<const uint16_t*>(x), static_cast<int>(M),
                              static_cast<int>(K), wq, static_cast<const uint16_t*>(scales),
                              static_cast<const uint16_t*>(biases), static_cast<int>(N),
                              group_size, bits, static_cast<const uint16_t*>(bias),
                              static_cast<uint16_t*>(y), static_cast<hipStream_t>(stream)));
}

int mxq_qmm(const void* x, int64_t M, int64_t K, const uint32_t* wq, const void* scales,
            const void* biases, int64_t N, int group_size, int bits, const void* bias, void* y,
            mxq_stream stream) {
  int rc = check_matmul("quantized_matmul", x, M, K, wq, scales, biases, N, group_size, bits,
                        bias, y);
  if (rc) return rc;
  if (M == 0 || N == 0) return ok();
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* xb = static_cast<const uint16_t*>(x);
  const auto* sc = static_cast<const uint16_t*>(scales);
  const auto* bi = static_cast<const uint16_t*>(biases);
  const auto* bs = static_cast<const uint16_t*>(bias);
  auto* yb = static_cast<uint16_t*>(y);
  if (!mxq::detail::qmm_supports_bits(bits)) {
    // a width the MFMA kernel does not take: the GEMV kernel handles any M in passes.
    return hip_status("quantized_matmul",
                      mxq::detail::launch_qmv(xb, static_cast<int>(M), static_cast<int>(K), wq,
                                              sc, bi, static_cast<int>(N), group_size, bits,
                                              bs, yb, s));
  }
  return hip_status("quantized_matmul",
                    mxq::detail::launch_qmm(xb, static_cast<int>(M), static_cast<int>(K), wq, sc,
                                            bi, static_cast<int>(N), group_size, bits, bs, yb,
                                            s));
}

int64_t mxq_tiled_bytes(int64_t N, int64_t K, int group_size, int bits) {
  int rc = check_bits_gs("tile", bits, group_size, K);
  if (rc) return rc;
  if (N < 0) return fail(MXQ_ERR_INVALID, "[tile] N must be non-negative.");
  if (!fits(N, K)) return fail(MXQ_ERR_INVALID, "[tile] N x K out of range.");
  if (K % 64 == 0 &&
      mxq::tiled::total_bytes(N, K, group_size, bits) > mxq::tiled::kMaxTiledBytes)
    return fail(MXQ_ERR_INVALID, "[tile] A tiled weight above 2 GiB is not supported.");
  if (K % 64 != 0)
    return fail(MXQ_ERR_INVALID,
                "[tile] The tiled layout needs K to be a multiple of 64 (got %lld).",
                static_cast<long long>(K));
  ok();
  return mxq::tiled::total_bytes(N, K, group_size, bits);
}

namespace {
int tile_impl(const uint32_t* wq, const void* scales, const void* biases, int64_t N, int64_t K,
              int group_size, int bits, bool pairs, void* tiled, mxq_stream stream) {
  const int64_t bytes = mxq_tiled_bytes(N, K, group_size, bits);
  if (bytes < 0) return static_cast<int>(bytes);
  if (pairs && N % 2 != 0)
    return fail(MXQ_ERR_INVALID,
                "[tile] A SwiGLU weight needs an even number of rows (gate, then up; got %lld).",
                static_cast<long long>(N));
  if (N == 0 || K == 0) return ok();
  if (!wq || !scales || !biases || !tiled)
    return fail(MXQ_ERR_NULL, "[tile] w, scales, biases and tiled must be non-NULL.");
  if (!aligned4(wq) || !aligned4(scales) || !aligned4(biases) ||
      (reinterpret_cast<uintptr_t>(tiled) & 15u) != 0)
    return fail(MXQ_ERR_ALIGNMENT,
                "[tile] w, scales and biases must be 4-byte aligned, tiled 16-byte aligned.");
  return hip_status("tile", mxq::detail::launch_tile(
                                wq, static_cast<const uint16_t*>(scales),
                                static_cast<const uint16_t*>(biases), N, K, group_size, bits,
                                pairs, tiled, static_cast<hipStream_t>(stream)));
}
}  // namespace

int mxq_tile(const uint32_t* wq, const void* scales, const void* biases, int64_t N, int64_t K,
             int group_size, int bits, void* tiled, mxq_stream stream) {
  return tile_impl(wq, scales, biases, N, K, group_size, bits, false, tiled, stream);
}

int mxq_tile_swiglu(const uint32_t* wq, const void* scales, const void* biases, int64_t N,
                    int64_t K, int group_size, int bits, void* tiled, mxq_stream stream) {
  return tile_impl(wq, scales, biases, N, K, group_size, bits, true, tiled, stream);
}

namespace {
int untile_impl(const void* tiled, int64_t N, int64_t K, int group_size, int bits, bool pairs,
                uint32_t* wq, void* scales, void* biases, mxq_stream stream) {
  const int64_t bytes = mxq_tiled_bytes(N, K, group_size, bits);
  if (bytes < 0) return static_cast<int>(bytes);
  if (pairs && N % 2 != 0)
    return fail(MXQ_ERR_INVALID,
                "[untile] A SwiGLU weight has an even number of rows (got %lld).",
                static_cast<long long>(N));
  if (N == 0 || K == 0) return ok();
  if (!wq || !scales || !biases || !tiled)
    return fail(MXQ_ERR_NULL, "[untile] tiled, w, scales and biases must be non-NULL.");
  if (!aligned4(wq) || !aligned4(scales) || !aligned4(biases) ||
      (reinterpret_cast<uintptr_t>(tiled) & 15u) != 0)
    return fail(MXQ_ERR_ALIGNMENT,
                "[untile] w, scales and biases must be 4-byte aligned, tiled 16-byte aligned.");
  return hip_status("untile", mxq::detail::launch_untile(
                                  tiled, N, K, group_size, bits, pairs, wq,
                                  static_cast<uint16_t*>(scales), static_cast<uint16_t*>(biases),
                                  static_cast<hipStream_t>(stream)));
}
}  // namespace

int mxq_untile(const void* tiled, int64_t N, int64_t K, int group_size, int bits, uint32_t* wq,
               void* scales, void* biases, mxq_stream stream) {
  return untile_impl(tiled, N, K, group_size, bits, false, wq, scales, biases, stream);
}

int mxq_untile_swiglu(const void* tiled, int64_t N, int64_t K, int group_size, int bits,
                      uint32_t* wq, void* scales, void* biases, mxq_stream stream) {
  return untile_impl(tiled, N, K, group_size, bits, true, wq, scales, biases, stream);
}

namespace {
int check_tiled(const char* op, const void* x, int64_t M, int64_t K, const void* tiled,
                int64_t N, int gs, int bits, const void* bias, const void* y) {
  if (M < 0 || N < 0 || K < 0)
    return fail(MXQ_ERR_INVALID, "[%s] Negative dimension.", op);
  int rc = check_bits_gs(op, bits, gs, K);
  if (rc) return rc;
  if (K == 0 || K % 64 != 0)
    return fail(MXQ_ERR_INVALID, "[%s] Tiled weights need K to be a positive multiple of 64.",
                op);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXQ_ERR_INVALID, "[%s] Dimensions above 2^31-1 are not supported.", op);
  if (K > kMaxK)
    return fail(MXQ_ERR_INVALID, "[%s] K above 2^22 (%lld) is not supported (got %lld).", op,
                static_cast<long long>(kMaxK), static_cast<long long>(K));
  if (mxq::tiled::total_bytes(N, K, gs, bits) > mxq::tiled::kMaxTiledBytes)
    return fail(MXQ_ERR_INVALID, "[%s] A tiled weight above 2 GiB is not supported.", op);
  if (M == 0 || N == 0) return MXQ_OK;
  if (!x || !tiled || !y) return fail(MXQ_ERR_NULL, "[%s] x, tiled and y must be non-NULL.", op);
  if (!aligned4(x) || !aligned4(y) || (bias && !aligned4(bias)) ||
      (reinterpret_cast<uintptr_t>(tiled) & 15u) != 0)
    return fail(MXQ_ERR_ALIGNMENT,
                "[%s] x, y and bias must be 4-byte aligned, tiled 16-byte aligned.", op);
  return MXQ_OK;
}
}  // namespace

int mxq_qmm_tiled_lora(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                       int group_size, int bits, const void* bias, int act, const void* xa,
                       const void* bt, int64_t R, void* y, mxq_stream stream) {
  int rc = check_tiled("quantized_matmul", x, M, K, tiled, N, group_size, bits, bias, y);
  if (rc) return rc;
  if (act != MXQ_ACT_NONE && act != MXQ_ACT_GELU_TANH && act != MXQ_ACT_SWIGLU)
    return fail(MXQ_ERR_INVALID, "[quantized_matmul] Unknown activation %d.", act);
  if (act == MXQ_ACT_SWIGLU && N % 2 != 0)
    return fail(MXQ_ERR_INVALID,
                "[quantized_matmul] SwiGLU needs an even number of weight rows (got %lld).",
                static_cast<long long>(N));
  if (xa || bt || R) {
    if (R <= 0 || R % 16 != 0 || R > 4096)
      return fail(MXQ_ERR_INVALID,
                  "[quantized_matmul] The low-rank update needs a rank R that is a positive "
                  "multiple of 16, at most 4096 (got %lld).",
                  static_cast<long long>(R));
    if (M * R * 2 > INT32_MAX || N * R * 2 > INT32_MAX)
      return fail(MXQ_ERR_INVALID, "[quantized_matmul] xa or bt above 2^31-1 bytes.");
    if (M > 0 && N > 0) {
      if (!xa || !bt) return fail(MXQ_ERR_NULL, "[quantized_matmul] xa and bt must be non-NULL.");
      if (!aligned4(xa) || !aligned4(bt))
        return fail(MXQ_ERR_ALIGNMENT, "[quantized_matmul] xa and bt must be 4-byte aligned.");
    }
  }
  if (M == 0 || N == 0) return ok();
  return hip_status("quantized_matmul",
                    mxq::detail::launch_qmm_tiled(
                        static_cast<const uint16_t*>(x), static_cast<int>(M),
                        static_cast<int>(K), tiled, static_cast<int>(N), group_size, bits,
                        static_cast<const uint16_t*>(bias), act,
                        static_cast<const uint16_t*>(xa), static_cast<const uint16_t*>(bt),
                        static_cast<int>(R), static_cast<uint16_t*>(y),
                        static_cast<hipStream_t>(stream)));
}

int mxq_qmm_tiled_act(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                      int group_size, int bits, const void* bias, int act, void* y,
                      mxq_stream stream) {
  return mxq_qmm_tiled_lora(x, M, K, tiled, N, group_size, bits, bias, act, nullptr, nullptr,
                            0, y, stream);
}

int mxq_qmm_tiled(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                  int group_size, int bits, const void* bias, void* y, mxq_stream stream) {
  return mxq_qmm_tiled_act(x, M, K, tiled, N, group_size, bits, bias, MXQ_ACT_NONE, y,
                           stream);
}

int mxq_qmv_tiled(const void* x, int64_t M, int64_t K, const void* tiled, int64_t N,
                  int group_size, int bits, const void* bias, void* y, mxq_stream stream) {
  int rc = check_tiled("quantized_matmul", x, M, K, tiled, N, group_size, bits, bias, y);
  if (rc) return rc;
  if (M > MXQ_QMV_MAX_M)
    return fail(MXQ_ERR_INVALID, "[qmv] M=%lld exceeds the GEMV limit %d.",
                static_cast<long long>(M), MXQ_QMV_MAX_M);
  if (M == 0 || N == 0) return ok();
  return hip_status("quantized_matmul",
                    mxq::detail::launch_qmv_tiled(
                        static_cast<const uint16_t*>(x), static_cast<int>(M),
                        static_cast<int>(K), tiled, static_cast<int>(N), group_size, bits,
                        static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                        static_cast<hipStream_t>(stream)));
}

}  // extern "C"

namespace {
// The GEMV or an MFMA kernel for M tokens. Up to 8 tokens the GEMV, one read of the
// weight, always wins. From 9 to MXQ_QMV_MAX_M (K % 64 == 0) it runs one pass of 16 or 32
// tokens, whose per-token work caps its rate (tiled layout: about 3.2 and 2.0 TB/s of
// weight), while the MFMA kernel at these M is bound by its K loop: about 0.8 us per
// 64-code step per round of 256 feature tiles. Measured on the tiled layout from
// N x K = 2048 x 2048 to 262144 x 3840: the GEMV takes 0.26-0.6 of the MFMA kernel's time
// for weights below about 120 MB at 32 tokens and below about 600 MB at 16. Both layouts
// take the same decision, so a weight gives the same result bits tiled or not (the GEMV
// applies the weights unrounded, the MFMA kernels as bf16).
bool gemv_preferred(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  if (M <= 8) return true;
  if (M > MXQ_QMV_MAX_M || K % 64 != 0 || gs <= 0) return false;
  const double wbytes = static_cast<double>(N) * K * bits / 8.0 + 4.0 * N * (K / gs);
  const double rounds = std::ceil(std::ceil(N / 256.0) / 256.0);
  const double t_mfma = 0.8e-6 * (K / 64.0) * rounds;
  const double t_gemv = wbytes / (M <= 16 ? 3.2e12 : 2.0e12);
  return t_gemv <= t_mfma;
}
}  // namespace

extern "C" {

int mxq_quantized_matmul_tiled(const void* x, int64_t M, int64_t K, const void* tiled,
                               int64_t N, int group_size, int bits, const void* bias, void* y,
                               mxq_stream stream) {
  if (gemv_preferred(M, N, K, group_size, bits))
    return mxq_qmv_tiled(x, M, K, tiled, N, group_size, bits, bias, y, stream);
  return mxq_qmm_tiled(x, M, K, tiled, N, group_size, bits, bias, y, stream);
}

}  // extern "C"

namespace {
// The MLX-layout operator without a workspace: the GEMV kernel where gemv_preferred says
// so, the in-place MFMA kernel otherwise. Allocates nothing.
int matmul_in_place(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                    const void* scales, const void* biases, int64_t N, int transpose,
                    int group_size, int bits, const void* bias, void* y, mxq_stream stream) {
  if (transpose != 1)
    return fail(MXQ_ERR_UNSUPPORTED,
                "[quantized_matmul] transpose=false (x * W with W stored [K, N]) is not "
                "implemented; the quantized linear layers use transpose=true.");
  if (gemv_preferred(M, N, K, group_size, bits))
    return mxq_qmv(x, M, K, wq, scales, biases, N, group_size, bits, bias, y, stream);
  return mxq_qmm(x, M, K, wq, scales, biases, N, group_size, bits, bias, y, stream);
}

// The workspace pools of mxq_quantized_matmul, one per GPU, created on a GPU's first
// large-M call and kept until the process ends. A pool keeps up to kPoolKeepBytes of
// freed workspace for the next call instead of returning it at each synchronisation.
constexpr int kPoolDevices = 64;
constexpr uint64_t kPoolKeepBytes = 256ull << 20;
std::mutex g_pool_mutex;
hipMemPool_t g_pool[kPoolDevices];
bool g_pool_tried[kPoolDevices];

// The pool of the device `stream` belongs to, or null where stream-ordered allocation
// is unavailable (the caller then runs the in-place kernel).
hipMemPool_t workspace_pool(hipStream_t stream) {
  int dev = 0;
  if ((stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev)) != hipSuccess ||
      dev < 0 || dev >= kPoolDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_pool_mutex);
  if (!g_pool_tried[dev]) {
    g_pool_tried[dev] = true;
    int supported = 0;
    hipMemPoolProps props;
    std::memset(&props, 0, sizeof(props));
    props.allocType = hipMemAllocationTypePinned;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    if (hipDeviceGetAttribute(&supported, hipDeviceAttributeMemoryPoolsSupported, dev) ==
            hipSuccess &&
        supported && hipMemPoolCreate(&pool, &props) == hipSuccess) {
      uint64_t keep = kPoolKeepBytes;
      (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
      g_pool[dev] = pool;
    }
    (void)hipGetLastError();
  }
  return g_pool[dev];
}

// Bytes of stream-ordered workspace a large-M mxq_quantized_matmul call tiles the weight
// into, or 0 where it runs in place: K % 64 == 0 and a tiled copy below 2 GiB (the caller
// takes this path only where the MFMA kernel beats the GEMV). The tiled kernel takes 0.36-0.95 of the in-place kernel's time,
// tiling included, from M = 16 (M = 16 to 1024; N x K from 2048 x 2048 to 5376 x 21504,
// 6-bit).
int64_t pooled_workspace_bytes(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  if (M <= 0 || M > INT32_MAX || N <= 0 || N > INT32_MAX || K <= 0 ||
      K % 64 != 0 || K > kMaxK || check_bits_gs("quantized_matmul", bits, gs, K) != MXQ_OK)
    return 0;
  const int64_t t = mxq::tiled::total_bytes(N, K, gs, bits);
  return t > mxq::tiled::kMaxTiledBytes ? 0 : t;
}

// The weight tiled into `workspace` (need bytes, 16-byte aligned, sharing no byte with an
// operand), then the tiled kernel: mxq_quantized_matmul_ws's work once it has a workspace.
int matmul_through_workspace(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                             const void* scales, const void* biases, int64_t N, int group_size,
                             int bits, const void* bias, void* y, void* workspace, int64_t need,
                             mxq_stream stream) {
  int rc = check_matmul("quantized_matmul", x, M, K, wq, scales, biases, N, group_size, bits,
                        bias, y);
  if (rc) return rc;
  // the tiler reads the weight triple while it writes the workspace, and the kernel
  // reads the workspace while it writes y: the workspace may share no byte with them
  const uintptr_t w0 = reinterpret_cast<uintptr_t>(workspace), w1 = w0 + static_cast<uintptr_t>(need);
  auto overlaps = [&](const void* p, int64_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    return p && bytes > 0 && a < w1 && w0 < a + static_cast<uintptr_t>(bytes);
  };
  const int64_t groups = N * (K / group_size);
  if (overlaps(x, M * K * 2) || overlaps(wq, N * K / 32 * bits * 4) ||
      overlaps(scales, groups * 2) || overlaps(biases, groups * 2) || overlaps(bias, N * 2) ||
      overlaps(y, M * N * 2))
    return fail(MXQ_ERR_INVALID,
                "[quantized_matmul] The workspace overlaps an input or the output.");
  rc = mxq_tile(wq, scales, biases, N, K, group_size, bits, workspace, stream);
  if (rc) return rc;
  return mxq_qmm_tiled(x, M, K, workspace, N, group_size, bits, bias, y, stream);
}
}  // namespace

extern "C" {

int mxq_quantized_matmul(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                         const void* scales, const void* biases, int64_t N, int transpose,
                         int group_size, int bits, const void* bias, void* y,
                         mxq_stream stream) {
  // Past the GEMV's range: the weight is tiled into a stream-ordered workspace and the
  // tiled kernel runs (the same result bits as the in-place kernel; about 1.7x faster at
  // M = 14400, K = 4096, N = 16384 and up to 2.8x at a few hundred tokens). Invalid arguments are refused before anything is allocated; where no
  // workspace can be had, the in-place kernel runs.
  if (transpose == 1 && !gemv_preferred(M, N, K, group_size, bits)) {
    const int64_t need = pooled_workspace_bytes(M, N, K, group_size, bits);
    if (need > 0) {
      int rc = check_matmul("quantized_matmul", x, M, K, wq, scales, biases, N, group_size,
                            bits, bias, y);
      if (rc) return rc;
      const hipStream_t s = static_cast<hipStream_t>(stream);
      void* ws = nullptr;
      // under graph capture nothing is allocated (mxq_quantized_matmul_noalloc is the
      // tiled path for captured code)
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(s, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
      const hipMemPool_t pool = cap == hipStreamCaptureStatusNone ? workspace_pool(s) : nullptr;
      if (pool && hipMallocFromPoolAsync(&ws, static_cast<size_t>(need), pool, s) == hipSuccess &&
          ws) {
        rc = matmul_through_workspace(x, M, K, wq, scales, biases, N, group_size, bits, bias, y,
                                      ws, need, stream);
        const hipError_t e = hipFreeAsync(ws, s);
        if (rc) return rc;
        return hip_status("quantized_matmul", e);
      }
      (void)hipGetLastError();  // a refused allocation leaves no error behind
    }
  }
  return matmul_in_place(x, M, K, wq, scales, biases, N, transpose, group_size, bits, bias, y,
                         stream);
}

int64_t mxq_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size,
                                            int bits) {
  int rc = check_bits_gs("quantized_matmul", bits, group_size, K);
  if (rc) return rc;
  if (M < 0 || N < 0 || K < 0) return fail(MXQ_ERR_INVALID, "[quantized_matmul] Negative dimension.");
  ok();
  // Tiling reads and writes the weight once; from about this many tokens the tiled MFMA
  // kernel saves more than that (the MLX-layout kernel takes about 1.7x its time). Both
  // MFMA kernels accumulate each output in the same order: the result bits are the same.
  constexpr int64_t kTileMinM = 1024;
  if (M < kTileMinM || M > INT32_MAX || N == 0 || N > INT32_MAX || K == 0 || K % 64 != 0 ||
      K > kMaxK || !mxq::detail::qmm_supports_bits(bits) ||
      mxq::tiled::total_bytes(N, K, group_size, bits) > mxq::tiled::kMaxTiledBytes)
    return 0;
  return mxq::tiled::total_bytes(N, K, group_size, bits);
}

int mxq_quantized_matmul_ws(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                            const void* scales, const void* biases, int64_t N, int transpose,
                            int group_size, int bits, const void* bias, void* y, void* workspace,
                            size_t ws_bytes, mxq_stream stream) {
  const int64_t need = mxq_quantized_matmul_workspace_size(M, N, K, group_size, bits);
  if (transpose != 1 || need <= 0 || !workspace || ws_bytes < static_cast<size_t>(need) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
    return matmul_in_place(x, M, K, wq, scales, biases, N, transpose, group_size, bits, bias, y,
                           stream);
  return matmul_through_workspace(x, M, K, wq, scales, biases, N, group_size, bits, bias, y,
                                  workspace, need, stream);
}

}  // extern "C"

// ---- the matmul that allocates nothing: mxq_quantized_matmul_ws with its
// workspace in a static device array, one per GPU (each GPU holds its copy until
// the process ends). Host code never uses the array's name as an address: the
// device address of each GPU's copy is looked up once, with that GPU current,
// and kept per device.
static __device__ __align__(256) uint8_t scratch[MXQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each GPU (null: not looked up)

// The scratch address on the device `stream` belongs to (the current device for
// the null stream).
int scratch_address(hipStream_t stream, void** out) {
  int cur = 0, dev = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess) e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status("quantized_matmul", e);
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MXQ_ERR_UNSUPPORTED, "[quantized_matmul] Device %d is beyond the %d this library "
                "keeps a scratch address for.", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return hip_status("quantized_matmul", e);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return hip_status("quantized_matmul", e);
    if (!p) return fail(MXQ_ERR_HIP, "[quantized_matmul] The scratch array has no device address.");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MXQ_OK;
}
}  // namespace

extern "C" {

int mxq_quantized_matmul_noalloc(const void* x, int64_t M, int64_t K, const uint32_t* wq,
                                 const void* scales, const void* biases, int64_t N,
                                 int transpose, int group_size, int bits, const void* bias,
                                 void* y, mxq_stream stream) {
  const int64_t need = mxq_quantized_matmul_workspace_size(M, N, K, group_size, bits);
  if (need < 0) return static_cast<int>(need);
  if (transpose != 1 || need == 0)  // no workspace used: the in-place operator
    return matmul_in_place(x, M, K, wq, scales, biases, N, transpose, group_size, bits, bias, y,
                           stream);
  if (need > MXQ_NOALLOC_SCRATCH_BYTES)
    return fail(MXQ_ERR_INVALID,
                "[quantized_matmul] The tiled weight (%lld bytes) exceeds the %lld-byte scratch "
                "of mxq_quantized_matmul_noalloc; pass a workspace to mxq_quantized_matmul_ws.",
                static_cast<long long>(need),
                static_cast<long long>(MXQ_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  const int rc = scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  return mxq_quantized_matmul_ws(x, M, K, wq, scales, biases, N, transpose, group_size, bits,
                                 bias, y, ws, static_cast<size_t>(need), stream);
}

}  // extern "C"

// ---- row-wise ops of the DiT block (mxq_blockops.hip)

namespace {
bool aligned2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }

int check_rows(const char* op, int64_t S, int64_t hidden,
               std::initializer_list<const void*> required) {
  if (S < 0 || hidden < 0) return fail(MXQ_ERR_INVALID, "[%s] Negative dimension.", op);
  if (hidden > INT32_MAX) return fail(MXQ_ERR_INVALID, "[%s] Row above 2^31-1 elements.", op);
  if (S == 0 || hidden == 0) return MXQ_OK;
  for (const void* p : required) {
    if (!p) return fail(MXQ_ERR_NULL, "[%s] A required tensor pointer is NULL.", op);
    if (!aligned2(p)) return fail(MXQ_ERR_ALIGNMENT, "[%s] bf16 tensors must be 2-byte aligned.", op);
  }
  return MXQ_OK;
}
}  // namespace

int mxq_norm_modscale(const void* x, int64_t S, int64_t hidden, const void* weight,
                      const void* shift, const void* scale, int64_t mod_rows,
                      const uint32_t* row_map, float eps, void* out, mxq_stream stream) {
  int rc = check_rows("norm_modscale", S, hidden, {x, weight, shift, scale, out});
  if (rc) return rc;
  if (S > 0 && hidden > 0 && mod_rows < 1)
    return fail(MXQ_ERR_INVALID, "[norm_modscale] mod_rows must be at least 1.");
  if (row_map && !aligned4(row_map))
    return fail(MXQ_ERR_ALIGNMENT, "[norm_modscale] row_map must be 4-byte aligned.");
  return hip_status("norm_modscale",
                    mxq::detail::launch_norm_modscale(
                        static_cast<const uint16_t*>(x), S, static_cast<int>(hidden),
                        static_cast<const uint16_t*>(weight), static_cast<const uint16_t*>(shift),
                        static_cast<const uint16_t*>(scale), row_map, mod_rows, eps,
                        static_cast<uint16_t*>(out), static_cast<hipStream_t>(stream)));
}

int mxq_mod_gate(const void* x, const void* other, int64_t S, int64_t hidden, const void* gate,
                 int64_t mod_rows, const uint32_t* row_map, void* out, mxq_stream stream) {
  int rc = check_rows("mod_gate", S, hidden, {x, other, gate, out});
  if (rc) return rc;
  if (S > 0 && hidden > 0 && mod_rows < 1)
    return fail(MXQ_ERR_INVALID, "[mod_gate] mod_rows must be at least 1.");
  if (row_map && !aligned4(row_map))
    return fail(MXQ_ERR_ALIGNMENT, "[mod_gate] row_map must be 4-byte aligned.");
  return hip_status("mod_gate", mxq::detail::launch_mod_gate(
                                    static_cast<const uint16_t*>(x),
                                    static_cast<const uint16_t*>(other), S,
                                    static_cast<int>(hidden), static_cast<const uint16_t*>(gate),
                                    row_map, mod_rows, static_cast<uint16_t*>(out),
                                    static_cast<hipStream_t>(stream)));
}

int mxq_rmsnorm_rope(const void* x, int64_t S, int64_t heads, int64_t head_dim,
                     const void* weight, const void* cos, const void* sin, int table_dtype,
                     int rot, float eps, void* out, mxq_stream stream) {
  if (S < 0 || heads < 0) return fail(MXQ_ERR_INVALID, "[rmsnorm_rope] Negative dimension.");
  if (heads > INT32_MAX || (heads > 0 && S > INT64_MAX / heads))
    return fail(MXQ_ERR_INVALID, "[rmsnorm_rope] S x heads rows out of range.");
  int rc = check_rows("rmsnorm_rope", S * heads, head_dim, {x, weight, out});
  if (rc) return rc;
  if (head_dim > 512)
    return fail(MXQ_ERR_UNSUPPORTED, "[rmsnorm_rope] head_dim %lld above 512.",
                static_cast<long long>(head_dim));
  if (rot < 0 || rot % 2 || rot > head_dim)
    return fail(MXQ_ERR_INVALID, "[rmsnorm_rope] rot must be even and at most head_dim (got %d).",
                rot);
  if (table_dtype != MXQ_FLOAT32 && table_dtype != MXQ_BFLOAT16)
    return fail(MXQ_ERR_INVALID, "[rmsnorm_rope] Unknown table dtype %d.", table_dtype);
  if (S * heads > 0 && head_dim > 0 && rot > 0 && (!cos || !sin))
    return fail(MXQ_ERR_NULL, "[rmsnorm_rope] cos and sin must be non-NULL.");
  if ((cos && !aligned2(cos)) || (sin && !aligned2(sin)) ||
      (table_dtype == MXQ_FLOAT32 && ((cos && !aligned4(cos)) || (sin && !aligned4(sin)))))
    return fail(MXQ_ERR_ALIGNMENT, "[rmsnorm_rope] cos and sin must be aligned to their dtype.");
  return hip_status("rmsnorm_rope",
                    mxq::detail::launch_rmsnorm_rope(
                        static_cast<const uint16_t*>(x), S, static_cast<int>(heads),
                        static_cast<int>(head_dim), static_cast<const uint16_t*>(weight), cos, sin,
                        table_dtype, rot, eps, static_cast<uint16_t*>(out),
                        static_cast<hipStream_t>(stream)));
}
