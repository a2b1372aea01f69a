// mxq_layout.hip — packer, unpacker, quantizer and dequantizer for the MLX
// affine layout (gfx950). These run at load time, not in the sampling loop;
// they are written for bit-exactness first and are HBM-bound.
//
// Reference behaviour:
//   quantize   : mx.quantize(w, group_size=64, bits=4) in
//                `model/minimax h3/tools/quantize_h3_g64.py:132`, and
//                quantize(model:) in `Packages/z-image-swift/Sources/ZImage/Weights.swift:31`
//   dequantize : MfLinear.dequantizedWeight, `model/minimax h3/H3Common.swift:382-401`
//                (w = q*scale + bias in fp32, then bf16)
//   layout     : `model/3模块/模型加载-通用.swift:178-185` (shape relations),
//                `model/minimax h3/H3Common.swift:389-394` (LSB-first codes)
#include "mxq_device.hpp"
#include "mxq_internal.hpp"
#include "mxq_tiled.hpp"

namespace mxq {
namespace {

constexpr int kThreads = 256;

inline unsigned grid_for(int64_t items) {
  return static_cast<unsigned>((items + kThreads - 1) / kThreads);
}

// One thread per output word: OR in every code whose bits overlap the word.
template <int BITS>
__global__ __launch_bounds__(kThreads) void pack_kernel(const uint8_t* __restrict__ codes,
                                                        int64_t rows, int64_t cols,
                                                        uint32_t* __restrict__ wq) {
  const int64_t W = cols * BITS / 32;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= rows * W) return;
  const int64_t n = idx / W, w = idx - n * W;
  const uint8_t* row = codes + n * cols;
  const int64_t bit0 = w * 32;
  const int64_t k0 = bit0 / BITS, k1 = (bit0 + 31) / BITS;
  uint32_t word = 0;
  for (int64_t k = k0; k <= k1; ++k) {
    const uint32_t c = row[k] & ((1u << BITS) - 1u);
    const int start = static_cast<int>(k * BITS - bit0);
    word |= start >= 0 ? (c << start) : (c >> -start);
  }
  wq[idx] = word;
}

// One thread per code.
template <int BITS>
__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint32_t* __restrict__ wq,
                                                          int64_t rows, int64_t cols,
                                                          uint8_t* __restrict__ codes) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= rows * cols) return;
  const int64_t n = idx / cols, k = idx - n * cols;
  const uint32_t* row = wq + n * (cols * BITS / 32);
  const int64_t p = k * BITS;
  const int off = static_cast<int>(p & 31);
  uint32_t v = row[p >> 5] >> off;
  if (off + BITS > 32) v |= row[(p >> 5) + 1] << (32 - off);
  codes[idx] = static_cast<uint8_t>(v & ((1u << BITS) - 1u));
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

template <typename T>
__device__ __forceinline__ void store_f32(T* p, float v);
template <>
__device__ __forceinline__ void store_f32<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_f32<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16(v); }

// One thread per (row, group): min/max, scale/bias, codes, packed words. A
// group of >= 32 codes always fills whole words, so no two threads share a word.
template <int BITS, typename TW, typename TSB>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const TW* __restrict__ w,
                                                            int64_t rows, int64_t cols, int gs,
                                                            int mode, uint32_t* __restrict__ wq,
                                                            TSB* __restrict__ scales,
                                                            TSB* __restrict__ biases) {
  const int64_t G = cols / gs;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= rows * G) return;
  const int64_t n = gid / G, g = gid - n * G;
  const TW* wg = w + n * cols + g * gs;
  const float nmax = static_cast<float>((1 << BITS) - 1);
  const float eps = 1e-7f;

  float mn = load_f32(wg), mx = mn;
  for (int i = 1; i < gs; ++i) {
    const float v = load_f32(wg + i);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  float s, b;
  if (mode == 0) {
    s = (mx - mn) / nmax;
    if (mx == mn) s = eps;
    b = mn;
  } else {
    s = fmaxf((mx - mn) / nmax, eps);
    const bool side = fabsf(mn) > fabsf(mx);
    s = side ? s : -s;
    const float edge = side ? mn : mx;
    const float q0 = rintf(edge / s);
    if (q0 != 0.0f) {
      s = edge / q0;
      b = edge;
    } else {
      b = 0.0f;
    }
  }

  uint32_t* out = wq + n * (cols * BITS / 32) + g * (gs * BITS / 32);
  uint64_t acc = 0;
  int nacc = 0, wo = 0;
  for (int i = 0; i < gs; ++i) {
    float q = rintf((load_f32(wg + i) - b) / s);
    q = fminf(fmaxf(q, 0.0f), nmax);
    acc |= static_cast<uint64_t>(static_cast<uint32_t>(q)) << nacc;
    nacc += BITS;
    if (nacc >= 32) {
      out[wo++] = static_cast<uint32_t>(acc);
      acc >>= 32;
      nacc -= 32;
    }
  }
  store_f32(scales + gid, s);
  store_f32(biases + gid, b);
}

// One thread per period (the smallest run of codes filling whole words).
template <int BITS, typename TSB, typename TO>
__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint32_t* __restrict__ wq,
                                                              const TSB* __restrict__ scales,
                                                              const TSB* __restrict__ biases,
                                                              int64_t rows, int64_t cols, int gs,
                                                              TO* __restrict__ out) {
  constexpr int PC = Period<BITS>::codes, PW = Period<BITS>::words;
  const int64_t per_row = cols / PC;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int64_t n = idx / per_row, j = idx - n * per_row;
  const int64_t k0 = j * PC;
  const int64_t gi = n * (cols / gs) + k0 / gs;
  const float s = load_f32(scales + gi), b = load_f32(biases + gi);
  uint32_t words[PW];
  const uint32_t* src = wq + n * (cols * BITS / 32) + j * PW;
#pragma unroll
  for (int i = 0; i < PW; ++i) words[i] = src[i];
  uint32_t q[PC];
  decode_codes<BITS, PC, PW>(words, q);
  TO* dst = out + n * cols + k0;
#pragma unroll
  for (int i = 0; i < PC; ++i) store_f32(dst + i, fmaf(static_cast<float>(q[i]), s, b));
}

// One thread per (row block, K step, half, unit): copies the unit's `BITS`
// words into its planes and, for the unit that owns it, writes the
// (scale, bias) pair. See mxq_tiled.hpp for the layout.
template <int BITS>
__global__ __launch_bounds__(kThreads) void tile_kernel(const uint32_t* __restrict__ wq,
                                                        const uint16_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ biases,
                                                        int64_t N, int64_t K, int gs,
                                                        bool pairs,
                                                        uint8_t* __restrict__ out) {
  const int64_t nk = K / 64;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t items = tiled::row_blocks(N) * nk * 128;
  if (idx >= items) return;
  const int u = static_cast<int>(idx & 63);
  const int h = static_cast<int>((idx >> 6) & 1);
  const int64_t rk = idx >> 7;  // rb * nk + kk (thread order; the record is step-major)
  const int64_t rb = rk / nk, kk = rk - rb * nk;
  const int r = u & 31, g = u >> 5;
  // source row of tiled row rb*64 + h*32 + r; with `pairs`, the halves of row
  // block rb are rows 32rb + r and N/2 + 32rb + r (gate and up of one output)
  const int64_t row = pairs ? h * (N / 2) + rb * 32 + r : rb * 64 + h * 32 + r;
  const bool valid = pairs ? rb * 32 + r < N / 2 : row < N;
  const int64_t W = K / 32 * BITS;
  constexpr int FP = tiled::full_planes(BITS), RW = tiled::rem_words(BITS);
  // the run's BITS words (dword-aligned in the MLX row): 16-byte loads, then the
  // remainder as one 8-byte, 4-byte or three 4-byte loads
  uint32_t words[BITS];
  const uint32_t* src = wq + (valid ? row : 0) * W + (kk * 64 + 32 * g) / 32 * BITS;
#pragma unroll
  for (int p = 0; p < FP; ++p) {
    const u32x4 v = valid ? *reinterpret_cast<const u32x4*>(src + 4 * p) : u32x4{0u, 0u, 0u, 0u};
    words[4 * p] = v.x; words[4 * p + 1] = v.y; words[4 * p + 2] = v.z; words[4 * p + 3] = v.w;
  }
  if constexpr (RW == 2) {
    const u32x2 v = valid ? *reinterpret_cast<const u32x2*>(src + 4 * FP) : u32x2{0u, 0u};
    words[4 * FP] = v.x; words[4 * FP + 1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < RW; ++i) words[4 * FP + i] = valid ? src[4 * FP + i] : 0u;
  }
  uint8_t* rec = out + tiled::record_index(rb, kk, tiled::row_blocks(N)) *
                           tiled::record_bytes(BITS, gs);
  uint8_t* half = rec + h * tiled::half_bytes(BITS);
  // one 16-byte store per plane (a wave writes 1 KiB of a plane contiguously); the
  // remainder plane holds RW words per unit
#pragma unroll
  for (int p = 0; p < FP; ++p)
    *reinterpret_cast<u32x4a*>(half + p * 1024 + u * 16) =
        u32x4a{words[4 * p], words[4 * p + 1], words[4 * p + 2], words[4 * p + 3]};
  if constexpr (RW == 2) {
    typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2a*>(half + FP * 1024 + u * 8) = u32x2a{words[4 * FP], words[4 * FP + 1]};
  } else if constexpr (RW > 0) {
    uint32_t* d = reinterpret_cast<uint32_t*>(half + FP * 1024 + u * 4 * RW);
#pragma unroll
    for (int i = 0; i < RW; ++i) d[i] = words[4 * FP + i];
  }
  const int G = tiled::gps(gs);
  if (G == 2 || g == 0) {
    const int64_t grp = (kk * 64 + 32 * g) / gs;
    const int64_t si = (valid ? row : 0) * (K / gs) + grp;
    const uint32_t sv = valid ? scales[si] : 0u;
    const uint32_t bv = valid ? biases[si] : 0u;
    uint32_t* e = reinterpret_cast<uint32_t*>(rec + tiled::code_bytes(BITS)) +
                  ((h * 32 + r) * G + (G == 2 ? g : 0));
    *e = sv | (bv << 16);
  }
}

// The same layout, one workgroup per (row block, group of kTileSteps K steps): the
// group's bytes of the block's 64 rows are read with consecutive lanes on consecutive
// 16-byte chunks of a row (rows are contiguous in the MLX layout; tile_kernel's one
// thread per unit reads 32 rows per load instruction), staged in LDS, then written
// unit by unit exactly as tile_kernel writes them.
constexpr int kTileSteps = 4;
template <int BITS>
__global__ __launch_bounds__(kThreads) void tile_rows_kernel(const uint32_t* __restrict__ wq,
                                                             const uint16_t* __restrict__ scales,
                                                             const uint16_t* __restrict__ biases,
                                                             int64_t N, int64_t K, int gs,
                                                             bool pairs,
                                                             uint8_t* __restrict__ out) {
  constexpr int CPR = kTileSteps * BITS / 2;  // 16-byte chunks of a row per group
  constexpr int RSTR = CPR * 16 + 16;         // staged row stride
  __shared__ __attribute__((aligned(16))) uint8_t st[64 * RSTR];
  const int64_t nk = K / 64;
  const int64_t ngrp = (nk + kTileSteps - 1) / kTileSteps;
  const int64_t rb = blockIdx.x / ngrp;
  const int64_t k0 = (blockIdx.x - rb * ngrp) * kTileSteps;
  const int64_t rowb = K / 8 * BITS;          // bytes per MLX row
  const int64_t W = K / 32 * BITS;            // words per MLX row
  // source row of block row t = 32 h + r; with `pairs`, the halves of row block rb
  // are rows 32rb + r and N/2 + 32rb + r (gate and up of one output)
  auto src_row = [&](int t, bool& valid) {
    const int h = t >> 5, r = t & 31;
    const int64_t row = pairs ? h * (N / 2) + rb * 32 + r : rb * 64 + t;
    valid = pairs ? rb * 32 + r < N / 2 : row < N;
    return row;
  };
  for (int c = threadIdx.x; c < 64 * CPR; c += kThreads) {
    const int t = c / CPR, j = c % CPR;
    bool valid;
    const int64_t row = src_row(t, valid);
    const int64_t off = k0 * 8 * BITS + j * 16;  // byte offset in the row
    u32x4a v = {0u, 0u, 0u, 0u};
    if (valid && off < rowb) {  // chunks past the row end belong to steps past K
      const uint32_t* p = wq + row * W + off / 4;
      if (off + 16 <= rowb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(p);
        v = u32x4a{a.x, a.y, a.z, a.w};
      } else {  // the row ends 8 bytes into this chunk (rowb is a multiple of 8)
        const u32x2 a = *reinterpret_cast<const u32x2*>(p);
        v = u32x4a{a.x, a.y, 0u, 0u};
      }
    }
    *reinterpret_cast<u32x4a*>(st + t * RSTR + j * 16) = v;
  }
  __syncthreads();
  constexpr int FP = tiled::full_planes(BITS), RW = tiled::rem_words(BITS);
  for (int e = threadIdx.x; e < 128 * kTileSteps; e += kThreads) {
    const int u = e & 63, h = (e >> 6) & 1, ks = e >> 7;
    const int64_t kk = k0 + ks;
    if (kk >= nk) continue;
    const int r = u & 31, g = u >> 5, t = h * 32 + r;
    bool valid;
    const int64_t row = src_row(t, valid);
    uint32_t words[BITS];
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(st + t * RSTR + (2 * ks + g) * BITS * 4);
#pragma unroll
    for (int i = 0; i < BITS; ++i) words[i] = sw[i];
    uint8_t* rec = out + tiled::record_index(rb, kk, tiled::row_blocks(N)) *
                             tiled::record_bytes(BITS, gs);
    uint8_t* half = rec + h * tiled::half_bytes(BITS);
#pragma unroll
    for (int p = 0; p < FP; ++p)
      *reinterpret_cast<u32x4a*>(half + p * 1024 + u * 16) =
          u32x4a{words[4 * p], words[4 * p + 1], words[4 * p + 2], words[4 * p + 3]};
    if constexpr (RW == 2) {
      typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2a*>(half + FP * 1024 + u * 8) = u32x2a{words[4 * FP], words[4 * FP + 1]};
    } else if constexpr (RW > 0) {
      uint32_t* d = reinterpret_cast<uint32_t*>(half + FP * 1024 + u * 4 * RW);
#pragma unroll
      for (int i = 0; i < RW; ++i) d[i] = words[4 * FP + i];
    }
    const int G = tiled::gps(gs);
    if (G == 2 || g == 0) {
      const int64_t grp = (kk * 64 + 32 * g) / gs;
      const int64_t si = (valid ? row : 0) * (K / gs) + grp;
      const uint32_t sv = valid ? scales[si] : 0u;
      const uint32_t bv = valid ? biases[si] : 0u;
      uint32_t* ep = reinterpret_cast<uint32_t*>(rec + tiled::code_bytes(BITS)) +
                     ((h * 32 + r) * G + (G == 2 ? g : 0));
      *ep = sv | (bv << 16);
    }
  }
}

// The inverse of tile_rows_kernel, for callers that keep only the tiled copy and
// need the MLX triple back: one workgroup per (row block, group of kTileSteps K
// steps) reads the records unit by unit (each plane a contiguous 1 KiB per wave),
// stages the block's rows in LDS, and writes them row by row with consecutive
// lanes on consecutive 16-byte chunks. The (scale, bias) pair of each group comes
// from the unit that starts the group. Rows past N (or past N/2 in a half, with
// `pairs`) are skipped.
template <int BITS>
__global__ __launch_bounds__(kThreads) void untile_rows_kernel(const uint8_t* __restrict__ in,
                                                               int64_t N, int64_t K, int gs,
                                                               bool pairs,
                                                               uint32_t* __restrict__ wq,
                                                               uint16_t* __restrict__ scales,
                                                               uint16_t* __restrict__ biases) {
  constexpr int CPR = kTileSteps * BITS / 2;
  constexpr int RSTR = CPR * 16 + 16;
  __shared__ __attribute__((aligned(16))) uint8_t st[64 * RSTR];
  const int64_t nk = K / 64;
  const int64_t ngrp = (nk + kTileSteps - 1) / kTileSteps;
  const int64_t rb = blockIdx.x / ngrp;
  const int64_t k0 = (blockIdx.x - rb * ngrp) * kTileSteps;
  const int64_t rowb = K / 8 * BITS;
  const int64_t W = K / 32 * BITS;
  auto dst_row = [&](int t, bool& valid) {
    const int h = t >> 5, r = t & 31;
    const int64_t row = pairs ? h * (N / 2) + rb * 32 + r : rb * 64 + t;
    valid = pairs ? rb * 32 + r < N / 2 : row < N;
    return row;
  };
  constexpr int FP = tiled::full_planes(BITS), RW = tiled::rem_words(BITS);
  const int G = tiled::gps(gs);
  for (int e = threadIdx.x; e < 128 * kTileSteps; e += kThreads) {
    const int u = e & 63, h = (e >> 6) & 1, ks = e >> 7;
    const int64_t kk = k0 + ks;
    if (kk >= nk) continue;
    const int r = u & 31, g = u >> 5, t = h * 32 + r;
    const uint8_t* rec = in + tiled::record_index(rb, kk, tiled::row_blocks(N)) *
                                  tiled::record_bytes(BITS, gs);
    const uint8_t* half = rec + h * tiled::half_bytes(BITS);
    uint32_t words[BITS];
#pragma unroll
    for (int p = 0; p < FP; ++p) {
      const u32x4a v = *reinterpret_cast<const u32x4a*>(half + p * 1024 + u * 16);
      words[4 * p] = v.x; words[4 * p + 1] = v.y; words[4 * p + 2] = v.z; words[4 * p + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < RW; ++i)
      words[4 * FP + i] = reinterpret_cast<const uint32_t*>(half + FP * 1024 + u * 4 * RW)[i];
    uint32_t* sw = reinterpret_cast<uint32_t*>(st + t * RSTR + (2 * ks + g) * BITS * 4);
#pragma unroll
    for (int i = 0; i < BITS; ++i) sw[i] = words[i];
    const int64_t c0 = kk * 64 + 32 * g;  // first code of the unit
    bool valid;
    const int64_t row = dst_row(t, valid);
    if (valid && c0 % gs == 0) {
      const uint32_t sb = reinterpret_cast<const uint32_t*>(rec + tiled::code_bytes(BITS))
          [(h * 32 + r) * G + (G == 2 ? g : 0)];
      const int64_t si = row * (K / gs) + c0 / gs;
      scales[si] = static_cast<uint16_t>(sb & 0xFFFFu);
      biases[si] = static_cast<uint16_t>(sb >> 16);
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < 64 * CPR; c += kThreads) {
    const int t = c / CPR, j = c % CPR;
    bool valid;
    const int64_t row = dst_row(t, valid);
    const int64_t off = k0 * 8 * BITS + j * 16;
    if (!valid || off >= rowb) continue;
    uint32_t* p = wq + row * W + off / 4;
    const u32x4a v = *reinterpret_cast<const u32x4a*>(st + t * RSTR + j * 16);
    if (off + 16 <= rowb) {
      *reinterpret_cast<u32x4*>(p) = u32x4{v.x, v.y, v.z, v.w};
    } else {  // the row ends 8 bytes into this chunk
      *reinterpret_cast<u32x2*>(p) = u32x2{v.x, v.y};
    }
  }
}

template <int BITS>
struct UntileRun {
  static hipError_t run(const void* in, int64_t N, int64_t K, int gs, bool pairs, uint32_t* wq,
                        uint16_t* sc, uint16_t* bi, hipStream_t s) {
    const int64_t blocks = tiled::row_blocks(N) * ((K / 64 + kTileSteps - 1) / kTileSteps);
    if (blocks == 0) return hipSuccess;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    untile_rows_kernel<BITS><<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
        static_cast<const uint8_t*>(in), N, K, gs, pairs, wq, sc, bi);
    return hipGetLastError();
  }
};

template <int BITS>
struct TileRun {
  static hipError_t run(const uint32_t* wq, const uint16_t* sc, const uint16_t* bi, int64_t N,
                        int64_t K, int gs, bool pairs, void* out, hipStream_t s) {
    const int64_t blocks = tiled::row_blocks(N) * ((K / 64 + kTileSteps - 1) / kTileSteps);
    if (blocks == 0) return hipSuccess;
    if (blocks > 0x7FFFFFFF) {  // one thread per unit then
      const int64_t items = tiled::row_blocks(N) * (K / 64) * 128;
      tile_kernel<BITS><<<grid_for(items), kThreads, 0, s>>>(wq, sc, bi, N, K, gs, pairs,
                                                             static_cast<uint8_t*>(out));
    } else {
      tile_rows_kernel<BITS><<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
          wq, sc, bi, N, K, gs, pairs, static_cast<uint8_t*>(out));
    }
    return hipGetLastError();
  }
};

template <template <int> class F, typename... A>
hipError_t by_bits(int bits, A... args) {
  switch (bits) {
    case 2: return F<2>::run(args...);
    case 3: return F<3>::run(args...);
    case 4: return F<4>::run(args...);
    case 5: return F<5>::run(args...);
    case 6: return F<6>::run(args...);
    case 8: return F<8>::run(args...);
    default: return hipErrorInvalidValue;
  }
}

template <int BITS>
struct PackRun {
  static hipError_t run(const uint8_t* codes, int64_t rows, int64_t cols, uint32_t* wq,
                        hipStream_t s) {
    const int64_t items = rows * (cols * BITS / 32);
    if (items == 0) return hipSuccess;
    pack_kernel<BITS><<<grid_for(items), kThreads, 0, s>>>(codes, rows, cols, wq);
    return hipGetLastError();
  }
};

template <int BITS>
struct UnpackRun {
  static hipError_t run(const uint32_t* wq, int64_t rows, int64_t cols, uint8_t* codes,
                        hipStream_t s) {
    const int64_t items = rows * cols;
    if (items == 0) return hipSuccess;
    unpack_kernel<BITS><<<grid_for(items), kThreads, 0, s>>>(wq, rows, cols, codes);
    return hipGetLastError();
  }
};

template <int BITS>
struct QuantizeRun {
  template <typename TW, typename TSB>
  static hipError_t go(const void* w, int64_t rows, int64_t cols, int gs, int mode,
                       uint32_t* wq, void* sc, void* bi, hipStream_t s) {
    const int64_t items = rows * (cols / gs);
    if (items == 0) return hipSuccess;
    quantize_kernel<BITS, TW, TSB><<<grid_for(items), kThreads, 0, s>>>(
        static_cast<const TW*>(w), rows, cols, gs, mode, wq, static_cast<TSB*>(sc),
        static_cast<TSB*>(bi));
    return hipGetLastError();
  }
  static hipError_t run(const void* w, int w_dtype, int64_t rows, int64_t cols, int gs,
                        int mode, uint32_t* wq, void* sc, void* bi, int sb_dtype,
                        hipStream_t s) {
    // dtype codes: 0 = fp32, 1 = bf16
    if (w_dtype == 0 && sb_dtype == 0)
      return go<float, float>(w, rows, cols, gs, mode, wq, sc, bi, s);
    if (w_dtype == 0 && sb_dtype == 1)
      return go<float, uint16_t>(w, rows, cols, gs, mode, wq, sc, bi, s);
    if (w_dtype == 1 && sb_dtype == 0)
      return go<uint16_t, float>(w, rows, cols, gs, mode, wq, sc, bi, s);
    return go<uint16_t, uint16_t>(w, rows, cols, gs, mode, wq, sc, bi, s);
  }
};

template <int BITS>
struct DequantizeRun {
  template <typename TSB, typename TO>
  static hipError_t go(const uint32_t* wq, const void* sc, const void* bi, int64_t rows,
                       int64_t cols, int gs, void* out, hipStream_t s) {
    const int64_t items = rows * (cols / Period<BITS>::codes);
    if (items == 0) return hipSuccess;
    dequantize_kernel<BITS, TSB, TO><<<grid_for(items), kThreads, 0, s>>>(
        wq, static_cast<const TSB*>(sc), static_cast<const TSB*>(bi), rows, cols, gs,
        static_cast<TO*>(out));
    return hipGetLastError();
  }
  static hipError_t run(const uint32_t* wq, const void* sc, const void* bi, int sb_dtype,
                        int64_t rows, int64_t cols, int gs, void* out, int out_dtype,
                        hipStream_t s) {
    if (sb_dtype == 0 && out_dtype == 0)
      return go<float, float>(wq, sc, bi, rows, cols, gs, out, s);
    if (sb_dtype == 0 && out_dtype == 1)
      return go<float, uint16_t>(wq, sc, bi, rows, cols, gs, out, s);
    if (sb_dtype == 1 && out_dtype == 0)
      return go<uint16_t, float>(wq, sc, bi, rows, cols, gs, out, s);
    return go<uint16_t, uint16_t>(wq, sc, bi, rows, cols, gs, out, s);
  }
};

}  // namespace

namespace detail {

hipError_t launch_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq,
                       hipStream_t s) {
  return by_bits<PackRun>(bits, codes, rows, cols, wq, s);
}

hipError_t launch_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits,
                         uint8_t* codes, hipStream_t s) {
  return by_bits<UnpackRun>(bits, wq, rows, cols, codes, s);
}

hipError_t launch_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols, int gs,
                           int bits, int mode, uint32_t* wq, void* scales, void* biases,
                           int sb_dtype, hipStream_t s) {
  return by_bits<QuantizeRun>(bits, w, w_dtype, rows, cols, gs, mode, wq, scales, biases,
                              sb_dtype, s);
}

hipError_t launch_tile(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                       int64_t N, int64_t K, int gs, int bits, bool pairs, void* out,
                       hipStream_t s) {
  return by_bits<TileRun>(bits, wq, scales, biases, N, K, gs, pairs, out, s);
}

hipError_t launch_untile(const void* tiled, int64_t N, int64_t K, int gs, int bits, bool pairs,
                         uint32_t* wq, uint16_t* scales, uint16_t* biases, hipStream_t s) {
  return by_bits<UntileRun>(bits, tiled, N, K, gs, pairs, wq, scales, biases, s);
}

hipError_t launch_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                             int sb_dtype, int64_t rows, int64_t cols, int gs, int bits,
                             void* out, int out_dtype, hipStream_t s) {
  return by_bits<DequantizeRun>(bits, wq, scales, biases, sb_dtype, rows, cols, gs, out,
                                out_dtype, s);
}

}  // namespace detail
}  // namespace mxq
