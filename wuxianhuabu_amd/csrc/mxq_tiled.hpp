// mxq_tiled.hpp — geometry of the tiled weight layout (host and device).
//
// The MLX layout stores each output row's codes contiguously along K. The
// large-M kernel reads, per 64-code K step, a 48-byte slice (6-bit) from each
// of 64 rows per wave, which touches ~40 cache lines per load instruction. The
// tiled layout reorders the same bits once, at load time, so that every
// weight load of both kernels is a fully coalesced 16-byte-per-lane access:
//
//   record (rb, kk) for row block rb = rows [64*rb, 64*rb+64) and K step kk =
//   codes [64*kk, 64*kk+64), stored at byte (kk * row_blocks + rb) * record_bytes
//   (step-major: the records of one K step, all row blocks, are adjacent, so the
//   GEMV's waves, which all start at the same K steps, read neighbouring bytes):
//     codes, 512*bits bytes: two halves h (rows 64*rb + 32*h + r, r < 32); in
//       each half, "units" u = 0..63 with row r = u % 32 and code half
//       g = u / 32 (codes [64*kk + 32*g, +32), i.e. `bits` whole words of the
//       MLX row). A half is `bits/4` planes of 16 bytes per unit (unit u at
//       plane*1024 + u*16) followed by a remainder plane of (bits % 4) words
//       per unit (unit u at (bits/4)*1024 + u*4*(bits%4)).
//     scale/bias pairs, 256*gps bytes (gps = 2 when group_size == 32, else 1):
//       entry ((h*32 + r) * gps + (gps == 2 ? g : 0)) is one dword, bf16 scale
//       in the low half and bf16 bias in the high half, for the group that
//       holds unit (h, r, g)'s codes.
//   Rows past N are zero (codes, scale and bias).
// Requires K % 64 == 0; the whole layout stays below 2 GiB (the kernels' 32-bit
// step offsets).
#pragma once

#include <stdint.h>

namespace mxq {
namespace tiled {

__host__ __device__ constexpr int gps(int gs) { return gs == 32 ? 2 : 1; }
__host__ __device__ constexpr int code_bytes(int bits) { return 512 * bits; }
__host__ __device__ constexpr int half_bytes(int bits) { return 256 * bits; }
__host__ __device__ constexpr int record_bytes(int bits, int gs) {
  return code_bytes(bits) + 256 * gps(gs);
}
__host__ __device__ constexpr int full_planes(int bits) { return bits / 4; }
__host__ __device__ constexpr int rem_words(int bits) { return bits % 4; }

__host__ __device__ inline int64_t row_blocks(int64_t N) { return (N + 63) / 64; }
__host__ __device__ inline int64_t total_bytes(int64_t N, int64_t K, int gs, int bits) {
  return row_blocks(N) * (K / 64) * static_cast<int64_t>(record_bytes(bits, gs));
}
// record index of (row block rb, K step kk) among rbs = row_blocks(N)
__host__ __device__ inline int64_t record_index(int64_t rb, int64_t kk, int64_t rbs) {
  return kk * rbs + rb;
}
constexpr int64_t kMaxTiledBytes = 0x7FFFFFFF;

}  // namespace tiled
}  // namespace mxq
