// mxq_device.hpp — device-side helpers shared by the libmxq kernels (gfx950).
//
// Packed layout (MLX affine): for row n, code k occupies stream bits
// [k*BITS, (k+1)*BITS) of the little-endian uint32 words of that row, LSB
// first. Every group of >= 32 codes starts on a word boundary, so a run of
// codes that is a multiple of the "period" (the smallest code count that fills
// whole words) can be decoded from whole words with compile-time offsets.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxq {

// 4-byte-aligned vector types for loads (the hardware runs in unaligned mode;
// only dword alignment is guaranteed by the API contract).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));  // 16-byte aligned (LDS)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN quieted). gfx950 lowers the
// __bf16 conversion to v_cvt_pk_bf16_f32, which rounds to nearest even.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2 in one dword (lo in bits 0..15): one
// v_cvt_pk_bf16_f32, round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Code i of a run of codes stored LSB-first in words w[0..]; all offsets are
// compile-time constants after unrolling, so this becomes v_bfe_u32 or
// v_alignbit_b32 + v_and_b32.
template <int BITS, int I, int NW>
__device__ __forceinline__ uint32_t code_of(const uint32_t (&w)[NW]) {
  constexpr int P = I * BITS;
  constexpr int WD = P / 32;
  constexpr int OFF = P % 32;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  static_assert(WD < NW, "code outside words");
  if constexpr (OFF + BITS <= 32) {
    return (w[WD] >> OFF) & MASK;
  } else {
    static_assert(WD + 1 < NW, "straddling code outside words");
    return __builtin_amdgcn_alignbit(w[WD + 1], w[WD], OFF) & MASK;
  }
}

// Same as code_of with the index as a value: used inside fully unrolled loops,
// where `i` folds to a constant (so `w` stays in registers).
template <int BITS, int NW>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[NW], int i) {
  const int p = i * BITS;
  const int wd = p >> 5, off = p & 31;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  if (off + BITS <= 32) return (w[wd] >> off) & MASK;
  return __builtin_amdgcn_alignbit(w[wd + 1], w[wd], off) & MASK;
}

// Codes i and i+1 (i even) of a run as one dword of two bf16 values
// (128 + q_i, 128 + q_{i+1}), for bits <= 7: their 2*BITS-bit field F is spread
// so the second code lands at bit 16, then 0x43 supplies each half's exponent
// (0x4300 | q is exactly 128 + q for q < 128).
// Three VALU instructions (bfe, lshl_or, and_or; four when the field straddles two
// words). `mask` and `magic` are the constants MASK | MASK << 16 and 0x43004300 held
// in VGPRs whose values the compiler does not know (VOP3 takes no literals here):
// knowing the mask, it splits the field into its two codes and spends four or five.
// Plain code, not inline assembly: the result feeds the MFMAs, and the compiler
// places the wait states a VALU result needs before an MFMA reads it only for
// instructions it generated itself. Written as inline assembly, the pair reached
// the MFMA one instruction later in some schedules and the MFMA read a stale
// register (wrong sums, depending on the build).
template <int BITS, int NW>
__device__ __forceinline__ uint32_t pair_at(const uint32_t (&w)[NW], int i, uint32_t mask,
                                            uint32_t magic) {
  static_assert(BITS <= 7, "0x4300 | q needs q < 128");
  const int p = i * BITS;
  const int wd = p >> 5, off = p & 31;
  constexpr uint32_t FMASK = (1u << (2 * BITS)) - 1u;
  const uint32_t f = off + 2 * BITS <= 32
                         ? (w[wd] >> off) & FMASK
                         : __builtin_amdgcn_alignbit(w[wd + 1], w[wd], off) & FMASK;
  return (((f << (16 - BITS)) | f) & mask) | magic;
}

template <int BITS, int NCODES, int NW, int I = 0>
__device__ __forceinline__ void decode_codes(const uint32_t (&w)[NW], uint32_t (&q)[NCODES]) {
  if constexpr (I < NCODES) {
    q[I] = code_of<BITS, I, NW>(w);
    decode_codes<BITS, NCODES, NW, I + 1>(w, q);
  }
}

// Smallest number of codes that fills whole 32-bit words, and those words.
template <int BITS>
struct Period {
  static constexpr int codes = (BITS == 3 || BITS == 5) ? 32 : (BITS == 6 ? 16 : 32 / BITS);
  static constexpr int words = codes * BITS / 32;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace mxq
