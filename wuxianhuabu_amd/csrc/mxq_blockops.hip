// mxq_blockops.hip — the row-wise ops of the H3 DiT block that feed and consume
// its quantized linears, fused as the reference fuses them
// (`model/2网络算子/网络算子-融合-RMSNormRoPE-通用.swift:41-343`, called at
// `model/minimax h3/H3Transformer.swift:455-480, 1117-1155`):
//   rmsnorm_rope    q/k path: rmsNormLast then the split-half rotary of
//                   applyRopePub (`model/minimax h3/H3Common.swift:502-508, 555-569`);
//   norm_modscale   rmsNormLast then x * (scale[m] + 1) + shift[m] (adaLN
//                   modulation, row m of the modulation table per token row);
//   mod_gate        x + other * gate[m] (gated residual).
// Arithmetic as the reference's kernels: fp32 mean of squares, rsqrt, the
// normalised value rounded to bf16 before the modulation / rotation, one more
// rounding at the end.
//
// All three are HBM-bound (a few flops per byte). One wave per token row, four
// rows per 256-thread workgroup; rows of x move in 16-byte pieces when the row
// length allows (8 bf16), else element-wise. The norm reads its row twice (the
// second pass hits L2: 4 rows of at most a few KiB per workgroup).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>

#include "mxq.h"
#include "mxq_device.hpp"
#include "mxq_internal.hpp"

namespace mxq {
namespace {

constexpr int kWaves = 4;  // rows per workgroup

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(16)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// mean of squares of one bf16 row (n elements), fp32, reduced over the wave
template <bool VEC>
__device__ __forceinline__ float row_sumsq(const uint16_t* xr, int n, int lane) {
  float s = 0.f;
  if constexpr (VEC) {
    const u32x4a* p = reinterpret_cast<const u32x4a*>(xr);
    for (int c = lane; c < n / 8; c += 64) {
      const u32x4a v = p[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = lo16(v[i]), b = hi16(v[i]);
        s = fmaf(a, a, s);
        s = fmaf(b, b, s);
      }
    }
  } else {
    for (int j = lane; j < n; j += 64) {
      const float a = bf16_to_f32(xr[j]);
      s = fmaf(a, a, s);
    }
  }
  return wave_sum(s);
}

// out = bf16( bf16(x * rstd * w) * (scale[m] + 1) + shift[m] )
template <bool VEC>
__global__ __launch_bounds__(64 * kWaves) void norm_modscale_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ shift, const uint16_t* __restrict__ scale,
    const uint32_t* __restrict__ map, int64_t mod_rows, int64_t S, int hidden, float eps,
    uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= S) return;
  const int64_t m = map ? min(static_cast<int64_t>(map[row]), mod_rows - 1) : 0;
  const uint16_t* xr = x + row * hidden;
  const uint16_t* sh = shift + m * hidden;
  const uint16_t* sc = scale + m * hidden;
  uint16_t* orow = out + row * hidden;
  const float rstd = rsqrtf(row_sumsq<VEC>(xr, hidden, lane) / hidden + eps);
  if constexpr (VEC) {
    for (int c = lane; c < hidden / 8; c += 64) {
      const u32x4a xv = reinterpret_cast<const u32x4a*>(xr)[c];
      const u32x4a wv = reinterpret_cast<const u32x4a*>(w)[c];
      const u32x4a hv = reinterpret_cast<const u32x4a*>(sh)[c];
      const u32x4a sv = reinterpret_cast<const u32x4a*>(sc)[c];
      u32x4a ov;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float n0 = round_bf16(lo16(xv[i]) * rstd * lo16(wv[i]));
        const float n1 = round_bf16(hi16(xv[i]) * rstd * hi16(wv[i]));
        ov[i] = pack_bf16x2(n0 * (lo16(sv[i]) + 1.f) + lo16(hv[i]),
                            n1 * (hi16(sv[i]) + 1.f) + hi16(hv[i]));
      }
      reinterpret_cast<u32x4a*>(orow)[c] = ov;
    }
  } else {
    for (int j = lane; j < hidden; j += 64) {
      const float nv = round_bf16(bf16_to_f32(xr[j]) * rstd * bf16_to_f32(w[j]));
      orow[j] = f32_to_bf16(nv * (bf16_to_f32(sc[j]) + 1.f) + bf16_to_f32(sh[j]));
    }
  }
}

// norm_modscale with the row in registers (hidden <= 512 * CPL, hidden % 8 == 0):
// one read of x instead of two.
template <int CPL>
__global__ __launch_bounds__(64 * kWaves) void norm_modscale_reg_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ shift, const uint16_t* __restrict__ scale,
    const uint32_t* __restrict__ map, int64_t mod_rows, int64_t S, int hidden, float eps,
    uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= S) return;
  const int64_t m = map ? min(static_cast<int64_t>(map[row]), mod_rows - 1) : 0;
  const int chunks = hidden / 8;
  const u32x4a* xr = reinterpret_cast<const u32x4a*>(x + row * hidden);
  u32x4a xv[CPL];
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + 64 * k;
    xv[k] = c < chunks ? xr[c] : u32x4a{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = lo16(xv[k][i]), b = hi16(xv[k][i]);
      sq = fmaf(a, a, sq);
      sq = fmaf(b, b, sq);
    }
  const float rstd = rsqrtf(wave_sum(sq) / hidden + eps);
  const u32x4a* wr = reinterpret_cast<const u32x4a*>(w);
  const u32x4a* hr = reinterpret_cast<const u32x4a*>(shift + m * hidden);
  const u32x4a* sr = reinterpret_cast<const u32x4a*>(scale + m * hidden);
  u32x4a* orow = reinterpret_cast<u32x4a*>(out + row * hidden);
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + 64 * k;
    if (c < chunks) {
      const u32x4a wv = wr[c], hv = hr[c], sv = sr[c];
      u32x4a ov;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float n0 = round_bf16(lo16(xv[k][i]) * rstd * lo16(wv[i]));
        const float n1 = round_bf16(hi16(xv[k][i]) * rstd * hi16(wv[i]));
        ov[i] = pack_bf16x2(n0 * (lo16(sv[i]) + 1.f) + lo16(hv[i]),
                            n1 * (hi16(sv[i]) + 1.f) + hi16(hv[i]));
      }
      orow[c] = ov;
    }
  }
}

// out = bf16( x + other * gate[m] )
template <bool VEC>
__global__ __launch_bounds__(64 * kWaves) void mod_gate_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ other,
    const uint16_t* __restrict__ gate, const uint32_t* __restrict__ map, int64_t mod_rows,
    int64_t S, int hidden, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= S) return;
  const int64_t m = map ? min(static_cast<int64_t>(map[row]), mod_rows - 1) : 0;
  const uint16_t* xr = x + row * hidden;
  const uint16_t* orr = other + row * hidden;
  const uint16_t* gr = gate + m * hidden;
  uint16_t* orow = out + row * hidden;
  if constexpr (VEC) {
    for (int c = lane; c < hidden / 8; c += 64) {
      const u32x4a xv = reinterpret_cast<const u32x4a*>(xr)[c];
      const u32x4a ov = reinterpret_cast<const u32x4a*>(orr)[c];
      const u32x4a gv = reinterpret_cast<const u32x4a*>(gr)[c];
      u32x4a r;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[i] = pack_bf16x2(lo16(xv[i]) + lo16(ov[i]) * lo16(gv[i]),
                           hi16(xv[i]) + hi16(ov[i]) * hi16(gv[i]));
      reinterpret_cast<u32x4a*>(orow)[c] = r;
    }
  } else {
    for (int j = lane; j < hidden; j += 64)
      orow[j] = f32_to_bf16(bf16_to_f32(xr[j]) + bf16_to_f32(orr[j]) * bf16_to_f32(gr[j]));
  }
}

// q/k rows [S, H, hd]: n = bf16(x * rstd * w); for j < rh (= rot/2)
//   out[j] = n[j] c[s, j] - n[j + rh] s[s, j],  out[j + rh] = n[j + rh] c[s, j] + n[j] s[s, j],
// out[j] = n[j] for j >= rot. The lane keeps its elements j = lane + 64 e in
// registers and the wave's normalised row goes through LDS for the partners.
template <int E, typename TT>
__global__ __launch_bounds__(64 * kWaves) void rmsnorm_rope_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const TT* __restrict__ ctab, const TT* __restrict__ stab, int64_t rows, int H, int hd,
    int rot, float eps, uint16_t* __restrict__ out) {
  __shared__ float nrm[kWaves][64 * E];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (row >= rows) return;
  const int64_t s = row / H;
  const int rh = rot / 2;
  const uint16_t* xr = x + row * hd;
  float xv[E];
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane + 64 * e;
    xv[e] = j < hd ? bf16_to_f32(xr[j]) : 0.f;
    sq = fmaf(xv[e], xv[e], sq);
  }
  const float rstd = rsqrtf(wave_sum(sq) / hd + eps);
  float* nw = nrm[wave];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane + 64 * e;
    if (j < hd) {
      xv[e] = round_bf16(xv[e] * rstd * bf16_to_f32(w[j]));
      nw[j] = xv[e];
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's row is in LDS
  __builtin_amdgcn_wave_barrier();
  auto tab = [&](const TT* t, int i) -> float {
    if constexpr (sizeof(TT) == 2)
      return bf16_to_f32(t[s * rh + i]);
    else
      return t[s * rh + i];
  };
  uint16_t* orow = out + row * hd;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane + 64 * e;
    if (j >= hd) continue;
    float o = xv[e];
    if (j < rh)
      o = xv[e] * tab(ctab, j) - nw[j + rh] * tab(stab, j);
    else if (j < rot)
      o = xv[e] * tab(ctab, j - rh) + nw[j - rh] * tab(stab, j - rh);
    orow[j] = f32_to_bf16(o);
  }
}

// rmsnorm_rope with G = hd / 8 lanes per row (64 / G rows per wave): each lane
// holds 8 consecutive elements (one 16-byte load), the mean of squares is
// reduced over the row's G lanes, and the rotation partner of element j
// (j +- rot/2, a multiple of 8) sits in lane +- rot/16 of the same row, read with
// lane shuffles. Used when hd and rot/2 are multiples of 8 and G divides 64.
template <int G, typename TT>
__global__ __launch_bounds__(64 * kWaves) void rmsnorm_rope_vec_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const TT* __restrict__ ctab, const TT* __restrict__ stab, int64_t rows, int H, int rot,
    float eps, uint16_t* __restrict__ out) {
  constexpr int hd = 8 * G;
  constexpr int RPW = 64 / G;  // rows per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gl = lane % G;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * RPW + lane / G;
  const bool valid = row < rows;
  const int j0 = gl * 8, rh = rot / 2;
  u32x4a xv = {0u, 0u, 0u, 0u};
  if (valid) xv = reinterpret_cast<const u32x4a*>(x + row * hd)[gl];
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = lo16(xv[i]);
    v[2 * i + 1] = hi16(xv[i]);
  }
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sq = fmaf(v[i], v[i], sq);
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
  const float rstd = rsqrtf(sq / hd + eps);
  const u32x4a wv = reinterpret_cast<const u32x4a*>(w)[gl];
  float n[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    n[2 * i] = round_bf16(v[2 * i] * rstd * lo16(wv[i]));
    n[2 * i + 1] = round_bf16(v[2 * i + 1] * rstd * hi16(wv[i]));
  }
  // partner lane within the row: j0 < rh -> j0 + rh; rh <= j0 < rot -> j0 - rh
  const int ph = rh / 8;
  const int pl = gl < ph ? gl + ph : (gl < 2 * ph ? gl - ph : gl);
  const int src = lane - gl + pl;
  float p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = __shfl(n[i], src, 64);
  u32x4a ov;
  if (j0 < rot) {
    const int64_t s = row / H;
    const int t0 = j0 < rh ? j0 : j0 - rh;
    const float sg = j0 < rh ? -1.f : 1.f;
    float c[8], sn[8];
    if (valid) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(TT) == 2) {
          c[i] = bf16_to_f32(ctab[s * rh + t0 + i]);
          sn[i] = bf16_to_f32(stab[s * rh + t0 + i]);
        } else {
          c[i] = ctab[s * rh + t0 + i];
          sn[i] = stab[s * rh + t0 + i];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = sn[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ov[i] = pack_bf16x2(n[2 * i] * c[2 * i] + sg * p[2 * i] * sn[2 * i],
                          n[2 * i + 1] * c[2 * i + 1] + sg * p[2 * i + 1] * sn[2 * i + 1]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) ov[i] = pack_bf16x2(n[2 * i], n[2 * i + 1]);
  }
  if (valid) reinterpret_cast<u32x4a*>(out + row * hd)[gl] = ov;
}

inline unsigned blocks_for(int64_t rows) {
  return static_cast<unsigned>((rows + kWaves - 1) / kWaves);
}

bool vec_ok(int n, std::initializer_list<const void*> ptrs) {
  if (n % 8) return false;
  for (const void* p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15u)) return false;
  return true;
}

}  // namespace

namespace detail {

hipError_t launch_norm_modscale(const uint16_t* x, int64_t S, int hidden, const uint16_t* w,
                                const uint16_t* shift, const uint16_t* scale,
                                const uint32_t* map, int64_t mod_rows, float eps, uint16_t* out,
                                hipStream_t s) {
  if (S == 0 || hidden == 0) return hipSuccess;
  if (vec_ok(hidden, {x, w, shift, scale, out}) && hidden <= 512 * 16) {
    const int cpl = (hidden / 8 + 63) / 64;
#define MXQ_NMS_REG(C)                                                                   \
  if (cpl <= C) {                                                                        \
    norm_modscale_reg_kernel<C><<<blocks_for(S), 64 * kWaves, 0, s>>>(                  \
        x, w, shift, scale, map, mod_rows, S, hidden, eps, out);                         \
    return hipGetLastError();                                                            \
  }
    MXQ_NMS_REG(2)
    MXQ_NMS_REG(4)
    MXQ_NMS_REG(8)
    MXQ_NMS_REG(12)
    MXQ_NMS_REG(16)
#undef MXQ_NMS_REG
  }
  if (vec_ok(hidden, {x, w, shift, scale, out}))
    norm_modscale_kernel<true><<<blocks_for(S), 64 * kWaves, 0, s>>>(
        x, w, shift, scale, map, mod_rows, S, hidden, eps, out);
  else
    norm_modscale_kernel<false><<<blocks_for(S), 64 * kWaves, 0, s>>>(
        x, w, shift, scale, map, mod_rows, S, hidden, eps, out);
  return hipGetLastError();
}

hipError_t launch_mod_gate(const uint16_t* x, const uint16_t* other, int64_t S, int hidden,
                           const uint16_t* gate, const uint32_t* map, int64_t mod_rows,
                           uint16_t* out, hipStream_t s) {
  if (S == 0 || hidden == 0) return hipSuccess;
  if (vec_ok(hidden, {x, other, gate, out}))
    mod_gate_kernel<true><<<blocks_for(S), 64 * kWaves, 0, s>>>(x, other, gate, map, mod_rows,
                                                                 S, hidden, out);
  else
    mod_gate_kernel<false><<<blocks_for(S), 64 * kWaves, 0, s>>>(x, other, gate, map, mod_rows,
                                                                  S, hidden, out);
  return hipGetLastError();
}

template <typename TT>
hipError_t rope_by_width(const uint16_t* x, int64_t rows, int H, int hd, const uint16_t* w,
                         const TT* c, const TT* sn, int rot, float eps, uint16_t* out,
                         hipStream_t s) {
  const bool vec = hd % 8 == 0 && (rot / 2) % 8 == 0 && 64 % (hd / 8 == 0 ? 3 : hd / 8) == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  if (vec) {
    const int G = hd / 8;
    const int64_t per_block = static_cast<int64_t>(kWaves) * (64 / G);
    const unsigned gv = static_cast<unsigned>((rows + per_block - 1) / per_block);
    switch (G) {
#define MXQ_ROPE_VEC(GG)                                                                    \
  case GG:                                                                                  \
    rmsnorm_rope_vec_kernel<GG, TT><<<gv, 64 * kWaves, 0, s>>>(x, w, c, sn, rows, H, rot, eps, \
                                                             out);                          \
    return hipGetLastError();
      MXQ_ROPE_VEC(1)
      MXQ_ROPE_VEC(2)
      MXQ_ROPE_VEC(4)
      MXQ_ROPE_VEC(8)
      MXQ_ROPE_VEC(16)
      MXQ_ROPE_VEC(32)
      MXQ_ROPE_VEC(64)
#undef MXQ_ROPE_VEC
      default: break;
    }
  }
  const unsigned g = blocks_for(rows);
  if (hd <= 64)
    rmsnorm_rope_kernel<1, TT><<<g, 64 * kWaves, 0, s>>>(x, w, c, sn, rows, H, hd, rot, eps, out);
  else if (hd <= 128)
    rmsnorm_rope_kernel<2, TT><<<g, 64 * kWaves, 0, s>>>(x, w, c, sn, rows, H, hd, rot, eps, out);
  else if (hd <= 256)
    rmsnorm_rope_kernel<4, TT><<<g, 64 * kWaves, 0, s>>>(x, w, c, sn, rows, H, hd, rot, eps, out);
  else
    rmsnorm_rope_kernel<8, TT><<<g, 64 * kWaves, 0, s>>>(x, w, c, sn, rows, H, hd, rot, eps, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rope(const uint16_t* x, int64_t S, int H, int hd, const uint16_t* w,
                               const void* c, const void* sn, int table_dtype, int rot,
                               float eps, uint16_t* out, hipStream_t s) {
  const int64_t rows = S * H;
  if (rows == 0 || hd == 0) return hipSuccess;
  if (table_dtype == MXQ_BFLOAT16)
    return rope_by_width(x, rows, H, hd, w, static_cast<const uint16_t*>(c),
                         static_cast<const uint16_t*>(sn), rot, eps, out, s);
  return rope_by_width(x, rows, H, hd, w, static_cast<const float*>(c),
                       static_cast<const float*>(sn), rot, eps, out, s);
}

}  // namespace detail
}  // namespace mxq
