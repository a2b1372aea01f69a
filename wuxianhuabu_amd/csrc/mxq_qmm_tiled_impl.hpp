// mxq_qmm_tiled_impl.hpp — large-M quantized matmul over the tiled weight layout:
//   y[m, n] = sum_k x[m, k] * (s[n, k/gs] * q[n, k] + b[n, k/gs])  (+ bias[n])
// with the same arithmetic as the MLX-layout kernel in mxq_qmm.hip (weights
// dequantized as fmaf(q, s, b) in fp32 and rounded once to bf16, bf16 MFMA
// with fp32 accumulation, bias added in fp32 before the single output
// rounding). It serves QuantizedLinear / MfLinear once their weights are
// resident (`model/minimax h3/H3Common.swift:358-368`,
// `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:177-188, 387-388`).
//
// Work decomposition (one workgroup = 4 waves, one per SIMD):
//   * the workgroup owns a BM x 256 output tile; wave w owns the 64 features
//     of tiled row block n0/64 + w, i.e. one tiled record per K step;
//   * every K step (64 codes) moves two operands HBM -> LDS with LDS-direct
//     loads (no VGPRs): the BM x 64 bf16 activation tile (shared by the four
//     waves) and each wave's weight record (a verbatim copy, 16 or 4 bytes per
//     lane), each into a 3-stage ring;
//   * each wave reads its record of step k+1 from LDS, unpacks it to bf16
//     (one slice per MFMA pair) while step k's MFMAs run, and reads the
//     activation fragments from LDS through a 4-deep register ring;
//   * v_mfma_f32_32x32x16_bf16: weights are the A operand, activations the B
//     operand; lane half g2 = lane/32 owns codes [32*g2, 32*g2 + 32) of the step
//     for both, so one lane unpacks one 32-code run (BITS whole words).
// Pipeline: step k requests activations of step k+2 and weights of step k+3,
// spread over its MFMA pairs. All global traffic is LDS-direct, so the only
// memory waits are the explicit ones: at the end of step k, vmcnt(L) (every
// request but step k's own L has landed) then a workgroup barrier.
#pragma once

#include <type_traits>

#include "mxq.h"
#include "mxq_device.hpp"
#include "mxq_internal.hpp"
#include "mxq_ring.hpp"
#include "mxq_tiled.hpp"

namespace mxq {
namespace {

constexpr int kRows = 256;    // output features per workgroup (4 waves x 64)
constexpr int kThreads = 256;
constexpr int kStages = 3;
constexpr int kGroupM = 4;    // token tiles swept together per XCD

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v3u __attribute__((ext_vector_type(3)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));  // y is 4-byte aligned

// One wave's record (64 rows x 64 codes) of the tiled layout, and how it is
// moved: CHUNKS loads of 1 KiB (16 B per lane), then TAIL loads of 256 B.
template <int BITS, int GP>
struct Rec {
  static constexpr int FP = tiled::full_planes(BITS), RW = tiled::rem_words(BITS);
  static constexpr int HALF = tiled::half_bytes(BITS);
  static constexpr int CODE = tiled::code_bytes(BITS);
  static constexpr int BYTES = CODE + 256 * GP;
  static constexpr int CHUNKS = BYTES / 1024;
  static constexpr int TAIL = (BYTES % 1024) / 256;
  static constexpr int LOADS = CHUNKS + TAIL;
};

// Activations fused into the epilogue (values in fp32, before the one bf16
// rounding): GELU with the tanh approximation
// 0.5 v (1 + tanh(u)), u = sqrt(2/pi) (v + 0.044715 v^3), as between the LTX
// feed-forward projections (`model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:392-401`),
// and silu(v) = v / (1 + e^{-v}) for silu(gate) * up on the fused fc1 output of
// the H3 MLP (`model/minimax h3/H3Transformer.swift:620-629`). Since
// 0.5 (1 + tanh(u)) = 1 / (1 + e^{-2u}), both are v / (1 + e^{-z}): one exp2
// and one reciprocal (v_exp_f32, v_rcp_f32; about 1 ulp each, far below the
// bf16 rounding that follows). e^{-z} = inf gives -0 / +0 in the limits.
__device__ __forceinline__ float act_sigmoid_times(float v, float z) {
  return __fdividef(v, 1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * z));
}
__device__ __forceinline__ float act_gelu_tanh(float v) {
  const float u = 0.7978845608028654f * fmaf(0.044715f * v, v * v, v);
  return act_sigmoid_times(v, 2.f * u);
}
__device__ __forceinline__ float act_silu(float v) { return act_sigmoid_times(v, v); }

template <int BITS>
struct RawRun {  // one lane's two 32-code runs and their scale/bias dwords
  uint32_t w[2][BITS];
  uint32_t sb[2];
};

// LORA: with the low-rank update (a separate instantiation: the update's rank
// loop over the accumulators costs the epilogue registers the plain kernel
// does not have to give up).
template <int BITS, int BM, int GP, bool EVEN, bool LORA>
__global__ __launch_bounds__(kThreads, 1) void qmm_tiled_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ tw,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int m_tiles, int n_tiles, int act, const uint16_t* __restrict__ xa,
    const uint16_t* __restrict__ bt, int rank) {
  using R = Rec<BITS, GP>;
  constexpr int MB = BM / 32;          // 32-token blocks per wave
  constexpr int XL = BM / 32;          // activation requests per wave per step (8 rows each)
  constexpr int XSTAGE = BM * 128;     // bytes per activation stage
  constexpr int WSTAGE = 4 * R::BYTES; // bytes per weight stage
  constexpr int L = XL + R::LOADS;     // requests per wave per step
  constexpr int SLOTS = MB * 4;        // MFMA pairs per step
  static_assert(L <= 2 * SLOTS, "two requests per MFMA pair at most");
  // epilogue staging: 4 KiB per wave, inside the consumed activation stage when
  // the wave's part of it is that large (BM >= 128), else a separate area
  constexpr bool OWN_STAGING = XL * 1024 < 4096;
  constexpr int LDS_BYTES = kStages * (XSTAGE + WSTAGE) + (OWN_STAGING ? 4 * 4096 : 0);
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
  uint8_t* const xl = lds;
  uint8_t* const wl = lds + kStages * XSTAGE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g2 = lane >> 5;

  // ---- persistent schedule: the tiles of the grouped order (see tile_of) are
  // split into 8 contiguous ranges, one per XCD (workgroup b runs on XCD b % 8);
  // the XCD's G/8 workgroups take its range round-robin, so in each round they
  // hold consecutive tiles and share operands in that XCD's L2.
  const int tiles = m_tiles * n_tiles;
  const int per_xcd = gridDim.x >> 3;  // gridDim.x is a multiple of 8
  const int t8 = (tiles + 7) >> 3;
  const int first = (blockIdx.x & 7) * t8 + (blockIdx.x >> 3);
  const int end = min(tiles, ((blockIdx.x & 7) + 1) * t8);
  if (first >= end) return;
  const int my_tiles = (end - first + per_xcd - 1) / per_xcd;
  const int nk = K >> 6;
  const int row_blocks = (N + 63) >> 6;
  // token / feature origin of this workgroup's r-th tile, packed as
  // m0 * 65536 + n0 / 64 (m0 < 2^15 tokens... see the host's limits): groups of
  // kGroupM token tiles sweep all feature tiles
  auto tile_of = [&](int r) -> int64_t {
    const int t = first + r * per_xcd;
    const int per_group = kGroupM * n_tiles;
    const int first_m = (t / per_group) * kGroupM;
    const int gsize = min(m_tiles - first_m, kGroupM);
    const int in_group = t % per_group;
    const int64_t m0 = static_cast<int64_t>(first_m + in_group % gsize) * BM;
    return (m0 << 32) | static_cast<uint32_t>((in_group / gsize) * kRows);
  };
  auto m0_of = [](int64_t t) { return static_cast<int>(t >> 32); };
  auto n0_of = [](int64_t t) { return static_cast<int>(t & 0xFFFFFFFF); };
  // activations of one token tile; rows past M lie outside the descriptor and
  // load as zeros (their outputs are never stored)
  auto x_rsrc = [&](int m0) {
    return ring::make_rsrc(x + static_cast<int64_t>(m0) * K,
                           static_cast<uint32_t>(min(BM, M - m0)) * K * 2);
  };
  // this wave's row block of one feature tile (clamped: a block past N computes
  // rows that are never stored), from its step-0 record to the end of the layout;
  // step kk's record lies kk * step_bytes further (records are step-major)
  const int step_bytes = row_blocks * R::BYTES;
  auto w_rsrc = [&](int n0) {
    const int rb = min((n0 >> 6) + wave, row_blocks - 1);
    return ring::make_rsrc(tw + static_cast<int64_t>(rb) * R::BYTES,
                           static_cast<uint32_t>(nk * row_blocks - rb) * R::BYTES);
  };

  // activation request i of this wave fills stage rows (wave*XL + i)*8 .. +8:
  // lane t writes physical chunk t%8 of row +t/8, i.e. logical chunk
  // (t%8) ^ swz(row). The row's low 3 bits are t/8 and bit 3 is the parity of
  // wave*XL + i, so the lane part of the offset takes two values (xvo) plus
  // (i & ~1) * 8 rows. The whole row offset stays in the vector offset, the
  // part of the address the buffer range check covers (the scalar offset, here
  // the K position, is not checked): rows past M then load as zeros.
  int xvo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave * XL + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ring::swz(r);
    xvo[i] = (r * K + 8 * c) * 2;
  }
  // fragment reads: token row mb*32 + l32, logical chunk 4*g2 + sl
  int xro[4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) xro[sl] = l32 * 128 + (((4 * g2 + sl) ^ ring::swz(l32)) * 16);

  f32x16 acc[2][MB];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x16{};
  uint32_t wu[2][2][16];  // unpacked bf16 pairs: [parity][row block][dword]
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) wu[p][nb][i] = 0u;
  // The third fill step (g = -1) multiplies activation stage 2 by wu[0]; both
  // hold exact zeros then, so that step adds +0 whatever the inputs.
  {
    v4u* z = reinterpret_cast<v4u*>(xl + 2 * XSTAGE);
#pragma unroll
    for (int i = tid; i < XSTAGE / 16; i += kThreads) z[i] = v4u{0u, 0u, 0u, 0u};
  }

  // Two request positions move through this workgroup's steps (tile r, K step
  // k) ahead of the step being multiplied (g): activations (step g+2) and
  // weights (step g+3). At the last step they stop and repeat it: a repeated
  // request is harmless and keeps every step's request count equal. Plain
  // scalars, advanced in place, so they stay in SGPRs, as do the buffer
  // descriptors of their current tiles (rebuilt only when a position moves on
  // to its next tile).
  int xs_r = 0, xs_k = 0, ws_r = 0, ws_k = 0;
  int64_t xs_t = tile_of(0), ws_t = xs_t;
  __amdgpu_buffer_rsrc_t xr_cur = x_rsrc(m0_of(xs_t)), wr_cur = w_rsrc(n0_of(ws_t));

  // request i of a step (activations first, needed a step sooner); st = the
  // step's ring index g mod 3: activations of step g+2 go to stage (g+2) mod 3,
  // weights of step g+3 to stage g mod 3
  auto request = [&](int i, int st, const __amdgpu_buffer_rsrc_t& xr, int kx,
                     const __amdgpu_buffer_rsrc_t& wr, int kw) __attribute__((always_inline)) {
    if (i < XL) {
      const int stage = st == 0 ? 2 : st - 1;
      ring::lds_load<16>(xr, xl + stage * XSTAGE + (wave * XL + i) * 1024,
                         xvo[i & 1] + (i & ~1) * 16 * K, kx * 128);
    } else {
      const int j = i - XL;
      const uint8_t* dst = wl + st * WSTAGE + wave * R::BYTES;
      if (j < R::CHUNKS) {
        ring::lds_load<16>(wr, dst + j * 1024, lane * 16, kw * step_bytes + j * 1024);
      } else {
        const int off = R::CHUNKS * 1024 + (j - R::CHUNKS) * 256;
        ring::lds_load<4>(wr, dst + off, lane * 4, kw * step_bytes + off);
      }
    }
  };
  auto read_frag = [&](const uint8_t* stage, int q) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8*>(stage + (q / 4) * 4096 + xro[q % 4]);
  };
  // this lane's two runs of one record, from LDS
  auto read_raw = [&](const uint8_t* rec, RawRun<BITS>& r) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const uint8_t* h = rec + nb * R::HALF;
#pragma unroll
      for (int p = 0; p < R::FP; ++p) {
        const v4u v = *reinterpret_cast<const v4u*>(h + p * 1024 + lane * 16);
        r.w[nb][4 * p] = v.x; r.w[nb][4 * p + 1] = v.y;
        r.w[nb][4 * p + 2] = v.z; r.w[nb][4 * p + 3] = v.w;
      }
      const uint8_t* t = h + R::FP * 1024 + lane * 4 * R::RW;
      if constexpr (R::RW == 1) {
        r.w[nb][4 * R::FP] = *reinterpret_cast<const uint32_t*>(t);
      } else if constexpr (R::RW == 2) {
        const v2u v = *reinterpret_cast<const v2u*>(t);
        r.w[nb][4 * R::FP] = v.x; r.w[nb][4 * R::FP + 1] = v.y;
      } else if constexpr (R::RW == 3) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          r.w[nb][4 * R::FP + i] = reinterpret_cast<const uint32_t*>(t)[i];
      }
      r.sb[nb] = *reinterpret_cast<const uint32_t*>(
          rec + R::CODE + ((nb * 32 + l32) * GP + (GP == 2 ? g2 : 0)) * 4);
    }
  };
  // ---- epilogue of one tile, one 32-token block (mb) at a time: the lane holds
  // acc for features n + nb*32 + 8a + 4*g2 + r (a, r = 0..3, n = n0 + 64*wave)
  // of token m0 + 32 mb + l32. The wave rounds its block to bf16 (bias added and
  // the activation applied in fp32 first) into LDS, reads it back as 16-byte row
  // pieces and stores whole row segments: 128 B (64 features) per row, or 64 B
  // for SwiGLU, whose record halves are the gate and up rows of the same 32
  // outputs (tiled by mxq_tile_swiglu) and whose output row has N/2 columns.
  // The staging area is this wave's own part of the activation stage the tile's
  // last step consumed: after that step's barrier no wave reads it, and only
  // this wave's requests of the next step write it (with BM = 64 that part is
  // too small and the block goes to its own area).
  auto store_tile = [&](auto actc, int m0, int n0, uint8_t* stage) __attribute__((always_inline)) {
    constexpr int ACT = decltype(actc)::value;
    constexpr bool GLU = ACT == MXQ_ACT_SWIGLU;
    constexpr int ROWB = GLU ? 64 : 128;  // staged bytes per token row
    constexpr int CPR = ROWB / 16;        // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;         // rows per read-back instruction
    uint8_t* const sb = OWN_STAGING ? lds + kStages * (XSTAGE + WSTAGE) + wave * 4096
                                    : stage + wave * XL * 1024;  // 16-byte aligned
    const int ncol = GLU ? N / 2 : N;                            // output columns
    const int c0 = GLU ? n0 / 2 + wave * 32 : n0 + wave * 64;    // this wave's first
    // lane-derived offsets are recomputed per tile (a few VALU) rather than
    // hoisted out of the tile loop, where they would be live across the steps
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int l32 = ln & 31, g2 = ln >> 5;
    // the lane's 32 bias values as bf16 pairs (features 2j, 2j+1 of its runs);
    // SwiGLU: gate bias [0, N/2), up bias [N/2, N)
    uint32_t bp[2][4][2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int j = 8 * a + 4 * g2 + 2 * h;
          const int n = GLU ? (nb ? ncol : 0) + c0 + j : c0 + nb * 32 + j;
          const int lim = GLU ? (nb ? N : ncol) : N;
          const uint32_t lo = bias && n < lim ? bias[n] : 0u;
          const uint32_t hi = bias && n + 1 < lim ? bias[n + 1] : 0u;
          bp[nb][a][h] = lo | (hi << 16);
        }
    auto bias_at = [&](int nb, int a, int r) __attribute__((always_inline)) {
      const uint32_t w = bp[nb][a][r >> 1];
      return __uint_as_float((r & 1) ? (w & 0xFFFF0000u) : (w << 16));
    };
    // read-back position: row rr = RPI i + lane / CPR, 16-byte chunk lane % CPR
    const int cr = ln % CPR, rr0 = ln / CPR;
    const int n = c0 + 8 * cr;
    const bool vec = n + 8 <= ncol;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if (m0 + mb * 32 < M) {
        if constexpr (GLU) {
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            const f32x16 cg = acc[0][mb], cu = acc[1][mb];
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
              o[r] = act_silu(cg[4 * a + r] + bias_at(0, a, r)) * (cu[4 * a + r] + bias_at(1, a, r));
            const int chunk = a ^ (l32 & 3);
            *reinterpret_cast<v2u*>(sb + l32 * 64 + chunk * 16 + g2 * 8) =
                v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          }
        } else {
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
              const f32x16 c = acc[nb][mb];
              float o[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                o[r] = c[4 * a + r] + bias_at(nb, a, r);
                if constexpr (ACT == MXQ_ACT_GELU_TANH) o[r] = act_gelu_tanh(o[r]);
              }
              const int chunk = (nb * 4 + a) ^ (l32 & 7);
              *reinterpret_cast<v2u*>(sb + l32 * 128 + chunk * 16 + g2 * 8) =
                  v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the block is in LDS
#pragma unroll
        for (int i = 0; i < 32 / RPI; ++i) {
          const int rr = RPI * i + rr0;
          const v4u v =
              *reinterpret_cast<const v4u*>(sb + rr * ROWB + ((cr ^ (rr & (CPR - 1))) * 16));
          const int m = m0 + mb * 32 + rr;
          if (m < M) {
            uint16_t* dst = y + static_cast<int64_t>(m) * ncol + n;
            if (vec && (reinterpret_cast<uintptr_t>(dst) & 3u) == 0) {
              // non-temporal: the output is not read again by this kernel, and all
              // workgroups store their tiles at about the same time, so keeping these
              // lines out of L2 leaves it to the operands of the next tiles
              __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(dst));
            } else {
              const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
              for (int e = 0; e < 8; ++e)
                if (n + e < ncol) dst[e] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[nb][mb] = f32x16{};
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- low-rank update of one tile (LoRA): acc += bt[rows] . xa[tokens]^T over
  // the rank (a multiple of 16), on the MFMAs, into the fp32 accumulators before the
  // epilogue. Operands come straight from global memory (each bt fragment is
  // reused by every 32-token block); rows past N and tokens past M read as zero
  // (vector offsets only, so the range check sees the whole offset).
  // SwiGLU tiles hold gate rows in half 0 and the matching up rows in half 1.
  auto lora_tile = [&](int m0, int n0) __attribute__((always_inline)) {
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int l32 = ln & 31, g2 = ln >> 5;
    const bool glu = act == MXQ_ACT_SWIGLU;
    const int c0 = glu ? n0 / 2 + wave * 32 : n0 + wave * 64;
    const __amdgpu_buffer_rsrc_t br =
        ring::make_rsrc(bt, static_cast<uint32_t>(N) * static_cast<uint32_t>(rank) * 2u);
    const __amdgpu_buffer_rsrc_t ar = ring::make_rsrc(
        xa + static_cast<int64_t>(m0) * rank, static_cast<uint32_t>(min(BM, M - m0)) * rank * 2u);
    int bo[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
      bo[nb] = ((glu ? (nb ? N / 2 : 0) + c0 : c0 + nb * 32) + l32) * rank * 2 + g2 * 16;
    const int ao = l32 * rank * 2 + g2 * 16;
    // chunk c + 16's operands are requested before chunk c's MFMAs (the last chunk is
    // requested twice: harmless), so each wait covers one chunk of MFMAs less latency
    bf16x8 bw[2], av[MB];
    auto fetch = [&](int c, bf16x8 (&b)[2], bf16x8 (&a)[MB]) __attribute__((always_inline)) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        b[nb] = __builtin_bit_cast(
            bf16x8, __builtin_amdgcn_raw_buffer_load_b128(br, bo[nb] + c * 2, 0, 0));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        a[mb] = __builtin_bit_cast(
            bf16x8,
            __builtin_amdgcn_raw_buffer_load_b128(ar, ao + c * 2 + mb * 32 * rank * 2, 0, 0));
    };
    fetch(0, bw, av);
    for (int c = 0; c < rank; c += 16) {
      bf16x8 bn[2], an[MB];
      fetch(min(c + 16, rank - 16), bn, an);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[nb], av[mb], acc[nb][mb], 0,
                                                                0, 0);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) bw[nb] = bn[nb];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) av[mb] = an[mb];
    }
  };

  // One K step g (st = g mod 3; J = g & 1 selects the unpack buffers). FULL
  // steps also read step g+1's record, multiply step g and unpack step g+1;
  // the first two fill steps (g = -3, -2) only request. Requests are spread
  // over the MFMA pairs. Pair q covers K slice sl = q / MB of token block
  // mb = q % MB, so an accumulator is reused 2*MB MFMAs later (not 2).
  auto step = [&](auto Jc, auto fullc, int g, int st) __attribute__((always_inline)) {
    constexpr int J = decltype(Jc)::value;
    constexpr bool FULL = decltype(fullc)::value;
    // this step's requests: activations (none before step 0), weights
    const __amdgpu_buffer_rsrc_t xr = xr_cur, wr = wr_cur;
    const int kx = xs_k, kw = ws_k;
    const bool x_on = g >= -2;
    if (x_on && ++xs_k == nk) {
      if (xs_r + 1 < my_tiles) {
        xs_k = 0;
        xs_t = tile_of(++xs_r);
        xr_cur = x_rsrc(m0_of(xs_t));
      } else {
        xs_k = nk - 1;
      }
    }
    if (++ws_k == nk) {
      if (ws_r + 1 < my_tiles) {
        ws_k = 0;
        ws_t = tile_of(++ws_r);
        wr_cur = w_rsrc(n0_of(ws_t));
      } else {
        ws_k = nk - 1;
      }
    }
    if constexpr (FULL) {
      const uint8_t* xb = xl + st * XSTAGE;
      const uint8_t* wb = wl + (st == 2 ? 0 : st + 1) * WSTAGE + wave * R::BYTES;
      auto fq = [](int q) { return (q % MB) * 4 + q / MB; };  // fragment of pair q
      bf16x8 f[4];
#pragma unroll
      for (int q = 0; q < 3; ++q) f[q] = read_frag(xb, fq(q));
      RawRun<BITS> raw;
      read_raw(wb, raw);
      const float s0 = __uint_as_float(raw.sb[0] << 16);
      const float b0 = __uint_as_float(raw.sb[0] & 0xFFFF0000u);
      const float s1 = __uint_as_float(raw.sb[1] << 16);
      const float b1 = __uint_as_float(raw.sb[1] & 0xFFFF0000u);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) {
#pragma unroll
        for (int i = 0; i < L; ++i)
          if (i * SLOTS / L == q) request(i, st, xr, kx, wr, kw);
        if (q + 3 < SLOTS) f[(q + 3) % 4] = read_frag(xb, fq(q + 3));
        const int mb = q % MB, sl = q / MB;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const bf16x8 wv = __builtin_bit_cast(
              bf16x8, v4u{wu[J][nb][4 * sl], wu[J][nb][4 * sl + 1], wu[J][nb][4 * sl + 2],
                          wu[J][nb][4 * sl + 3]});
          acc[nb][mb] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(wv, f[q % 4], acc[nb][mb], 0, 0, 0);
        }
        // unpack slices start two pairs in, when the record reads have landed
        if (q >= 2) {
#pragma unroll
          for (int d = (q - 2) * 32 / (SLOTS - 2); d < (q - 1) * 32 / (SLOTS - 2); ++d) {
            const int nb = d / 16, i = d % 16;
            const float sc = nb ? s1 : s0, bi = nb ? b1 : b0;
            wu[J ^ 1][nb][i] =
                pack_bf16x2(fmaf(static_cast<float>(code_at<BITS>(raw.w[nb], 2 * i)), sc, bi),
                            fmaf(static_cast<float>(code_at<BITS>(raw.w[nb], 2 * i + 1)), sc, bi));
            // pinned here: otherwise the compiler sinks the unpack into the next
            // step (its only user), doubling that step's VALU work
            asm volatile("" : "+v"(wu[J ^ 1][nb][i]));
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i)
        if (i >= XL || x_on) request(i, st, xr, kx, wr, kw);
    }
    // every request older than this step's own has landed, for all waves
    ring::ring_barrier<L>();
  };
  using J0 = std::integral_constant<int, 0>;
  using J1 = std::integral_constant<int, 1>;
  using Full = std::true_type;
  using Fill = std::false_type;

  ring::ring_barrier<0>();  // stage 2 zeroed by all waves
  // fill: g = -3, -2 request; g = -1 (st = 2, wu[1] = 0) also unpacks step 0
  step(J1{}, Fill{}, -3, 0);
  step(J0{}, Fill{}, -2, 1);
  step(J1{}, Full{}, -1, 2);
  // tiles: the epilogue stays out of the step loop. With an even number of K
  // steps (EVEN) every tile starts on unpack parity 0; otherwise a tile with an
  // odd count leaves the next one starting on the other parity.
  int g = 0, st = 0;
  auto next = [&] __attribute__((always_inline)) {
    ++g;
    st = st == 2 ? 0 : st + 1;
  };
  for (int r = 0; r < my_tiles; ++r) {
    int left = nk;
    if (!EVEN && (g & 1)) {
      step(J1{}, Full{}, g, st);
      next();
      --left;
    }
    for (; left >= 2; left -= 2) {
      step(J0{}, Full{}, g, st);
      next();
      step(J1{}, Full{}, g, st);
      next();
    }
    if (!EVEN && left) {
      step(J0{}, Full{}, g, st);
      next();
    }
    const int64_t t = tile_of(r);
    if constexpr (LORA) lora_tile(m0_of(t), n0_of(t));
    uint8_t* const stage = xl + (st == 0 ? 2 : st - 1) * XSTAGE;
    if (act == MXQ_ACT_GELU_TANH)
      store_tile(std::integral_constant<int, MXQ_ACT_GELU_TANH>{}, m0_of(t), n0_of(t), stage);
    else if (act == MXQ_ACT_SWIGLU)
      store_tile(std::integral_constant<int, MXQ_ACT_SWIGLU>{}, m0_of(t), n0_of(t), stage);
    else
      store_tile(std::integral_constant<int, MXQ_ACT_NONE>{}, m0_of(t), n0_of(t), stage);
  }
  // the last steps' requests (repeats of the last step) must land before the
  // workgroup's LDS is released
  ring::wait_vmcnt<0>();
}

inline int cu_count() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    return n;
  }();
  return cus;
}

// Low-rank update operands (xa == nullptr: none): xa [M, R], bt [N, R] bf16.
struct Lora {
  const uint16_t* xa;
  const uint16_t* bt;
  int R;
};

// One workgroup per CU (rounded to whole XCD sets), never more than the tiles.
inline int persistent_blocks(int tiles) { return ring::grid_blocks(min(tiles, cu_count())); }

template <int BITS, int BM, int GP>
hipError_t run_tiled(const uint16_t* x, int M, int K, const void* tw, int N,
                     const uint16_t* bias, int act, const Lora& lo, uint16_t* y,
                     hipStream_t s) {
  const int m_tiles = (M + BM - 1) / BM, n_tiles = (N + kRows - 1) / kRows;
  const int blocks = persistent_blocks(m_tiles * n_tiles);
  const uint8_t* w = static_cast<const uint8_t*>(tw);
  const bool even = (K >> 6) % 2 == 0;
#define MXQ_LAUNCH(E, L)                                                \
  qmm_tiled_kernel<BITS, BM, GP, E, L><<<blocks, kThreads, 0, s>>>(     \
      x, w, bias, y, M, N, K, m_tiles, n_tiles, act, lo.xa, lo.bt, lo.R)
  if (lo.xa) {
    if (even) MXQ_LAUNCH(true, true); else MXQ_LAUNCH(false, true);
  } else {
    if (even) MXQ_LAUNCH(true, false); else MXQ_LAUNCH(false, false);
  }
#undef MXQ_LAUNCH
  return hipGetLastError();
}

// Time of one 32-, 64- or 128-token tile relative to a 256-token tile (same K,
// same 256 features): the weight loads and unpacking do not shrink with the tile,
// and a short step is bound by the ring's latency (K = 4096, N = 16384, 6-bit:
// 48.7 us for 32 tokens in 32-row tiles, 50.4 us for 64 tokens in 32-row tiles and
// 52.9 us in 64-row tiles, against 1.52 ms for 14 rounds of 256-row tiles).
constexpr double kTileCost32 = 0.45, kTileCost64 = 0.6, kTileCost128 = 0.75;

// Token tiles of 32, 64, 128 or 256 rows, chosen by estimated time: rounds of
// tiles over the CUs times the relative cost of one tile. Small problems (few
// 256-row tiles, e.g. M = 256 with N = 2048: 8 tiles for 256 CUs) take the
// smaller tiles, which spread the same work over more CUs. When M % 256
// leaves a remainder of at most 128 rows and the full tiles alone fill whole
// rounds better, the remainder runs as a second launch with smaller tiles
// instead of as a last round of mostly empty 256-row tiles. Every tile height
// accumulates each output in the same order, so the choice never changes a
// result bit.
template <int BITS, int GP>
hipError_t run_rows(int bm, const uint16_t* x, int M, int K, const void* tw, int N,
                    const uint16_t* bias, int act, const Lora& lo, uint16_t* y, hipStream_t s) {
  switch (bm) {
    case 32: return run_tiled<BITS, 32, GP>(x, M, K, tw, N, bias, act, lo, y, s);
    case 64: return run_tiled<BITS, 64, GP>(x, M, K, tw, N, bias, act, lo, y, s);
    case 128: return run_tiled<BITS, 128, GP>(x, M, K, tw, N, bias, act, lo, y, s);
    default: return run_tiled<BITS, 256, GP>(x, M, K, tw, N, bias, act, lo, y, s);
  }
}

template <int BITS, int GP>
hipError_t pick_rows(const uint16_t* x, int M, int K, const void* tw, int N,
                     const uint16_t* bias, int act, const Lora& lo, uint16_t* y,
                     hipStream_t s) {
  const int64_t cus = cu_count(), n_tiles = (N + kRows - 1) / kRows;
  auto rounds = [&](int64_t tiles) { return static_cast<double>((tiles + cus - 1) / cus); };
  const int heights[4] = {32, 64, 128, 256};
  const double costs[4] = {kTileCost32, kTileCost64, kTileCost128, 1.0};
  // one launch of the best height for `rows` tokens: (estimated time, height)
  auto best = [&](int64_t rows, int max_bm, int& bm_out) {
    double t_best = 0;
    bm_out = 0;
    for (int h = 0; h < 4 && heights[h] <= max_bm; ++h) {
      const double t = rounds((rows + heights[h] - 1) / heights[h] * n_tiles) * costs[h];
      if (bm_out == 0 || t < t_best) {
        t_best = t;
        bm_out = heights[h];
      }
    }
    return t_best;
  };
  int bm = 0;
  const double t_one = best(M, 256, bm);
  const int full = M / 256, rem = M % 256;
  if (full > 0 && rem > 0 && rem <= 128) {
    int bm_rem = 0;
    const double t_two = rounds(static_cast<int64_t>(full) * n_tiles) + best(rem, 128, bm_rem);
    if (t_two < t_one) {
      const hipError_t e = run_rows<BITS, GP>(256, x, full * 256, K, tw, N, bias, act, lo, y, s);
      if (e != hipSuccess) return e;
      const int64_t r0 = static_cast<int64_t>(full) * 256;
      const int64_t ldy = act == MXQ_ACT_SWIGLU ? N / 2 : N;
      const Lora rl{lo.xa ? lo.xa + r0 * lo.R : nullptr, lo.bt, lo.R};
      return run_rows<BITS, GP>(bm_rem, x + r0 * K, rem, K, tw, N, bias, act, rl, y + r0 * ldy,
                                s);
    }
  }
  return run_rows<BITS, GP>(bm, x, M, K, tw, N, bias, act, lo, y, s);
}

template <int BITS>
hipError_t pick_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                      const uint16_t* bias, int act, const Lora& lo, uint16_t* y,
                      hipStream_t s) {
  if (gs == 32) return pick_rows<BITS, 2>(x, M, K, tw, N, bias, act, lo, y, s);
  return pick_rows<BITS, 1>(x, M, K, tw, N, bias, act, lo, y, s);
}

}  // namespace


// The entry point of one code width, compiled in its own translation unit
// (mxq_qmm_tiled_b<BITS>.hip) so the widths build in parallel.
namespace detail {
#define MXQ_TILED_CAT2(a, b) a##b
#define MXQ_TILED_CAT(a, b) MXQ_TILED_CAT2(a, b)
hipError_t MXQ_TILED_CAT(launch_qmm_tiled_b, MXQ_TILED_BITS)(
    const uint16_t* x, int M, int K, const void* tw, int N, int gs, const uint16_t* bias,
    int act, const uint16_t* xa, const uint16_t* bt, int R, uint16_t* y, hipStream_t s) {
  const Lora lo{xa && R > 0 ? xa : nullptr, bt, R};
  return pick_tiled<MXQ_TILED_BITS>(x, M, K, tw, N, gs, bias, act, lo, y, s);
}
}  // namespace detail
}  // namespace mxq
