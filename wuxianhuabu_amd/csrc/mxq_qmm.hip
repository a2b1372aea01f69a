// mxq_qmm.hip — large-M quantized matmul on gfx950 bf16 MFMA:
//   y[m, n] = sum_k x[m, k] * (s[n, k/gs] * q[n, k] + b[n, k/gs])  (+ bias[n])
//
// Replaces mlx's qmm path behind quantizedMM(x, w, scales:, biases:,
// transpose: true, ...) for the DiT projections and MLP GEMMs
// (`model/minimax h3/H3Common.swift:358-359`, called from
// `model/minimax h3/H3Transformer.swift:448, 580, 622, 627`, and MLXNN
// QuantizedLinear in `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:177-188, 387-388`).
//
// Work decomposition (one workgroup = 4 waves = 256 threads, one per SIMD):
//   * the workgroup owns a BM x 256 output tile (BM tokens x 256 features);
//   * each wave owns BM x 64: it loads the packed codes of its 64 feature rows
//     with buffer loads (one 32-code run per lane per 32-row block), unpacks
//     them in registers to bf16 (w = q*s + b in fp32, then round) and keeps
//     them as MFMA operands for the whole K step;
//   * the BM x 64 activation tile of each K step is staged once through LDS
//     (double-buffered) and read by all four waves;
//   * v_mfma_f32_32x32x16_bf16 with the weights as the A operand and the
//     activations as the B operand; each lane's 16 accumulators hold one token
//     and four runs of 4 consecutive output features (8-byte stores).
// K is consumed 64 codes at a time. Inside one 64-wide step, lane half
// g2 = lane/32 owns codes [32*g2, 32*g2+32) of its row for both the weight and
// the activation fragments, so each lane unpacks one contiguous 32-code run
// (BITS whole words, for every supported width) and reads 64 contiguous
// activation bytes. The loop is software-pipelined: packed weights for step
// k+2 are loaded and step k+1 is unpacked while step k's MFMAs run.
#include <type_traits>

#include "mxq_device.hpp"
#include "mxq_internal.hpp"
#include "mxq_ring.hpp"

namespace mxq {
namespace {

constexpr int kBN = 256;       // output features per workgroup
constexpr int kKS = 64;        // K step
constexpr int kXPitch = 72;    // LDS row pitch in bf16 (64 + 8 padding)
constexpr int kThreads = 256;
constexpr int kGroupM = 4;     // token tiles swept together per XCD

typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t v3u __attribute__((ext_vector_type(3)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Raw buffer loads: 64-bit base in the (wave-uniform) descriptor, a per-lane
// 32-bit byte offset computed once, and the K-step advance as a scalar offset.
template <int NW>
__device__ __forceinline__ void buf_load_words(__amdgpu_buffer_rsrc_t r, int voff, int soff,
                                               uint32_t (&w)[NW]) {
  if constexpr (NW == 2) {
    const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (NW == 3) {
    const v3u v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z;
  } else if constexpr (NW == 4) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (NW == 5) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    w[4] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 16, soff, 0);
  } else if constexpr (NW == 6) {
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    const v2u u = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 16, soff, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w; w[4] = u.x; w[5] = u.y;
  } else {
    static_assert(NW == 8, "unsupported run");
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    const v4u u = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    w[4] = u.x; w[5] = u.y; w[6] = u.z; w[7] = u.w;
  }
}

using ring::make_rsrc;
using ring::ring_barrier;
using ring::swz;
using ring::wait_vmcnt;

// 32 codes -> four MFMA operands of 8 bf16 (w = q*s + b, fp32 then RNE).
template <int BITS>
__device__ __forceinline__ void unpack32(const uint32_t (&w)[BITS], float s, float b,
                                         bf16x8 (&f)[4]) {
  uint32_t q[32];
  decode_codes<BITS, 32, BITS>(w, q);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      p[i] = pack_bf16x2(fmaf(static_cast<float>(q[8 * j + 2 * i]), s, b),
                         fmaf(static_cast<float>(q[8 * j + 2 * i + 1]), s, b));
    const v4u v = {p[0], p[1], p[2], p[3]};
    f[j] = __builtin_bit_cast(bf16x8, v);
  }
}

// Packed weights of one K step as loaded: 2 row blocks x one 32-code run, plus
// the raw bf16 scale and bias bits (converted only when unpacked).
template <int BITS>
struct RawW {
  uint32_t w[2][BITS];
  uint32_t s[2], b[2];
};

template <int BITS, int BM, bool KTAIL>
__global__ __launch_bounds__(kThreads, 1) void qmm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int gs_log2, int m_tiles, int n_tiles) {
  constexpr int MB = BM / 32;       // 32-token blocks per wave
  constexpr int XL = BM / 32;       // 16-byte activation loads per thread per K step
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * kXPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g2 = lane >> 5;

  int m_tile, n_tile;
  if (!ring::tile_coords<kGroupM>(m_tiles, n_tiles, m_tile, n_tile)) return;
  const int m0 = m_tile * BM, n0 = n_tile * kBN;

  const int WB = K / 32 * BITS * 4;  // packed row bytes
  const int G = K >> gs_log2;
  const int nk = (K + kKS - 1) / kKS;
  const int rows_m = min(BM, M - m0), rows_n = min(kBN, N - n0);

  // descriptors rebased at the tile so all offsets fit in 32 bits
  const __amdgpu_buffer_rsrc_t xrs =
      make_rsrc(x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(rows_m) * K * 2);
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(reinterpret_cast<const char*>(wq) + static_cast<int64_t>(n0) * WB,
                static_cast<uint32_t>(rows_n) * WB);
  const __amdgpu_buffer_rsrc_t srs =
      make_rsrc(scales + static_cast<int64_t>(n0) * G, static_cast<uint32_t>(rows_n) * G * 2);
  const __amdgpu_buffer_rsrc_t brs =
      make_rsrc(biases + static_cast<int64_t>(n0) * G, static_cast<uint32_t>(rows_n) * G * 2);

  // per-lane byte offsets (rows clamped into the tile: every access is in range)
  int wvo[2], svo[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int r = min(wave * 64 + nb * 32 + l32, rows_n - 1);
    wvo[nb] = r * WB + g2 * BITS * 4;
    svo[nb] = r * G * 2 + ((32 * g2) >> gs_log2) * 2;
  }
  const int xc = (tid & 7) * 8;  // activation column staged by this thread
  int xvo[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) xvo[i] = (min((tid >> 3) + 32 * i, rows_m - 1) * K + xc) * 2;

  f32x16 acc[2][MB];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x16{};

  u32x4 xr[XL];

  auto load_w = [&](int kk, RawW<BITS>& r) {
    int so = kk * (8 * BITS);                   // 2 runs of BITS words per step
    int ss = ((kk * kKS) >> gs_log2) * 2;
    if constexpr (KTAIL) {
      // a half step at the end: lanes past K re-read the previous run (in range)
      const bool past = kk * kKS + 32 * g2 >= K;
      so -= past ? 4 * BITS : 0;
      ss -= past ? (((32 * g2) >> gs_log2) * 2) : 0;
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      buf_load_words<BITS>(wrs, wvo[nb] + (KTAIL ? so : 0), KTAIL ? 0 : so, r.w[nb]);
      r.s[nb] = __builtin_amdgcn_raw_buffer_load_b16(srs, svo[nb] + (KTAIL ? ss : 0),
                                                     KTAIL ? 0 : ss, 0);
      r.b[nb] = __builtin_amdgcn_raw_buffer_load_b16(brs, svo[nb] + (KTAIL ? ss : 0),
                                                     KTAIL ? 0 : ss, 0);
    }
  };
  auto load_x = [&](int kk) {
    if constexpr (!KTAIL) {
#pragma unroll
      for (int i = 0; i < XL; ++i)
        xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              xrs, xvo[i], kk * kKS * 2, 0));
    } else {
      const int col = min(kk * kKS, K - 8 - xc) * 2;
#pragma unroll
      for (int i = 0; i < XL; ++i)
        xr[i] = __builtin_bit_cast(u32x4,
                                   __builtin_amdgcn_raw_buffer_load_b128(xrs, xvo[i] + col, 0, 0));
    }
  };
  auto store_x = [&](int buf, int kk) {
    const bool ok = !KTAIL || (kk * kKS + xc < K);
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      u32x4 v = xr[i];
      if (KTAIL && !ok) v = u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4a*>(&xs[buf][((tid >> 3) + 32 * i) * kXPitch + xc]) = v;
    }
  };
  auto dequant = [&](int kk, const RawW<BITS>& r, bf16x8 (&wf)[2][4]) {
    const bool ok = !KTAIL || (kk * kKS + 32 * g2 < K);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float s = __uint_as_float(r.s[nb] << 16), b = __uint_as_float(r.b[nb] << 16);
      if (KTAIL && !ok) {
        s = 0.f;
        b = 0.f;
      }
      unpack32<BITS>(r.w[nb], s, b, wf[nb]);
    }
  };
  // One K step: MFMAs of step kk (operands wf + LDS buffer kk&1) with the
  // unpacking of step kk+1 (raw `cur`) interleaved; the loads of step kk+2
  // go out first, into `nxt`.
  auto step = [&](int kk, const bf16x8 (&wf)[2][4], bf16x8 (&wn)[2][4], const RawW<BITS>& cur,
                  RawW<BITS>& nxt) {
    load_w(min(kk + 2, nk - 1), nxt);
    dequant(min(kk + 1, nk - 1), cur, wn);
    const uint16_t* xb = xs[kk & 1] + l32 * kXPitch + 32 * g2;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) {
        const bf16x8 xv = *reinterpret_cast<const bf16x8*>(xb + mb * 32 * kXPitch + 8 * sl);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[nb][sl], xv, acc[nb][mb], 0, 0, 0);
      }
    }
    // schedule: weight loads first, then per 32-token block four LDS reads
    // and 8 MFMAs, each MFMA followed by up to four VALU (the unpacking)
    __builtin_amdgcn_sched_group_barrier(0x020, 2 * ((BITS + 3) / 4) + 4, 0);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
    }
    store_x((kk + 1) & 1, kk + 1);
    load_x(min(kk + 2, nk - 1));
    __syncthreads();
  };

  // ---- prologue: step 0 staged and unpacked, step 1 in flight ----
  RawW<BITS> ra, rb;
  bf16x8 wa[2][4], wb[2][4];
  load_w(0, ra);
  load_x(0);
  store_x(0, 0);
  dequant(0, ra, wa);
  load_w(min(1, nk - 1), ra);
  load_x(min(1, nk - 1));
  __syncthreads();

  // ---- main loop, unrolled by two so the register roles swap without copies ----
  int kk = 0;
  for (; kk + 1 < nk; kk += 2) {
    step(kk, wa, wb, ra, rb);
    step(kk + 1, wb, wa, rb, ra);
  }
  if (kk < nk) step(kk, wa, wb, ra, rb);

  // ---- epilogue: lane holds y[m, n + 8a + 4*g2 + r] (a, r = 0..3) for one token m ----
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int n = n0 + wave * 64 + nb * 32 + 8 * a + 4 * g2;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bv[r] = n + r < N ? bf16_to_f32(bias[n + r]) : 0.f;
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = m0 + mb * 32 + l32;
        if (m >= M) continue;
        uint16_t* dst = y + static_cast<int64_t>(m) * N + n;
        const f32x16 c = acc[nb][mb];
        const float v0 = c[4 * a] + bv[0], v1 = c[4 * a + 1] + bv[1];
        const float v2 = c[4 * a + 2] + bv[2], v3 = c[4 * a + 3] + bv[3];
        if (n + 3 < N && ((reinterpret_cast<uintptr_t>(dst) & 3u) == 0)) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
        } else {
          const float v[4] = {v0, v1, v2, v3};
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) dst[r] = f32_to_bf16(v[r]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Ring-pipelined variant for K % 64 == 0 (every DiT projection shape).
//
// Latency is hidden by distance, since each SIMD runs a single wave:
//   * activations go HBM -> LDS directly (buffer_load_dwordx4 ... lds, no
//     VGPRs) into a 4-stage ring; step k+3 is requested while step k computes;
//   * packed weights go HBM -> VGPRs into a 4-slot ring; step k+3 is requested
//     while step k+1 is unpacked under step k's MFMAs;
//   * the LDS fragments of 32-token block b+1 are read while block b's MFMAs
//     issue.
// LDS rows are 128 B (64 bf16) with the 16-byte chunks XOR-swizzled by
// swz(r) = (r & 7) ^ ((r >> 3) & 1), so both the fragment reads (32 rows, same
// logical chunk) and the staging writes are bank-conflict free.
// ---------------------------------------------------------------------------
constexpr int kXStages = 4;
constexpr int kWSlots = 4;

template <int BITS>
struct RunLoads {  // VMEM instructions per 32-code run load
  static constexpr int value = BITS == 5 || BITS == 6 || BITS == 8 ? 2 : 1;
};

template <int BITS, int BM>
__global__ __launch_bounds__(kThreads, 1) void qmm_ring_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int M, int N, int K, int gs_log2, int m_tiles, int n_tiles) {
  constexpr int MB = BM / 32;            // 32-token blocks per wave
  constexpr int XL = BM / 32;            // LDS-direct loads per wave per K step (8 rows each)
  constexpr int STAGE = BM * 64;         // bf16 elements per LDS stage
  // weight VMEM instructions per K step per lane
  constexpr int WLOADS = 2 * (RunLoads<BITS>::value + 2);
  constexpr int LOADS_PER_STEP = WLOADS + XL;
  __shared__ __attribute__((aligned(16))) uint16_t xs[kXStages * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g2 = lane >> 5;

  int m_tile, n_tile;
  if (!ring::tile_coords<kGroupM>(m_tiles, n_tiles, m_tile, n_tile)) return;
  const int m0 = m_tile * BM, n0 = n_tile * kBN;

  const int WB = K / 32 * BITS * 4;  // packed row bytes
  const int G = K >> gs_log2;
  const int nk = K / kKS;
  const int rows_m = min(BM, M - m0), rows_n = min(kBN, N - n0);

  const __amdgpu_buffer_rsrc_t xrs =
      make_rsrc(x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(rows_m) * K * 2);
  // weights: the MLX rows of this tile (all offsets per lane fixed; the K
  // step is a scalar offset)
  __amdgpu_buffer_rsrc_t wrs, srs, brs;
  int wvo[2], svo[2];
  {
    wrs = make_rsrc(reinterpret_cast<const char*>(wq) + static_cast<int64_t>(n0) * WB,
                    static_cast<uint32_t>(rows_n) * WB);
    srs = make_rsrc(scales + static_cast<int64_t>(n0) * G, static_cast<uint32_t>(rows_n) * G * 2);
    brs = make_rsrc(biases + static_cast<int64_t>(n0) * G, static_cast<uint32_t>(rows_n) * G * 2);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int r = min(wave * 64 + nb * 32 + l32, rows_n - 1);
      wvo[nb] = r * WB + g2 * BITS * 4;
      svo[nb] = r * G * 2 + ((32 * g2) >> gs_log2) * 2;
    }
  }
  // staging: instruction i of this wave fills LDS rows (wave*XL + i)*8 .. +8;
  // lane t writes physical chunk t%8 of row +t/8 with logical chunk ^ swz(row)
  int xvo[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int r = (wave * XL + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ swz(r);
    xvo[i] = (min(r, rows_m - 1) * K + 8 * c) * 2;
  }
  // fragment reads: row mb*32 + l32, logical chunk 4*g2 + sl
  int xro[4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) xro[sl] = l32 * 128 + (((4 * g2 + sl) ^ swz(l32)) * 16);

  f32x16 acc[2][MB];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x16{};

  // The issue order of every load is pinned (sched_barrier after each): the
  // compiler derives its vmcnt waits from program order, and a prologue whose
  // loads were reordered relative to the loop body would make those waits, which
  // are the minimum over both paths, far stricter than the ring needs.
  auto load_w = [&](int kk, RawW<BITS>& r) {
    {
      const int so = kk * (8 * BITS);
      const int ss = ((kk * kKS) >> gs_log2) * 2;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        buf_load_words<BITS>(wrs, wvo[nb], so, r.w[nb]);
        __builtin_amdgcn_sched_barrier(0);
        r.s[nb] = __builtin_amdgcn_raw_buffer_load_b16(srs, svo[nb], ss, 0);
        __builtin_amdgcn_sched_barrier(0);
        r.b[nb] = __builtin_amdgcn_raw_buffer_load_b16(brs, svo[nb], ss, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // scale and bias of row block nb from the raw bf16 bits
  auto scale_bias = [&](const RawW<BITS>& r, int nb, float& sc, float& bi) {
    sc = __uint_as_float(r.s[nb] << 16);
    bi = __uint_as_float(r.b[nb] << 16);
  };
  auto load_x = [&](int kk, int stage) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      uint16_t* dst = xs + stage * STAGE + (wave * XL + i) * 512;
      ring::lds_load<16>(xrs, dst, xvo[i], kk * kKS * 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto read_frags = [&](int stage, int mb, bf16x8 (&f)[4]) {
    const char* base = reinterpret_cast<const char*>(xs + stage * STAGE) + mb * 32 * 128;
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) f[sl] = *reinterpret_cast<const bf16x8*>(base + xro[sl]);
  };

  RawW<BITS> rw[kWSlots];
#pragma unroll
  for (int i = 0; i < kWSlots; ++i) rw[i] = RawW<BITS>{};
  uint32_t wu[2][2][16];  // unpacked bf16 pairs: [buffer][row block][dword]
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int k = 0; k < 16; ++k) wu[i][j][k] = 0u;
  // the pipeline's third fill step multiplies stage 2 by wu[0]: both start at
  // exact zeros, so that step adds +0 to every accumulator whatever the inputs
  {
    u32x4a* st2 = reinterpret_cast<u32x4a*>(xs + 2 * STAGE);
#pragma unroll
    for (int i = tid; i < STAGE / 8; i += kThreads) st2[i] = u32x4a{0u, 0u, 0u, 0u};
  }

  // unpack dwords [d0, d1) of raw slot r into wu buffer b
  // (the bounds are constants once the callers' loops are unrolled)
  auto unpack = [&](const RawW<BITS>& r, uint32_t (&dst)[2][16], float s0, float b0, float s1,
                    float b1, int d0, int d1) {
#pragma unroll
    for (int d = d0; d < d1; ++d) {
      const int nb = d / 16, i = d % 16;
      const float sc = nb ? s1 : s0, bi = nb ? b1 : b0;
      dst[nb][i] = pack_bf16x2(fmaf(static_cast<float>(code_at<BITS>(r.w[nb], 2 * i)), sc, bi),
                               fmaf(static_cast<float>(code_at<BITS>(r.w[nb], 2 * i + 1)), sc, bi));
    }
  };

  // One K step. J = (kk + 3) mod 4 picks the register/LDS slots at compile
  // time. Step kk requests step kk+3's weights and activations, unpacks step
  // kk+1's weights (requested two steps earlier) and multiplies step kk's.
  // Source order is the schedule (sched_barrier fences keep it): per 32-token
  // block, the next block's LDS reads, then four pairs of MFMAs each followed by
  // one 2-code slice of the unpacking. The pipeline fill (kk = -3, -2, -1) runs
  // this same code, so the compiler's vmcnt waits and the ring barrier's count
  // follow one fixed issue order: steps -3 and -2 only request; step -1 also
  // unpacks step 0 and multiplies the zeroed stage 2 by the zeroed wu[0].
  auto step = [&](auto Jc, int kk) {
    constexpr int J = decltype(Jc)::value;
    constexpr int XS = J % kXStages;        // stage holding step kk
    constexpr int F = J % 2, FN = (J + 1) % 2;
    const RawW<BITS>& nr = rw[(J + 1) % kWSlots];
    // requests for step kk+3 (clamped at the end: a repeated request is
    // harmless and keeps every step's request count equal)
    const int kl = min(kk + 3, nk - 1);
    load_w(kl, rw[(J + 3) % kWSlots]);
    load_x(kl, (J + 3) % kXStages);
    float s0, b0, s1, b1;
    scale_bias(nr, 0, s0, b0);
    scale_bias(nr, 1, s1, b1);
    if (kk >= -1) {
      bf16x8 xa[4], xb[4];
      read_frags(XS, 0, xa);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        bf16x8 (&cur)[4] = (mb & 1) ? xb : xa;
        bf16x8 (&nxt)[4] = (mb & 1) ? xa : xb;
        if (mb + 1 < MB) read_frags(XS, mb + 1, nxt);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const bf16x8 wv = __builtin_bit_cast(
                bf16x8, v4u{wu[F][nb][4 * sl], wu[F][nb][4 * sl + 1], wu[F][nb][4 * sl + 2],
                            wu[F][nb][4 * sl + 3]});
            acc[nb][mb] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(wv, cur[sl], acc[nb][mb], 0, 0, 0);
          }
          // slices: (MB * 4) slots cover the 32 dwords of the next step's operands
          constexpr int SLOTS = MB * 4;
          unpack(nr, wu[FN], s0, b0, s1, b1, (mb * 4 + sl) * 32 / SLOTS,
                 (mb * 4 + sl + 1) * 32 / SLOTS);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // step kk+1's stage was requested in step kk-2: wait for this wave's part
    // of it (the requests of steps kk-1 and kk may stay in flight), then publish
    ring_barrier<2 * LOADS_PER_STEP>();
  };

  // stage 2 zeroed by every wave before anyone multiplies it
  ring_barrier<0>();
  for (int kk = -3;;) {
    step(std::integral_constant<int, 0>{}, kk);
    if (++kk >= nk) break;
    step(std::integral_constant<int, 1>{}, kk);
    if (++kk >= nk) break;
    step(std::integral_constant<int, 2>{}, kk);
    if (++kk >= nk) break;
    step(std::integral_constant<int, 3>{}, kk);
    if (++kk >= nk) break;
  }
  // no LDS-direct load may still be in flight when the workgroup's LDS is
  // released (the last steps' requests repeat step nk-1 and are never read)
  wait_vmcnt<0>();

  // ---- epilogue: lane holds y[m, n + 8a + 4*g2 + r] (a, r = 0..3) for one token m ----
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int n = n0 + wave * 64 + nb * 32 + 8 * a + 4 * g2;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bv[r] = n + r < N ? bf16_to_f32(bias[n + r]) : 0.f;
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = m0 + mb * 32 + l32;
        if (m >= M) continue;
        uint16_t* dst = y + static_cast<int64_t>(m) * N + n;
        const f32x16 c = acc[nb][mb];
        const float v0 = c[4 * a] + bv[0], v1 = c[4 * a + 1] + bv[1];
        const float v2 = c[4 * a + 2] + bv[2], v3 = c[4 * a + 3] + bv[3];
        if (n + 3 < N && ((reinterpret_cast<uintptr_t>(dst) & 3u) == 0)) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
        } else {
          const float v[4] = {v0, v1, v2, v3};
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) dst[r] = f32_to_bf16(v[r]);
        }
      }
    }
  }
}

// Launch geometry shared by both kernels.
struct Grid {
  int m_tiles, n_tiles, blocks, gs_log2;
};

inline Grid grid_for(int M, int N, int BM, int gs) {
  Grid g;
  g.m_tiles = (M + BM - 1) / BM;
  g.n_tiles = (N + kBN - 1) / kBN;
  g.blocks = ring::grid_blocks(g.m_tiles * g.n_tiles);
  g.gs_log2 = gs == 32 ? 5 : (gs == 64 ? 6 : 7);
  return g;
}

template <int BITS, int BM>
hipError_t run_ring(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                    const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                    hipStream_t s) {
  const Grid g = grid_for(M, N, BM, gs);
  qmm_ring_kernel<BITS, BM><<<g.blocks, kThreads, 0, s>>>(x, wq, sc, bi, bias, y, M, N, K,
                                                          g.gs_log2, g.m_tiles, g.n_tiles);
  return hipGetLastError();
}

template <int BITS, int BM>
hipError_t run_step(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                    const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                    hipStream_t s) {
  const Grid g = grid_for(M, N, BM, gs);
  if (K % kKS == 0)
    qmm_kernel<BITS, BM, false><<<g.blocks, kThreads, 0, s>>>(x, wq, sc, bi, bias, y, M, N, K,
                                                              g.gs_log2, g.m_tiles, g.n_tiles);
  else
    qmm_kernel<BITS, BM, true><<<g.blocks, kThreads, 0, s>>>(x, wq, sc, bi, bias, y, M, N, K,
                                                             g.gs_log2, g.m_tiles, g.n_tiles);
  return hipGetLastError();
}

// K a multiple of 64 (every DiT projection) and more than 64 tokens: ring
// kernel with 256- or 128-token tiles. Otherwise (a half step at the end of K,
// or few tokens): the two-deep kernel with tiles of at most 128 tokens.
template <int BITS>
hipError_t pick_bm(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                   const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                   hipStream_t s) {
  if (K % kKS == 0 && M > 64) {
    if (M <= 128) return run_ring<BITS, 128>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
    return run_ring<BITS, 256>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  }
  if (M <= 64) return run_step<BITS, 64>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  return run_step<BITS, 128>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
}

}  // namespace

namespace detail {

bool qmm_supports_bits(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

hipError_t launch_qmm(const uint16_t* x, int M, int K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int N, int gs, int bits,
                      const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (bits) {
    case 2: return pick_bm<2>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 3: return pick_bm<3>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 5: return pick_bm<5>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 4: return pick_bm<4>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 6: return pick_bm<6>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 8: return pick_bm<8>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace detail
}  // namespace mxq
