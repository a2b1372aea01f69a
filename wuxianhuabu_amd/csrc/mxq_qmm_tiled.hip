// mxq_qmm_tiled.hip — large-M quantized matmul over the tiled weight layout:
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
#include <type_traits>

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

template <int BITS>
struct RawRun {  // one lane's two 32-code runs and their scale/bias dwords
  uint32_t w[2][BITS];
  uint32_t sb[2];
};

template <int BITS, int BM, int GP>
__global__ __launch_bounds__(kThreads, 1) void qmm_tiled_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ tw,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int m_tiles, int n_tiles) {
  using R = Rec<BITS, GP>;
  constexpr int MB = BM / 32;          // 32-token blocks per wave
  constexpr int XL = BM / 32;          // activation requests per wave per step (8 rows each)
  constexpr int XSTAGE = BM * 128;     // bytes per activation stage
  constexpr int WSTAGE = 4 * R::BYTES; // bytes per weight stage
  constexpr int L = XL + R::LOADS;     // requests per wave per step
  constexpr int SLOTS = MB * 4;        // MFMA pairs per step
  static_assert(L <= SLOTS, "one request per MFMA pair at most");
  static_assert(kStages * (XSTAGE + WSTAGE) <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kStages * (XSTAGE + WSTAGE)];
  uint8_t* const xl = lds;
  uint8_t* const wl = lds + kStages * XSTAGE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g2 = lane >> 5;

  int m_tile, n_tile;
  if (!ring::tile_coords<kGroupM>(m_tiles, n_tiles, m_tile, n_tile)) return;
  const int m0 = m_tile * BM, n0 = n_tile * kRows;
  const int nk = K >> 6;
  const int rows_m = min(BM, M - m0);

  const __amdgpu_buffer_rsrc_t xrs =
      ring::make_rsrc(x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(rows_m) * K * 2);
  // this wave's row block (clamped: a block past N computes rows never stored)
  const int rb = min((n0 >> 6) + wave, (N + 63) / 64 - 1);
  const __amdgpu_buffer_rsrc_t wrs = ring::make_rsrc(
      tw + static_cast<int64_t>(rb) * nk * R::BYTES, static_cast<uint32_t>(nk) * R::BYTES);

  // activation request i of this wave fills stage rows (wave*XL + i)*8 .. +8:
  // lane t writes physical chunk t%8 of row +t/8, i.e. logical chunk
  // (t%8) ^ swz(row); rows past the tile repeat its last row
  int xvo[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int r = (wave * XL + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ring::swz(r);
    xvo[i] = (min(r, rows_m - 1) * K + 8 * c) * 2;
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
  // The third fill step (kk = -1) multiplies activation stage 2 by wu[0]; both
  // hold exact zeros then, so that step adds +0 whatever the inputs.
  {
    v4u* z = reinterpret_cast<v4u*>(xl + 2 * XSTAGE);
#pragma unroll
    for (int i = tid; i < XSTAGE / 16; i += kThreads) z[i] = v4u{0u, 0u, 0u, 0u};
  }

  // request i of step kk (activations of step kk+2 first, needed a step
  // sooner, then this wave's weight record of step kk+3); st = kk mod 3
  auto request = [&](int i, int kk, int st) {
    if (i < XL) {
      const int kx = min(kk + 2, nk - 1);
      const int stage = st == 0 ? 2 : st - 1;  // (kk + 2) mod 3
      ring::lds_load<16>(xrs, xl + stage * XSTAGE + (wave * XL + i) * 1024, xvo[i], kx * 128);
    } else {
      const int j = i - XL;
      const int kw = min(kk + 3, nk - 1);
      const uint8_t* dst = wl + st * WSTAGE + wave * R::BYTES;  // (kk + 3) mod 3
      if (j < R::CHUNKS) {
        ring::lds_load<16>(wrs, dst + j * 1024, lane * 16, kw * R::BYTES + j * 1024);
      } else {
        const int off = R::CHUNKS * 1024 + (j - R::CHUNKS) * 256;
        ring::lds_load<4>(wrs, dst + off, lane * 4, kw * R::BYTES + off);
      }
    }
  };
  auto read_frag = [&](const uint8_t* stage, int q) {
    return *reinterpret_cast<const bf16x8*>(stage + (q / 4) * 4096 + xro[q % 4]);
  };
  // this lane's two runs of one record, from LDS
  auto read_raw = [&](const uint8_t* rec, RawRun<BITS>& r) {
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

  // One K step; J = parity of kk + 3 selects the unpack buffers, st = kk mod 3
  // the ring stages. Fill steps (kk = -3, -2) only request; from kk = -1 on the
  // step also reads step kk+1's record, multiplies step kk and unpacks kk+1.
  auto step = [&](auto Jc, int kk, int st) {
    constexpr int J = decltype(Jc)::value;
    if (kk >= -1) {
      const uint8_t* xb = xl + st * XSTAGE;
      const uint8_t* wb = wl + (st == 2 ? 0 : st + 1) * WSTAGE + wave * R::BYTES;
      bf16x8 f[4];
#pragma unroll
      for (int q = 0; q < 3; ++q) f[q] = read_frag(xb, q);
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
          if (i * SLOTS / L == q) request(i, kk, st);
        if (q + 3 < SLOTS) f[(q + 3) % 4] = read_frag(xb, q + 3);
        const int mb = q / 4, sl = q % 4;
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
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i)
        if (i >= XL || kk >= -2) request(i, kk, st);  // no activations of step -1
    }
    // every request older than this step's own has landed, for all waves
    ring::ring_barrier<L>();
  };

  ring::ring_barrier<0>();  // stage 2 zeroed by all waves
  for (int kk = -3, st = 0;;) {
    step(std::integral_constant<int, 0>{}, kk, st);
    if (++kk >= nk) break;
    st = st == 2 ? 0 : st + 1;
    step(std::integral_constant<int, 1>{}, kk, st);
    if (++kk >= nk) break;
    st = st == 2 ? 0 : st + 1;
  }
  // the last steps' requests (repeats of step nk-1) must land before the
  // workgroup's LDS is released
  ring::wait_vmcnt<0>();

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

template <int BITS, int BM, int GP>
hipError_t run_tiled(const uint16_t* x, int M, int K, const void* tw, int N,
                     const uint16_t* bias, uint16_t* y, hipStream_t s) {
  const int m_tiles = (M + BM - 1) / BM, n_tiles = (N + kRows - 1) / kRows;
  qmm_tiled_kernel<BITS, BM, GP><<<ring::grid_blocks(m_tiles * n_tiles), kThreads, 0, s>>>(
      x, static_cast<const uint8_t*>(tw), bias, y, M, N, K, m_tiles, n_tiles);
  return hipGetLastError();
}

template <int BITS>
hipError_t pick_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                      const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (gs == 32) {
    if (M <= 128) return run_tiled<BITS, 128, 2>(x, M, K, tw, N, bias, y, s);
    return run_tiled<BITS, 256, 2>(x, M, K, tw, N, bias, y, s);
  }
  if (M <= 128) return run_tiled<BITS, 128, 1>(x, M, K, tw, N, bias, y, s);
  return run_tiled<BITS, 256, 1>(x, M, K, tw, N, bias, y, s);
}

}  // namespace

namespace detail {

hipError_t launch_qmm_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                            int bits, const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (bits) {
    case 2: return pick_tiled<2>(x, M, K, tw, N, gs, bias, y, s);
    case 3: return pick_tiled<3>(x, M, K, tw, N, gs, bias, y, s);
    case 4: return pick_tiled<4>(x, M, K, tw, N, gs, bias, y, s);
    case 5: return pick_tiled<5>(x, M, K, tw, N, gs, bias, y, s);
    case 6: return pick_tiled<6>(x, M, K, tw, N, gs, bias, y, s);
    case 8: return pick_tiled<8>(x, M, K, tw, N, gs, bias, y, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace detail
}  // namespace mxq
