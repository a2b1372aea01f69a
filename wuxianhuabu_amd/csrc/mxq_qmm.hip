// mxq_qmm.hip — large-M quantized matmul on gfx950 bf16 MFMA:
//   y[m, n] = sum_k x[m, k] * (s[n, k/gs] * q[n, k] + b[n, k/gs])  (+ bias[n])
//
// Replaces mlx's qmm path behind quantizedMM(x, w, scales:, biases:,
// transpose: true, ...) for the DiT projections and MLP GEMMs
// (`model/minimax h3/H3Common.swift:358-359`, called from
// `model/minimax h3/H3Transformer.swift:448, 580, 622, 627`, and MLXNN
// QuantizedLinear in `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:177-188, 387-388`).
//
// Work decomposition (one workgroup = 4 waves = 256 threads):
//   * the workgroup owns a BM x 256 output tile (BM tokens x 256 features);
//   * each wave owns BM x 64: it loads the packed codes of its 64 feature rows
//     straight from HBM (one 16-code chunk per lane per 16-row block), unpacks
//     them in registers to bf16 (w = q*s + b in fp32, then round) and keeps
//     them as MFMA operands for the whole K step;
//   * the BM x 64 activation tile of each K step is staged once through LDS
//     (double-buffered) and read by all four waves;
//   * v_mfma_f32_16x16x32_bf16 with the weights as the A operand and the
//     activations as the B operand, so each lane's accumulator holds 4
//     consecutive output features of one token (8-byte stores).
// K is consumed 64 codes at a time. Inside one 64-wide step, lane group
// g4 = lane/16 owns codes [16*g4, 16*g4+16) of its row for both the weight and
// the activation fragments, so each lane unpacks one contiguous 16-code run
// (BITS/2 whole words) and reads 32 contiguous activation bytes.
#include "mxq_device.hpp"
#include "mxq_internal.hpp"

namespace mxq {
namespace {

constexpr int kBN = 256;       // output features per workgroup
constexpr int kKS = 64;        // K step
constexpr int kXPitch = 72;    // LDS row pitch in bf16 (64 + 8 padding)
constexpr int kThreads = 256;

template <int NW>
__device__ __forceinline__ void load_chunk(const uint32_t* p, uint32_t (&w)[NW]) {
  if constexpr (NW == 1) {
    w[0] = p[0];
  } else if constexpr (NW == 2) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (NW == 3) {
    const u32x3 v = *reinterpret_cast<const u32x3*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z;
  } else {
    static_assert(NW == 4, "unsupported chunk");
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  }
}

// 16 codes -> two MFMA operands of 8 bf16 each (w = q*s + b, fp32 then RNE).
template <int BITS, int NW>
__device__ __forceinline__ void unpack16(const uint32_t (&w)[NW], float s, float b,
                                         bf16x8& lo, bf16x8& hi) {
  uint32_t q[16];
  decode_codes<BITS, 16, NW>(w, q);
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    p[i] = pack_bf16x2(fmaf(static_cast<float>(q[2 * i]), s, b),
                       fmaf(static_cast<float>(q[2 * i + 1]), s, b));
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v a = {p[0], p[1], p[2], p[3]};
  const u32x4v c = {p[4], p[5], p[6], p[7]};
  lo = __builtin_bit_cast(bf16x8, a);
  hi = __builtin_bit_cast(bf16x8, c);
}

template <int BITS, int BM>
__global__ __launch_bounds__(kThreads, 1) void qmm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K, int gs,
    int m_tiles, int n_tiles) {
  constexpr int NW = BITS / 2;      // words per 16-code run
  constexpr int MB = BM / 16;       // 16-token blocks per wave
  constexpr int XL = BM / 32;       // 16-byte activation loads per thread per K step
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * kXPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;

  // ---- tile order: XCD-contiguous ranges, then groups of 8 token tiles ----
  const int tiles = m_tiles * n_tiles;
  int bid = blockIdx.x;
  const int nblk = gridDim.x;  // padded to a multiple of 8 by the launcher
  bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  if (bid >= tiles) return;
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * n_tiles;
  const int first_m = (bid / per_group) * GROUP_M;
  const int gsize = min(m_tiles - first_m, GROUP_M);
  const int in_group = bid % per_group;
  const int m_tile = first_m + in_group % gsize;
  const int n_tile = in_group / gsize;
  const int m0 = m_tile * BM, n0 = n_tile * kBN;

  const int64_t W = static_cast<int64_t>(K) * BITS / 32;
  const int G = K / gs;
  const int nk = (K + kKS - 1) / kKS;

  const uint32_t* wrow[4];
  const uint16_t* srow[4];
  const uint16_t* brow[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int n = min(n0 + wave * 64 + nb * 16 + l16, N - 1);
    wrow[nb] = wq + n * W;
    srow[nb] = scales + static_cast<int64_t>(n) * G;
    brow[nb] = biases + static_cast<int64_t>(n) * G;
  }
  const int xc = (tid & 7) * 8;  // activation column handled by this thread
  const uint16_t* xrow[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int m = min(m0 + (tid >> 3) + 32 * i, M - 1);
    xrow[i] = x + static_cast<int64_t>(m) * K + xc;
  }

  f32x4 acc[4][MB];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 xr[XL];
  uint32_t wr[4][NW];
  float sr[4], br[4];

  auto load_x = [&](int kk) {
    const int k0 = kk * kKS;
    const bool ok = k0 + xc < K;
#pragma unroll
    for (int i = 0; i < XL; ++i)
      xr[i] = ok ? *reinterpret_cast<const u32x4*>(xrow[i] + k0) : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XL; ++i)
      *reinterpret_cast<u32x4a*>(&xs[buf][((tid >> 3) + 32 * i) * kXPitch + xc]) = xr[i];
  };
  auto load_w = [&](int kk) {
    const int kc = kk * kKS + 16 * g4;
    const bool ok = kc < K;
    const int g = ok ? kc / gs : 0;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      if (ok) {
        load_chunk<NW>(wrow[nb] + (kc / 16) * NW, wr[nb]);
        sr[nb] = bf16_to_f32(srow[nb][g]);
        br[nb] = bf16_to_f32(brow[nb][g]);
      } else {
#pragma unroll
        for (int j = 0; j < NW; ++j) wr[nb][j] = 0u;
        sr[nb] = 0.f;
        br[nb] = 0.f;
      }
    }
  };

  load_x(0);
  load_w(0);
  store_x(0);
  __syncthreads();

  for (int kk = 0; kk < nk; ++kk) {
    bf16x8 wf[4][2];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) unpack16<BITS, NW>(wr[nb], sr[nb], br[nb], wf[nb][0], wf[nb][1]);

    const bool more = kk + 1 < nk;
    if (more) {
      load_x(kk + 1);
      load_w(kk + 1);
    }

    const uint16_t* xb = xs[kk & 1] + l16 * kXPitch + 16 * g4;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const bf16x8 x0 = *reinterpret_cast<const bf16x8*>(xb + mb * 16 * kXPitch);
      const bf16x8 x1 = *reinterpret_cast<const bf16x8*>(xb + mb * 16 * kXPitch + 8);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[nb][0], x0, acc[nb][mb], 0, 0, 0);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[nb][1], x1, acc[nb][mb], 0, 0, 0);
    }

    if (more) store_x((kk + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds y[m, n..n+3] for one token m ----
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int n = n0 + wave * 64 + nb * 16 + 4 * g4;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bv[r] = n + r < N ? bf16_to_f32(bias[n + r]) : 0.f;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = m0 + mb * 16 + l16;
      if (m >= M) continue;
      uint16_t* dst = y + static_cast<int64_t>(m) * N + n;
      const f32x4 a = acc[nb][mb];
      if (n + 3 < N && ((reinterpret_cast<uintptr_t>(dst) & 3u) == 0)) {
        const uint32_t lo = pack_bf16x2(a[0] + bv[0], a[1] + bv[1]);
        const uint32_t hi = pack_bf16x2(a[2] + bv[2], a[3] + bv[3]);
        *reinterpret_cast<u32x2*>(dst) = u32x2{lo, hi};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) dst[r] = f32_to_bf16(a[r] + bv[r]);
      }
    }
  }
}

template <int BITS, int BM>
hipError_t run_qmm(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                   const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                   hipStream_t s) {
  const int m_tiles = (M + BM - 1) / BM;
  const int n_tiles = (N + kBN - 1) / kBN;
  const int tiles = m_tiles * n_tiles;
  const int grid = (tiles + 7) / 8 * 8;
  qmm_kernel<BITS, BM><<<grid, kThreads, 0, s>>>(x, wq, sc, bi, bias, y, M, N, K, gs, m_tiles,
                                                 n_tiles);
  return hipGetLastError();
}

template <int BITS>
hipError_t pick_bm(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                   const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                   hipStream_t s) {
  if (M <= 64) return run_qmm<BITS, 64>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  if (M <= 128) return run_qmm<BITS, 128>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  return run_qmm<BITS, 256>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
}

}  // namespace

namespace detail {

bool qmm_supports_bits(int bits) { return bits == 2 || bits == 4 || bits == 6 || bits == 8; }

hipError_t launch_qmm(const uint16_t* x, int M, int K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int N, int gs, int bits,
                      const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (bits) {
    case 2: return pick_bm<2>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 4: return pick_bm<4>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 6: return pick_bm<6>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 8: return pick_bm<8>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace detail
}  // namespace mxq
