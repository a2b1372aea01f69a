// mxq_qmv_impl.hpp — small-M quantized matmul (GEMV), y = x * W^T (+ bias): the kernels,
// compiled once per code width (mxq_qmv_b{2,3,4,5,6,8}.hip); mxq_qmv.hip dispatches.
//
// Replaces mlx's qmv path behind quantizedMM for M <= 8: the H3 adaLN /
// timestep-modulation projection (M = number of unique timesteps,
// `model/minimax h3/H3Transformer.swift:389-402, 957-988`) and the Gemma-4
// tied-embedding logits (M = 1, N = 262144,
// `model/3模块/ltx2.5专属/gemma4文本-(ltx专属).swift:306-312`).
//
// HBM-bound: every packed weight byte is read once. Two kernels:
//   * qmv_tiled_kernel (below): one workgroup per 32-row half of a 64-row block,
//     64-code K steps, the dot products on the matrix cores. It reads the tiled
//     layout, or (MLX = true) the MLX layout in place when K % 64 == 0;
//   * qmv_kernel (this section): the MLX layout for any K (K an odd multiple of
//     32 included), with coalesced loads (consecutive lanes read consecutive
//     16-code chunks of a row) and no MFMA.
// qmv_kernel splits K: the K dimension of each row is spread over the 64 lanes
// of a wave (and, when N is small, over the 4 waves of a block); partial sums
// meet in wavefront shuffles and, across waves, in LDS.
//
// Per 16-code chunk the affine form is factored:
//   sum_k x_k (s q_k + b) = s * sum_k x_k q_k + b * sum_k x_k
// so each weight costs one decode and MT fused multiply-adds.
#pragma once

#include <type_traits>

#include "mxq_device.hpp"
#include "mxq_internal.hpp"
#include "mxq_ring.hpp"
#include "mxq_tiled.hpp"

namespace mxq {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// Codes per chunk: 16, or 32 for the widths whose 16 codes do not fill whole
// words (3 and 5 bits). A chunk never straddles a group (group size >= 32).
template <int BITS>
struct Chunk {
  static constexpr int codes = (BITS == 3 || BITS == 5) ? 32 : 16;
  static constexpr int words = codes * BITS / 32;
};

template <int NW>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t (&w)[NW]) {
  if constexpr (NW == 1) {
    w[0] = p[0];
  } else if constexpr (NW == 2) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (NW == 3) {
    const u32x3 v = *reinterpret_cast<const u32x3*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z;
  } else if constexpr (NW == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
#pragma unroll
    for (int i = 4; i < NW; ++i) w[i] = p[i];
  }
}

// MT: rows of x handled per launch row-block (1, 2, 4 or 8); R: weight rows per
// wave; KSPLIT: waves of a block sharing the same R rows (1 or 4).
template <int BITS, int MT, int R, int KSPLIT>
__global__ __launch_bounds__(kThreads) void qmv_kernel(
    const uint16_t* __restrict__ x, int M, int K, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases, int N, int gs,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y) {
  constexpr int CC = Chunk<BITS>::codes, CW = Chunk<BITS>::words;
  constexpr int HALVES = CC / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rows_per_block = R * (kWaves / KSPLIT);
  const int n0 = blockIdx.x * rows_per_block + (KSPLIT == 1 ? wave : 0) * R;
  const int m0 = blockIdx.y * MT;
  const int mcount = min(MT, M - m0);
  const int64_t W = static_cast<int64_t>(K) * BITS / 32;
  const int G = K / gs;
  const int nchunks = K / CC;

  const uint32_t* wrow[R];
  const uint16_t* srow[R];
  const uint16_t* brow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(n0 + r, N - 1);
    wrow[r] = wq + n * W;
    srow[r] = scales + static_cast<int64_t>(n) * G;
    brow[r] = biases + static_cast<int64_t>(n) * G;
  }
  const uint16_t* xrow[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) xrow[m] = x + static_cast<int64_t>(m0 + min(m, mcount - 1)) * K;

  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

  const int cstep = 64 * KSPLIT;
  for (int c = lane + 64 * (KSPLIT == 1 ? 0 : wave); c < nchunks; c += cstep) {
    const int k0 = c * CC;
    uint32_t words[R][CW];
    float sc[R], bi[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      load_words<CW>(wrow[r] + static_cast<int64_t>(c) * CW, words[r]);
      sc[r] = bf16_to_f32(srow[r][k0 / gs]);
      bi[r] = bf16_to_f32(brow[r][k0 / gs]);
    }
    float dot[R][MT], xs[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      xs[m] = 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) dot[r][m] = 0.0f;
    }
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      // 16 activations per row of x, as 8 dwords of bf16 pairs
      uint32_t xv[MT][8];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const u32x4* p = reinterpret_cast<const u32x4*>(xrow[m] + k0 + 16 * h);
        const u32x4 a = p[0], b = p[1];
        xv[m][0] = a.x; xv[m][1] = a.y; xv[m][2] = a.z; xv[m][3] = a.w;
        xv[m][4] = b.x; xv[m][5] = b.y; xv[m][6] = b.z; xv[m][7] = b.w;
      }
      float xf[MT][16];
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xf[m][2 * i] = __uint_as_float(xv[m][i] << 16);
          xf[m][2 * i + 1] = __uint_as_float(xv[m][i] & 0xFFFF0000u);
          xs[m] += xf[m][2 * i] + xf[m][2 * i + 1];
        }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint32_t q[CC];
        decode_codes<BITS, CC, CW>(words[r], q);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float qf = static_cast<float>(q[16 * h + i]);
#pragma unroll
          for (int m = 0; m < MT; ++m) dot[r][m] = fmaf(xf[m][i], qf, dot[r][m]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r][m] = fmaf(sc[r], dot[r][m], fmaf(bi[r], xs[m], acc[r][m]));
  }

  // wave reduction: afterwards every lane holds every total
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = wave_sum(acc[r][m]);

  if constexpr (KSPLIT > 1) {
    __shared__ float part[KSPLIT][R * MT];
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) part[wave][r * MT + m] = acc[r][m];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < KSPLIT; ++w) t += part[w][r * MT + m];
        acc[r][m] = t;
      }
  }

  // lane j writes output j = r*MT + m
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (lane == r * MT + m) {
        const int n = n0 + r;
        if (n < N && m < mcount) {
          float v = acc[r][m];
          if (bias) v += bf16_to_f32(bias[n]);
          y[static_cast<int64_t>(m0 + m) * N + n] = f32_to_bf16(v);
        }
      }
    }
}

template <int BITS, int MT, int R, int KSPLIT>
hipError_t run_qmv(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                   const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                   hipStream_t s) {
  const int rows_per_block = R * (kWaves / KSPLIT);
  dim3 grid((N + rows_per_block - 1) / rows_per_block, (M + MT - 1) / MT);
  qmv_kernel<BITS, MT, R, KSPLIT><<<grid, kThreads, 0, s>>>(x, M, K, wq, sc, bi, N, gs, bias, y);
  return hipGetLastError();
}

template <int BITS, int MT>
hipError_t pick_split(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                      const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                      hipStream_t s) {
  constexpr int R = MT >= 4 ? 4 : 8;
  // Enough waves to cover every CU several times over without splitting K
  // across waves; otherwise split each row's K range over the 4 waves.
  const int64_t waves = (static_cast<int64_t>(N) + R - 1) / R;
  if (waves >= 2048) return run_qmv<BITS, MT, R, 1>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  return run_qmv<BITS, MT, R, 4>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
}

template <int BITS>
hipError_t pick_mt(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                   const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                   hipStream_t s) {
  if (M <= 1) return pick_split<BITS, 1>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  if (M <= 2) return pick_split<BITS, 2>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  if (M <= 4) return pick_split<BITS, 4>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  return pick_split<BITS, 8>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
}

// ---------------------------------------------------------------------------
// GEMV on the tiled layout (mxq_tiled.hpp). HBM-bound, so the design goal is
// bytes in flight with as little VALU work per byte as possible: one
// workgroup of a few waves per 32-row record half; the waves take the K steps
// in chunks of 4, round robin. Each
// wave works in batches of up to SPW steps, with two register sets: while
// batch b computes, every load of batch b+1 (its activation slice, MT rows x
// SPW steps x 128 B, and its weight units) is in flight. Computing a batch
// writes its activation slice to the wave's own LDS region (no other wave
// reads it: no barrier), sums each activation half-run once, and consumes the
// records.
// Per step a lane owns one unit (row l32 of the half, code half g2): 32 codes
// from a coalesced 16-byte plane plus remainder words.
//
// Codes become bf16 pairs without float arithmetic: 0x4300 | q is the bf16
// value 128 + q for q < 128. The dot products run on the matrix cores: per
// step, four v_mfma_f32_32x32x16_bf16 with the activations as A (rows = tokens,
// zero past M) and the code pairs as B (columns = the 32 rows of the half).
// Operand lane l supplies K slots 8*(l/32) .. +7 of MFMA c; both operands map
// slot (g2, c, j) to code 32*g2 + 8c + j of the step, so the MFMA sums the
// step's 64 codes. Lane (l32, g2) then holds tokens 4*g2 .. 4*g2+3 of row l32:
//   sum_k x_k (s q_k + b) = s * sum_k x_k (128 + q_k) + (b - 128 s) * sum_k x_k.
// 8-bit codes (up to 255) are converted exactly instead, with offset 0.
// ---------------------------------------------------------------------------
// Cache policy of the tiled weight loads: non-temporal, since each weight byte is read
// once (M = 2, K = 4096, N = 24576, 6-bit: 16.3 against 17.5 us; the Gemma logits
// shape 95.9 against 106.3 us). The MLX-layout form keeps the default: its batches
// split a row's 128-byte lines, and the next batch reads the rest of a line from L2
// (25.6 us; 38.1 with non-temporal loads). The activations, which every workgroup
// reads, keep the default too.
constexpr int kTiledWeightAux = 2;
// K steps per chunk of the waves' round-robin split. Against one contiguous K quarter
// per wave (6-bit, same box): K = 4096, N = 24576, tiled 14.82 -> 14.58 us at M = 2
// (15.9 -> 14.8 at M = 3), MLX layout 21.5 -> 20.3 us; K = 21504, N = 5376, M = 1, MLX
// layout 31.9 -> 28.0 us; 8 and 16 tokens within 1 %.
constexpr int kQmvChunk = 4;
typedef uint32_t v2u_t __attribute__((ext_vector_type(2)));
typedef uint32_t v3u_t __attribute__((ext_vector_type(3)));
typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), c, false);
}

// NH record halves (32 rows each) per workgroup of WPB waves; batches of SPW
// steps per wave; MT <= 32 tokens (one pass; larger M runs ceil(M / MT) passes).
//
// MLX: the same kernel over the MLX layout itself (wq [N, K*BITS/32], scales and
// biases [N, K/gs], K % 64 == 0), for callers that keep no tiled copy. A wave
// loads a batch's bytes of its 32 rows (SPW * 8 * BITS contiguous bytes per row)
// with consecutive lanes on consecutive 16-byte chunks, stages them in its own
// LDS region, and lane (l32, g2) reads back the BITS words of codes
// [64k + 32 g2, +32) of its row l32 (a run of 32 codes is BITS whole words);
// it loads that row's scale and bias of step k's group(s) itself. Everything
// else is shared. gshift = log2(gs / 64) for gs >= 64. With batches of 2 or 4 steps, a
// lane loads its row's scales (and biases) of the whole batch at once: a dword-aligned
// window holding the batch's groups (12 bytes for 4 steps, 16 for 4 steps at gs = 32,
// 8 for 2 steps), split where used. A row's scales for all of K lie in one or two
// 128-byte lines, which one 2-byte load per step asked L2 for once per step.
template <int BITS, int MT, int GP, int NH, int WPB, int SPW, bool MLX>
__global__ __launch_bounds__(64 * WPB) void qmv_tiled_kernel(
    const uint16_t* __restrict__ x, int M, int K, const uint8_t* __restrict__ tw, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
    const uint32_t* __restrict__ wq, const uint16_t* __restrict__ scs,
    const uint16_t* __restrict__ bis, int gshift) {
  static_assert(MT <= 32, "the MFMA output has 32 token rows");
  constexpr int FP = tiled::full_planes(BITS), RW = tiled::rem_words(BITS);
  constexpr int RB = tiled::code_bytes(BITS) + 256 * GP;      // record bytes
  // activation bytes per wave, a whole number of 1 KiB pieces (64 lanes x
  // 16 B each): the padding of small MT x SPW receives repeats of valid rows
  constexpr int XW = (MT * SPW * 128 + 1023) / 1024 * 1024;
  constexpr int XLOADS = XW / 1024;                           // 16-byte loads per lane per batch
  constexpr int NSUM = MT * SPW * 2;                          // half-run sums per batch
  // output registers per lane that hold tokens: register k of lane (l32, g2) is token
  // tok(k, g2) = 8 (k / 4) + 4 g2 + k % 4 of the MFMA's 32 rows
  constexpr int RPL = MT < 4 ? MT : MT <= 8 ? 4 : MT / 2;
  static_assert(NH * 32 * MT * 4 <= XW, "partials reuse the activation region");
  __shared__ __attribute__((aligned(16))) uint8_t lds[WPB * XW];
  __shared__ __attribute__((aligned(16))) uint8_t zero_chunk[WPB][SPW * 128];
  __shared__ float xsum_all[WPB][NSUM];
  // MLX layout: a batch's weight bytes of the wave's rows (CPR 16-byte chunks of each
  // row, loaded with consecutive lanes on consecutive chunks), staged row by row at a
  // padded stride and read back as each lane's runs
  constexpr int CPR = SPW * BITS / 2;          // 16-byte chunks of a row per batch
  constexpr int NCL = 32 * CPR / 64;           // coalesced 16-byte loads per lane per half
  constexpr int RSTR = CPR * 16 + 16;          // staged row stride
  static_assert(!MLX || (SPW * BITS) % 4 == 0, "whole loads of 64 lanes per batch");
  // MLX: batches of 2 or 4 steps load their scales and biases as whole windows
  constexpr bool kWin = MLX && (SPW == 2 || SPW == 4);
  __shared__ __attribute__((aligned(16))) uint8_t wl_all[WPB][MLX ? NH * 32 * RSTR : 16];

  // Naming an AGPR keeps the MFMA results in AGPRs. A kernel that names none may
  // be given VGPR-form MFMAs, and with 8-wave workgroups the compiler then wrote
  // some MFMA results over their own A or B operand registers, which gave
  // timing-dependent wrong sums.
  asm volatile("" ::: "a0");
  constexpr int kWeightAux = MLX ? 0 : kTiledWeightAux;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, g2 = lane >> 5;
  auto tok = [&](int k) { return 8 * (k >> 2) + 4 * g2 + (k & 3); };
  const int rb = NH == 2 ? blockIdx.x : blockIdx.x >> 1;     // record row block
  const int h0 = NH == 2 ? 0 : (blockIdx.x & 1);             // first half of this workgroup
  const int m0 = blockIdx.y * MT;
  const int mcount = min(MT, M - m0);
  const int nk = K >> 6;
  uint8_t* const xw = lds + wave * XW;
  float* const xsum = xsum_all[wave];

  const __amdgpu_buffer_rsrc_t xrs = ring::make_rsrc(
      x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(mcount) * K * 2);
  // weight (and, MLX layout, scale and bias) sources of this workgroup's rows;
  // the lane parts of the offsets stay in the vector offset, which the buffer
  // range check covers
  __amdgpu_buffer_rsrc_t wrs, srs, brs;
  int wvo[NH], rvo[NH], svo[NH];
  // MLX: piece i of half nb; lane l loads chunk q % CPR of row q / CPR (q = 64 i + l)
  // of the batch: cro = its row's offset, cco = the chunk's, clo = where it is staged
  // packed as (row within the half) | (chunk << 8), unpacked where used
  int tcq[MLX ? NCL : 1];
  int rows = 0, rowb = 0, step_bytes = 0;
  // MLX, one group per step or fewer: the block's last scale and bias (halfword s_last).
  // When rows * G is odd it shares its dword with the two bytes past the descriptor's
  // end, and the range check returns that whole dword as zero to the window loads; it is
  // loaded once on its own and used in place of the window's value.
  int s_last = -1;
  uint32_t s_tail = 0, b_tail = 0;
  if constexpr (MLX) {
    rowb = K / 8 * BITS;                                // bytes per weight row
    const int G = GP == 2 ? K >> 5 : K >> (6 + gshift);  // groups per row
    const int r0 = rb * 64;
    rows = min(64, N - r0);
    wrs = ring::make_rsrc(wq + static_cast<int64_t>(r0) * (rowb / 4),
                          static_cast<uint32_t>(rows) * rowb);
    srs = ring::make_rsrc(scs + static_cast<int64_t>(r0) * G, static_cast<uint32_t>(rows) * G * 2);
    brs = ring::make_rsrc(bis + static_cast<int64_t>(r0) * G, static_cast<uint32_t>(rows) * G * 2);
    if constexpr (GP == 1 && kWin) {
      s_last = rows * G - 1;
      s_tail = __builtin_amdgcn_raw_buffer_load_b16(srs, s_last * 2, 0, 0);
      b_tail = __builtin_amdgcn_raw_buffer_load_b16(brs, s_last * 2, 0, 0);
    }
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) {
      const int r = min((h0 + nb) * 32 + l32, rows - 1);  // rows past N repeat the last one
      wvo[nb] = r * rowb + g2 * BITS * 4;
      rvo[nb] = wvo[nb] + FP * 16;
      svo[nb] = r * G * 2;
    }
#pragma unroll
    for (int i = 0; i < NCL; ++i) {
      const int q = 64 * i + lane;
      tcq[i] = (q / CPR) | ((q % CPR) << 8);
    }
  } else {
    // from the row block's step-0 record to the end of the layout (step-major records)
    const int rbs = (N + 63) >> 6;
    wrs = ring::make_rsrc(tw + static_cast<int64_t>(rb) * RB,
                          static_cast<uint32_t>(nk * rbs - rb) * RB);
    step_bytes = rbs * RB;
    srs = brs = wrs;
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) {
      const int h = h0 + nb;
      wvo[nb] = h * tiled::half_bytes(BITS) + lane * 16;
      rvo[nb] = h * tiled::half_bytes(BITS) + FP * 1024 + lane * 4 * RW;
      svo[nb] = tiled::code_bytes(BITS) + (h * 32 + l32) * GP * 4;  // both groups if GP == 2
    }
  }
  // A operand rows: token l32 of the batch's activations, zeros past MT. With
  // two groups per step (GP == 2) each code half gets its own MFMA set, whose A
  // is zero in the other half's K slots.
  {
    v4u_t* z = reinterpret_cast<v4u_t*>(zero_chunk[wave]);
    for (int i = lane; i < SPW * 8; i += 64) z[i] = v4u_t{0u, 0u, 0u, 0u};
  }
  const uint8_t* xa[GP];
#pragma unroll
  for (int e = 0; e < GP; ++e)
    xa[e] = (l32 < MT && (GP == 1 || g2 == e) ? xw + l32 * (SPW * 128) : zero_chunk[wave]) +
            g2 * 64;

  // The waves take the K steps in chunks of kQmvChunk, round robin: wave w sums chunks
  // w, w + WPB, w + 2 WPB, ... in step order, whatever its batch size, so both layouts
  // (1-step batches tiled, 2 or 4 steps over the MLX layout) give the same bits. At any
  // time a workgroup's waves read neighbouring chunks of its rows.
  static_assert(kQmvChunk % SPW == 0, "batches tile the chunks");
  const int k_begin = wave * kQmvChunk, k_end = nk;
  // the batch after the one at b0: the next SPW steps of its chunk, else the wave's next chunk
  auto next_batch = [&](int b) {
    const int n = b + SPW;
    return n % kQmvChunk == 0 ? n + kQmvChunk * (WPB - 1) : n;
  };
  // pair_at's constants, in VGPRs
  uint32_t kPairMask = ((1u << BITS) - 1u) * 0x10001u, kMagic = 0x43004300u;
  asm volatile("" : "+v"(kPairMask), "+v"(kMagic));

  float acc[NH][RPL];
#pragma unroll
  for (int nb = 0; nb < NH; ++nb)
#pragma unroll
    for (int r = 0; r < RPL; ++r) acc[nb][r] = 0.f;

  // One batch of loads, into registers (the compiler waits for each register
  // where it is first used): the activations of steps b0 .. b0+SPW-1 (clamped;
  // rows past M repeat a valid row, whose sums are never stored), 16 bytes per
  // lane per 1 KiB piece, and every weight unit of the batch (clamped: repeats
  // are never used). Piece i, lane byte o = i*1024 + lane*16 holds row
  // o / (SPW*128), step (o / 128) % SPW, 16-byte chunk (o / 16) % 8.
  // lane part of the activation offsets of a whole batch (row, step within the
  // batch, chunk); the batch's first step comes in as the scalar offset
  int xvo[XLOADS];
#pragma unroll
  for (int i = 0; i < XLOADS; ++i) {
    const int o = i * 1024 + lane * 16;
    xvo[i] = (min(o / (SPW * 128), mcount - 1) * K + ((o / 128) % SPW) * 64) * 2 +
             ((o / 16) % 8) * 16;
  }
  // sb: tiled, the unit's scale (low half) and bias (high half) dword per group;
  // MLX, sb[..][0] the scale(s) and sb[..][GP - 1] the bias(es) as loaded (GP == 2:
  // both groups' values in one dword; GP == 1: one value, zero-extended). They
  // are split where used, so the loads stay in flight until then.
  struct Batch {
    v4u_t x[XLOADS];
    uint32_t w[MLX ? 1 : SPW][NH][BITS];     // tiled: each step's unit words
    v4u_t wc[MLX ? NH : 1][MLX ? NCL : 1];   // MLX: the batch's row chunks
    uint32_t sb[SPW][NH][MLX ? 2 : GP];
  };
  auto load = [&](Batch& B, int b0) __attribute__((always_inline)) {
    if (b0 + SPW <= k_end) {  // whole batch: the step offset is uniform (soffset)
#pragma unroll
      for (int i = 0; i < XLOADS; ++i)
        B.x[i] = __builtin_amdgcn_raw_buffer_load_b128(
            xrs, xvo[i], __builtin_amdgcn_readfirstlane(b0 * 128), 0);
    } else {
#pragma unroll
      for (int i = 0; i < XLOADS; ++i) {
        const int o = i * 1024 + lane * 16;
        const int m = min(o / (SPW * 128), mcount - 1);
        const int st = min(b0 + (o / 128) % SPW, k_end - 1);
        B.x[i] = __builtin_amdgcn_raw_buffer_load_b128(
            xrs, (m * K + st * 64) * 2 + ((o / 16) % 8) * 16, 0, 0);
      }
    }
    if constexpr (MLX) {
      // the batch's bytes of each row. Chunks past a row's end hold the next row's
      // bytes or, past the last row, zeros (the whole offset is in the vector offset,
      // which the buffer range check covers); they are staged where steps past K
      // would be, and never used.
      const int sb0 = __builtin_amdgcn_readfirstlane(b0 * 8 * BITS);
#pragma unroll
      for (int i = 0; i < NCL; ++i) {
        int tc = tcq[i];
        asm volatile("" : "+v"(tc));  // unpacked here, not held across the loop
#pragma unroll
        for (int nb = 0; nb < NH; ++nb)
          B.wc[nb][i] = __builtin_amdgcn_raw_buffer_load_b128(
              wrs, min((h0 + nb) * 32 + (tc & 0xFF), rows - 1) * rowb + sb0 + (tc >> 8) * 16, 0,
              kWeightAux);
      }
    }
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      // uniform, kept in an SGPR (a VGPR soffset would become a readfirstlane loop)
      const int kj = min(b0 + j, k_end - 1);
      const int so = __builtin_amdgcn_readfirstlane(MLX ? kj * 8 * BITS : kj * step_bytes);
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) {
        if constexpr (!MLX) {
#pragma unroll
          for (int p = 0; p < FP; ++p) {
            const v4u_t v =
                __builtin_amdgcn_raw_buffer_load_b128(wrs, wvo[nb] + p * 1024, so, kWeightAux);
            B.w[j][nb][4 * p] = v.x; B.w[j][nb][4 * p + 1] = v.y;
            B.w[j][nb][4 * p + 2] = v.z; B.w[j][nb][4 * p + 3] = v.w;
          }
          if constexpr (RW == 1) {
            B.w[j][nb][4 * FP] = __builtin_amdgcn_raw_buffer_load_b32(wrs, rvo[nb], so, kWeightAux);
          } else if constexpr (RW == 2) {
            const v2u_t v = __builtin_amdgcn_raw_buffer_load_b64(wrs, rvo[nb], so, kWeightAux);
            B.w[j][nb][4 * FP] = v.x; B.w[j][nb][4 * FP + 1] = v.y;
          } else if constexpr (RW == 3) {
            const v3u_t v = __builtin_amdgcn_raw_buffer_load_b96(wrs, rvo[nb], so, kWeightAux);
            B.w[j][nb][4 * FP] = v.x; B.w[j][nb][4 * FP + 1] = v.y;
            B.w[j][nb][4 * FP + 2] = v.z;
          }
        }
        if constexpr (MLX) {
          if constexpr (kWin) {
            // whole-batch windows, below
          } else if constexpr (GP == 2) {  // groups 2k and 2k + 1
            const int ss = __builtin_amdgcn_readfirstlane(kj * 4);
            B.sb[j][nb][0] = __builtin_amdgcn_raw_buffer_load_b32(srs, svo[nb], ss, kWeightAux);
            B.sb[j][nb][1] = __builtin_amdgcn_raw_buffer_load_b32(brs, svo[nb], ss, kWeightAux);
          } else {                  // group k >> gshift
            const int ss = __builtin_amdgcn_readfirstlane((kj >> gshift) * 2);
            B.sb[j][nb][0] = __builtin_amdgcn_raw_buffer_load_b16(srs, svo[nb], ss, kWeightAux);
            B.sb[j][nb][1] = __builtin_amdgcn_raw_buffer_load_b16(brs, svo[nb], ss, kWeightAux);
          }
        } else if constexpr (GP == 2) {
          const v2u_t v = __builtin_amdgcn_raw_buffer_load_b64(wrs, svo[nb], so, kWeightAux);
          B.sb[j][nb][0] = v.x;
          B.sb[j][nb][GP - 1] = v.y;
        } else {
          B.sb[j][nb][0] = __builtin_amdgcn_raw_buffer_load_b32(wrs, svo[nb], so, kWeightAux);
        }
      }
    }
    if constexpr (MLX && SPW == 4) {
      // the batch's scales and biases of the lane's row, one window each; the whole
      // offset is in the vector offset, which the range check covers (past the last
      // row: zeros, never used). GP == 2: dword j = groups 2(b0+j), 2(b0+j)+1, as one
      // load per step gives them. GP == 1: three dwords from the even halfword at or
      // below the batch's first group, b0 >> gshift (sb[0..2][nb]).
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) {
        if constexpr (GP == 2) {
          const v4u_t sv = __builtin_amdgcn_raw_buffer_load_b128(srs, svo[nb] + 4 * b0, 0,
                                                                 kWeightAux);
          const v4u_t bv = __builtin_amdgcn_raw_buffer_load_b128(brs, svo[nb] + 4 * b0, 0,
                                                                 kWeightAux);
          B.sb[0][nb][0] = sv.x; B.sb[1][nb][0] = sv.y; B.sb[2][nb][0] = sv.z;
          B.sb[3][nb][0] = sv.w;
          B.sb[0][nb][1] = bv.x; B.sb[1][nb][1] = bv.y; B.sb[2][nb][1] = bv.z;
          B.sb[3][nb][1] = bv.w;
        } else {
          const int a = (((svo[nb] >> 1) + (b0 >> gshift)) & ~1) * 2;
          const v3u_t sv = __builtin_amdgcn_raw_buffer_load_b96(srs, a, 0, kWeightAux);
          const v3u_t bv = __builtin_amdgcn_raw_buffer_load_b96(brs, a, 0, kWeightAux);
          B.sb[0][nb][0] = sv.x; B.sb[1][nb][0] = sv.y; B.sb[2][nb][0] = sv.z;
          B.sb[0][nb][1] = bv.x; B.sb[1][nb][1] = bv.y; B.sb[2][nb][1] = bv.z;
        }
      }
    } else if constexpr (kWin) {
      // 2-step batches, the same windows: GP == 2, two dwords; GP == 1, two dwords from
      // the even halfword at or below group b0 >> gshift
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) {
        const int a = GP == 2 ? svo[nb] + 4 * b0 : (((svo[nb] >> 1) + (b0 >> gshift)) & ~1) * 2;
        const v2u_t sv = __builtin_amdgcn_raw_buffer_load_b64(srs, a, 0, kWeightAux);
        const v2u_t bv = __builtin_amdgcn_raw_buffer_load_b64(brs, a, 0, kWeightAux);
        B.sb[0][nb][0] = sv.x; B.sb[1][nb][0] = sv.y;
        B.sb[0][nb][1] = bv.x; B.sb[1][nb][1] = bv.y;
      }
    }
  };
  // The batch's arithmetic: the activations go to this wave's LDS region (LDS
  // operations of one wave run in order, so the previous batch's reads of it
  // are done first), then half-run sums: item t = (m, step, half) is the sum
  // of its four 16-byte chunks, one chunk per lane, met by two lane swaps.
  // FULLB: all SPW steps lie before k_end (true of every batch but a wave's last)
  auto consume = [&](auto fullc, const Batch& B, int b0) __attribute__((always_inline)) {
    constexpr bool FULLB = decltype(fullc)::value;
    uint8_t* const wl = wl_all[wave];
    if constexpr (MLX) {  // this wave's own region: its earlier reads of it come first
#pragma unroll
      for (int i = 0; i < NCL; ++i) {
        int tc = tcq[i];
        asm volatile("" : "+v"(tc));
#pragma unroll
        for (int nb = 0; nb < NH; ++nb)
          *reinterpret_cast<v4u_t*>(wl + nb * 32 * RSTR + (tc & 0xFF) * RSTR + (tc >> 8) * 16) =
              B.wc[nb][i];
      }
    }
#pragma unroll
    for (int i = 0; i < XLOADS; ++i)
      *reinterpret_cast<v4u_t*>(xw + i * 1024 + lane * 16) = B.x[i];
#pragma unroll
    for (int t0 = 0; t0 < NSUM * 4; t0 += 64) {
      const int u = t0 + lane;                 // (item, chunk) = (u / 4, u % 4)
      float v = 0.f;
      if (u < NSUM * 4) {
        const v4u_t c = *reinterpret_cast<const v4u_t*>(xw + u * 16);
        v = dot2_bf16(c.x, 0x3F803F80u, dot2_bf16(c.y, 0x3F803F80u,
            dot2_bf16(c.z, 0x3F803F80u, dot2_bf16(c.w, 0x3F803F80u, 0.f))));
      }
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      if (u < NSUM * 4 && (u & 3) == 0) xsum[u / 4] = v;
    }
    __builtin_amdgcn_s_waitcnt((15 & 15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if (!FULLB && b0 + j >= k_end) break;
      // step sums of this lane's tokens 4*g2 + r (zero past MT), per group
      float xs[GP][RPL];
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int m = tok(r), mc = min(m, MT - 1);
        const float h0s = xsum[(mc * SPW + j) * 2], h1s = xsum[(mc * SPW + j) * 2 + 1];
        if constexpr (GP == 2) {
          xs[0][r] = m < MT ? h0s : 0.f;
          xs[GP - 1][r] = m < MT ? h1s : 0.f;
        } else {
          xs[0][r] = m < MT ? h0s + h1s : 0.f;
        }
      }
      bf16x8 av[GP][4];
#pragma unroll
      for (int e = 0; e < GP; ++e)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          av[e][c] = *reinterpret_cast<const bf16x8*>(xa[e] + j * 128 + c * 16);
      // this step's BITS words of the lane's run: tiled, as loaded; MLX, from the
      // staged rows (row l32, run 2j + g2 of the batch)
      uint32_t wv[NH][BITS];
#pragma unroll
      for (int nb = 0; nb < NH; ++nb)
#pragma unroll
        for (int i = 0; i < BITS; ++i)
          wv[nb][i] = MLX ? reinterpret_cast<const uint32_t*>(
                                wl + nb * 32 * RSTR + l32 * RSTR + (2 * j + g2) * BITS * 4)[i]
                          : B.w[MLX ? 0 : j][nb][i];
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) {
        bf16x8 bv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          uint32_t pr[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int q = 8 * c + 2 * i;
            if constexpr (BITS == 8)  // codes up to 255: exact bf16 integers, offset 0
              pr[i] = pack_bf16x2(static_cast<float>(code_at<BITS>(wv[nb], q)),
                                  static_cast<float>(code_at<BITS>(wv[nb], q + 1)));
            else
              pr[i] = pair_at<BITS>(wv[nb], q, kPairMask, kMagic);
          }
          bv[c] = __builtin_bit_cast(bf16x8, v4u_t{pr[0], pr[1], pr[2], pr[3]});
        }
#pragma unroll
        for (int e = 0; e < GP; ++e) {
          f32x16_t d;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[e][c], bv[c], c == 0 ? f32x16_t{} : d,
                                                        0, 0, 0);
          float sc, bi;
          if constexpr (MLX) {
            uint32_t sv = B.sb[j][nb][0], bv2 = B.sb[j][nb][1];
            if constexpr (GP == 1 && kWin) {
              // halfword h of the window: group (b0 + j) >> gshift, counted from the
              // window's first (even) halfword
              const int hw0 = (svo[nb] >> 1) + (b0 >> gshift);
              const int h = ((b0 + j) >> gshift) - (b0 >> gshift) + (hw0 & 1);
              const int d = h >> 1;
              // values, not lvalues: a choice between elements would index the batch
              // at run time and move it to scratch memory
              const uint32_t s0 = B.sb[0][nb][0], s1 = B.sb[1][nb][0];
              const uint32_t c0 = B.sb[0][nb][1], c1 = B.sb[1][nb][1];
              uint32_t ws, wb;
              if constexpr (SPW == 4) {
                const uint32_t s2 = B.sb[2][nb][0], c2 = B.sb[2][nb][1];
                ws = d == 0 ? s0 : d == 1 ? s1 : s2;
                wb = d == 0 ? c0 : d == 1 ? c1 : c2;
              } else {
                ws = d == 0 ? s0 : s1;
                wb = d == 0 ? c0 : c1;
              }
              sv = (h & 1) ? ws >> 16 : ws;
              bv2 = (h & 1) ? wb >> 16 : wb;
              if ((hw0 & ~1) + h == s_last) {
                sv = s_tail;
                bv2 = b_tail;
              }
            }
            sc = __uint_as_float(e ? sv & 0xFFFF0000u : sv << 16);
            bi = __uint_as_float(e ? bv2 & 0xFFFF0000u : bv2 << 16);
          } else {
            sc = __uint_as_float(B.sb[j][nb][e] << 16);
            bi = __uint_as_float(B.sb[j][nb][e] & 0xFFFF0000u);
          }
          const float b2 = fmaf(BITS == 8 ? 0.f : -128.f, sc, bi);
#pragma unroll
          for (int r = 0; r < RPL; ++r)
            acc[nb][r] = fmaf(sc, d[r], fmaf(b2, xs[e][r], acc[nb][r]));
        }
      }
      // 5-bit codes, 16-token passes over the MLX layout (4-step batches): each step's
      // operand reads stay after the previous step's products, which keeps the kernel in
      // fewer registers (K = 4096, N = 24576, M = 16: 46.5 -> 38.8 us; N = 7168: 15.7 ->
      // 14.7 us; K = 21504, N = 5376: 55.9 -> 51.2 us). 3-bit codes were 3-8 % slower so.
      if constexpr (MLX && MT >= 16 && BITS == 5) __builtin_amdgcn_sched_barrier(0);
    }
  };
  // two register sets: batch b+1's loads are in flight while batch b computes.
  // Each consume follows its prefetch (or the absence of one) in straight-line
  // code, and a batch with a prefetch behind it is whole (no early exit that
  // would leave its loads unwaited), so the compiler's wait before the batch's
  // first use counts the prefetch as still in flight instead of waiting for it.
  using Whole = std::true_type;
  using Part = std::false_type;
  Batch ba, bb;
  int b0 = k_begin;
  if (b0 < k_end) {
    load(ba, b0);
    for (;;) {
      int b1 = next_batch(b0);
      if (b1 >= k_end) {
        consume(Part{}, ba, b0);
        break;
      }
      load(bb, b1);
      consume(Whole{}, ba, b0);
      b0 = b1;
      b1 = next_batch(b0);
      if (b1 >= k_end) {
        consume(Part{}, bb, b0);
        break;
      }
      load(ba, b1);
      consume(Whole{}, bb, b0);
      b0 = b1;
    }
  }

  // the waves' partials meet in LDS (each wave reuses its own activation
  // region): lane (l32, g2) holds tokens 4*g2 + r of row l32
  float* part = reinterpret_cast<float*>(xw);
  __builtin_amdgcn_s_waitcnt((15 & 15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
#pragma unroll
  for (int nb = 0; nb < NH; ++nb)
#pragma unroll
    for (int r = 0; r < RPL; ++r)
      if (tok(r) < MT) part[(nb * 32 + l32) * MT + tok(r)] = acc[nb][r];
  __syncthreads();
  if (wave != 0 || lane >= NH * 32) return;
  const int n = rb * 64 + h0 * 32 + lane;
  if (n >= N) return;
  const float bv = bias ? bf16_to_f32(bias[n]) : 0.f;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m >= mcount) break;
    float t = bv;
#pragma unroll
    for (int v = 0; v < WPB; ++v)
      t += reinterpret_cast<const float*>(lds + v * XW)[lane * MT + m];
    y[static_cast<int64_t>(m0 + m) * N + n] = f32_to_bf16(t);
  }
}

// Launch shape: one workgroup per 32-row record half (768 workgroups at N = 24576,
// three per CU), 4 waves, batches of 1 step (two steps in flight per wave). Measured
// with non-temporal weight loads in a same-box A/B at K = 4096, N = 24576, 6-bit, five
// rotated copies (median of 7 x 50 launches): 1-step batches 14.4 us at M = 2 (14.4 at
// M = 1, 15.4 at M = 8); 2-step 14.9 (14.6, 17.8); 3-step 16.1; 4-step 15.7; 8 waves
// with 2-step batches 15.1 (21.4 at M = 8), with 1-step 15.2. Results are the same bits
// for every batch size (each wave sums its chunks in step order).
#ifndef MXQ_QMV_WAVES
#define MXQ_QMV_WAVES 4
#endif
#ifndef MXQ_QMV_SPW
#define MXQ_QMV_SPW 1
#endif
constexpr int kTiledNH = 1, kTiledWaves = MXQ_QMV_WAVES, kTiledSPW = MXQ_QMV_SPW;

// Waves per workgroup: 8 where fewer than 512 workgroups would run and K holds 32 steps
// or more (each wave keeps at least one whole chunk), else 4. A small grid then keeps more
// loads in flight (M = 1, N = 5376, K = 21504: 25.3 against 36.7 us; 16 waves, 21.8 us,
// do not fit the MLX layout's staging in LDS); large grids are faster with 4 (N = 24576:
// 16.7 against 18.8 us). The tiled and MLX-layout launches use the same rule, so they split
// K alike and give the same result bits.
inline int qmv_waves(int N, int M, int MT, int K) {
  const int64_t wgs = static_cast<int64_t>((N + 63) / 64 * 2) * ((M + MT - 1) / MT);
  return wgs < 512 && (K >> 6) >= 32 ? 8 : 4;
}

template <int BITS, int MT>
hipError_t run_qmv_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                         const uint16_t* bias, uint16_t* y, hipStream_t s) {
  constexpr int NH = kTiledNH, SPW = kTiledSPW;
  dim3 grid((N + 63) / 64 * (2 / NH), (M + MT - 1) / MT);
  const uint8_t* t = static_cast<const uint8_t*>(tw);
#define MXQ_QMV_LAUNCH(G, W)                                                   \
  qmv_tiled_kernel<BITS, MT, G, NH, W, SPW, false><<<grid, 64 * W, 0, s>>>(    \
      x, M, K, t, N, bias, y, nullptr, nullptr, nullptr, 0)
  const bool eight = qmv_waves(N, M, MT, K) == 8;
  if (gs == 32) {
    if (eight) MXQ_QMV_LAUNCH(2, 8); else MXQ_QMV_LAUNCH(2, kTiledWaves);
  } else {
    if (eight) MXQ_QMV_LAUNCH(1, 8); else MXQ_QMV_LAUNCH(1, kTiledWaves);
  }
#undef MXQ_QMV_LAUNCH
  return hipGetLastError();
}

// The same kernel reading the MLX layout in place (K % 64 == 0).
template <int BITS, int MT>
hipError_t run_qmv_mlx(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                       const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                       hipStream_t s) {
  // batches of 4 steps: a batch reads 4 x 8 * BITS contiguous bytes of each row (192 B
  // at 6 bits), so fewer of a row's 128-byte lines are split between batches
  // (M = 2, N = 24576: 31.4 us against 32.8 us with 2 steps; 8 or 16 steps, two
  // record halves per workgroup or 2 waves per workgroup were slower). 16-token passes
  // of even code widths take batches of 2: two 4-step batches of 16 tokens' activations
  // (64 VGPRs) and codes held 273-308 VGPRs per lane at 4 waves, one wave per SIMD, and
  // spilled at 8 waves; with 2 steps, 184-204 and no spills (6-bit, K = 4096: N = 24576
  // 48.8 -> 38.5 us, N = 7168 19.5 -> 13.5 us; K = 21504, N = 5376: 74.8 -> 52.6 us).
  // 8-token passes stay at 4 steps (2 steps: 38.7 -> 45.5 us at K = 21504).
  constexpr int NH = 1, SPW = (MT >= 16 && BITS % 2 == 0) ? 2 : 4;
  dim3 grid((N + 63) / 64 * (2 / NH), (M + MT - 1) / MT);
#define MXQ_QMV_LAUNCH(G, W, GSH)                                              \
  qmv_tiled_kernel<BITS, MT, G, NH, W, SPW, true><<<grid, 64 * W, 0, s>>>(     \
      x, M, K, nullptr, N, bias, y, wq, sc, bi, GSH)
  const bool eight = qmv_waves(N, M, MT, K) == 8;  // the tiled launch's rule
  const int gsh = gs == 128 ? 1 : 0;
  if (gs == 32) {
    if (eight) MXQ_QMV_LAUNCH(2, 8, 0); else MXQ_QMV_LAUNCH(2, kTiledWaves, 0);
  } else {
    if (eight) MXQ_QMV_LAUNCH(1, 8, gsh); else MXQ_QMV_LAUNCH(1, kTiledWaves, gsh);
  }
#undef MXQ_QMV_LAUNCH
  return hipGetLastError();
}

template <int BITS>
hipError_t pick_mt_mlx(const uint16_t* x, int M, int K, const uint32_t* wq, const uint16_t* sc,
                       const uint16_t* bi, int N, int gs, const uint16_t* bias, uint16_t* y,
                       hipStream_t s) {
  if (M <= 1) return run_qmv_mlx<BITS, 1>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  if (M <= 2) return run_qmv_mlx<BITS, 2>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  if (M <= 4) return run_qmv_mlx<BITS, 4>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  if (M <= 8) return run_qmv_mlx<BITS, 8>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
  // 16 tokens per pass: the 4-step batches of 32 would take 16 KiB of LDS per wave
  return run_qmv_mlx<BITS, 16>(x, M, K, wq, sc, bi, N, gs, bias, y, s);
}

template <int BITS>
hipError_t pick_mt_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                         const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (M <= 1) return run_qmv_tiled<BITS, 1>(x, M, K, tw, N, gs, bias, y, s);
  if (M <= 2) return run_qmv_tiled<BITS, 2>(x, M, K, tw, N, gs, bias, y, s);
  if (M <= 4) return run_qmv_tiled<BITS, 4>(x, M, K, tw, N, gs, bias, y, s);
  if (M <= 8) return run_qmv_tiled<BITS, 8>(x, M, K, tw, N, gs, bias, y, s);
  if (M <= 16) return run_qmv_tiled<BITS, 16>(x, M, K, tw, N, gs, bias, y, s);
  return run_qmv_tiled<BITS, 32>(x, M, K, tw, N, gs, bias, y, s);
}

}  // namespace

namespace detail {
#define MXQ_QMV_CAT2(a, b) a##b
#define MXQ_QMV_CAT(a, b) MXQ_QMV_CAT2(a, b)
// the MLX layout: whole 64-code steps run the step kernel over the layout in place;
// otherwise (K an odd multiple of 32, gs = 32) the lane-per-chunk kernel
hipError_t MXQ_QMV_CAT(launch_qmv_b, MXQ_QMV_BITS)(const uint16_t* x, int M, int K,
                                                   const uint32_t* wq, const uint16_t* scales,
                                                   const uint16_t* biases, int N, int gs,
                                                   const uint16_t* bias, uint16_t* y,
                                                   hipStream_t s) {
  if (K % 64 == 0)
    return pick_mt_mlx<MXQ_QMV_BITS>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
  return pick_mt<MXQ_QMV_BITS>(x, M, K, wq, scales, biases, N, gs, bias, y, s);
}
hipError_t MXQ_QMV_CAT(launch_qmv_tiled_b, MXQ_QMV_BITS)(const uint16_t* x, int M, int K,
                                                         const void* tw, int N, int gs,
                                                         const uint16_t* bias, uint16_t* y,
                                                         hipStream_t s) {
  return pick_mt_tiled<MXQ_QMV_BITS>(x, M, K, tw, N, gs, bias, y, s);
}
}  // namespace detail
}  // namespace mxq
