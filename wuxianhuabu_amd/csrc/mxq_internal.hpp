// mxq_internal.hpp — launchers behind the C ABI. Arguments are validated by
// mxq_api.cpp before any of these is called; launchers only pick a kernel
// instantiation and enqueue it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxq {
namespace detail {

hipError_t launch_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq,
                       hipStream_t s);
hipError_t launch_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits,
                         uint8_t* codes, hipStream_t s);
hipError_t launch_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols, int gs,
                           int bits, int mode, uint32_t* wq, void* scales, void* biases,
                           int sb_dtype, hipStream_t s);
hipError_t launch_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                             int sb_dtype, int64_t rows, int64_t cols, int gs, int bits,
                             void* out, int out_dtype, hipStream_t s);

// MLX layout -> tiled layout (mxq_tiled.hpp). K % 64 == 0, bf16 scales/biases.
// With `pairs`, row block rb takes rows 32rb.. (first half) and N/2 + 32rb..
// (second half) of an [N, K] weight with N even.
hipError_t launch_tile(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                       int64_t N, int64_t K, int gs, int bits, bool pairs, void* out,
                       hipStream_t s);

// tiled layout -> MLX layout, the inverse of launch_tile (same `pairs` meaning).
hipError_t launch_untile(const void* tiled, int64_t N, int64_t K, int gs, int bits, bool pairs,
                         uint32_t* wq, uint16_t* scales, uint16_t* biases, hipStream_t s);

// y[M,N] = x[M,K] * W^T (+ bias): small-M split-K GEMV (any M; rows of x are
// processed in blocks of up to 8).
hipError_t launch_qmv(const uint16_t* x, int M, int K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int N, int gs, int bits,
                      const uint16_t* bias, uint16_t* y, hipStream_t s);

// Large-M bf16 MFMA kernel. Returns hipErrorNotSupported for widths it does
// not implement (the caller then falls back to launch_qmv).
hipError_t launch_qmm(const uint16_t* x, int M, int K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int N, int gs, int bits,
                      const uint16_t* bias, uint16_t* y, hipStream_t s);
bool qmm_supports_bits(int bits);

// Both kernels on tiled weights (K % 64 == 0): any M for the MFMA kernel,
// M <= 8 for the GEMV.
// act: MXQ_ACT_* (mxq.h), applied in the MFMA kernel's epilogue; xa [M, R] and
// bt [N, R] (bf16, R % 16 == 0; xa == nullptr for none) add xa . bt^T first.
hipError_t launch_qmm_tiled(const uint16_t* x, int M, int K, const void* tiled, int N, int gs,
                            int bits, const uint16_t* bias, int act, const uint16_t* xa,
                            const uint16_t* bt, int R, uint16_t* y, hipStream_t s);
hipError_t launch_qmv_tiled(const uint16_t* x, int M, int K, const void* tiled, int N, int gs,
                            int bits, const uint16_t* bias, uint16_t* y, hipStream_t s);

// Row-wise ops of the DiT block around the linears (mxq_blockops.hip): bf16 rows.
hipError_t launch_norm_modscale(const uint16_t* x, int64_t S, int hidden, const uint16_t* w,
                                const uint16_t* shift, const uint16_t* scale,
                                const uint32_t* map, int64_t mod_rows, float eps, uint16_t* out,
                                hipStream_t s);
hipError_t launch_mod_gate(const uint16_t* x, const uint16_t* other, int64_t S, int hidden,
                           const uint16_t* gate, const uint32_t* map, int64_t mod_rows,
                           uint16_t* out, hipStream_t s);
hipError_t launch_rmsnorm_rope(const uint16_t* x, int64_t S, int H, int hd, const uint16_t* w,
                               const void* c, const void* sn, int table_dtype, int rot,
                               float eps, uint16_t* out, hipStream_t s);

}  // namespace detail
}  // namespace mxq
