// mxq_qmv.hip — dispatch of the GEMV kernels by code width. The kernels
// (mxq_qmv_impl.hpp) are compiled once per width in mxq_qmv_b{2,3,4,5,6,8}.hip.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "mxq_internal.hpp"

namespace mxq {
namespace detail {

#define MXQ_QMV_DECL(B)                                                                      \
  hipError_t launch_qmv_b##B(const uint16_t* x, int M, int K, const uint32_t* wq,            \
                             const uint16_t* scales, const uint16_t* biases, int N, int gs,  \
                             const uint16_t* bias, uint16_t* y, hipStream_t s);              \
  hipError_t launch_qmv_tiled_b##B(const uint16_t* x, int M, int K, const void* tw, int N,   \
                                   int gs, const uint16_t* bias, uint16_t* y, hipStream_t s);
MXQ_QMV_DECL(2)
MXQ_QMV_DECL(3)
MXQ_QMV_DECL(4)
MXQ_QMV_DECL(5)
MXQ_QMV_DECL(6)
MXQ_QMV_DECL(8)
#undef MXQ_QMV_DECL

hipError_t launch_qmv(const uint16_t* x, int M, int K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int N, int gs, int bits,
                      const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (bits) {
    case 2: return launch_qmv_b2(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 3: return launch_qmv_b3(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 4: return launch_qmv_b4(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 5: return launch_qmv_b5(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 6: return launch_qmv_b6(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    case 8: return launch_qmv_b8(x, M, K, wq, scales, biases, N, gs, bias, y, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_qmv_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                            int bits, const uint16_t* bias, uint16_t* y, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (bits) {
    case 2: return launch_qmv_tiled_b2(x, M, K, tw, N, gs, bias, y, s);
    case 3: return launch_qmv_tiled_b3(x, M, K, tw, N, gs, bias, y, s);
    case 4: return launch_qmv_tiled_b4(x, M, K, tw, N, gs, bias, y, s);
    case 5: return launch_qmv_tiled_b5(x, M, K, tw, N, gs, bias, y, s);
    case 6: return launch_qmv_tiled_b6(x, M, K, tw, N, gs, bias, y, s);
    case 8: return launch_qmv_tiled_b8(x, M, K, tw, N, gs, bias, y, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace detail
}  // namespace mxq
