// mxq_qmm_tiled.hip — dispatch of the tiled MFMA kernels by code width. The
// kernels (mxq_qmm_tiled_impl.hpp) are compiled once per width in
// mxq_qmm_tiled_b{2,3,4,5,6,8}.hip.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "mxq_internal.hpp"

namespace mxq {
namespace detail {

#define MXQ_TILED_DECL(B)                                                                    \
  hipError_t launch_qmm_tiled_b##B(const uint16_t* x, int M, int K, const void* tw, int N,    \
                                   int gs, const uint16_t* bias, int act, const uint16_t* xa, \
                                   const uint16_t* bt, int R, uint16_t* y, hipStream_t s);
MXQ_TILED_DECL(2)
MXQ_TILED_DECL(3)
MXQ_TILED_DECL(4)
MXQ_TILED_DECL(5)
MXQ_TILED_DECL(6)
MXQ_TILED_DECL(8)
#undef MXQ_TILED_DECL

hipError_t launch_qmm_tiled(const uint16_t* x, int M, int K, const void* tw, int N, int gs,
                            int bits, const uint16_t* bias, int act, const uint16_t* xa,
                            const uint16_t* bt, int R, uint16_t* y, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (bits) {
    case 2: return launch_qmm_tiled_b2(x, M, K, tw, N, gs, bias, act, xa, bt, R, y, s);
    case 3: return launch_qmm_tiled_b3(x, M, K, tw, N, gs, bias, act, xa, bt, R, y, s);
    case 4: return launch_qmm_tiled_b4(x, M, K, tw, N, gs, bias, act, xa, bt, R, y, s);
    case 5: return launch_qmm_tiled_b5(x, M, K, tw, N, gs, bias, act, xa, bt, R, y, s);
    case 6: return launch_qmm_tiled_b6(x, M, K, tw, N, gs, bias, act, xa, bt, R, y, s);
    case 8: return launch_qmm_tiled_b8(x, M, K, tw, N, gs, bias, act, xa, bt, R, y, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace detail
}  // namespace mxq
