// mxq_qmm_tiled_b3.hip — the tiled MFMA kernels for 3-bit codes (one
// translation unit per width; the kernels are in mxq_qmm_tiled_impl.hpp).
#define MXQ_TILED_BITS 3
#include "mxq_qmm_tiled_impl.hpp"
