// mxq_qmm_tiled_b2.hip — the tiled MFMA kernels for 2-bit codes (one
// translation unit per width; the kernels are in mxq_qmm_tiled_impl.hpp).
#define MXQ_TILED_BITS 2
#include "mxq_qmm_tiled_impl.hpp"
