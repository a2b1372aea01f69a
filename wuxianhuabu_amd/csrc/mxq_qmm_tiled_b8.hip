// mxq_qmm_tiled_b8.hip — the tiled MFMA kernels for 8-bit codes (one
// translation unit per width; the kernels are in mxq_qmm_tiled_impl.hpp).
#define MXQ_TILED_BITS 8
#include "mxq_qmm_tiled_impl.hpp"
