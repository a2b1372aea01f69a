// mxq_qmm_tiled_b6.hip — the tiled MFMA kernels for 6-bit codes (one
// translation unit per width; the kernels are in mxq_qmm_tiled_impl.hpp).
#define MXQ_TILED_BITS 6
#include "mxq_qmm_tiled_impl.hpp"
