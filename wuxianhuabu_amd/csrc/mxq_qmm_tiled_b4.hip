// mxq_qmm_tiled_b4.hip — the tiled MFMA kernels for 4-bit codes (one
// translation unit per width; the kernels are in mxq_qmm_tiled_impl.hpp).
#define MXQ_TILED_BITS 4
#include "mxq_qmm_tiled_impl.hpp"
