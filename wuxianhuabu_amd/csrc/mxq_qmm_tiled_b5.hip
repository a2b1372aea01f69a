// mxq_qmm_tiled_b5.hip — the tiled MFMA kernels for 5-bit codes (one
// translation unit per width; the kernels are in mxq_qmm_tiled_impl.hpp).
#define MXQ_TILED_BITS 5
#include "mxq_qmm_tiled_impl.hpp"
