// mxq_qmv_b6.hip — the GEMV kernels for 6-bit codes (one translation unit per width;
// the kernels are in mxq_qmv_impl.hpp).
#define MXQ_QMV_BITS 6
#include "mxq_qmv_impl.hpp"
