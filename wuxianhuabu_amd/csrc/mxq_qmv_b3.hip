// mxq_qmv_b3.hip — the GEMV kernels for 3-bit codes (one translation unit per width;
// the kernels are in mxq_qmv_impl.hpp).
#define MXQ_QMV_BITS 3
#include "mxq_qmv_impl.hpp"
