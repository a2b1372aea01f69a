// mxq_qmv_b2.hip — the GEMV kernels for 2-bit codes (one translation unit per width;
// the kernels are in mxq_qmv_impl.hpp).
#define MXQ_QMV_BITS 2
#include "mxq_qmv_impl.hpp"
