// mxq_qmv_b5.hip — the GEMV kernels for 5-bit codes (one translation unit per width;
// the kernels are in mxq_qmv_impl.hpp).
#define MXQ_QMV_BITS 5
#include "mxq_qmv_impl.hpp"
