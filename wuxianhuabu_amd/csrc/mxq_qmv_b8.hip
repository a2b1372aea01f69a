// mxq_qmv_b8.hip — the GEMV kernels for 8-bit codes (one translation unit per width;
// the kernels are in mxq_qmv_impl.hpp).
#define MXQ_QMV_BITS 8
#include "mxq_qmv_impl.hpp"
