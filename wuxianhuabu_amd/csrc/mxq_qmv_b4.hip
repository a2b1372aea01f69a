// mxq_qmv_b4.hip — the GEMV kernels for 4-bit codes (one translation unit per width;
// the kernels are in mxq_qmv_impl.hpp).
#define MXQ_QMV_BITS 4
#include "mxq_qmv_impl.hpp"
