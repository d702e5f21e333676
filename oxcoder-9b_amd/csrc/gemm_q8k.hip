// Prefill GEMM (int8 MFMA) -- placeholder translation unit; kq_gemm_q8k currently runs the
// batched GEMV kernels in groups of four tokens.
#include "kq_device.h"
#include "kq_internal.h"
