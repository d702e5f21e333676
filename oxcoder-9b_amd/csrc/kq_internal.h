// Host-side internals of libkq: status codes, error text, argument checks, launch helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/kq.h"

namespace kq {

// Records the message for kq_last_error() (thread-local) and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Validates (w, R, C, type) as a Kindi-layout quantized tensor.
int check_matrix(const void* w, int R, int C, int type, const char* fn);
int check_ptr(const void* p, size_t align, const char* what, const char* fn);

// Reports a failed launch (hipGetLastError) as KQ_ERR_HIP.
int check_launch(const char* fn);

// Compute units of the current device (cached per device).
int device_cus();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline int block_bytes(int type) { return type == KQ_TYPE_Q4_K ? 144 : 210; }

// Launchers implemented by the kernel translation units.  Arguments are already validated.
void launch_q8k_quantize(const float* x, int64_t ldx, int C, int N, uint8_t* xq, hipStream_t s);
// The same for M rows, also writing the prefill GEMM's fragment copy xf (Mpad >= M rows, the rows past
// M zero).
void launch_q8k_quantize_frag(const float* x, int64_t ldx, int C, int M, int Mpad, uint8_t* xq, uint8_t* xf,
                              hipStream_t s);
// Fused producers of Q8_K activations (RMSNorm with optional residual add; SwiGLU).
void launch_rms_q8k(float* h, const float* res, int add, const float* w, int D, int N, int64_t ld, float* xn,
                    uint8_t* xq, hipStream_t s);
void launch_swiglu_q8k(const float* gate, const float* up, int n, int N, int64_t ld, float* y, uint8_t* xq,
                       hipStream_t s);
void launch_gemv_q8k(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int N, float* y,
                     int64_t ldy, hipStream_t s);
// n (1..3) matrices of one type sharing xq; one launch per group of up to 4 tokens.
void launch_gemv_q8k_group(int n, const uint8_t* const* w, const int* R, int C, int type,
                           const uint8_t* xq, int N, float* const* y, const int64_t* ldy, hipStream_t s);
// n (2..3) matrices of both types sharing xq, one token, C <= 4096: one launch when one type has
// a single matrix; false (nothing launched) otherwise.  Outputs bit-identical to the group above.
bool launch_gemv_q8k_mixed(int n, const uint8_t* const* w, const int* R, const int* type, int C, const uint8_t* xq,
                           float* const* y, hipStream_t s);
// The same with fp32 activations.
bool launch_gemv_f32_mixed(int n, const uint8_t* const* w, const int* R, const int* type, int C, const float* x,
                           float* const* y, hipStream_t s);
// One token of fp32 activations, n (1..3) matrices of one type, C <= 4096: the quantization to Q8_K
// inside the GEMV launch (bit-identical to launch_q8k_quantize + launch_gemv_q8k_group); xqo
// (nullable) receives the Q8_K bytes.
void launch_gemv_q8k_x_group(int n, const uint8_t* const* w, const int* R, int C, int type, const float* x,
                             float* const* y, uint8_t* xqo, hipStream_t s);
// The same for both weight types in one launch (as launch_gemv_q8k_mixed); false (nothing launched)
// when the group does not have that form.
bool launch_gemv_q8k_x_mixed(int n, const uint8_t* const* w, const int* R, const int* type, int C, const float* x,
                             float* const* y, uint8_t* xqo, hipStream_t s);
// Small-batch GEMV on MFMA (C <= 16384, N <= 16): rows bit-identical to the GEMV above.
void launch_gemv_mfma_group(int n, const uint8_t* const* w, const int* R, int C, int type, const uint8_t* xq,
                            int N, float* const* y, const int64_t* ldy, hipStream_t s);
// Prefill GEMM; ws (or nullptr) holds gemm_q8k_workspace(R, C, M) bytes (256-byte aligned): the
// activation fragments and, for grids too small to fill the GPU, the partial sums of the K split.
size_t gemm_q8k_workspace(int R, int C, int M);
void launch_gemm_q8k(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int M, float* y, int64_t ldy,
                     uint8_t* ws, hipStream_t s);
// The same over n (1..3) matrices sharing xq: one fragment copy, one GEMM launch per weight type;
// each matrix's results equal those of its own launch_gemm_q8k call bit for bit.
size_t gemm_q8k_group_workspace(int n, const int* R, int C, int M);
void launch_gemm_q8k_group(int n, const uint8_t* const* w, const int* R, int C, const int* type, const uint8_t* xq,
                           int M, float* const* y, const int64_t* ldy, uint8_t* ws, hipStream_t s,
                           bool frag_ready = false);
// From fp32 activations: x (M rows, stride ldx) quantized once into the workspace, as Q8_K rows and
// the fragment copy in one launch, then the grouped GEMM.  Workspace: the Q8_K rows (256-byte
// aligned), then gemm_q8k_group_workspace.
size_t gemm_f32_group_workspace(int n, const int* R, int C, int M);
void launch_gemm_f32_group(int n, const uint8_t* const* w, const int* R, int C, const int* type, const float* x,
                           int64_t ldx, int M, float* const* y, const int64_t* ldy, uint8_t* ws, hipStream_t s);
// Device address of the static GEMM workspace on the current device (KQ_GEMM_STATIC_SCRATCH_BYTES),
// looked up on the first call per device; fails with KQ_ERR_HIP when the lookup fails.
int gemm_static_scratch(uint8_t** out, const char* fn);
// Argmax (argmax_block.h): ws holds argmax_workspace_bytes() bytes, its first word zero.
size_t argmax_workspace_bytes();
void launch_argmax(const float* y, int n, uint8_t* ws, int* out, hipStream_t s);
// One-token GEMV of one matrix plus the argmax of its outputs.
void launch_gemv_q8k_argmax(const uint8_t* w, int R, int C, int type, const uint8_t* xq, float* y, uint8_t* ws,
                            int* out, hipStream_t s);
void launch_subblock_sums(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int N,
                          int32_t* sums, hipStream_t s);
// fp32-activation GEMV (Kindi numerics) of n (1..3) matrices of one type sharing x: the kernels of
// the Q8_K GEMV with fp32 activations, one launch.
void launch_gemv_f32_group(int n, const uint8_t* const* w, const int* R, int C, int type, const float* x,
                           float* const* y, hipStream_t s);
void launch_dequant_rows(const uint8_t* w, int R, int C, int type, int row0, int nrows, float* y,
                         int64_t ldy, hipStream_t s);

}  // namespace kq
