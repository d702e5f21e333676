/*
 * kq.h -- C ABI of libkq.so, the MI355X (gfx950) quantized matrix products of the Kindi Q4 path.
 *
 * Every entry point takes device pointers and sizes, enqueues its kernels on `stream` (a
 * hipStream_t passed as void*; NULL = the default stream), allocates nothing, and returns 0 or a
 * negative KQ_ERR_* code whose text kq_last_error() returns.  Arguments are validated before any
 * launch, the way the reference validates a pack before touching native buffers
 * (scripts/kindi_q4/kindi/q4pack.py:86-108).
 *
 * Weights use the Kindi losslessly repacked layout [R/8][C/256][8][block] (q4pack.py:151-160,
 * q4kernels.h:8-10) with GGML Q4_K (type 12, 144 B / 256 weights) or Q6_K (type 14, 210 B)
 * blocks.  Requirements: R % 8 == 0, C % 256 == 0, 256 <= C <= 61440, w 16-byte aligned.
 *
 * Q8_K activations are GGML block_q8_K: float d, int8 qs[256], int16 bsums[16] (292 B per 256
 * values); N rows of C values occupy N*(C/256) consecutive blocks.
 *
 * Numerical contract of the Q8_K products: per (row, super-block) the integer sums are exact and
 * the fp32 value is v = fma(d*dx, I1, -(dmin*dx)*I2) (Q4_K) or (d*dx)*I (Q6_K); the row result
 * is a pairwise tree of the v over super-block columns in natural order.  A row's result does not
 * depend on N or on which kernel computed it.
 */
#ifndef KQ_H
#define KQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KQ_TYPE_Q4_K 12
#define KQ_TYPE_Q6_K 14

#define KQ_OK 0
#define KQ_ERR_ARG (-1)   /* invalid shape, type, pointer or alignment */
#define KQ_ERR_HIP (-2)   /* the HIP runtime reported an error */

#define KQ_MAX_BATCH 16   /* tokens per kq_gemv_q8k call */

/* Text of the last error raised on the calling thread ("" when none). */
const char* kq_last_error(void);

/* Library version, (major << 16) | minor. */
int kq_version(void);

/*
 * Hash of the sources the library was built from (kernels, their headers, this file): a change of
 * the arithmetic changes it.  For the engine's state-cache fingerprint, which keys saved states on
 * the code of the arithmetic (engine_fingerprint and _ARITH, scripts/kindi_q4/kindi/cache.py:51-95).
 */
const char* kq_source_hash(void);

/*
 * y[r] = sum_j w[r][j] * x[j] with fp32 activations: Kindi's decode GEMV.
 * Replaces the CUDA kernel q4_gemv(w, x, y, R, C, type) (scripts/kindi_q4/kindi/q4.cu:18-27) as
 * launched by Engine.gemv (gpu4.py:95-99), and kc_matvec (kcpu4.c:337-340).  Weights decode as
 * in q4kernels.h:12-33; the sum is fp32 (not bit-identical to the reference's order, within
 * 1e-5 * max|y|).  x: C floats, y: R floats, both 4-byte aligned.
 */
int kq_gemv(const void* w, int R, int C, int type, const float* x, float* y, void* stream);

/*
 * Up to 3 matrices sharing one input, as the CPU engine's gemv(m, n, A, y, x) does
 * (kcpu4.c:100-118).  C is common; R[i], type[i] per matrix.  One launch per weight type (one for
 * both when C <= 4096 and one type has a single matrix); every y[i] equals kq_gemv on that matrix
 * bit for bit.
 */
int kq_gemv_multi(int n, const void* const* w, const int* R, int C, const int* type,
                  const float* x, float* const* y, void* stream);

/*
 * Q8_K activation quantizer (GGML quantize_row_q8_K_ref semantics; no counterpart in the
 * reference, whose Q4 path keeps activations in fp32, q4kernels.h:37-83).  x: N rows of C floats
 * with row stride ldx (floats), 4-byte aligned; xq: N*(C/256) blocks of 292 B, 4-byte aligned.
 * Inputs must be finite.
 */
int kq_q8k_quantize(const float* x, int64_t ldx, int C, int N, void* xq, void* stream);

/*
 * RMSNorm producing the GEMV input directly in Q8_K: for each of N rows (row stride ld floats),
 * if add: h += residual (written back to h); s = 1 / sqrtf((float)(sum h^2 / D) + 1e-6f) with the
 * squares summed in double; xn = (h * s) * w; xq = Q8_K(xn) (as kq_q8k_quantize).  Replaces the
 * Q4 engine's q4_rms(h, residual, w, xn, xp, D, add) (scripts/kindi_q4/kindi/q4.cu:39-46, launched
 * by Engine.rmsfold, gpu4.py:104-106) followed by the quantization of xp; the double sum follows
 * that kernel's order (256 strided partial sums, then a halving tree), so h and xn are
 * bit-identical to it.  The CPU engine's rmsfold (kcpu4.c:123-139) is the same computation with a
 * sequential double sum.  D % 256 == 0, D <= 16384; xn may be NULL (only xq is produced) or h itself;
 * residual (read only when add != 0) must not overlap h.  All pointers 4-byte aligned.
 */
int kq_rms_q8k(float* h, const float* residual, int add, const float* w, int D, int N, int64_t ld, float* xn,
               void* xq, void* stream);

/*
 * SwiGLU producing the down-projection input directly in Q8_K: y = (g / (1 + exp(-g))) * u
 * elementwise for N rows of n values (row stride ld floats), xq = Q8_K(y).  Replaces q4_silu
 * (q4.cu:36-38, launched as k_smfold by the FFN, engine.py:287) and the CPU engine's
 * silu(ffg) * ffu (kcpu4.c:77, 292) followed by the quantization.  exp is the library's own
 * binary32 exp (within 2 ulp of the exact value, like CUDA's and glibc's expf), so y agrees with
 * the reference to a few ulp and exactly with the repository's CPU oracle.  n % 256 == 0; y may
 * be NULL.  All pointers 4-byte aligned.
 */
int kq_swiglu_q8k(const float* gate, const float* up, int n, int N, int64_t ld, float* y, void* xq,
                  void* stream);

/*
 * Y[n][r] (row stride ldy floats) for N = 1..16 Q8_K activation rows: batch-1 decode (N = 1)
 * and speculative-verify GEMV.  Same role as q4_gemv with quantized activations; the batched
 * form follows the ternary engine's k_tc_mv{2,4,8}(..., y[ntok][R]) (tc.cu:306-310).
 */
int kq_gemv_q8k(const void* w, int R, int C, int type, const void* xq, int N, float* y,
                int64_t ldy, void* stream);

/*
 * Up to 3 matrices sharing one Q8_K input in one launch per type (q/k/v, gate/up; with one token,
 * C <= 4096 and one of the two types holding a single matrix, as a Q4_K_M layer's q, k and Q6_K v,
 * one launch for both): the Q8_K form of the CPU engine's multi-matrix gemv(m, n, A, y, x)
 * (kcpu4.c:100-118).  C and N are common; R[i], type[i], y[i] and ldy[i] per matrix.  Every y[i]
 * equals kq_gemv_q8k on that matrix alone bit for bit.
 */
int kq_gemv_q8k_multi(int n, const void* const* w, const int* R, int C, const int* type, const void* xq,
                      int N, float* const* y, const int64_t* ldy, void* stream);

/*
 * Batch-1 decode GEMV from fp32 activations with Q8_K arithmetic, the quantization inside the GEMV
 * launch: gpu4.Engine.gemv(names, x, outs) (scripts/kindi_q4/kindi/gpu4.py:95-99) takes fp32 x;
 * here up to 3 matrices sharing x (fp32[C], 16-byte aligned) in one launch per type, each
 * workgroup quantizing x itself (the bytes of kq_q8k_quantize), instead of a quantizer launch
 * followed by kq_gemv_q8k_multi; every y[i] equals that pair's bit for bit.  xq (C/256*292 bytes,
 * dword aligned, or NULL) receives the Q8_K bytes; it is required for C > 4096, where the call
 * runs the quantizer and the GEMV as two launches.
 */
int kq_gemv_q8k_x(int n, const void* const* w, const int* R, int C, const int* type, const float* x,
                  float* const* y, void* xq, void* stream);

/*
 * Greedy pick over the logits: *out = index of the largest y[i] (i < n), the smallest index among
 * equal largest values; NaN is never chosen and an input with no value above -1e30 gives 0.  The
 * rule of k_argmax (scripts/kindi_q4/kindi/kindi.cu:637-661), launched after the head GEMV by
 * Engine.head (engine.py:323-331).  One launch: workgroups reduce their share and the last one to
 * finish reduces the partials.  ws: kq_argmax_workspace() bytes (8320: 64 keys and a counter, each
 * on its own cache line, so that atomics on one address stay few), 256-byte aligned, zero-filled
 * before its first use (each call leaves it ready for the next); calls sharing a workspace must be
 * ordered (same stream or synchronised).  out: one device int.
 */
size_t kq_argmax_workspace(void);
int kq_argmax(const float* y, int n, void* ws, int* out, void* stream);

/*
 * Output head with the greedy pick fused: y = W xq for one Q8_K token (as kq_gemv_q8k, same bits)
 * and *out = argmax(y) as kq_argmax, which the GEMV workgroups compute from the values they store
 * when C <= 4096 (one column pass), saving the argmax launch and the logits read-back; for larger C
 * a separate argmax launch follows.  Replaces gemv([head]) + k_argmax in Engine.head
 * (engine.py:326-328).  ws and out as for kq_argmax.
 */
int kq_gemv_q8k_argmax(const void* w, int R, int C, int type, const void* xq, float* y, void* ws, int* out,
                       void* stream);

/*
 * Prefill GEMM: Y[m][r] for M >= 1 activation rows (row stride ldy), int8 products with int32
 * accumulation and the fp32 epilogue above.  Slot of the ternary engine's chunk GEMM
 * k_mm_g5q (chunk.cu:820) driven by chunk.feed (chunk.py:378); the Q4 engine itself prefills
 * token by token (gpu4.py:109-110).  Allocates nothing; kq_gemm_q8k_ws below is the faster form.
 */
int kq_gemm_q8k(const void* w, int R, int C, int type, const void* xq, int M, float* y,
                int64_t ldy, void* stream);

/* Bytes of device workspace kq_gemm_q8k_ws needs for R weight rows, C columns, M activation rows
 * (0 for invalid sizes). */
size_t kq_gemm_q8k_workspace(int R, int C, int M);

/*
 * kq_gemm_q8k with a caller-provided workspace (ws 256-byte aligned, ws_bytes at least
 * kq_gemm_q8k_workspace(R, C, M): about M*C bytes with M rounded up to 256, plus S*M*R*4 bytes when
 * the output tiles (64 rows x 128 tokens) are too few to fill the GPU and the K dimension is split
 * S ways (S <= 8, at least 4 super-blocks each; fixed by R, C and M)).  The call first copies the
 * activation quants into ws in MFMA fragment order, so that every operand load of the GEMM is one
 * contiguous 1 KB; a split GEMM writes S partial sums into ws and adds them in order.  The result
 * depends only on the inputs and (R, C, M); it equals kq_gemm_q8k's bit for bit when S = 1 and
 * within the 1e-5 bar otherwise (fp32 sums in another order).  Allocates nothing; calls sharing a
 * workspace must be ordered (same stream or synchronised).
 */
int kq_gemm_q8k_ws(const void* w, int R, int C, int type, const void* xq, int M, float* y,
                   int64_t ldy, void* ws, size_t ws_bytes, void* stream);

/*
 * Up to 3 matrices sharing one Q8_K input (q/k/v, gate/up of a prefill chunk): the prefill GEMM of
 * each, with one fragment copy of the activations for all of them and one GEMM launch per weight
 * type, so the small matrices' tiles fill the GPU together.  The chunked prefill runs one GEMM per
 * projection on each chunk's shared input (chunk.py:165-177, ternary k_mm_g5q chunk.cu:820); the
 * reference's GPU operator takes several matrices on one input the same way
 * (Engine.gemv(names, x, outs), gpu4.py:95-99).  C and M are common; R[i], type[i], y[i] and
 * ldy[i] per matrix.  ws (256-byte aligned) holds kq_gemm_q8k_multi_workspace(n, R, C, M) bytes.
 * Every y[i] equals what kq_gemm_q8k_ws gives for that matrix alone, bit for bit.
 */
size_t kq_gemm_q8k_multi_workspace(int n, const int* R, int C, int M);
int kq_gemm_q8k_multi_ws(int n, const void* const* w, const int* R, int C, const int* type, const void* xq, int M,
                         float* const* y, const int64_t* ldy, void* ws, size_t ws_bytes, void* stream);

/*
 * The same from fp32 activations: x holds M rows of C floats (row stride ldx, 4-byte aligned), which
 * one launch quantizes to Q8_K (as kq_q8k_quantize, same bytes) into the workspace, writing the GEMM's
 * fragment copy at the same time; then the grouped GEMM.  This is the chunked prefill's step: each
 * chunk's hidden states quantized once for the projections that share them (chunk.py:165-177).  ws
 * (256-byte aligned) holds kq_gemm_f32_multi_workspace(n, R, C, M) bytes; every y[i] equals
 * kq_q8k_quantize followed by kq_gemm_q8k_ws on that matrix, bit for bit.
 */
size_t kq_gemm_f32_multi_workspace(int n, const int* R, int C, int M);
int kq_gemm_f32_multi(int n, const void* const* w, const int* R, int C, const int* type, const float* x, int64_t ldx,
                      int M, float* const* y, const int64_t* ldy, void* ws, size_t ws_bytes, void* stream);

/*
 * kq_gemm_q8k_ws without a caller workspace and without any allocation: the workspace is the
 * library's static device array of KQ_GEMM_STATIC_SCRATCH_BYTES (one per device, held until the
 * process ends; a 256-token prefill chunk of every 9B-model matrix fits).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Results are bit-identical to
 * kq_gemm_q8k_ws on the same inputs.  A GEMM whose kq_gemm_q8k_workspace(R, C, M) exceeds the
 * array is rejected with KQ_ERR_ARG before any launch.  The device address of the array is looked
 * up on the first call on each device (the current device; `stream` must belong to it).  Calls on
 * one device share the array: calls that overlap in time on one GPU (different streams, or
 * different threads without ordering) race and give wrong results; calls ordered on one stream are
 * safe.  Nothing in the array needs to start at zero: each call writes what it reads.
 */
#define KQ_GEMM_STATIC_SCRATCH_BYTES (32u << 20)
int kq_gemm_q8k_static(const void* w, int R, int C, int type, const void* xq, int M, float* y,
                       int64_t ldy, void* stream);

/*
 * Exact integer sub-block sums, for parity checks:
 *   Q4_K: sums[((n*R + r)*G + g)*8 + s]  = sum_{j<32} q4 * q8 over sub-block s (q4 in 0..15)
 *   Q6_K: sums[((n*R + r)*G + g)*16 + t] = sum_{j<16} (q6 - 32) * q8 over sub-block t
 * computed by the same per-lane code as kq_gemv_q8k.  No reference counterpart (the reference has
 * no integer dot); these are GGML's aux32 terms before scaling.
 */
int kq_subblock_sums(const void* w, int R, int C, int type, const void* xq, int N, int32_t* sums,
                     void* stream);

/*
 * Decode rows row0 .. row0+nrows-1 to fp32 (row stride ldy floats), bit-identical to
 * kc_dequant (kcpu4.c:341, q4kernels.h:34-36).  With nrows = 1 this is q4_embed
 * (q4.cu:28-32, gpu4.py:100-103).
 */
int kq_dequant_rows(const void* w, int R, int C, int type, int row0, int nrows, float* y,
                    int64_t ldy, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KQ_H */
