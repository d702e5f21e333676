// extern "C" entry points of libkq.so (declared in include/kq.h): argument checks, then launches.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "kq_internal.h"

namespace kq {

// Compute units of the current device (cached per device).
int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

static thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_ptr(const void* p, size_t align, const char* what, const char* fn) {
    if (!p) return fail(KQ_ERR_ARG, "%s: %s is NULL", fn, what);
    if (reinterpret_cast<uintptr_t>(p) % align)
        return fail(KQ_ERR_ARG, "%s: %s must be %zu-byte aligned", fn, what, align);
    return KQ_OK;
}

// Shape rules of the packed tensor (q4pack.py:97-103: rows % 8, ne0 % 256; type in {12, 14}).
int check_matrix(const void* w, int R, int C, int type, const char* fn) {
    if (type != KQ_TYPE_Q4_K && type != KQ_TYPE_Q6_K)
        return fail(KQ_ERR_ARG, "%s: type %d is not Q4_K (12) or Q6_K (14)", fn, type);
    if (R <= 0 || R % 8) return fail(KQ_ERR_ARG, "%s: R=%d must be a positive multiple of 8", fn, R);
    if (C <= 0 || C % 256) return fail(KQ_ERR_ARG, "%s: C=%d must be a positive multiple of 256", fn, C);
    if (C > 61440) return fail(KQ_ERR_ARG, "%s: C=%d exceeds the supported maximum 61440", fn, C);
    return check_ptr(w, 16, "w", fn);
}

int check_launch(const char* fn) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(KQ_ERR_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
    g_err[0] = 0;
    return KQ_OK;
}

}  // namespace kq

using namespace kq;

#define KQ_TRY(expr)            \
    do {                        \
        const int _rc = (expr); \
        if (_rc) return _rc;    \
    } while (0)

extern "C" {

const char* kq_last_error(void) { return g_err; }

int kq_version(void) { return (1 << 16) | 0; }

#ifndef KQ_SOURCE_HASH
#define KQ_SOURCE_HASH "unknown"
#endif
const char* kq_source_hash(void) { return KQ_SOURCE_HASH; }

int kq_gemv(const void* w, int R, int C, int type, const float* x, float* y, void* stream) {
    static const char* fn = "kq_gemv";
    KQ_TRY(check_matrix(w, R, C, type, fn));
    KQ_TRY(check_ptr(x, 4, "x", fn));
    KQ_TRY(check_ptr(y, 4, "y", fn));
    if (R / 8 > (1 << 27)) return fail(KQ_ERR_ARG, "%s: R=%d too large for one call", fn, R);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    launch_gemv_f32_group(1, &wb, &R, C, type, x, &y, as_stream(stream));
    return check_launch(fn);
}

int kq_gemv_multi(int n, const void* const* w, const int* R, int C, const int* type,
                  const float* x, float* const* y, void* stream) {
    static const char* fn = "kq_gemv_multi";
    if (n < 1 || n > 3) return fail(KQ_ERR_ARG, "%s: n=%d must be 1..3", fn, n);
    if (!w || !R || !type || !y) return fail(KQ_ERR_ARG, "%s: NULL array argument", fn);
    int64_t tiles = 0;
    for (int i = 0; i < n; i++) {
        KQ_TRY(check_matrix(w[i], R[i], C, type[i], fn));
        KQ_TRY(check_ptr(y[i], 4, "y[i]", fn));
        tiles += R[i] / 8;
    }
    if (tiles > (1 << 27)) return fail(KQ_ERR_ARG, "%s: too many rows in one call", fn);
    KQ_TRY(check_ptr(x, 4, "x", fn));
    // both weight types (a Q4_K_M layer's q, k and Q6_K v): one launch where possible
    {
        const uint8_t* wa[3];
        for (int i = 0; i < n; i++) wa[i] = static_cast<const uint8_t*>(w[i]);
        if (launch_gemv_f32_mixed(n, wa, R, type, C, x, y, as_stream(stream))) return check_launch(fn);
    }
    // matrices of the same type share a launch
    for (int ty : {KQ_TYPE_Q4_K, KQ_TYPE_Q6_K}) {
        const uint8_t* ws[3];
        int rs[3];
        float* ys[3];
        int k = 0;
        for (int i = 0; i < n; i++)
            if (type[i] == ty) { ws[k] = static_cast<const uint8_t*>(w[i]); rs[k] = R[i]; ys[k] = y[i]; k++; }
        if (k) launch_gemv_f32_group(k, ws, rs, C, ty, x, ys, as_stream(stream));
    }
    return check_launch(fn);
}

int kq_q8k_quantize(const float* x, int64_t ldx, int C, int N, void* xq, void* stream) {
    static const char* fn = "kq_q8k_quantize";
    if (C <= 0 || C % 256) return fail(KQ_ERR_ARG, "%s: C=%d must be a positive multiple of 256", fn, C);
    if (N <= 0) return fail(KQ_ERR_ARG, "%s: N=%d must be positive", fn, N);
    if (ldx < C) return fail(KQ_ERR_ARG, "%s: ldx=%lld is smaller than C=%d", fn, (long long)ldx, C);
    if ((int64_t)N * (C / 256) > 0x7fffffffLL)
        return fail(KQ_ERR_ARG, "%s: N*C/256 exceeds 2^31-1 blocks", fn);
    KQ_TRY(check_ptr(x, 4, "x", fn));
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    launch_q8k_quantize(x, ldx, C, N, static_cast<uint8_t*>(xq), as_stream(stream));
    return check_launch(fn);
}

int kq_rms_q8k(float* h, const float* residual, int add, const float* w, int D, int N, int64_t ld, float* xn,
               void* xq, void* stream) {
    static const char* fn = "kq_rms_q8k";
    if (D <= 0 || D % 256 || D > 16384)   // the kernel's per-thread row share (RMS_DMAX)
        return fail(KQ_ERR_ARG, "%s: D=%d must be a positive multiple of 256, at most 16384", fn, D);
    if (N <= 0 || N > 65535) return fail(KQ_ERR_ARG, "%s: N=%d must be 1..65535", fn, N);
    if (ld < D) return fail(KQ_ERR_ARG, "%s: ld=%lld is smaller than D=%d", fn, (long long)ld, D);
    KQ_TRY(check_ptr(h, 4, "h", fn));
    KQ_TRY(check_ptr(w, 4, "w", fn));
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    if (add) KQ_TRY(check_ptr(residual, 4, "residual", fn));
    if (xn) KQ_TRY(check_ptr(xn, 4, "xn", fn));
    launch_rms_q8k(h, add ? residual : nullptr, add ? 1 : 0, w, D, N, ld, xn, static_cast<uint8_t*>(xq),
                   as_stream(stream));
    return check_launch(fn);
}

int kq_swiglu_q8k(const float* gate, const float* up, int n, int N, int64_t ld, float* y, void* xq,
                  void* stream) {
    static const char* fn = "kq_swiglu_q8k";
    if (n <= 0 || n % 256) return fail(KQ_ERR_ARG, "%s: n=%d must be a positive multiple of 256", fn, n);
    if (N <= 0) return fail(KQ_ERR_ARG, "%s: N=%d must be positive", fn, N);
    if (ld < n) return fail(KQ_ERR_ARG, "%s: ld=%lld is smaller than n=%d", fn, (long long)ld, n);
    if ((int64_t)N * (n / 256) > 0x7fffffffLL) return fail(KQ_ERR_ARG, "%s: N*n/256 exceeds 2^31-1 blocks", fn);
    KQ_TRY(check_ptr(gate, 4, "gate", fn));
    KQ_TRY(check_ptr(up, 4, "up", fn));
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    if (y) KQ_TRY(check_ptr(y, 4, "y", fn));
    launch_swiglu_q8k(gate, up, n, N, ld, y, static_cast<uint8_t*>(xq), as_stream(stream));
    return check_launch(fn);
}

size_t kq_argmax_workspace(void) { return argmax_workspace_bytes(); }

static int check_argmax_ws(const void* ws, const int* out, const char* fn) {
    KQ_TRY(check_ptr(ws, 256, "ws", fn));
    return check_ptr(out, 4, "out", fn);
}

int kq_argmax(const float* y, int n, void* ws, int* out, void* stream) {
    static const char* fn = "kq_argmax";
    if (n <= 0) return fail(KQ_ERR_ARG, "%s: n=%d must be positive", fn, n);
    KQ_TRY(check_ptr(y, 4, "y", fn));
    KQ_TRY(check_argmax_ws(ws, out, fn));
    launch_argmax(y, n, static_cast<uint8_t*>(ws), out, as_stream(stream));
    return check_launch(fn);
}

int kq_gemv_q8k_argmax(const void* w, int R, int C, int type, const void* xq, float* y, void* ws, int* out,
                       void* stream) {
    static const char* fn = "kq_gemv_q8k_argmax";
    KQ_TRY(check_matrix(w, R, C, type, fn));
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    KQ_TRY(check_ptr(y, 4, "y", fn));
    KQ_TRY(check_argmax_ws(ws, out, fn));
    launch_gemv_q8k_argmax(static_cast<const uint8_t*>(w), R, C, type, static_cast<const uint8_t*>(xq), y,
                           static_cast<uint8_t*>(ws), out, as_stream(stream));
    return check_launch(fn);
}

int kq_gemv_q8k(const void* w, int R, int C, int type, const void* xq, int N, float* y,
                int64_t ldy, void* stream) {
    static const char* fn = "kq_gemv_q8k";
    KQ_TRY(check_matrix(w, R, C, type, fn));
    if (N < 1 || N > KQ_MAX_BATCH) return fail(KQ_ERR_ARG, "%s: N=%d must be 1..%d", fn, N, KQ_MAX_BATCH);
    if (N > 1 && ldy < R) return fail(KQ_ERR_ARG, "%s: ldy=%lld is smaller than R=%d", fn, (long long)ldy, R);
    if (R / 8 > (1 << 27)) return fail(KQ_ERR_ARG, "%s: R=%d too large for one call", fn, R);
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    KQ_TRY(check_ptr(y, 4, "y", fn));
    launch_gemv_q8k(static_cast<const uint8_t*>(w), R, C, type, static_cast<const uint8_t*>(xq), N, y,
                    ldy, as_stream(stream));
    return check_launch(fn);
}

int kq_gemv_q8k_x(int n, const void* const* w, const int* R, int C, const int* type, const float* x,
                  float* const* y, void* xq, void* stream) {
    static const char* fn = "kq_gemv_q8k_x";
    if (n < 1 || n > 3) return fail(KQ_ERR_ARG, "%s: n=%d must be 1..3", fn, n);
    if (!w || !R || !type || !y) return fail(KQ_ERR_ARG, "%s: NULL array argument", fn);
    int64_t tiles = 0;
    for (int i = 0; i < n; i++) {
        KQ_TRY(check_matrix(w[i], R[i], C, type[i], fn));
        KQ_TRY(check_ptr(y[i], 4, "y[i]", fn));
        tiles += R[i] / 8;
    }
    if (tiles > (1 << 27)) return fail(KQ_ERR_ARG, "%s: too many rows in one call", fn);
    KQ_TRY(check_ptr(x, 16, "x", fn));
    if (xq) KQ_TRY(check_ptr(xq, 4, "xq", fn));
    uint8_t* xq8 = static_cast<uint8_t*>(xq);
    if (C > 4096) {   // more than one column pass: the quantizer's own launch, then the grouped GEMV
        if (!xq8) return fail(KQ_ERR_ARG, "%s: C=%d > 4096 needs the xq buffer", fn, C);
        launch_q8k_quantize(x, C, C, 1, xq8, as_stream(stream));
        const int64_t ld[3] = {R[0], n > 1 ? R[1] : 0, n > 2 ? R[2] : 0};
        return kq_gemv_q8k_multi(n, w, R, C, type, xq8, 1, y, ld, stream);
    }
    {   // both weight types: one launch where possible
        const uint8_t* wa[3];
        for (int i = 0; i < n; i++) wa[i] = static_cast<const uint8_t*>(w[i]);
        if (launch_gemv_q8k_x_mixed(n, wa, R, type, C, x, y, xq8, as_stream(stream))) return check_launch(fn);
    }
    bool first = true;
    for (int ty : {KQ_TYPE_Q4_K, KQ_TYPE_Q6_K}) {
        const uint8_t* ws[3];
        int rs[3];
        float* ys[3];
        int k = 0;
        for (int i = 0; i < n; i++)
            if (type[i] == ty) { ws[k] = static_cast<const uint8_t*>(w[i]); rs[k] = R[i]; ys[k] = y[i]; k++; }
        if (!k) continue;
        launch_gemv_q8k_x_group(k, ws, rs, C, ty, x, ys, first ? xq8 : nullptr, as_stream(stream));
        first = false;
    }
    return check_launch(fn);
}

int kq_gemv_q8k_multi(int n, const void* const* w, const int* R, int C, const int* type, const void* xq,
                      int N, float* const* y, const int64_t* ldy, void* stream) {
    static const char* fn = "kq_gemv_q8k_multi";
    if (n < 1 || n > 3) return fail(KQ_ERR_ARG, "%s: n=%d must be 1..3", fn, n);
    if (!w || !R || !type || !y || !ldy) return fail(KQ_ERR_ARG, "%s: NULL array argument", fn);
    if (N < 1 || N > KQ_MAX_BATCH) return fail(KQ_ERR_ARG, "%s: N=%d must be 1..%d", fn, N, KQ_MAX_BATCH);
    int64_t tiles = 0;
    for (int i = 0; i < n; i++) {
        KQ_TRY(check_matrix(w[i], R[i], C, type[i], fn));
        KQ_TRY(check_ptr(y[i], 4, "y[i]", fn));
        if (N > 1 && ldy[i] < R[i]) return fail(KQ_ERR_ARG, "%s: ldy[%d] is smaller than R", fn, i);
        tiles += R[i] / 8;
    }
    if (tiles > (1 << 27)) return fail(KQ_ERR_ARG, "%s: too many rows in one call", fn);
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    // one token over both weight types (a Q4_K_M layer's q, k and Q6_K v): one launch where possible
    if (N == 1) {
        const uint8_t* wa[3];
        for (int i = 0; i < n; i++) wa[i] = static_cast<const uint8_t*>(w[i]);
        if (launch_gemv_q8k_mixed(n, wa, R, type, C, static_cast<const uint8_t*>(xq), y, as_stream(stream)))
            return check_launch(fn);
    }
    // matrices of the same type share a launch
    for (int ty : {KQ_TYPE_Q4_K, KQ_TYPE_Q6_K}) {
        const uint8_t* ws[3];
        int rs[3];
        float* ys[3];
        int64_t ls[3];
        int k = 0;
        for (int i = 0; i < n; i++)
            if (type[i] == ty) {
                ws[k] = static_cast<const uint8_t*>(w[i]); rs[k] = R[i]; ys[k] = y[i]; ls[k] = N > 1 ? ldy[i] : R[i];
                k++;
            }
        if (k) launch_gemv_q8k_group(k, ws, rs, C, ty, static_cast<const uint8_t*>(xq), N, ys, ls, as_stream(stream));
    }
    return check_launch(fn);
}

// A GEMM's matrix, M and output (the activations are checked by the caller).
static int check_gemm_out(const void* w, int R, int C, int type, int M, const float* y, int64_t ldy, const char* fn) {
    KQ_TRY(check_matrix(w, R, C, type, fn));
    if (M < 1) return fail(KQ_ERR_ARG, "%s: M=%d must be positive", fn, M);
    if (M > 1 && ldy < R) return fail(KQ_ERR_ARG, "%s: ldy=%lld is smaller than R=%d", fn, (long long)ldy, R);
    KQ_TRY(check_ptr(y, 4, "y", fn));
    if ((int64_t)M * (C / 256) > 0x7fffffffLL) return fail(KQ_ERR_ARG, "%s: M*C/256 too large", fn);
    return KQ_OK;
}

static int check_gemm(const void* w, int R, int C, int type, const void* xq, int M, const float* y, int64_t ldy,
                      const char* fn) {
    KQ_TRY(check_gemm_out(w, R, C, type, M, y, ldy, fn));
    return check_ptr(xq, 4, "xq", fn);
}

int kq_gemm_q8k(const void* w, int R, int C, int type, const void* xq, int M, float* y,
                int64_t ldy, void* stream) {
    static const char* fn = "kq_gemm_q8k";
    KQ_TRY(check_gemm(w, R, C, type, xq, M, y, ldy, fn));
    launch_gemm_q8k(static_cast<const uint8_t*>(w), R, C, type, static_cast<const uint8_t*>(xq), M, y, ldy,
                    nullptr, as_stream(stream));
    return check_launch(fn);
}

size_t kq_gemm_q8k_workspace(int R, int C, int M) {
    if (R < 8 || R % 8 || C < 256 || C % 256 || M < 1) return 0;
    return gemm_q8k_workspace(R, C, M);
}

int kq_gemm_q8k_ws(const void* w, int R, int C, int type, const void* xq, int M, float* y,
                   int64_t ldy, void* ws, size_t ws_bytes, void* stream) {
    static const char* fn = "kq_gemm_q8k_ws";
    KQ_TRY(check_gemm(w, R, C, type, xq, M, y, ldy, fn));
    KQ_TRY(check_ptr(ws, 256, "ws", fn));
    const size_t need = gemm_q8k_workspace(R, C, M);
    if (ws_bytes < need) return fail(KQ_ERR_ARG, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
    launch_gemm_q8k(static_cast<const uint8_t*>(w), R, C, type, static_cast<const uint8_t*>(xq), M, y, ldy,
                    static_cast<uint8_t*>(ws), as_stream(stream));
    return check_launch(fn);
}

size_t kq_gemm_q8k_multi_workspace(int n, const int* R, int C, int M) {
    if (n < 1 || n > 3 || !R || C < 256 || C % 256 || M < 1) return 0;
    for (int i = 0; i < n; i++)
        if (R[i] < 8 || R[i] % 8) return 0;
    return gemm_q8k_group_workspace(n, R, C, M);
}

int kq_gemm_q8k_multi_ws(int n, const void* const* w, const int* R, int C, const int* type, const void* xq, int M,
                         float* const* y, const int64_t* ldy, void* ws, size_t ws_bytes, void* stream) {
    static const char* fn = "kq_gemm_q8k_multi_ws";
    if (n < 1 || n > 3) return fail(KQ_ERR_ARG, "%s: n=%d must be 1..3", fn, n);
    if (!w || !R || !type || !y || !ldy) return fail(KQ_ERR_ARG, "%s: NULL array argument", fn);
    for (int i = 0; i < n; i++) KQ_TRY(check_gemm(w[i], R[i], C, type[i], xq, M, y[i], ldy[i], fn));
    KQ_TRY(check_ptr(ws, 256, "ws", fn));
    const size_t need = gemm_q8k_group_workspace(n, R, C, M);
    if (ws_bytes < need) return fail(KQ_ERR_ARG, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
    const uint8_t* wb[3];
    for (int i = 0; i < n; i++) wb[i] = static_cast<const uint8_t*>(w[i]);
    launch_gemm_q8k_group(n, wb, R, C, type, static_cast<const uint8_t*>(xq), M, y, ldy, static_cast<uint8_t*>(ws),
                          as_stream(stream));
    return check_launch(fn);
}

size_t kq_gemm_f32_multi_workspace(int n, const int* R, int C, int M) {
    if (!kq_gemm_q8k_multi_workspace(n, R, C, M)) return 0;
    return gemm_f32_group_workspace(n, R, C, M);
}

int kq_gemm_f32_multi(int n, const void* const* w, const int* R, int C, const int* type, const float* x, int64_t ldx,
                      int M, float* const* y, const int64_t* ldy, void* ws, size_t ws_bytes, void* stream) {
    static const char* fn = "kq_gemm_f32_multi";
    if (n < 1 || n > 3) return fail(KQ_ERR_ARG, "%s: n=%d must be 1..3", fn, n);
    if (!w || !R || !type || !y || !ldy) return fail(KQ_ERR_ARG, "%s: NULL array argument", fn);
    KQ_TRY(check_ptr(x, 4, "x", fn));
    if (M > 1 && ldx < C) return fail(KQ_ERR_ARG, "%s: ldx=%lld is smaller than C=%d", fn, (long long)ldx, C);
    for (int i = 0; i < n; i++) KQ_TRY(check_gemm_out(w[i], R[i], C, type[i], M, y[i], ldy[i], fn));
    KQ_TRY(check_ptr(ws, 256, "ws", fn));
    const size_t need = gemm_f32_group_workspace(n, R, C, M);
    if (ws_bytes < need) return fail(KQ_ERR_ARG, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
    const uint8_t* wb[3];
    for (int i = 0; i < n; i++) wb[i] = static_cast<const uint8_t*>(w[i]);
    launch_gemm_f32_group(n, wb, R, C, type, x, ldx, M, y, ldy, static_cast<uint8_t*>(ws), as_stream(stream));
    return check_launch(fn);
}

int kq_gemm_q8k_static(const void* w, int R, int C, int type, const void* xq, int M, float* y,
                       int64_t ldy, void* stream) {
    static const char* fn = "kq_gemm_q8k_static";
    KQ_TRY(check_gemm(w, R, C, type, xq, M, y, ldy, fn));
    const size_t need = gemm_q8k_workspace(R, C, M);
    if (need > KQ_GEMM_STATIC_SCRATCH_BYTES)
        return fail(KQ_ERR_ARG,
                    "%s: R=%d C=%d M=%d needs %zu bytes of workspace, more than the %u-byte static scratch "
                    "(split M into chunks, or use kq_gemm_q8k_ws)", fn, R, C, M, need,
                    (unsigned)KQ_GEMM_STATIC_SCRATCH_BYTES);
    uint8_t* ws = nullptr;
    KQ_TRY(gemm_static_scratch(&ws, fn));
    launch_gemm_q8k(static_cast<const uint8_t*>(w), R, C, type, static_cast<const uint8_t*>(xq), M, y, ldy, ws,
                    as_stream(stream));
    return check_launch(fn);
}

int kq_subblock_sums(const void* w, int R, int C, int type, const void* xq, int N, int32_t* sums,
                     void* stream) {
    static const char* fn = "kq_subblock_sums";
    KQ_TRY(check_matrix(w, R, C, type, fn));
    if (N < 1) return fail(KQ_ERR_ARG, "%s: N=%d must be positive", fn, N);
    KQ_TRY(check_ptr(xq, 4, "xq", fn));
    KQ_TRY(check_ptr(sums, 4, "sums", fn));
    launch_subblock_sums(static_cast<const uint8_t*>(w), R, C, type, static_cast<const uint8_t*>(xq), N,
                         sums, as_stream(stream));
    return check_launch(fn);
}

int kq_dequant_rows(const void* w, int R, int C, int type, int row0, int nrows, float* y,
                    int64_t ldy, void* stream) {
    static const char* fn = "kq_dequant_rows";
    KQ_TRY(check_matrix(w, R, C, type, fn));
    if (nrows < 1 || nrows > 65535) return fail(KQ_ERR_ARG, "%s: nrows=%d must be 1..65535", fn, nrows);
    if (row0 < 0 || row0 > R - nrows)
        return fail(KQ_ERR_ARG, "%s: rows [%d, %d) outside [0, %d)", fn, row0, row0 + nrows, R);
    if (nrows > 1 && ldy < C) return fail(KQ_ERR_ARG, "%s: ldy=%lld is smaller than C=%d", fn, (long long)ldy, C);
    KQ_TRY(check_ptr(y, 4, "y", fn));
    launch_dequant_rows(static_cast<const uint8_t*>(w), R, C, type, row0, nrows, y, ldy, as_stream(stream));
    return check_launch(fn);
}

}  // extern "C"
