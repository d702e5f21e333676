/*
 * kq_oracle.c -- CPU oracle for the Kindi Q4 quantized matrix products.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the oracle: tests/, the smoke check
 * and the CPU-baseline leg of bench.py may call it.  Nothing in the product
 * library (libkq.so) links it, and no product code path falls back to it.
 *
 * It restates, in plain C with every floating-point step spelled out:
 *   - Q4_K / Q6_K block decode               scripts/kindi_q4/kindi/q4kernels.h:12-33
 *   - row decode (kc_dequant)                 q4kernels.h:34-36, kcpu4.c:341
 *   - block addressing of the 8-row layout    q4kernels.h:7-10, q4pack.py:151-160
 *   - the fp32-activation row dot q4_dot      q4kernels.h:37-71 (AVX2 branch: one
 *     8-lane accumulator per row, element e goes to lane e%8 in ascending e, then
 *     a sequential sum of the 8 lanes, multiply-then-add with no contraction)
 *   - kc_matvec (row loop)                    kcpu4.c:337-340
 *   - the Q8_K activation quantizer, GGML block_q8_K semantics (quantize_row_q8_K_ref
 *     in ggml-quants.c of llama.cpp 5e7f6271c06b9104862ab799278a1b7f1323a449, the
 *     commit tests/kindi_q4/reference.cpp and README.md:75 name; ggml is not vendored)
 *   - the integer Q4_K x Q8_K / Q6_K x Q8_K sub-block dot sums (ggml_vec_dot_q4_K_q8_K
 *     and ggml_vec_dot_q6_K_q8_K generic versions, same commit), exposed per sub-block,
 *     and the output evaluated in double from those exact integers;
 *   - the same GGML dot with GGML's own fp32 accumulation order (8 partial lanes),
 *     kept to show that the double evaluation and GGML's fp32 one agree to tolerance;
 *   - the producers of the GEMV inputs: RMSNorm with residual add (q4_rms, q4.cu:39-46,
 *     and the CPU engine's rmsfold, kcpu4.c:123-139) and SwiGLU (q4_silu, q4.cu:36-38;
 *     kcpu4.c:77, 292), with a binary32 exp built from IEEE single operations;
 *   - the greedy pick over the logits, k_argmax (kindi.cu:637-661).
 *
 * Build: gcc -O2 -ffp-contract=off -fopenmp -shared -fPIC (oracle/Makefile).
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>

#define QK 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210
#define Q8K_BYTES 292

static int block_bytes(int type) { return type == 12 ? Q4K_BYTES : Q6K_BYTES; }

/* IEEE binary16 -> binary32, exact for every input (the role of h2f, kcpu4.c:63-69). */
static float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = s;
        else {                                   /* subnormal: renormalise */
            int sh = 0; uint32_t mm = m;
            while (!(mm & 1024)) { mm <<= 1; sh++; }
            u = s | ((uint32_t)(113 - sh) << 23) | ((mm & 1023) << 13);
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &u, 4); return f;
}

static uint16_t rd16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }

/* Block (row, group) of a tensor in the 8-row interleaved layout [R/8][G][8][bs]
 * (q4kernels.h:8-10). */
static const uint8_t* block_at(const uint8_t* W, int C, int type, int row, int g) {
    const size_t G = (size_t)(C / QK);
    return W + (((size_t)(row / 8) * G + (size_t)g) * 8 + (size_t)(row % 8)) * (size_t)block_bytes(type);
}

/* 6-bit scale and min of Q4_K sub-block k (q4kernels.h:17-18). */
static void q4k_scale_min(const uint8_t* s, int k, int* sc, int* mn) {
    if (k < 4) { *sc = s[k] & 63; *mn = s[k + 4] & 63; }
    else { *sc = (s[k + 4] & 15) | ((s[k - 4] >> 6) << 4); *mn = (s[k + 4] >> 4) | ((s[k] >> 6) << 4); }
}

/* Q4_K quant of element e in [0,256): nibble (k%2) of qs[(k/2)*32 + j] (q4kernels.h:20-21). */
static int q4k_quant(const uint8_t* b, int e) {
    const int k = e / 32, j = e % 32;
    return (b[16 + (k / 2) * 32 + j] >> ((k % 2) * 4)) & 15;
}

/* Q6_K unsigned 6-bit quant (0..63) of element e = h*128 + k*32 + j (q4kernels.h:26-28). */
static int q6k_quant(const uint8_t* b, int e) {
    const int h = e / 128, k = (e % 128) / 32, j = e % 32;
    const int low = (b[h * 64 + (k % 2) * 32 + j] >> ((k / 2) * 4)) & 15;
    const int high = (b[128 + h * 32 + j] >> (2 * k)) & 3;
    return low | (high << 4);
}

/* q4_decode (q4kernels.h:12-33): w = (d*sc)*q - (dmin*m) for Q4_K, (d*sc)*(q-32) for Q6_K. */
void kqo_decode_block(const uint8_t* b, int type, float* y) {
    if (type == 12) {
        const float d = h2f(rd16(b)), dm = h2f(rd16(b + 2));
        for (int k = 0; k < 8; k++) {
            int sc, mn; q4k_scale_min(b + 4, k, &sc, &mn);
            const float ds = d * (float)sc, ms = dm * (float)mn;
            for (int j = 0; j < 32; j++) {
                const float t = ds * (float)q4k_quant(b, k * 32 + j);
                y[k * 32 + j] = t - ms;
            }
        }
    } else {
        const float d = h2f(rd16(b + 208));
        const int8_t* s = (const int8_t*)(b + 192);
        for (int e = 0; e < QK; e++) {
            const float ds = d * (float)s[e / 16];
            y[e] = ds * (float)(q6k_quant(b, e) - 32);
        }
    }
}

/* kc_dequant: one row, all groups (q4kernels.h:34-36, kcpu4.c:341). */
void kqo_dequant_row(const uint8_t* W, int R, int C, int type, int row, float* y) {
    (void)R;
    for (int g = 0; g < C / QK; g++) kqo_decode_block(block_at(W, C, type, row, g), type, y + (size_t)g * QK);
}

/* q4_dot AVX2 branch (q4kernels.h:38-71), restated lane by lane.  Lane l of the 8-wide
 * accumulator receives elements e = l (mod 8) in ascending order; each weight is formed as
 * (ds*q) - ms (Q4_K) or ds*q (Q6_K) and added as acc + w*x, two roundings each. */
float kqo_dot_f32(const uint8_t* W, int C, int type, int row, const float* x) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int g = 0; g < C / QK; g++) {
        const uint8_t* b = block_at(W, C, type, row, g);
        const float* in = x + (size_t)g * QK;
        if (type == 12) {
            const float d = h2f(rd16(b)), dm = h2f(rd16(b + 2));
            for (int k = 0; k < 8; k++) {
                int sc, mn; q4k_scale_min(b + 4, k, &sc, &mn);
                const float ds = d * (float)sc, ms = dm * (float)mn;
                for (int j = 0; j < 32; j++) {
                    const int e = k * 32 + j;
                    const float t = ds * (float)q4k_quant(b, e);
                    const float w = t - ms;
                    const float p = w * in[e];
                    lane[e & 7] = lane[e & 7] + p;
                }
            }
        } else {
            const float d = h2f(rd16(b + 208));
            const int8_t* s = (const int8_t*)(b + 192);
            for (int e = 0; e < QK; e++) {
                const float ds = d * (float)s[e / 16];
                const float w = ds * (float)(q6k_quant(b, e) - 32);
                const float p = w * in[e];
                lane[e & 7] = lane[e & 7] + p;
            }
        }
    }
    float total = 0;
    for (int i = 0; i < 8; i++) total += lane[i];
    return total;
}

/* kc_matvec (kcpu4.c:337-340): y[r] = q4_dot(row r), rows split over OpenMP threads. */
void kqo_matvec_f32(const uint8_t* W, int R, int C, int type, const float* x, float* y) {
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < R; r++) y[r] = kqo_dot_f32(W, C, type, r, x);
}

/* ---------------------------------------------------------------- Q8_K (GGML block_q8_K) */
/* Block: float d; int8 qs[256]; int16 bsums[16]  (292 bytes, packed). */

static int nearest_int(float v) {                /* GGML nearest_int: round half to even */
    const float t = v + 12582912.f;              /* 1.5 * 2^23 */
    int32_t i; memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* quantize_row_q8_K_ref: max is the signed value of the first element of largest |x|;
 * iscale = -127/max; q = min(127, nearest_int(iscale*x)); d = 1/iscale; bsums are sums of 16
 * consecutive q.  An all-zero block gives d = 0, q = 0 (GGML leaves bsums unwritten there;
 * here they are written as 0, the sum of the zero quants). */
void kqo_quantize_q8k(const float* x, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n / QK; i++) {
        const float* xb = x + i * QK;
        uint8_t* ob = out + i * Q8K_BYTES;
        float amax = 0, max = 0;
        for (int j = 0; j < QK; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        int8_t qs[QK]; int16_t bs[16]; float d;
        if (amax == 0.0f) {
            d = 0; memset(qs, 0, sizeof qs); memset(bs, 0, sizeof bs);
        } else {
            const float iscale = -127.f / max;
            for (int j = 0; j < QK; j++) {
                const float t = iscale * xb[j];
                const int v = nearest_int(t);
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            for (int j = 0; j < 16; j++) {
                int s = 0;
                for (int l = 0; l < 16; l++) s += qs[j * 16 + l];
                bs[j] = (int16_t)s;
            }
            d = 1 / iscale;
        }
        memcpy(ob, &d, 4); memcpy(ob + 4, qs, QK); memcpy(ob + 4 + QK, bs, 32);
    }
}

/* Integer sub-block sums for row `row` against one Q8_K activation row `xq` (G blocks):
 *   Q4_K: S[g*8 + s]  = sum_{j<32} q4(32s+j) * q8(32s+j)          (unsigned nibble x int8)
 *   Q6_K: S[g*16 + t] = sum_{j<16} (q6(16t+j) - 32) * q8(16t+j)   (signed 6-bit x int8)
 * These are the aux32 contributions before the scale multiply in GGML's generic dots. */
static void row_subblock_sums(const uint8_t* W, int C, int type, int row, const uint8_t* xq, int32_t* S) {
    const int G = C / QK;
    for (int g = 0; g < G; g++) {
        const uint8_t* b = block_at(W, C, type, row, g);
        const int8_t* q8 = (const int8_t*)(xq + (size_t)g * Q8K_BYTES + 4);
        if (type == 12) {
            for (int s = 0; s < 8; s++) {
                int32_t acc = 0;
                for (int j = 0; j < 32; j++) acc += q4k_quant(b, s * 32 + j) * (int32_t)q8[s * 32 + j];
                S[g * 8 + s] = acc;
            }
        } else {
            for (int t = 0; t < 16; t++) {
                int32_t acc = 0;
                for (int j = 0; j < 16; j++) acc += (q6k_quant(b, t * 16 + j) - 32) * (int32_t)q8[t * 16 + j];
                S[g * 16 + t] = acc;
            }
        }
    }
}

/* Sub-block sums for N activation rows: S[((n*R + r) * G + g) * nsub + s], nsub = 8 or 16. */
void kqo_subblock_sums(const uint8_t* W, int R, int C, int type, const uint8_t* xq, int N, int32_t* S) {
    const int G = C / QK, nsub = type == 12 ? 8 : 16;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++)
        for (int r = 0; r < R; r++)
            row_subblock_sums(W, C, type, r, xq + (size_t)n * G * Q8K_BYTES,
                              S + ((size_t)n * R + r) * (size_t)G * nsub);
}

/* y[n][r] from the exact integer sums, epilogue in double:
 *   Q4_K: sum_g d*dx * sum_s sc_s*S_s  -  dmin*dx * sum_s m_s*(b_{2s} + b_{2s+1})
 *   Q6_K: sum_g d*dx * sum_t sc_t*S_t
 * d, dmin are the fp16 block scales widened exactly, dx the Q8_K block's fp32 d. */
void kqo_gemv_q8k(const uint8_t* W, int R, int C, int type, const uint8_t* xq, int N, double* y, int64_t ldy) {
    const int G = C / QK;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++)
        for (int r = 0; r < R; r++) {
            int32_t S[16];
            double acc = 0;
            for (int g = 0; g < G; g++) {
                const uint8_t* b = block_at(W, C, type, r, g);
                const uint8_t* xb = xq + ((size_t)n * G + g) * Q8K_BYTES;
                float dxf; memcpy(&dxf, xb, 4);
                const double dx = dxf;
                const int16_t* bs = (const int16_t*)(xb + 4 + QK);
                const int8_t* q8 = (const int8_t*)(xb + 4);
                if (type == 12) {
                    int64_t I1 = 0, I2 = 0;
                    for (int s = 0; s < 8; s++) {
                        int32_t acc_s = 0;
                        for (int j = 0; j < 32; j++) acc_s += q4k_quant(b, s * 32 + j) * (int32_t)q8[s * 32 + j];
                        S[s] = acc_s;
                        int sc, mn; q4k_scale_min(b + 4, s, &sc, &mn);
                        I1 += (int64_t)sc * S[s];
                        I2 += (int64_t)mn * ((int64_t)bs[2 * s] + bs[2 * s + 1]);
                    }
                    acc += (double)h2f(rd16(b)) * dx * (double)I1 - (double)h2f(rd16(b + 2)) * dx * (double)I2;
                } else {
                    const int8_t* sc = (const int8_t*)(b + 192);
                    int64_t I = 0;
                    for (int t = 0; t < 16; t++) {
                        int32_t acc_t = 0;
                        for (int j = 0; j < 16; j++) acc_t += (q6k_quant(b, t * 16 + j) - 32) * (int32_t)q8[t * 16 + j];
                        I += (int64_t)sc[t] * acc_t;
                    }
                    acc += (double)h2f(rd16(b + 208)) * dx * (double)I;
                }
            }
            y[(size_t)n * ldy + r] = acc;
        }
}

/* GGML's generic fp32 order for one row (ggml_vec_dot_q{4,6}_K_q8_K_generic): per block the
 * integer products accumulate into 8 int32 lanes (aux32[l], l = element % 8 within each group
 * of 8, scaled by the sub-block scale); then sums[l] += (d*dx) * aux32[l]; Q4_K also keeps
 * sumf -= (dmin*dx) * sumi with sumi = sum_j bsums[j]*m[j/2]; finally sumf += sums[l]. */
float kqo_dot_q8k_ggml(const uint8_t* W, int C, int type, int row, const uint8_t* xq) {
    const int G = C / QK;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sumf = 0;
    for (int g = 0; g < G; g++) {
        const uint8_t* b = block_at(W, C, type, row, g);
        const uint8_t* xb = xq + (size_t)g * Q8K_BYTES;
        float dx; memcpy(&dx, xb, 4);
        const int8_t* q8 = (const int8_t*)(xb + 4);
        const int16_t* bs = (const int16_t*)(xb + 4 + QK);
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (type == 12) {
            int sumi = 0;
            for (int j = 0; j < 16; j++) { int sc, mn; q4k_scale_min(b + 4, j / 2, &sc, &mn); sumi += bs[j] * mn; }
            for (int e = 0; e < QK; e++) {
                int sc, mn; q4k_scale_min(b + 4, e / 32, &sc, &mn);
                aux32[e & 7] += sc * (int32_t)(int16_t)(q8[e] * q4k_quant(b, e));
            }
            const float d = h2f(rd16(b)) * dx;
            for (int l = 0; l < 8; l++) { const float t = d * (float)aux32[l]; sums[l] = sums[l] + t; }
            const float dmin = h2f(rd16(b + 2)) * dx;
            const float t = dmin * (float)sumi;
            sumf = sumf - t;
        } else {
            const int8_t* sc = (const int8_t*)(b + 192);
            for (int e = 0; e < QK; e++)
                aux32[e & 7] += sc[e / 16] * (int32_t)(int16_t)(q8[e] * (q6k_quant(b, e) - 32));
            const float d = h2f(rd16(b + 208)) * dx;
            for (int l = 0; l < 8; l++) { const float t = d * (float)aux32[l]; sums[l] = sums[l] + t; }
        }
    }
    for (int l = 0; l < 8; l++) sumf += sums[l];
    return sumf;
}

void kqo_gemv_q8k_ggml(const uint8_t* W, int R, int C, int type, const uint8_t* xq, int N, float* y, int64_t ldy) {
    const int G = C / QK;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++)
        for (int r = 0; r < R; r++)
            y[(size_t)n * ldy + r] = kqo_dot_q8k_ggml(W, C, type, r, xq + (size_t)n * G * Q8K_BYTES);
}

/* ------------------------------------------------------------------ producers of the GEMV inputs */

/* exp(x) in binary32 from IEEE single operations in a fixed order: Cody-Waite reduction
 * r = x - n ln2 (ln2 split in 0x1.62e4p-1, whose 15 significant bits make n * it exact, and
 * 0x1.7f7d1cp-20), e^r by its degree-7 Taylor polynomial in Horner form (|r| <= ln2/2, truncation
 * below 0.1 ulp), then exact scaling by 2^n (two steps below the normal range, one rounding).
 * The library's kernels evaluate the same steps, so both give the same bits.  Compiled with
 * -ffp-contract=off: no step is fused. */
static float pow2i(int k) { uint32_t u = (uint32_t)(k + 127) << 23; float f; memcpy(&f, &u, 4); return f; }

float kqo_expf(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep+6f) return INFINITY;
    if (x < -0x1.9fe368p+6f) return 0.0f;
    const float n = rintf(x * 0x1.715476p+0f);
    const float r = (x - n * 0x1.62e4p-1f) - n * 0x1.7f7d1cp-20f;
    float p = 0x1.a01a02p-13f;
    p = p * r + 0x1.6c16c2p-10f;
    p = p * r + 0x1.111112p-7f;
    p = p * r + 0x1.555556p-5f;
    p = p * r + 0x1.555556p-3f;
    p = p * r + 0x1p-1f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    int k = (int)n;
    if (k > 127) { p = p * 2.0f; k -= 1; }
    if (k < -126) return (p * pow2i(k + 64)) * 0x1p-64f;
    return p * pow2i(k);
}

/* q4_rms (scripts/kindi_q4/kindi/q4.cu:39-46) for one row: optional residual add into h, sum of
 * squares in double in that kernel's order (thread t of 256 adds i = t, t+256, ... in sequence,
 * then sums[t] += sums[t+n] for n = 128, 64, ..., 1), s = 1/sqrtf((float)(sum/D) + 1e-6f),
 * xn = (h*s)*w.  order = 1 sums sequentially instead, as the CPU engine's rmsfold does
 * (kcpu4.c:123-139). */
void kqo_rms_norm(float* h, const float* res, int add, const float* w, int D, float* xn, int order) {
    double acc;
    if (add) for (int i = 0; i < D; i++) h[i] = h[i] + res[i];
    if (order == 1) {
        acc = 0.0;
        for (int i = 0; i < D; i++) acc += (double)h[i] * (double)h[i];
    } else {
        double sums[256];
        for (int t = 0; t < 256; t++) {
            double s = 0.0;
            for (int i = t; i < D; i += 256) s += (double)h[i] * (double)h[i];
            sums[t] = s;
        }
        for (int n = 128; n; n >>= 1)
            for (int t = 0; t < n; t++) sums[t] += sums[t + n];
        acc = sums[0];
    }
    const float s = 1.0f / sqrtf((float)(acc / D) + 1e-6f);
    for (int i = 0; i < D; i++) xn[i] = (h[i] * s) * w[i];
}

/* silu(g) * u (q4_silu, q4.cu:36-38; kcpu4.c:77, 292) with kqo_expf. */
void kqo_swiglu(const float* g, const float* u, int64_t n, float* y) {
    for (int64_t i = 0; i < n; i++) y[i] = (g[i] / (1.0f + kqo_expf(-g[i]))) * u[i];
}

void kqo_expf_n(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; i++) y[i] = kqo_expf(x[i]);
}

/* ------------------------------------------------------------------ greedy pick */

/* k_argmax (scripts/kindi_q4/kindi/kindi.cu:637-661): 1024 threads, thread t scans
 * e = t, t+1024, ... keeping the first strictly larger value (start -1e30, index 0), then a
 * halving tree that prefers the larger value and, on equal values, the smaller index. */
int kqo_argmax(const float* y, int64_t n) {
    float bval[1024];
    int bidx[1024];
    for (int t = 0; t < 1024; t++) {
        float bv = -1e30f;
        int bi = 0;
        for (int64_t e = t; e < n; e += 1024) {
            const float v = y[e];
            if (v > bv) { bv = v; bi = (int)e; }
        }
        bval[t] = bv; bidx[t] = bi;
    }
    for (int st = 512; st > 0; st >>= 1)
        for (int t = 0; t < st; t++) {
            const int i2 = t + st;
            if (bval[i2] > bval[t] || (bval[i2] == bval[t] && bidx[i2] < bidx[t])) {
                bval[t] = bval[i2]; bidx[t] = bidx[i2];
            }
        }
    return bidx[0];
}
