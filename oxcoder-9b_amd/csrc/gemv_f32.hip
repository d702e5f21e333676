// Row decode (kc_dequant / q4_embed) and the exact integer sub-block sums for parity checks.  The
// fp32-activation GEMV itself (kq_gemv, Kindi's q4_gemv numerics) runs on the kernels of the Q8_K
// GEMV with fp32 activations (gemv_q8k.hip, ActF32).
#include "kq_device.h"
#include "kq_internal.h"
#include "q4_lanes.h"

namespace kq {

// ----------------------------------------------------------------------------- row decode
// One thread per element, the arithmetic of q4_decode (q4kernels.h:12-33) step for step:
// Q4_K y = (d*sc)*q - (dmin*m), Q6_K y = (d*sc)*(q-32); compiled without contraction.
__global__ void __launch_bounds__(256)
k_dequant_rows(const uint8_t* __restrict__ W, int C, int type, int row0, float* __restrict__ Y, int64_t ldy) {
    const int G = C / QK;
    const int n = blockIdx.y;
    const int row = row0 + n;
    const int g = blockIdx.x, e = threadIdx.x;
    const int bs = type == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    const uint8_t* b = W + (((int64_t)(row / 8) * G + g) * 8 + (row % 8)) * bs;
    float out;
    if (type == TYPE_Q4_K) {
        const float d = f16_lo((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        const float dm = f16_lo((uint32_t)b[2] | ((uint32_t)b[3] << 8));
        const uint8_t* s = b + 4;
        const int k = e >> 5, j = e & 31;
        const int sc = k < 4 ? (s[k] & 63) : ((s[k + 4] & 15) | ((s[k - 4] >> 6) << 4));
        const int mn = k < 4 ? (s[k + 4] & 63) : ((s[k + 4] >> 4) | ((s[k] >> 6) << 4));
        const int q = (b[16 + (k >> 1) * 32 + j] >> ((k & 1) * 4)) & 15;
        const float ds = d * (float)sc, ms = dm * (float)mn;
        out = ds * (float)q - ms;
    } else {
        const float d = f16_lo((uint32_t)b[208] | ((uint32_t)b[209] << 8));
        const int h = e >> 7, k = (e & 127) >> 5, j = e & 31;
        const int low = (b[h * 64 + (k & 1) * 32 + j] >> ((k >> 1) * 4)) & 15;
        const int high = (b[128 + h * 32 + j] >> (2 * k)) & 3;
        const float ds = d * (float)(int8_t)b[192 + (e >> 4)];
        out = ds * (float)((low | (high << 4)) - 32);
    }
    Y[(int64_t)n * ldy + (int64_t)g * QK + e] = out;
}

void launch_dequant_rows(const uint8_t* w, int R, int C, int type, int row0, int nrows, float* y,
                         int64_t ldy, hipStream_t s) {
    (void)R;
    dim3 grid(C / QK, nrows), block(QK);
    hipLaunchKernelGGL(k_dequant_rows, grid, block, 0, s, w, C, type, row0, y, ldy);
}

// ----------------------------------------------------------------------------- sub-block sums
// One wave per (token, row); lanes as in the Q8_K GEMV, writing the exact per-sub-block sums.
__global__ void __launch_bounds__(256)
k_subblock_sums(const uint8_t* __restrict__ W, int R, int G, int type, const uint8_t* __restrict__ XQ,
                int N, int32_t* __restrict__ S) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (wave >= (int64_t)N * R) return;
    const int n = (int)(wave / R), row = (int)(wave - (int64_t)n * R);
    const int p = lane & 3, slot = lane >> 2;
    const int bs = type == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    for (int g = slot; g < G; g += 16) {
        const uint8_t* bk = W + (((int64_t)(row / 8) * G + g) * 8 + (row % 8)) * bs;
        const uint8_t* xb = XQ + ((int64_t)n * G + g) * Q8K_BYTES;
        int32_t* out = S + (((int64_t)n * R + row) * G + g) * (type == TYPE_Q4_K ? 8 : 16);
        if (type == TYPE_Q4_K) {
            const u32x4 qa = ld16(bk + 16 + 32 * p), qb = ld16(bk + 32 + 32 * p);
            uint32_t xl[8], xh[8];
            const u32x4 a0 = ld16_a4(xb + 4 + 64 * p), a1 = ld16_a4(xb + 20 + 64 * p);
            const u32x4 a2 = ld16_a4(xb + 36 + 64 * p), a3 = ld16_a4(xb + 52 + 64 * p);
            xl[0] = a0.x; xl[1] = a0.y; xl[2] = a0.z; xl[3] = a0.w;
            xl[4] = a1.x; xl[5] = a1.y; xl[6] = a1.z; xl[7] = a1.w;
            xh[0] = a2.x; xh[1] = a2.y; xh[2] = a2.z; xh[3] = a2.w;
            xh[4] = a3.x; xh[5] = a3.y; xh[6] = a3.z; xh[7] = a3.w;
            int plo, phi;
            q4k_lane_dots(qa, qb, xl, xh, plo, phi);
            out[2 * p] = plo;
            out[2 * p + 1] = phi;
        } else {
            const int h = p >> 1, jj = p & 1;
            const u32x4 l0 = ld16_a2(bk + h * 64 + 16 * jj);
            const u32x4 l1 = ld16_a2(bk + h * 64 + 32 + 16 * jj);
            const u32x4 hb = ld16_a2(bk + 128 + h * 32 + 16 * jj);
            uint32_t xa[16];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const u32x4 a = ld16_a4(xb + 4 + h * 128 + k * 32 + 16 * jj);
                xa[4 * k + 0] = a.x; xa[4 * k + 1] = a.y; xa[4 * k + 2] = a.z; xa[4 * k + 3] = a.w;
            }
            const u32x4 bsv = ld16_a4(xb + 260 + 16 * h);
            const uint32_t bw[4] = {bsv.x, bsv.y, bsv.z, bsv.w};
            int P[4];
            q6k_lane_dots(l0, l1, hb, xa, P);
#pragma unroll
            for (int k = 0; k < 4; k++) out[8 * h + 2 * k + jj] = P[k] - 32 * shalf(bw[k], jj);
        }
    }
}

void launch_subblock_sums(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int N,
                          int32_t* sums, hipStream_t s) {
    const int64_t waves = (int64_t)N * R;
    const int wpb = 4;
    dim3 grid((unsigned)((waves + wpb - 1) / wpb)), block(64 * wpb);
    hipLaunchKernelGGL(k_subblock_sums, grid, block, 0, s, w, R, C / QK, type, xq, N, sums);
}

}  // namespace kq
