// fp32-activation Q4_K / Q6_K GEMV for gfx950: the numerics of Kindi's q4_gemv / q4_dot
// (scripts/kindi_q4/kindi/q4.cu:18-27, q4kernels.h:37-83) with the work laid out for wave64.
//
// Same lane mapping as the Q8_K GEMV (slot = lane >> 2 walks super-block columns, four lanes per
// super-block).  Per sub-block the weight is w = ds*q - ms (Q4_K) or ds*(q - 32) (Q6_K), so
//   sum_j w_j x_j = ds * sum_j q_j x_j - ms * sum_j x_j        (Q4_K)
//                 = ds * (sum_j q6u_j x_j - 32 * sum_j x_j)     (Q6_K, q6u = q + 32)
// Each lane loads its 64 activations once per column pass, forms their sums, and reuses both for
// every row of the wave; the quants are converted with v_cvt_f32_ubyte and accumulated with fp32
// FMA.  The row result differs from the reference's accumulation order only by fp32 rounding.
#include "kq_device.h"
#include "kq_internal.h"
#include "q4_lanes.h"

namespace kq {

__device__ __forceinline__ float ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xffu); }

// sum over 4 nibble bytes (already masked to 0..15 or 0..63) times 4 activations
__device__ __forceinline__ float dot_bytes(uint32_t q, const float* x, float acc) {
    acc = __builtin_fmaf(ub(q, 0), x[0], acc);
    acc = __builtin_fmaf(ub(q, 1), x[1], acc);
    acc = __builtin_fmaf(ub(q, 2), x[2], acc);
    return __builtin_fmaf(ub(q, 3), x[3], acc);
}

template <int RPW>
__global__ void __launch_bounds__(256)
k_gemv_q4k_f32(const uint8_t* __restrict__ W, const float* __restrict__ X, float* __restrict__ Y, int R, int G) {
    constexpr int WPT = 8 / RPW;
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t tile = wave / WPT;
    if (tile >= R / 8) return;
    const int r0 = (int)(wave - tile * WPT) * RPW;
    const int p = lane & 3, slot = lane >> 2;
    const uint8_t* Wt = W + tile * (int64_t)G * (8 * Q4K_BYTES) + r0 * Q4K_BYTES;

    PassTree tree[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) tree_init(tree[r]);
    const int passes = (G + 15) >> 4;
    for (int pass = 0; pass < passes; pass++) {
        const int g = slot + 16 * pass;
        const bool valid = g < G;
        float xl[32], xh[32];
        float sxl = 0.0f, sxh = 0.0f;
        if (valid) {
            const float* xg = X + (int64_t)g * QK + 64 * p;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const f32x4 a = *reinterpret_cast<const f32x4_a4*>(xg + 4 * k);
                const f32x4 b = *reinterpret_cast<const f32x4_a4*>(xg + 32 + 4 * k);
                xl[4 * k] = a.x; xl[4 * k + 1] = a.y; xl[4 * k + 2] = a.z; xl[4 * k + 3] = a.w;
                xh[4 * k] = b.x; xh[4 * k + 1] = b.y; xh[4 * k + 2] = b.z; xh[4 * k + 3] = b.w;
            }
#pragma unroll
            for (int j = 0; j < 32; j++) { sxl += xl[j]; sxh += xh[j]; }
        } else {
#pragma unroll
            for (int j = 0; j < 32; j++) xl[j] = xh[j] = 0.0f;
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float v = 0.0f;
            if (valid) {
                const uint8_t* bk = Wt + (int64_t)g * (8 * Q4K_BYTES) + r * Q4K_BYTES;
                const u32x4 hdr = ld16(bk), qa = ld16(bk + 16 + 32 * p), qb = ld16(bk + 32 + 32 * p);
                const ScMin sm = q4k_scmin_pair(hdr.y, hdr.z, hdr.w, p);
                const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                float plo = 0.0f, phi = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    plo = dot_bytes(q[k] & 0x0f0f0f0fu, xl + 4 * k, plo);
                    phi = dot_bytes((q[k] >> 4) & 0x0f0f0f0fu, xh + 4 * k, phi);
                }
                const float d = f16_lo(hdr.x), dm = f16_hi(hdr.x);
                const float dsl = d * (float)sm.sc_lo, dsh = d * (float)sm.sc_hi;
                const float msl = dm * (float)sm.m_lo, msh = dm * (float)sm.m_hi;
                v = dsl * plo - msl * sxl + (dsh * phi - msh * sxh);
            }
            v = __fadd_rn(v, __shfl_xor(v, 1, 64));
            v = __fadd_rn(v, __shfl_xor(v, 2, 64));
            tree_push(tree[r], slot_tree_f32(v));
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float y = tree_final(tree[r]);
        if (lane == 0) Y[tile * 8 + r0 + r] = y;
    }
}

template <int RPW>
__global__ void __launch_bounds__(256)
k_gemv_q6k_f32(const uint8_t* __restrict__ W, const float* __restrict__ X, float* __restrict__ Y, int R, int G) {
    constexpr int WPT = 8 / RPW;
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t tile = wave / WPT;
    if (tile >= R / 8) return;
    const int r0 = (int)(wave - tile * WPT) * RPW;
    const int p = lane & 3, slot = lane >> 2;
    const int h = p >> 1, jj = p & 1;
    const uint8_t* Wt = W + tile * (int64_t)G * (8 * Q6K_BYTES) + r0 * Q6K_BYTES;

    PassTree tree[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) tree_init(tree[r]);
    const int passes = (G + 15) >> 4;
    for (int pass = 0; pass < passes; pass++) {
        const int g = slot + 16 * pass;
        const bool valid = g < G;
        float xa[64];           // group k (k=0..3), element j (0..15): xa[16k + j]
        float sx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (valid) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float* xg = X + (int64_t)g * QK + h * 128 + k * 32 + 16 * jj;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const f32x4 a = *reinterpret_cast<const f32x4_a4*>(xg + 4 * w);
                    xa[16 * k + 4 * w] = a.x; xa[16 * k + 4 * w + 1] = a.y;
                    xa[16 * k + 4 * w + 2] = a.z; xa[16 * k + 4 * w + 3] = a.w;
                }
#pragma unroll
                for (int j = 0; j < 16; j++) sx[k] += xa[16 * k + j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 64; j++) xa[j] = 0.0f;
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float v = 0.0f;
            if (valid) {
                const uint8_t* bk = Wt + (int64_t)g * (8 * Q6K_BYTES) + r * Q6K_BYTES;
                const u32x4 l0 = ld16_a2(bk + h * 64 + 16 * jj);
                const u32x4 l1 = ld16_a2(bk + h * 64 + 32 + 16 * jj);
                const u32x4 hb = ld16_a2(bk + 128 + h * 32 + 16 * jj);
                const u32x4 s = ld16_a2(bk + 192);
                const uint32_t dsh = uint32_t(reinterpret_cast<uintptr_t>(bk) & 3);
                const uint32_t dw = ld4(bk + 208 - dsh);
                const float d = f16_lo(dw >> (8 * dsh));
                const uint32_t w0 = h ? s.z : s.x, w1 = h ? s.w : s.y;
                const int sc[4] = {sbyte(w0, jj), sbyte(w0, jj + 2), sbyte(w1, jj), sbyte(w1, jj + 2)};
                const uint32_t L0[4] = {l0.x, l0.y, l0.z, l0.w}, L1[4] = {l1.x, l1.y, l1.z, l1.w};
                const uint32_t H[4] = {hb.x, hb.y, hb.z, hb.w};
                float P[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t m4 = 0x0f0f0f0fu, m2 = 0x30303030u;
                    const uint32_t q0 = (L0[w] & m4) | ((H[w] << 4) & m2);
                    const uint32_t q1 = (L1[w] & m4) | ((H[w] << 2) & m2);
                    const uint32_t q2 = ((L0[w] >> 4) & m4) | (H[w] & m2);
                    const uint32_t q3 = ((L1[w] >> 4) & m4) | ((H[w] >> 2) & m2);
                    P[0] = dot_bytes(q0, xa + 0 * 16 + 4 * w, P[0]);
                    P[1] = dot_bytes(q1, xa + 1 * 16 + 4 * w, P[1]);
                    P[2] = dot_bytes(q2, xa + 2 * 16 + 4 * w, P[2]);
                    P[3] = dot_bytes(q3, xa + 3 * 16 + 4 * w, P[3]);
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float ds = d * (float)sc[k];
                    v += ds * (P[k] - 32.0f * sx[k]);
                }
            }
            v = __fadd_rn(v, __shfl_xor(v, 1, 64));
            v = __fadd_rn(v, __shfl_xor(v, 2, 64));
            tree_push(tree[r], slot_tree_f32(v));
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float y = tree_final(tree[r]);
        if (lane == 0) Y[tile * 8 + r0 + r] = y;
    }
}

template <int RPW>
static void launch_f32_rpw(const uint8_t* w, int R, int G, int type, const float* x, float* y, hipStream_t s) {
    const int64_t waves = (int64_t)(R / 8) * (8 / RPW);
    const int wpb = 4;
    dim3 grid((unsigned)((waves + wpb - 1) / wpb)), block(64 * wpb);
    if (type == TYPE_Q4_K)
        hipLaunchKernelGGL(k_gemv_q4k_f32<RPW>, grid, block, 0, s, w, x, y, R, G);
    else
        hipLaunchKernelGGL(k_gemv_q6k_f32<RPW>, grid, block, 0, s, w, x, y, R, G);
}

void launch_gemv_f32(const uint8_t* w, int R, int C, int type, const float* x, float* y,
                     int rows_per_wave, hipStream_t s) {
    const int G = C / QK;
    int rpw = rows_per_wave;
    if (rpw <= 0) {
        rpw = 4;
        while (rpw > 1 && (int64_t)(R / 8) * (8 / rpw) < 2048) rpw >>= 1;
    }
    switch (rpw) {
        case 1: launch_f32_rpw<1>(w, R, G, type, x, y, s); break;
        case 2: launch_f32_rpw<2>(w, R, G, type, x, y, s); break;
        case 4: launch_f32_rpw<4>(w, R, G, type, x, y, s); break;
        default: launch_f32_rpw<8>(w, R, G, type, x, y, s); break;
    }
}

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
