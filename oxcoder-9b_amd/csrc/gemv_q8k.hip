// Q4_K / Q6_K x Q8_K GEMV for gfx950 (batch-1 decode and small-batch speculative verify).
//
// Work split: one wave owns RPW consecutive rows of one 8-row tile; the wave walks the
// super-block columns 16 at a time (slot = lane >> 2, g = slot + 16*pass) with four lanes per
// super-block.  Each lane streams its share of every tile column with 16-byte loads (a Q4_K tile
// column is 1152 B = 9 cache lines, read once), keeps the RPW rows' quants in registers and runs
// them against each token's Q8_K activations with v_dot4_i32_i8.  Per (row, super-block) the four
// lanes' int32 partials are summed exactly (quad shuffle), turned into one fp32 value, and the
// values are reduced by the pairwise column tree of q4_lanes.h.  HBM traffic per call is the
// weight bytes once plus activations and outputs; activations are re-read from L1/L2 per row group.
#include "kq_device.h"
#include "kq_internal.h"
#include "q4_lanes.h"

namespace kq {

// ----------------------------------------------------------------------------- Q4_K
template <int NT, int RPW>
__global__ void __launch_bounds__(256)
k_gemv_q4k_q8k(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ, float* __restrict__ Y,
               int R, int G, int64_t ldy) {
    constexpr int WPT = 8 / RPW;  // waves per 8-row tile
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t tile = wave / WPT;
    if (tile >= R / 8) return;
    const int r0 = (int)(wave - tile * WPT) * RPW;
    const int p = lane & 3, slot = lane >> 2;
    const uint8_t* Wt = W + tile * (int64_t)G * (8 * Q4K_BYTES) + r0 * Q4K_BYTES;

    PassTree tree[NT][RPW];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < RPW; r++) tree_init(tree[t][r]);

    const int passes = (G + 15) >> 4;
    for (int pass = 0; pass < passes; pass++) {
        const int g = slot + 16 * pass;
        const bool valid = g < G;
        u32x4 hdr[RPW], qa[RPW], qb[RPW];
        if (valid) {
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const uint8_t* bk = Wt + (int64_t)g * (8 * Q4K_BYTES) + r * Q4K_BYTES;
                hdr[r] = ld16(bk);
                qa[r] = ld16(bk + 16 + 32 * p);
                qb[r] = ld16(bk + 32 + 32 * p);
            }
        } else {
#pragma unroll
            for (int r = 0; r < RPW; r++) hdr[r] = qa[r] = qb[r] = u32x4{0, 0, 0, 0};
        }
        ScMin sm[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) sm[r] = q4k_scmin_pair(hdr[r].y, hdr[r].z, hdr[r].w, p);

#pragma unroll
        for (int t = 0; t < NT; t++) {
            uint32_t xl[8], xh[8];
            float dx = 0.0f;
            int blo = 0, bhi = 0;
            if (valid) {
                const uint8_t* xb = XQ + ((int64_t)t * G + g) * Q8K_BYTES;
                dx = __builtin_bit_cast(float, ld4(xb));
                const u32x4 a0 = ld16_a4(xb + 4 + 64 * p), a1 = ld16_a4(xb + 20 + 64 * p);
                const u32x4 a2 = ld16_a4(xb + 36 + 64 * p), a3 = ld16_a4(xb + 52 + 64 * p);
                xl[0] = a0.x; xl[1] = a0.y; xl[2] = a0.z; xl[3] = a0.w;
                xl[4] = a1.x; xl[5] = a1.y; xl[6] = a1.z; xl[7] = a1.w;
                xh[0] = a2.x; xh[1] = a2.y; xh[2] = a2.z; xh[3] = a2.w;
                xh[4] = a3.x; xh[5] = a3.y; xh[6] = a3.z; xh[7] = a3.w;
                const uint32_t b01 = ld4(xb + 260 + 8 * p), b23 = ld4(xb + 264 + 8 * p);
                blo = shalf(b01, 0) + shalf(b01, 1);
                bhi = shalf(b23, 0) + shalf(b23, 1);
            } else {
#pragma unroll
                for (int k = 0; k < 8; k++) xl[k] = xh[k] = 0;
            }
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                int plo, phi;
                q4k_lane_dots(qa[r], qb[r], xl, xh, plo, phi);
                const int i1 = quad_sum_i32((int)sm[r].sc_lo * plo + (int)sm[r].sc_hi * phi);
                const int i2 = quad_sum_i32((int)sm[r].m_lo * blo + (int)sm[r].m_hi * bhi);
                const float v = valid ? q4k_value(hdr[r].x, dx, i1, i2) : 0.0f;
                tree_push(tree[t][r], slot_tree_f32(v));
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const float y = tree_final(tree[t][r]);
            if (lane == 0) Y[(int64_t)t * ldy + tile * 8 + r0 + r] = y;
        }
}

// ----------------------------------------------------------------------------- Q6_K
// Block bytes of row r start at an offset = 2r (mod 16) inside a 16-byte aligned tile column,
// so the lane fields (16 B each) are read with dword-aligned loads plus a funnel shift.  Every
// such read stays inside the 8-row tile column: the last field of a block ends at byte 192 and
// the scale/d window [192, 210) is read from the dword containing byte 192 or 190.
template <int NT, int RPW>
__global__ void __launch_bounds__(256)
k_gemv_q6k_q8k(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ, float* __restrict__ Y,
               int R, int G, int64_t ldy) {
    constexpr int WPT = 8 / RPW;
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t tile = wave / WPT;
    if (tile >= R / 8) return;
    const int r0 = (int)(wave - tile * WPT) * RPW;
    const int p = lane & 3, slot = lane >> 2;
    const int h = p >> 1, jj = p & 1;
    const uint8_t* Wt = W + tile * (int64_t)G * (8 * Q6K_BYTES) + r0 * Q6K_BYTES;

    PassTree tree[NT][RPW];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < RPW; r++) tree_init(tree[t][r]);

    const int passes = (G + 15) >> 4;
    for (int pass = 0; pass < passes; pass++) {
        const int g = slot + 16 * pass;
        const bool valid = g < G;
        u32x4 l0[RPW], l1[RPW], hb[RPW];
        int sc[RPW][4];
        float d[RPW];
        if (valid) {
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const uint8_t* bk = Wt + (int64_t)g * (8 * Q6K_BYTES) + r * Q6K_BYTES;
                l0[r] = ld16_a2(bk + h * 64 + 16 * jj);
                l1[r] = ld16_a2(bk + h * 64 + 32 + 16 * jj);
                hb[r] = ld16_a2(bk + 128 + h * 32 + 16 * jj);
                const u32x4 s = ld16_a2(bk + 192);       // 16 int8 scales
                const uintptr_t da = reinterpret_cast<uintptr_t>(bk + 208);
                const uint32_t dw = ld4(reinterpret_cast<const uint8_t*>(da & ~uintptr_t(3)));
                d[r] = f16_lo(dw >> (8 * (da & 3)));
                const uint32_t w0 = h ? s.z : s.x, w1 = h ? s.w : s.y;   // scales 8h .. 8h+7
                sc[r][0] = sbyte(w0, jj);
                sc[r][1] = sbyte(w0, jj + 2);
                sc[r][2] = sbyte(w1, jj);
                sc[r][3] = sbyte(w1, jj + 2);
            }
        } else {
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                l0[r] = l1[r] = hb[r] = u32x4{0, 0, 0, 0};
                sc[r][0] = sc[r][1] = sc[r][2] = sc[r][3] = 0;
                d[r] = 0.0f;
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            uint32_t xa[16];
            int corr[4];
            float dx = 0.0f;
            if (valid) {
                const uint8_t* xb = XQ + ((int64_t)t * G + g) * Q8K_BYTES;
                dx = __builtin_bit_cast(float, ld4(xb));
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const u32x4 a = ld16_a4(xb + 4 + h * 128 + k * 32 + 16 * jj);
                    xa[4 * k + 0] = a.x; xa[4 * k + 1] = a.y; xa[4 * k + 2] = a.z; xa[4 * k + 3] = a.w;
                }
                // bsums of sub-blocks 8h + 2k + jj, k = 0..3 (dword k of bsums[8h..8h+7])
                const u32x4 bs = ld16_a4(xb + 260 + 16 * h);
                corr[0] = 32 * shalf(bs.x, jj);
                corr[1] = 32 * shalf(bs.y, jj);
                corr[2] = 32 * shalf(bs.z, jj);
                corr[3] = 32 * shalf(bs.w, jj);
            } else {
#pragma unroll
                for (int k = 0; k < 16; k++) xa[k] = 0;
                corr[0] = corr[1] = corr[2] = corr[3] = 0;
            }
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                int P[4];
                q6k_lane_dots(l0[r], l1[r], hb[r], xa, P);
                int I = sc[r][0] * (P[0] - corr[0]);
                I += sc[r][1] * (P[1] - corr[1]);
                I += sc[r][2] * (P[2] - corr[2]);
                I += sc[r][3] * (P[3] - corr[3]);
                I = quad_sum_i32(I);
                const float v = valid ? q6k_value(d[r], dx, I) : 0.0f;
                tree_push(tree[t][r], slot_tree_f32(v));
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const float y = tree_final(tree[t][r]);
            if (lane == 0) Y[(int64_t)t * ldy + tile * 8 + r0 + r] = y;
        }
}

// ----------------------------------------------------------------------------- launch
template <int NT, int RPW>
static void launch_nt(const uint8_t* w, int R, int G, int type, const uint8_t* xq, float* y,
                      int64_t ldy, hipStream_t s) {
    const int64_t waves = (int64_t)(R / 8) * (8 / RPW);
    const int wpb = 4;
    dim3 grid((unsigned)((waves + wpb - 1) / wpb)), block(64 * wpb);
    if (type == TYPE_Q4_K)
        hipLaunchKernelGGL((k_gemv_q4k_q8k<NT, RPW>), grid, block, 0, s, w, xq, y, R, G, ldy);
    else
        hipLaunchKernelGGL((k_gemv_q6k_q8k<NT, RPW>), grid, block, 0, s, w, xq, y, R, G, ldy);
}

template <int NT>
static void launch_rpw(const uint8_t* w, int R, int G, int type, const uint8_t* xq, float* y,
                       int64_t ldy, int rpw, hipStream_t s) {
    switch (rpw) {
        case 1: launch_nt<NT, 1>(w, R, G, type, xq, y, ldy, s); break;
        case 2: launch_nt<NT, 2>(w, R, G, type, xq, y, ldy, s); break;
        case 4: launch_nt<NT, 4>(w, R, G, type, xq, y, ldy, s); break;
        default: launch_nt<NT, 8>(w, R, G, type, xq, y, ldy, s); break;
    }
}

// Rows per wave: enough waves to cover the chip (>= 2048) for the given row count, and a
// register budget of NT*RPW <= 16 outputs per lane.
static int pick_rpw(int R, int nt) {
    int rpw = 8;
    while (rpw > 1 && ((int64_t)(R / 8) * (8 / rpw) < 2048 || nt * rpw > 16)) rpw >>= 1;
    return rpw;
}

void launch_gemv_q8k(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int N, float* y,
                     int64_t ldy, int rows_per_wave, hipStream_t s) {
    const int G = C / QK;
    // Tokens go in groups of up to 4 per launch; each group is an independent launch over the
    // same weights, so every token's arithmetic is the same as in a single-token call.
    for (int n0 = 0; n0 < N; n0 += 4) {
        const int nt = N - n0 < 4 ? N - n0 : 4;
        const int rpw = rows_per_wave > 0 ? rows_per_wave : pick_rpw(R, nt);
        const uint8_t* xg = xq + (int64_t)n0 * G * Q8K_BYTES;
        float* yg = y + (int64_t)n0 * ldy;
        switch (nt) {
            case 1: launch_rpw<1>(w, R, G, type, xg, yg, ldy, rpw, s); break;
            case 2: launch_rpw<2>(w, R, G, type, xg, yg, ldy, rpw, s); break;
            case 3: launch_rpw<3>(w, R, G, type, xg, yg, ldy, rpw, s); break;
            default: launch_rpw<4>(w, R, G, type, xg, yg, ldy, rpw, s); break;
        }
    }
}

}  // namespace kq
